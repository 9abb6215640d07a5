"""StateTune training recurrence, importable as ``flashrwkv2.tmix.wkv7.statetune``.

``statetune_recurrent_fp32io16`` keeps the reference's signature, error
contract and outputs ``(y, S_T, boundary, state_dot_a)`` (reference
``flashrwkv2/tmix/wkv7/statetune.py:11-236``). Head size 64 runs the chunked
bf16-MFMA kernels, 128 the bf16-MFMA kernels over 16-token pieces, 256 the
per-token fp32 training kernels; every backward recomputes each chunk from
stored states instead of dividing by the decay.

Caller chunks may have any length. The kernels walk a chunk in pieces of P
tokens (P = 64 at head size 64, 16 at 128 and 256); the forward keeps the
state at each interior piece start in a buffer indexed by (piece start) / P,
which the backward reads. That buffer holds ceil(N / P) x H x D x D fp32
values from the forward to the backward (16 KiB per 64 token-heads at D = 64,
64 KiB per 16 token-heads at D = 128, 256 KiB at D = 256) whether or not a
chunk is longer than P. Callers whose chunks never exceed P tokens pass
``max_chunk_len`` to ``statetune_recurrent_internal``: the forward then keeps
no buffer, and the backward recomputes any interior state it needs into a
temporary workspace, so a wrong hint costs time, never correctness.

Nothing reads the chunk metadata on the host, so a training step never
synchronises. It does not run under HIP graph capture: the chunked kernels are
not validated inside a captured graph, and the operator raises RuntimeError
when called on a capturing stream.
"""

from __future__ import annotations

import torch

from ... import _contract as C
from ..._contract import Each, check
from . import DECAY_LOGITS, DECAY_RAW_W

_METADATA_NAMES = ("sequence_chunk_offsets", "chunk_token_starts", "chunk_token_ends")


def _cuda(arg: str | None) -> tuple:
    return (
        C.is_tensor(arg),
        check(arg, C.cuda_contiguous, ValueError, "{name} must be contiguous CUDA"),
    )


# Reference ``statetune.py:41-76``.
TOKENS = (
    *_cuda("state"),
    check("state", C.dtype_is(torch.float32), TypeError, "state must be float32"),
    check("state", lambda x, ns: x.ndim == 4 and x.shape[0] > 0 and x.shape[1] > 0,
          ValueError, "state must have shape [B,H,D,D]"),
    check("state", lambda x, ns: x.shape[2] == x.shape[3] and x.shape[2] in (64, 128, 256),
          ValueError, "state head size must be 64, 128, or 256"),
    Each(C.PACKED_TOKENS, (
        *_cuda(None),
        check(None, C.same_device_as("state"), ValueError, "{name} must share the state device"),
        check(None, C.dtype_is(torch.float16, torch.bfloat16), TypeError,
              "{name} must be float16 or bfloat16"),
        check(None, C.same_shape_as("r"), ValueError, "{name} must match r shape"),
    )),
    check("r", lambda x, ns: x.ndim == 3 and x.shape[0] > 0
          and x.shape[1:] == ns["state"].shape[1:3], ValueError,
          "token tensors must have shape [total_tokens,H,D]"),
)

# Reference ``statetune.py:19-38`` plus the entry's own checks (``:224-229``).
METADATA = (
    Each(_METADATA_NAMES, (
        *_cuda(None),
        check(None, C.dtype_is(torch.int32), TypeError, "{name} must be int32"),
        check(None, C.same_device_as("state"), ValueError, "{name} must share the state device"),
    )),
    check("sequence_chunk_offsets", C.ndim_is(1), ValueError,
          "sequence_chunk_offsets must be one-dimensional"),
    check("chunk_token_starts", lambda x, ns: x.ndim == 1
          and ns["chunk_token_ends"].shape == x.shape, ValueError,
          "chunk token metadata must have matching shape [C]"),
    check("chunk_token_starts", lambda x, ns: x.numel() > 0, ValueError,
          "at least one training chunk is required"),
    check("sequence_chunk_offsets", lambda x, ns: x.numel() == ns["state"].shape[0] + 1,
          ValueError, "sequence_chunk_offsets must have shape [B+1]"),
    check("scale", C.finite_number, ValueError, "scale must be finite"),
)


def _piece_len(head_size: int) -> int:
    """Piece length of the training kernels for this head size."""
    return 64 if head_size == 64 else 16


def _interior(r: torch.Tensor, heads: int, d: int,
              max_chunk_len: int | None) -> torch.Tensor | None:
    """Buffer for the interior piece-start states: ceil(N / P) slots of
    [D, D] fp32 (bf16 at head size 128, in the kernels' own order), as a flat
    float32 tensor, or None when the caller states that no chunk is longer than
    one piece."""
    p = _piece_len(d)
    if max_chunk_len is not None and max_chunk_len <= p:
        return None
    slots = (r.shape[0] + p - 1) // p
    elems = slots * heads * d * d
    if d == 128:
        elems //= 2
    return torch.empty((elems,), device=r.device, dtype=torch.float32)


class _StateTune(torch.autograd.Function):
    """Forward keeps the chunk-start and interior piece-start states; backward
    recomputes each piece from them (reference ``statetune.py:79-199``
    divides by the decay instead)."""

    @staticmethod
    def forward(ctx, initial_state, offsets, starts, ends, r, decay, k, v, a, b, scale,
                decay_mode, max_chunk_len):
        state = initial_state.detach().contiguous().clone()
        heads, d = state.shape[1], state.shape[2]
        boundary = torch.empty((starts.numel(), heads, d, d), device=state.device,
                               dtype=torch.float32)
        interior = _interior(r, heads, d, max_chunk_len)
        output = torch.empty_like(v)
        state_dot_a = torch.empty_like(r, dtype=torch.float32)
        C.native().statetune_forward_internal(offsets, starts, ends, state, r, decay, k, v, a, b,
                                              output, boundary, state_dot_a, interior,
                                              float(scale), int(decay_mode))
        ctx.save_for_backward(offsets, starts, ends, r, decay, k, v, a, b, boundary, interior)
        ctx.scale, ctx.decay_mode = float(scale), int(decay_mode)
        ctx.mark_non_differentiable(boundary, state_dot_a)
        # Outputs without a gradient reach backward as None instead of zero
        # tensors: boundary and state_dot_a are 16 KiB per chunk-head and 256 B
        # per token-head, whose zero fills would cost more HBM traffic than the
        # backward's own gradient writes; a None dY or dS_T is a zero input
        # of the backward kernel.
        ctx.set_materialize_grads(False)
        return output, state, boundary, state_dot_a

    @staticmethod
    def backward(ctx, grad_output, grad_final_state, _grad_boundary, _grad_state_dot_a):
        offsets, starts, ends, r, decay, k, v, a, b, boundary, interior = ctx.saved_tensors
        grads = [torch.empty_like(t) for t in (r, decay, k, v, a, b)]
        d = r.shape[2]
        grad_state = torch.empty((offsets.numel() - 1, r.shape[1], d, d), device=r.device,
                                 dtype=torch.float32)
        dy = None if grad_output is None else grad_output.contiguous()
        ds = None if grad_final_state is None else grad_final_state.contiguous().float()
        C.native().statetune_backward_internal(offsets, starts, ends, r, decay, k, v, a, b, dy,
                                               ds, boundary, *grads, grad_state, interior,
                                               ctx.scale, ctx.decay_mode)
        return (grad_state, None, None, None, *grads, None, None, None)


def _run(ns: dict, decay_mode: int):
    C.enforce(TOKENS, ns)
    C.enforce(METADATA, ns)
    max_chunk_len = ns.get("max_chunk_len")
    if max_chunk_len is not None and not (isinstance(max_chunk_len, int)
                                          and not isinstance(max_chunk_len, bool)
                                          and max_chunk_len > 0):
        raise ValueError("max_chunk_len must be a positive integer or None")
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError("statetune_recurrent_fp32io16 does not run under HIP graph "
                           "capture: its chunked kernels are not validated inside a "
                           "captured graph; run the training step eagerly")
    return _StateTune.apply(ns["state"], *(ns[n] for n in _METADATA_NAMES),
                            *(ns[n] for n in C.PACKED_TOKENS), float(ns["scale"]), decay_mode,
                            max_chunk_len)


def statetune_recurrent_fp32io16(initial_state, sequence_chunk_offsets, chunk_token_starts,
                                 chunk_token_ends, r, decay_logits, k, v, a, b, *,
                                 scale: float = 1.0):
    """StateTune with a nonzero initial state and its gradient.

    Reference ``statetune.py:202-236``. Returns ``(y, final_state, boundary,
    state_dot_a)``; ``boundary`` and ``state_dot_a`` are not differentiable.
    """
    ns = dict(locals())
    ns["state"] = ns.pop("initial_state")
    return _run(ns, DECAY_LOGITS)


def statetune_recurrent_internal(initial_state, sequence_chunk_offsets, chunk_token_starts,
                                 chunk_token_ends, r, decay, k, v, a, b, *,
                                 scale: float = 1.0, decay_mode: int = DECAY_RAW_W,
                                 max_chunk_len: int | None = None):
    """StateTune with an explicit decay mode (not reference API):
    ``DECAY_RAW_W`` takes the retention itself, and its gradient is dL/dw.
    ``max_chunk_len`` is an optional upper bound on the chunk lengths: at or
    below the kernels' piece length (64 tokens at head size 64, 16 at 128 and
    256) the forward keeps no interior-state buffer for the backward."""
    if decay_mode not in (DECAY_LOGITS, DECAY_RAW_W):
        raise ValueError("decay_mode must be DECAY_LOGITS or DECAY_RAW_W")
    ns = dict(locals())
    ns["state"] = ns.pop("initial_state")
    ns["decay_logits"] = ns.pop("decay")
    return _run(ns, int(decay_mode))


__all__ = ["statetune_recurrent_fp32io16"]
