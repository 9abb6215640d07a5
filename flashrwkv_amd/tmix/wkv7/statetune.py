"""StateTune training recurrence, mirroring ``flashrwkv2.tmix.wkv7.statetune``.

``statetune_recurrent_fp32io16`` keeps the reference's signature, validation
(error types and messages) and outputs ``(y, S_T, boundary, state_dot_a)``
(reference ``flashrwkv2/tmix/wkv7/statetune.py:11-236``). Head size 64 runs
the chunked bf16-MFMA kernels, 128 and 256 the per-token fp32 training
kernels; either backward recomputes every chunk from the stored boundary
states instead of dividing by the decay.

The backward kernels work on chunks of at most 64 tokens (head size 64) or 16
tokens (128, 256). Caller chunks that are longer are split internally (one
device-to-host copy of the chunk metadata per forward); the boundary output
still holds the state at each caller chunk start.
"""

from __future__ import annotations

import math

import torch

from . import DECAY_LOGITS, DECAY_RAW_W, _extension


def _kernel_chunk(head_size: int) -> int:
    """Longest chunk the backward kernels take for this head size."""
    return 64 if head_size == 64 else 16


def _check_cuda_contiguous(tensor: torch.Tensor, name: str) -> None:
    if not isinstance(tensor, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if not tensor.is_cuda or not tensor.is_contiguous():
        raise ValueError(f"{name} must be contiguous CUDA")


def _check_metadata(sequence_chunk_offsets, chunk_token_starts, chunk_token_ends, state):
    """Reference ``statetune.py:19-38``."""
    for name, tensor in (
        ("sequence_chunk_offsets", sequence_chunk_offsets),
        ("chunk_token_starts", chunk_token_starts),
        ("chunk_token_ends", chunk_token_ends),
    ):
        _check_cuda_contiguous(tensor, name)
        if tensor.dtype != torch.int32:
            raise TypeError(f"{name} must be int32")
        if tensor.device != state.device:
            raise ValueError(f"{name} must share the state device")
    if sequence_chunk_offsets.ndim != 1:
        raise ValueError("sequence_chunk_offsets must be one-dimensional")
    if chunk_token_starts.ndim != 1 or chunk_token_ends.shape != chunk_token_starts.shape:
        raise ValueError("chunk token metadata must have matching shape [C]")
    if chunk_token_starts.numel() == 0:
        raise ValueError("at least one training chunk is required")


def _check_token_inputs(state, r, decay_logits, k, v, a, b) -> None:
    """Reference ``statetune.py:41-76``."""
    _check_cuda_contiguous(state, "state")
    if state.dtype != torch.float32:
        raise TypeError("state must be float32")
    if state.ndim != 4 or state.shape[0] <= 0 or state.shape[1] <= 0:
        raise ValueError("state must have shape [B,H,D,D]")
    if state.shape[2] != state.shape[3] or state.shape[2] not in (64, 128, 256):
        raise ValueError("state head size must be 64, 128, or 256")
    tensors = {"r": r, "decay_logits": decay_logits, "k": k, "v": v, "a": a, "b": b}
    for name, tensor in tensors.items():
        _check_cuda_contiguous(tensor, name)
        if tensor.device != state.device:
            raise ValueError(f"{name} must share the state device")
        if tensor.dtype not in (torch.float16, torch.bfloat16):
            raise TypeError(f"{name} must be float16 or bfloat16")
        if tensor.shape != r.shape:
            raise ValueError(f"{name} must match r shape")
    if r.ndim != 3 or r.shape[0] <= 0 or r.shape[1:] != state.shape[1:3]:
        raise ValueError("token tensors must have shape [total_tokens,H,D]")


def _kernel_chunks(sequence_chunk_offsets, chunk_token_starts, chunk_token_ends, limit):
    """Kernel chunk metadata (chunks of at most ``limit`` tokens).

    Returns ``(offsets, starts, ends, first)`` where ``first[c]`` is the
    kernel chunk that starts caller chunk ``c``, or ``None`` when every
    caller chunk already fits (then the caller metadata is used as is).
    """
    starts = chunk_token_starts.cpu()
    ends = chunk_token_ends.cpu()
    if int((ends - starts).max()) <= limit:
        return None
    offsets = sequence_chunk_offsets.cpu().tolist()
    starts, ends = starts.tolist(), ends.tolist()
    k_off, k_start, k_end, first = [0], [], [], []
    for seq in range(len(offsets) - 1):
        for c in range(offsets[seq], offsets[seq + 1]):
            first.append(len(k_start))
            s, e = starts[c], ends[c]
            if e <= s:
                k_start.append(s)
                k_end.append(s)
            for t in range(s, e, limit):
                k_start.append(t)
                k_end.append(min(t + limit, e))
        k_off.append(len(k_start))
    dev = sequence_chunk_offsets.device

    def as_tensor(values):
        return torch.tensor(values, dtype=torch.int32, device=dev)

    return as_tensor(k_off), as_tensor(k_start), as_tensor(k_end), as_tensor(first)


class _StateTune(torch.autograd.Function):
    """Reference ``statetune.py:79-199`` with a recompute-based backward."""

    @staticmethod
    def forward(ctx, initial_state, sequence_chunk_offsets, chunk_token_starts,
                chunk_token_ends, r, decay, k, v, a, b, scale, decay_mode):
        state = initial_state.detach().contiguous().clone()
        output = torch.empty_like(v)
        n_chunks = chunk_token_starts.numel()
        heads, d = state.shape[1], state.shape[2]
        state_dot_a = torch.empty_like(r, dtype=torch.float32)
        split = _kernel_chunks(sequence_chunk_offsets, chunk_token_starts, chunk_token_ends,
                               _kernel_chunk(d))
        if split is None:
            meta = (sequence_chunk_offsets, chunk_token_starts, chunk_token_ends)
            checkpoint = torch.empty((n_chunks, heads, d, d), device=state.device,
                                     dtype=torch.float32)
        else:
            meta = split[:3]
            checkpoint = torch.empty((split[1].numel(), heads, d, d), device=state.device,
                                     dtype=torch.float32)
        _extension().statetune_forward_internal(
            *meta, state, r, decay, k, v, a, b, output, checkpoint, state_dot_a,
            float(scale), int(decay_mode))
        boundary = checkpoint if split is None else checkpoint.index_select(0, split[3])
        ctx.save_for_backward(*meta, r, decay, k, v, a, b, checkpoint)
        ctx.scale = float(scale)
        ctx.decay_mode = int(decay_mode)
        ctx.mark_non_differentiable(boundary, state_dot_a)
        return output, state, boundary, state_dot_a

    @staticmethod
    def backward(ctx, grad_output, grad_final_state, _grad_boundary, _grad_state_dot_a):
        offsets, starts, ends, r, decay, k, v, a, b, checkpoint = ctx.saved_tensors
        grads = [torch.empty_like(t) for t in (r, decay, k, v, a, b)]
        batch = offsets.numel() - 1
        grad_state = torch.empty((batch, r.shape[1], r.shape[2], r.shape[2]), device=r.device,
                                 dtype=torch.float32)
        dy = None if grad_output is None else grad_output.contiguous()
        ds = None if grad_final_state is None else grad_final_state.contiguous().float()
        _extension().statetune_backward_internal(
            offsets, starts, ends, r, decay, k, v, a, b, dy, ds, checkpoint, *grads,
            grad_state, ctx.scale, ctx.decay_mode)
        return (grad_state, None, None, None, *grads, None, None)


def statetune_recurrent_fp32io16(initial_state, sequence_chunk_offsets, chunk_token_starts,
                                 chunk_token_ends, r, decay_logits, k, v, a, b, *,
                                 scale: float = 1.0):
    """Run StateTune with a nonzero state and direct initial-state gradient.

    Reference ``statetune.py:202-236``. Returns ``(y, final_state, boundary,
    state_dot_a)``; ``boundary`` and ``state_dot_a`` are not differentiable.
    """
    _check_token_inputs(initial_state, r, decay_logits, k, v, a, b)
    _check_metadata(sequence_chunk_offsets, chunk_token_starts, chunk_token_ends,
                    initial_state)
    if sequence_chunk_offsets.numel() != initial_state.shape[0] + 1:
        raise ValueError("sequence_chunk_offsets must have shape [B+1]")
    if not isinstance(scale, (int, float)) or not math.isfinite(float(scale)):
        raise ValueError("scale must be finite")
    return _StateTune.apply(initial_state, sequence_chunk_offsets, chunk_token_starts,
                            chunk_token_ends, r, decay_logits, k, v, a, b, float(scale),
                            DECAY_LOGITS)


def statetune_recurrent_internal(initial_state, sequence_chunk_offsets, chunk_token_starts,
                                 chunk_token_ends, r, decay, k, v, a, b, *,
                                 scale: float = 1.0, decay_mode: int = DECAY_RAW_W):
    """StateTune with an explicit decay mode (``DECAY_RAW_W`` takes the
    retention itself; its gradient is dL/dw). Not part of the reference API."""
    _check_token_inputs(initial_state, r, decay, k, v, a, b)
    _check_metadata(sequence_chunk_offsets, chunk_token_starts, chunk_token_ends,
                    initial_state)
    if sequence_chunk_offsets.numel() != initial_state.shape[0] + 1:
        raise ValueError("sequence_chunk_offsets must have shape [B+1]")
    if decay_mode not in (DECAY_LOGITS, DECAY_RAW_W):
        raise ValueError("decay_mode must be DECAY_LOGITS or DECAY_RAW_W")
    return _StateTune.apply(initial_state, sequence_chunk_offsets, chunk_token_starts,
                            chunk_token_ends, r, decay, k, v, a, b, float(scale),
                            int(decay_mode))


__all__ = ["statetune_recurrent_fp32io16"]
