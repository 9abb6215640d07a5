"""WKV7 operators (MI355X-native), importable as ``flashrwkv2.tmix.wkv7``.

The public functions keep the names, keyword arguments, return values and
error contract of the reference's ``flashrwkv2/tmix/wkv7/__init__.py``
(cited per function). Argument checks are the contract tables below, run by
:func:`flashrwkv_amd._contract.enforce`; the work goes through
``flashrwkv_amd._C`` into hand-written gfx950 HIP kernels. There is no CPU or
Python fallback: without the native library every operator raises
RuntimeError.
"""

from __future__ import annotations

import torch

from ... import _contract as C
from ..._contract import Each, check, is_tensor

DECAY_LOGITS = 0
DECAY_RAW_W = 1

# Reference name of the native-facade accessor (``__init__.py:8-17``).
_extension = C.native

# ------------------------------------------------------------------ tables
_TOKENS = Each(C.PACKED_TOKENS, (
    is_tensor(),
    check(None, C.ndim_is(3), ValueError, "{name} must have packed shape [total_tokens,H,D]"),
    check(None, C.contiguous, ValueError, "{name} must be contiguous"),
))


def _pool_rules(dtype: torch.dtype, dtype_message: str) -> tuple:
    return (
        is_tensor("state_pool"),
        check("state_pool", C.contiguous, ValueError, "state_pool must be contiguous"),
        check("state_pool", C.dtype_is(dtype), TypeError, dtype_message),
    )


# fp32-state recurrence (reference ``__init__.py:20-38, 200-242``).
RECURRENT_FP32 = (
    _TOKENS,
    *_pool_rules(torch.float32, "state_pool must have dtype float32"),
    *C.METADATA,
)

# fp16-state recurrence (reference ``__init__.py:41-62, 280-330``).
RECURRENT_FP16 = (
    _TOKENS,
    *_pool_rules(torch.float16, "FP16-state state_pool must have dtype float16"),
    is_tensor("elapsed_state_pool"),
    check("elapsed_state_pool", C.dtype_is(torch.int32), TypeError,
          "elapsed_state_pool must have dtype torch.int32"),
    check("elapsed_state_pool", C.cuda_contiguous, ValueError,
          "elapsed_state_pool must be contiguous CUDA int32"),
    check("elapsed_state_pool", C.same_device_as("state_pool"), ValueError,
          "elapsed_state_pool must share state_pool's device"),
    check("elapsed_state_pool",
          lambda x, ns: x.ndim == 1 and x.shape[0] == ns["state_pool"].shape[0], ValueError,
          "elapsed_state_pool must have shape [state_pool_slots]"),
    *C.METADATA,
    C.when(lambda ns: ns["max_seqlen"] is not None,
           check("max_seqlen", C.positive_int, ValueError,
                 "max_seqlen must be a positive integer")),
)

# elapsed-phase advance (reference ``__init__.py:65-81``).
ADVANCE = (
    is_tensor("elapsed_state"),
    check("elapsed_state", C.dtype_is(torch.int32), TypeError,
          "elapsed_state must have dtype torch.int32"),
    check("elapsed_state", C.cuda_contiguous, ValueError,
          "elapsed_state must be contiguous CUDA int32"),
    check("elapsed_state", lambda x, ns: x.numel() > 0, ValueError,
          "elapsed_state must be non-empty"),
    check("amount", C.plain_int, TypeError, "amount must be an int"),
)


def _int32_cuda(x, ns) -> bool:
    return x.dtype == torch.int32 and x.is_cuda and x.is_contiguous()


# varlen elapsed-phase advance (reference ``__init__.py:83-130``).
ADVANCE_VARLEN = (
    is_tensor("elapsed_state_pool"),
    check("elapsed_state_pool",
          lambda x, ns: _int32_cuda(x, ns) and x.ndim == 1 and x.numel() > 0, ValueError,
          "elapsed_state_pool must be non-empty contiguous CUDA int32"),
    *C.METADATA,
    check("cu_seqlens", _int32_cuda, ValueError, "cu_seqlens must be contiguous CUDA int32"),
    check("state_indices", _int32_cuda, ValueError,
          "state_indices must be contiguous CUDA int32"),
    check(None, lambda _, ns: (ns["cu_seqlens"].device == ns["elapsed_state_pool"].device
                               and ns["state_indices"].device
                               == ns["elapsed_state_pool"].device), ValueError,
          "elapsed metadata tensors must share a CUDA device"),
    check(None, lambda _, ns: (ns["cu_seqlens"].ndim == 1 and ns["state_indices"].ndim == 1
                               and ns["cu_seqlens"].numel()
                               == ns["state_indices"].numel() + 1), ValueError,
          "cu_seqlens must have shape [B+1] and state_indices shape [B]"),
    check("total_tokens", C.positive_int, ValueError,
          "total_tokens must be a positive integer"),
)

# fp16 add-vector helper (reference ``__init__.py:133-151``).
ADD_VEC = (
    Each(("x", "vec"), (
        is_tensor(),
        check(None, C.dtype_is(torch.float16), TypeError,
              "{name} must have dtype torch.float16"),
        check(None, C.cuda_contiguous, ValueError, "{name} must be contiguous CUDA float16"),
        check(None, C.same_device_as("x"), ValueError, "{name} must share x's device"),
    )),
    check("x", lambda x, ns: C.packed_rows(x, ns) and x.shape[1] % 2 == 0, ValueError,
          "x must have packed shape [total_tokens,C] with even C"),
    check("vec", lambda x, ns: x.shape == (ns["x"].shape[1],), ValueError,
          "vec must have shape [C]"),
)


# ------------------------------------------------------------------ entries
def _max_seqlen_arg(max_seqlen: int | None) -> int:
    return -1 if max_seqlen is None else int(max_seqlen)


def prepare_recurrent_metadata(
    cu_seqlens: torch.Tensor,
    state_indices: torch.Tensor,
    *,
    total_tokens: int,
    state_pool_size: int,
    max_seqlen: int | None = None,
) -> object:
    """Validate packed metadata once and return a reusable native ticket.

    Reference ``__init__.py:180-197``. The ticket pins the metadata tensors
    (identity, data pointer, shape, version), the launch sizes, the device and
    the current stream; reusing it after any of these change raises
    RuntimeError. With a ticket, launches neither validate nor synchronise.
    """
    C.enforce(C.METADATA, {"cu_seqlens": cu_seqlens, "state_indices": state_indices})
    return C.native().prepare_recurrent_metadata(
        cu_seqlens, state_indices, total_tokens, state_pool_size,
        _max_seqlen_arg(max_seqlen))


def _ticket_for(validated_metadata, cu_seqlens, state_indices, total_tokens, slots,
                max_seqlen):
    if validated_metadata is not None:
        return validated_metadata
    return prepare_recurrent_metadata(cu_seqlens, state_indices, total_tokens=total_tokens,
                                      state_pool_size=slots, max_seqlen=max_seqlen)


def _recurrent_fp32(ns: dict, decay_mode: int | None) -> torch.Tensor:
    C.enforce(RECURRENT_FP32, ns)
    pool, r = ns["state_pool"], ns["r"]
    ticket = _ticket_for(ns["validated_metadata"], ns["cu_seqlens"], ns["state_indices"],
                         r.shape[0], pool.shape[0], ns["max_seqlen"])
    tokens = tuple(ns[name] for name in C.PACKED_TOKENS)
    output = torch.empty_like(ns["v"])
    facade = C.native()
    common = (ns["cu_seqlens"], ns["state_indices"], pool, *tokens, output, float(ns["scale"]))
    if decay_mode is None:
        facade.recurrent_fp32_from_decay_logits(*common, ns["decay_bias"], ticket,
                                                _max_seqlen_arg(ns["max_seqlen"]))
    else:
        facade.recurrent_fp32_forward_internal(*common, int(decay_mode), ns["decay_bias"],
                                               ticket, _max_seqlen_arg(ns["max_seqlen"]))
    return output


# Routes of long sequences in the fp32-state recurrent op (not reference API).
LONG_ROUTE_CHUNKED = "chunked"
LONG_ROUTE_PER_TOKEN = "per_token"
_ROUTE_CODES = {LONG_ROUTE_CHUNKED: 0, LONG_ROUTE_PER_TOKEN: 1}


def set_recurrent_long_route(route: str) -> str:
    """Choose how ``infer_recurrent_fp32io16_forward_varlen`` runs long calls.

    Not reference API. Calls with bf16 tokens, head size 64 and a longest
    sequence of 64 tokens or more run, by default (``"chunked"``), on the
    split-precision chunk kernel: its outputs meet the reference's
    relative-RMSE gate of 0.002, but the pool it leaves differs from the
    per-token fp32 recurrence by about 4e-4 relative RMSE (1e-7 on the
    per-token kernel). ``"per_token"`` runs every call on the per-token fp32
    kernel, as the reference computes it, at several times the time for long
    sequences. Decode, short sequences, fp16 tokens and other head sizes run
    the per-token kernel either way, and so does any call made under HIP
    graph capture. The setting is process-wide; returns the previous route.
    """
    if route not in _ROUTE_CODES:
        raise ValueError(f"route must be one of {sorted(_ROUTE_CODES)}, got {route!r}")
    previous = C.native().set_recurrent_long_route(_ROUTE_CODES[route])
    return LONG_ROUTE_PER_TOKEN if previous == 1 else LONG_ROUTE_CHUNKED


def recurrent_long_route() -> str:
    """The current route of long calls (see :func:`set_recurrent_long_route`)."""
    return LONG_ROUTE_PER_TOKEN if C.native().recurrent_long_route() == 1 else LONG_ROUTE_CHUNKED


def infer_recurrent_fp32io16_forward_varlen(
    r: torch.Tensor,
    decay_logits: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    *,
    state_pool: torch.Tensor,
    cu_seqlens: torch.Tensor,
    state_indices: torch.Tensor,
    scale: float = 1.0,
    decay_bias: torch.Tensor | None = None,
    max_seqlen: int | None = None,
    validated_metadata: object | None = None,
) -> torch.Tensor:
    """Packed RWKV-7 recurrence from raw decay logits, state pool in place.

    Reference ``__init__.py:245-277``: fp16/bf16 ``[N,H,D]`` tokens, fp32
    ``[slots,H,D,D]`` pool ([K,V]) updated at ``state_indices``; returns the
    output shaped like ``v``.
    """
    return _recurrent_fp32(dict(locals()), None)


def recurrent_forward_internal(
    r: torch.Tensor,
    decay: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    *,
    state_pool: torch.Tensor,
    cu_seqlens: torch.Tensor,
    state_indices: torch.Tensor,
    decay_mode: int = DECAY_RAW_W,
    scale: float = 1.0,
    decay_bias: torch.Tensor | None = None,
    max_seqlen: int | None = None,
    validated_metadata: object | None = None,
) -> torch.Tensor:
    """fp32-state recurrence with an explicit decay mode (not reference API).

    ``decay_mode=DECAY_RAW_W`` takes the retention ``w`` itself (needed for
    retentions below the logits floor ``exp(-e^{-1/2})``), and fp32 tokens are
    accepted (the public op rejects them, reference ``csrc/validation.cpp:100-103``).
    """
    ns = dict(locals())
    ns["decay_logits"] = ns.pop("decay")
    return _recurrent_fp32(ns, decay_mode)


def infer_recurrent_fp16_forward_varlen(
    r: torch.Tensor,
    decay_logits: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    *,
    state_pool: torch.Tensor,
    elapsed_state_pool: torch.Tensor,
    cu_seqlens: torch.Tensor,
    state_indices: torch.Tensor,
    scale: float = 1.0,
    decay_bias: torch.Tensor | None = None,
    max_seqlen: int | None = None,
    validated_metadata: object | None = None,
) -> torch.Tensor:
    """Packed recurrence with an fp16 state pool (the Albatross family).

    Reference ``__init__.py:280-339``: fp16 ``[N,H,D]`` tokens and decay
    logits, fp16 ``[slots,H,D,D]`` pool ([K,V]) updated at ``state_indices``,
    int32 ``elapsed_state_pool`` phase origins (read, not advanced); returns
    the fp16 output shaped like ``v``. Without ``max_seqlen`` the ticket
    infers it, so a launch never reads the offsets on the host.
    """
    ns = dict(locals())
    C.enforce(RECURRENT_FP16, ns)
    ticket = _ticket_for(validated_metadata, cu_seqlens, state_indices, r.shape[0],
                         state_pool.shape[0], max_seqlen)
    output = torch.empty_like(v)
    C.native().recurrent_fp16_from_decay_logits(
        cu_seqlens, state_indices, elapsed_state_pool, state_pool,
        *(ns[name] for name in C.PACKED_TOKENS), output, float(scale), decay_bias, ticket,
        _max_seqlen_arg(max_seqlen))
    return output


def infer_recurrent_fp16_advance_i32(elapsed_state: torch.Tensor, amount: int) -> None:
    """Advance fp16-state phase origins in place by ``amount`` (int32, wrapping).

    Reference ``__init__.py:65-81``.
    """
    C.enforce(ADVANCE, {"elapsed_state": elapsed_state, "amount": amount})
    C.native().recurrent_fp16_advance_i32(elapsed_state, amount)


def infer_recurrent_fp16_advance_i32_varlen(
    elapsed_state_pool: torch.Tensor,
    cu_seqlens: torch.Tensor,
    state_indices: torch.Tensor,
    *,
    total_tokens: int,
    validated_metadata: object | None = None,
) -> None:
    """Advance each selected slot's phase origin by its sequence length.

    Reference ``__init__.py:83-130``.
    """
    C.enforce(ADVANCE_VARLEN, dict(locals()))
    ticket = _ticket_for(validated_metadata, cu_seqlens, state_indices, total_tokens,
                         elapsed_state_pool.shape[0], None)
    C.native().recurrent_fp16_advance_i32_varlen(cu_seqlens, state_indices,
                                                 elapsed_state_pool, total_tokens, ticket)


def infer_recurrent_add_vec_forward_varlen(x: torch.Tensor, vec: torch.Tensor) -> torch.Tensor:
    """``fp16(x + vec)`` over packed ``[N,C]`` rows (reference ``__init__.py:133-151``)."""
    C.enforce(ADD_VEC, {"x": x, "vec": vec})
    return C.native().recurrent_add_vec_forward_varlen(x, vec)


__all__ = [
    "infer_recurrent_fp16_advance_i32",
    "infer_recurrent_fp16_advance_i32_varlen",
    "infer_recurrent_add_vec_forward_varlen",
    "infer_recurrent_fp32io16_forward_varlen",
    "infer_recurrent_fp16_forward_varlen",
    "prepare_recurrent_metadata",
]

# The pretraining and chunked entries are exported here too, as in the
# reference (``tmix/wkv7/__init__.py:350-354``).
from .pretrain import pretrain_recurrent_bf16  # noqa: E402
from .chunk import infer_chunk_bf16_forward_varlen  # noqa: E402

__all__ += ["pretrain_recurrent_bf16", "infer_chunk_bf16_forward_varlen"]
