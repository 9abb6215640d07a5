"""Chunked WKV7 prefill, importable as ``flashrwkv2.tmix.wkv7.chunk``.

``infer_chunk_bf16_forward_varlen`` keeps the reference's signature, error
contract and bf16 state-pool contract (reference
``flashrwkv2/tmix/wkv7/chunk.py:17-125``); its checks are the contract table
``CHUNK_PREFILL`` below. The kernel behind it is the exact chunk form of the
recurrence on bf16 MFMA with an fp32 state between 64-token chunks, so
``chunk_size`` is validated but does not change the result (the reference's
K1/K2 kernels depend on it).
"""

from __future__ import annotations

import torch

from ... import _contract as C
from ..._contract import Each, check, is_tensor
from . import DECAY_LOGITS, DECAY_RAW_W, prepare_recurrent_metadata


def _bf16_cuda(x, ns) -> bool:
    return x.dtype == torch.bfloat16 and x.is_cuda and x.is_contiguous()


def _pool_ok(x, ns) -> bool:
    r = ns["r"]
    return (isinstance(x, torch.Tensor) and _bf16_cuda(x, ns) and x.ndim == 4
            and x.shape[1:] == (r.shape[1], 64, 64) and x.device == r.device)


def _metadata_ok(_, ns) -> bool:
    dev = ns["r"].device
    return all(t.dtype == torch.int32 and t.is_cuda and t.is_contiguous() and t.device == dev
               for t in (ns["cu_seqlens"], ns["state_indices"]))


def _bias_ok(x, ns) -> bool:
    heads = ns["r"].shape[1]
    return (_bf16_cuda(x, ns) and x.device == ns["r"].device
            and tuple(x.shape) in {(heads, 64), (heads * 64,)})


# Reference ``chunk.py:41-109`` (plus ``_resolve_max_seqlen``, ``__init__.py:166-177``).
CHUNK_PREFILL = (
    check("chunk_size", C.plain_int, TypeError, "chunk_size must be an integer"),
    check("chunk_size", lambda x, ns: x > 0, ValueError, "chunk_size must be positive"),
    check("scale", C.finite, ValueError, "scale must be finite"),
    Each(C.PACKED_TOKENS, (
        is_tensor(),
        check(None, _bf16_cuda, ValueError, "{name} must be contiguous CUDA bfloat16"),
        check(None, C.same_device_as("r"), ValueError, "{name} must share r's device"),
        check(None, C.same_shape_as("r"), ValueError, "{name} must have the same shape as r"),
    )),
    check("r", lambda x, ns: x.ndim == 3 and x.shape[0] > 0 and x.shape[1] > 0
          and x.shape[2] == 64, ValueError,
          "packed chunk inputs must have shape [total_tokens,H,64]"),
    check("state_pool", _pool_ok, ValueError,
          "state_pool must be contiguous CUDA bfloat16 [slots,H,64,64]"),
    *C.METADATA,
    check(None, _metadata_ok, ValueError, "chunk metadata must be contiguous CUDA int32"),
    C.when(lambda ns: ns["max_seqlen"] is not None,
           check("max_seqlen", lambda x, ns: int(x) > 0, ValueError,
                 "max_seqlen must be positive")),
    C.when(lambda ns: ns["max_seqlen"] is None,
           check("cu_seqlens", lambda x, ns: x.numel() >= 2, ValueError,
                 "cu_seqlens must contain at least one sequence")),
)

CHUNK_BIAS = (
    C.when(lambda ns: ns["decay_bias"] is not None,
           check("decay_bias", _bias_ok, ValueError,
                 "decay_bias must be contiguous CUDA bfloat16 [H,64] or [H*64]")),
)


def infer_chunk_bf16_forward_varlen(
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
    chunk_size: int = 16,
    max_seqlen: int | None = None,
    scale: float = 1.0,
    decay_bias: torch.Tensor | None = None,
    validated_metadata: object | None = None,
) -> torch.Tensor:
    """Packed RWKV-7 bf16 chunked prefill; ``state_pool`` is updated in place.

    Invalid metadata is rejected by the ticket's validation (or, with a
    caller ticket, fails closed on the device: NaN output, pool untouched).
    The longest sequence comes from ``max_seqlen`` or the ticket.
    """
    ns = dict(locals())
    C.enforce(CHUNK_PREFILL, ns)
    ticket = validated_metadata
    if ticket is None:
        ticket = prepare_recurrent_metadata(cu_seqlens, state_indices,
                                            total_tokens=r.shape[0],
                                            state_pool_size=state_pool.shape[0],
                                            max_seqlen=max_seqlen)
    launch_max = int(max_seqlen) if max_seqlen is not None else int(ticket.max_seqlen())
    C.enforce(CHUNK_BIAS, ns)
    output, _ = C.native().infer_chunk_bf16_forward_varlen(
        r, decay_logits, k, v, a, b, state_pool, cu_seqlens, state_indices,
        int(chunk_size), launch_max, float(scale), decay_bias=decay_bias)
    return output


def chunk_forward_internal(
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
) -> torch.Tensor:
    """Chunked forward with an explicit decay mode, fp16/bf16 tokens and an fp32
    or bf16 pool (not reference API; the measurement harness and parity tests
    use it)."""
    if decay_mode not in (DECAY_LOGITS, DECAY_RAW_W):
        raise ValueError("decay_mode must be DECAY_LOGITS or DECAY_RAW_W")
    return C.native().chunk_forward_internal(
        r, decay, k, v, a, b, state_pool, cu_seqlens, state_indices, float(scale),
        int(decay_mode), decay_bias)


__all__ = ["infer_chunk_bf16_forward_varlen"]
