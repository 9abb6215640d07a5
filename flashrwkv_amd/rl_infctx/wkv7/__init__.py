"""RL/infctx packed chunk family, importable as ``flashrwkv2.rl_infctx.wkv7``.

``rl_infctx_chunk_fp32io16`` keeps the reference's signature, error contract
and return value ``(output, final_pool)``: a cloned pool updated at
``state_indices`` (reference ``flashrwkv2/rl_infctx/wkv7/__init__.py:11-159``).
``chunk_size`` and ``strategy`` are validated and passed on, but the result
does not depend on them: head size 64 runs the exact chunked bf16-MFMA
kernel, 128 and 256 the fp32 per-token kernel.

The contract checks values of ``cu_seqlens`` and ``state_indices`` (zero
start, total end, non-empty sequences, distinct in-range slots), so the
call reads both to the host once; the chunk lists are then built from those
host copies with vectorised integer arithmetic and sent back in one copy.
"""

from __future__ import annotations

import numpy as np
import torch

from ... import _contract as C
from ..._contract import Each, check, is_tensor

CHUNK_SIZES = {16, 32, 64}
STRATEGIES = {"materialized": 0, "recompute": 1}


def _cuda_tensor_rules(arg: str | None, dtype: torch.dtype | None = None) -> tuple:
    rules = (
        is_tensor(arg),
        check(arg, C.cuda_contiguous, ValueError, "{name} must be contiguous CUDA"),
    )
    if dtype is not None:
        rules += (check(arg, C.dtype_is(dtype), TypeError, f"{{name}} must have dtype {dtype}"),)
    return rules


def _token_shape(x, ns) -> bool:
    return x.ndim == 3 and x.shape[0] > 0 and x.shape[1] > 0 and x.shape[2] in {64, 128, 256}


def _bias_shape(x, ns) -> bool:
    _, heads, d = ns["r"].shape
    return tuple(x.shape) in {(heads * d,), (heads, d)}


_BIAS_GIVEN = lambda ns: ns["decay_bias"] is not None  # noqa: E731

# Reference ``__init__.py:88-115`` (structure of every argument).
STRUCTURE = (
    check("chunk_size", C.one_of(CHUNK_SIZES), ValueError,
          "chunk_size must be one of 16, 32, or 64"),
    check("strategy", C.one_of(STRATEGIES), ValueError,
          "strategy must be 'materialized' or 'recompute'"),
    check("scale", C.finite, ValueError, "scale must be finite"),
    Each(C.PACKED_TOKENS, (
        *_cuda_tensor_rules(None),
        check(None, C.dtype_is(torch.float16, torch.bfloat16), TypeError,
              "{name} must be float16 or bfloat16"),
    )),
    check("r", _token_shape, ValueError, "RL/Infctx token tensors must have shape [N,H,D]"),
    check(None, lambda _, ns: all(ns[n].shape == ns["r"].shape and ns[n].device == ns["r"].device
                                  for n in C.PACKED_TOKENS), ValueError,
          "RL/Infctx token tensors must match r and share a device"),
    *(C.when(_BIAS_GIVEN, rule) for rule in _cuda_tensor_rules("decay_bias")),
    C.when(_BIAS_GIVEN, check("decay_bias", lambda x, ns: x.dtype == ns["r"].dtype
                              and x.device == ns["r"].device, TypeError,
                              "decay_bias must match token dtype and device")),
    C.when(_BIAS_GIVEN, check("decay_bias", _bias_shape, ValueError,
                              "decay_bias must have shape [H*D] or [H,D]")),
    *_cuda_tensor_rules("cu_seqlens", torch.int32),
    check("cu_seqlens", lambda x, ns: x.is_cuda and x.is_contiguous(), ValueError,
          "cu_seqlens must be contiguous CUDA int32"),
    check("cu_seqlens", C.same_device_as("r"), ValueError, "cu_seqlens must share the token device"),
    check("cu_seqlens", lambda x, ns: x.ndim == 1 and x.numel() >= 2, ValueError,
          "cu_seqlens must have shape [B+1]"),
)

# Reference ``_validate_cu_seqlens`` value checks, on the host copy.
OFFSET_VALUES = (
    check("offsets", lambda x, ns: x[0] == 0, ValueError, "cu_seqlens must start at zero"),
    check("offsets", lambda x, ns: x[-1] == ns["r"].shape[0], ValueError,
          "cu_seqlens must end at total_tokens"),
    check("offsets", lambda x, ns: bool(np.all(np.diff(x) > 0)), ValueError,
          "each RL/Infctx sequence must be non-empty"),
)

# Reference ``__init__.py:124-148``: slots, then the pool.
SLOTS = (
    *_cuda_tensor_rules("state_indices", torch.int32),
    check("state_indices", lambda x, ns: x.ndim == 1 and x.numel() == ns["batch"], ValueError,
          "state_indices must have shape [B]"),
    check("state_indices", C.same_device_as("r"), ValueError,
          "state_indices must share the token device"),
)
SLOT_VALUES = (
    check("slots", lambda x, ns: np.unique(x).size == x.size, ValueError,
          "state_indices must not contain duplicates"),
)
POOL = (
    *_cuda_tensor_rules("state_pool", torch.float32),
    check("state_pool", lambda x, ns: x.ndim == 4 and x.shape[1:] == (ns["r"].shape[1],
                                                                    ns["r"].shape[2],
                                                                    ns["r"].shape[2]),
          ValueError, "state_pool must have shape [slots,H,D,D]"),
    check("slots", lambda x, ns: x.size == 0 or (x.min() >= 0 and x.max() < ns["state_pool"].shape[0]),
          ValueError, "state_indices must be within state_pool"),
)


def chunk_lists(offsets: np.ndarray, chunk_size: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Per-sequence chunk lists of a packed batch (no padding).

    Sequence ``s`` (tokens ``offsets[s] .. offsets[s+1]-1``) is cut into
    ``ceil(len / chunk_size)`` chunks from its start, the last one short.
    Returns ``(sequence_chunk_offsets [B+1], chunk_token_starts [C],
    chunk_token_ends [C])``: the reference's chunk metadata
    (``__init__.py:38-63``), computed here as array arithmetic.
    """
    offsets = offsets.astype(np.int64)
    lengths = np.diff(offsets)
    counts = (lengths + chunk_size - 1) // chunk_size
    seq_offsets = np.zeros(counts.size + 1, dtype=np.int64)
    np.cumsum(counts, out=seq_offsets[1:])
    owner = np.repeat(np.arange(counts.size), counts)
    rank = np.arange(seq_offsets[-1]) - seq_offsets[owner]
    starts = offsets[owner] + rank * chunk_size
    ends = np.minimum(starts + chunk_size, offsets[owner + 1])
    return seq_offsets, starts, ends


def rl_infctx_chunk_fp32io16(r, decay_logits, k, v, a, b, *, state_pool=None, cu_seqlens,
                             state_indices=None, chunk_size: int = 16,
                             strategy: str = "recompute", scale: float = 1.0,
                             decay_bias=None):
    """Packed RL/infctx chunk forward (reference ``__init__.py:66-152``).

    Returns ``(output, final_pool)``; the input pool is not modified.
    """
    ns = dict(locals())
    C.enforce(STRUCTURE, ns)
    ns["offsets"] = cu_seqlens.detach().cpu().numpy()
    C.enforce(OFFSET_VALUES, ns)
    batch = ns["batch"] = cu_seqlens.numel() - 1
    device = r.device
    if state_indices is None:
        state_indices = ns["state_indices"] = torch.arange(batch, device=device, dtype=torch.int32)
    C.enforce(SLOTS, ns)
    ns["slots"] = state_indices.detach().cpu().numpy()
    C.enforce(SLOT_VALUES, ns)
    if state_pool is None:
        d = r.shape[2]
        state_pool = ns["state_pool"] = torch.zeros(batch, r.shape[1], d, d, device=device,
                                                    dtype=torch.float32)
    C.enforce(POOL, ns)

    seq_offsets, starts, ends = chunk_lists(ns["offsets"], chunk_size)
    packed = torch.from_numpy(np.concatenate([seq_offsets, starts, ends]).astype(np.int32))
    packed = packed.to(device)
    n_chunks = starts.size
    metadata = (packed[: batch + 1], packed[batch + 1: batch + 1 + n_chunks],
                packed[batch + 1 + n_chunks:])
    gather = state_indices.to(torch.int64)
    working = state_pool.index_select(0, gather)
    output, final_working = C.native().rl_infctx_chunk_fp32io16_forward(
        *metadata, working, r, decay_logits, k, v, a, b, STRATEGIES[strategy], float(scale),
        decay_bias)
    return output, state_pool.clone().index_copy(0, gather, final_working)


def rl_infctx_chunk_fp32io16_factor_recompute(*args, **kwargs):
    """``rl_infctx_chunk_fp32io16`` with ``strategy="recompute"`` (reference ``__init__.py:155-159``)."""
    return rl_infctx_chunk_fp32io16(*args, **{**kwargs, "strategy": "recompute"})


__all__ = ["rl_infctx_chunk_fp32io16", "rl_infctx_chunk_fp32io16_factor_recompute"]
