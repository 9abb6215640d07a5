"""Chunked WKV7 prefill, mirroring ``flashrwkv2.tmix.wkv7.chunk``.

``infer_chunk_bf16_forward_varlen`` keeps the reference's signature, checks,
error types and messages (reference ``flashrwkv2/tmix/wkv7/chunk.py:17-125``)
and its bf16 state-pool contract. The kernel behind it is the exact chunk
form of the recurrence on bf16 MFMA with an fp32 state between 64-token
chunks, so ``chunk_size`` is validated but does not change the result (the
reference's K1/K2 kernels depend on it).
"""

from __future__ import annotations

import math

import torch

from . import (
    DECAY_LOGITS,
    DECAY_RAW_W,
    _check_metadata_inputs,
    _extension,
    _resolve_max_seqlen,
    prepare_recurrent_metadata,
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
    """Run packed RWKV-7 bf16 chunked prefill; ``state_pool`` is updated in place."""
    if not isinstance(chunk_size, int) or isinstance(chunk_size, bool):
        raise TypeError("chunk_size must be an integer")
    if chunk_size <= 0:
        raise ValueError("chunk_size must be positive")
    if not math.isfinite(float(scale)):
        raise ValueError("scale must be finite")
    tensors = {"r": r, "decay_logits": decay_logits, "k": k, "v": v, "a": a, "b": b}
    for name, tensor in tensors.items():
        if not isinstance(tensor, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
        if tensor.dtype != torch.bfloat16 or not tensor.is_cuda or not tensor.is_contiguous():
            raise ValueError(f"{name} must be contiguous CUDA bfloat16")
        if tensor.device != r.device:
            raise ValueError(f"{name} must share r's device")
        if tensor.shape != r.shape:
            raise ValueError(f"{name} must have the same shape as r")
    if r.ndim != 3 or r.shape[0] <= 0 or r.shape[1] <= 0 or r.shape[2] != 64:
        raise ValueError("packed chunk inputs must have shape [total_tokens,H,64]")
    if (
        not isinstance(state_pool, torch.Tensor)
        or state_pool.dtype != torch.bfloat16
        or not state_pool.is_cuda
        or not state_pool.is_contiguous()
        or state_pool.ndim != 4
        or state_pool.shape[1:] != (r.shape[1], 64, 64)
        or state_pool.device != r.device
    ):
        raise ValueError("state_pool must be contiguous CUDA bfloat16 [slots,H,64,64]")
    _check_metadata_inputs(cu_seqlens, state_indices)
    if (
        cu_seqlens.dtype != torch.int32
        or state_indices.dtype != torch.int32
        or not cu_seqlens.is_cuda
        or not state_indices.is_cuda
        or not cu_seqlens.is_contiguous()
        or not state_indices.is_contiguous()
        or cu_seqlens.device != r.device
        or state_indices.device != r.device
    ):
        raise ValueError("chunk metadata must be contiguous CUDA int32")
    launch_max_seqlen = _resolve_max_seqlen(cu_seqlens, max_seqlen)
    ticket = (
        validated_metadata
        if validated_metadata is not None
        else prepare_recurrent_metadata(
            cu_seqlens,
            state_indices,
            total_tokens=r.shape[0],
            state_pool_size=state_pool.shape[0],
            max_seqlen=launch_max_seqlen,
        )
    )
    del ticket  # the native op validates and snapshots the metadata on device
    if decay_bias is not None:
        if (
            decay_bias.dtype != torch.bfloat16
            or not decay_bias.is_cuda
            or not decay_bias.is_contiguous()
            or decay_bias.device != r.device
            or decay_bias.shape not in {(r.shape[1], 64), (r.shape[1] * 64,)}
        ):
            raise ValueError("decay_bias must be contiguous CUDA bfloat16 [H,64] or [H*64]")
    output, _ = _extension().infer_chunk_bf16_forward_varlen(
        r, decay_logits, k, v, a, b, state_pool, cu_seqlens, state_indices,
        int(chunk_size), int(launch_max_seqlen), float(scale), decay_bias=decay_bias)
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
    """Internal chunked forward: explicit decay mode, fp16/bf16 tokens, fp32 or
    bf16 pool (not part of the reference API; used by the measurement harness
    and parity tests)."""
    if decay_mode not in (DECAY_LOGITS, DECAY_RAW_W):
        raise ValueError("decay_mode must be DECAY_LOGITS or DECAY_RAW_W")
    return _extension().chunk_forward_internal(
        r, decay, k, v, a, b, state_pool, cu_seqlens, state_indices, float(scale),
        int(decay_mode), decay_bias)


__all__ = ["infer_chunk_bf16_forward_varlen"]
