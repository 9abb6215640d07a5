"""Pretraining recurrence (clampw v3), mirroring ``flashrwkv2.tmix.wkv7.pretrain``.

``pretrain_recurrent_bf16`` keeps the reference's signature, validation
(error types and messages) and autograd contract (reference
``flashrwkv2/tmix/wkv7/pretrain.py:14-129``): dense bf16 ``[B,T,C]`` tokens
with decay logits ``w`` (retention ``exp(-e^{-1/2} sigmoid(w))``), zero initial
state, output ``[B,T,C]``. The forward and backward run through
``torch.ops.rwkv7_clampw_v3``: head size 64 on the chunked bf16-MFMA kernels,
128 and 256 on the per-token fp32 training kernels. Either backward recomputes
its chunks from the saved boundary states (every 16 tokens).
"""

from __future__ import annotations

import torch

from . import _extension

CHUNK_LEN = 16


def _validate_inputs(tensors: tuple[torch.Tensor, ...], head_size: int) -> tuple[int, int, int]:
    """Reference ``pretrain.py:14-48``."""
    if head_size not in {64, 128, 256}:
        raise ValueError("head_size must be one of 64, 128, or 256")
    if len(tensors) != 6:
        raise ValueError("clampw requires r, w, k, v, a, and b")
    r = tensors[0]
    if not isinstance(r, torch.Tensor):
        raise TypeError("r must be a torch.Tensor")
    if r.ndim != 3 or min(r.shape) <= 0:
        raise ValueError("r must have shape [B,T,C] with nonzero dimensions")
    if r.dtype != torch.bfloat16:
        raise TypeError("r must be bfloat16")
    if not r.is_cuda or not r.is_contiguous():
        raise ValueError("r must be contiguous CUDA")
    for name, tensor in zip(("w", "k", "v", "a", "b"), tensors[1:]):
        if not isinstance(tensor, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
        if tensor.dtype != torch.bfloat16:
            raise TypeError(f"{name} must be bfloat16")
        if not tensor.is_cuda or not tensor.is_contiguous():
            raise ValueError(f"{name} must be contiguous CUDA")
        if tensor.shape != r.shape:
            raise ValueError(f"{name} must match r shape")
        if tensor.device != r.device:
            raise ValueError(f"{name} must share the r device")
    batch, tokens, channels = r.shape
    if channels % head_size != 0:
        raise ValueError("C must be divisible by head_size")
    if tokens % CHUNK_LEN != 0:
        raise ValueError("T must be divisible by the canonical chunk length 16")
    return batch, tokens, channels


class _PretrainRecurrent(torch.autograd.Function):
    """Reference ``pretrain.py:50-106``."""

    @staticmethod
    def forward(ctx, r, w, k, v, a, b, head_size):
        batch, tokens, channels = _validate_inputs((r, w, k, v, a, b), head_size)
        _extension()
        heads = channels // head_size
        values = tuple(t.view(batch, tokens, heads, head_size) for t in (r, w, k, v, a, b))
        output = torch.empty_like(values[3])
        boundary = torch.empty((batch, heads, tokens // CHUNK_LEN, head_size, head_size),
                               device=r.device, dtype=torch.float32)
        state_dot_a = torch.empty((batch, tokens, heads, head_size), device=r.device,
                                  dtype=torch.float32)
        torch.ops.rwkv7_clampw_v3.forward(*values, output, boundary, state_dot_a, head_size)
        ctx.save_for_backward(*values, boundary, state_dot_a)
        ctx.input_shape = (batch, tokens, channels)
        ctx.head_size = head_size
        return output.view(batch, tokens, channels)

    @staticmethod
    def backward(ctx, grad_output):
        r, w, k, v, a, b, boundary, state_dot_a = ctx.saved_tensors
        batch, tokens, channels = ctx.input_shape
        head_size = ctx.head_size
        heads = channels // head_size
        dy = grad_output.contiguous().view(batch, tokens, heads, head_size)
        grads = tuple(torch.empty_like(t) for t in (r, w, k, v, a, b))
        torch.ops.rwkv7_clampw_v3.backward(r, w, k, v, a, b, dy, boundary, state_dot_a,
                                           *grads, head_size)
        return tuple(g.view(batch, tokens, channels) for g in grads) + (None,)


def pretrain_recurrent_bf16(r: torch.Tensor, w: torch.Tensor, k: torch.Tensor,
                            v: torch.Tensor, a: torch.Tensor, b: torch.Tensor, *,
                            head_size: int = 64) -> torch.Tensor:
    """Run the clampw v3 pretraining forward/backward (reference ``pretrain.py:109-126``)."""
    _validate_inputs((r, w, k, v, a, b), head_size)
    return _PretrainRecurrent.apply(r, w, k, v, a, b, head_size)


__all__ = ["pretrain_recurrent_bf16"]
