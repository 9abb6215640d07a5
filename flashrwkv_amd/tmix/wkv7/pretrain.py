"""Pretraining recurrence (clampw v3), importable as ``flashrwkv2.tmix.wkv7.pretrain``.

``pretrain_recurrent_bf16`` keeps the reference's signature, error contract
and autograd behaviour (reference ``flashrwkv2/tmix/wkv7/pretrain.py:14-129``):
dense bf16 ``[B,T,C]`` tokens with decay logits ``w`` (retention
``exp(-e^{-1/2} sigmoid(w))``), zero initial state, output ``[B,T,C]``.

Both directions run through ``torch.ops.rwkv7_clampw_v3``: head size 64 on
the chunked bf16-MFMA kernels, 128 on the bf16-MFMA kernels over 16-token
pieces, 256 on the per-token fp32 training kernels. The forward saves the state every 16 tokens; the backward recomputes
from those states and never divides by the decay.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from ... import _contract as C
from ..._contract import check, is_tensor

CHUNK_LEN = 16
_DECAY_AND_FRIENDS = ("w", "k", "v", "a", "b")


def _bf16(x, ns) -> bool:
    return x.dtype == torch.bfloat16


def _cuda_contig(x, ns) -> bool:
    return x.is_cuda and x.is_contiguous()


# Reference ``pretrain.py:14-48``.
PRETRAIN = (
    check("head_size", C.one_of({64, 128, 256}), ValueError,
          "head_size must be one of 64, 128, or 256"),
    check(None, lambda _, ns: len(ns["tensors"]) == 6, ValueError,
          "clampw requires r, w, k, v, a, and b"),
    is_tensor("r"),
    check("r", lambda x, ns: x.ndim == 3 and min(x.shape) > 0, ValueError,
          "r must have shape [B,T,C] with nonzero dimensions"),
    check("r", _bf16, TypeError, "r must be bfloat16"),
    check("r", _cuda_contig, ValueError, "r must be contiguous CUDA"),
    C.Each(_DECAY_AND_FRIENDS, (
        is_tensor(),
        check(None, _bf16, TypeError, "{name} must be bfloat16"),
        check(None, _cuda_contig, ValueError, "{name} must be contiguous CUDA"),
        check(None, C.same_shape_as("r"), ValueError, "{name} must match r shape"),
        check(None, C.same_device_as("r"), ValueError, "{name} must share the r device"),
    )),
    check("r", lambda x, ns: x.shape[2] % ns["head_size"] == 0, ValueError,
          "C must be divisible by head_size"),
    check("r", lambda x, ns: x.shape[1] % CHUNK_LEN == 0, ValueError,
          "T must be divisible by the canonical chunk length 16"),
)


@dataclass(frozen=True)
class _Layout:
    """Shapes of one pretraining call: dense [B,T,C] seen as [B,T,H,D]."""

    batch: int
    tokens: int
    heads: int
    head_size: int

    @classmethod
    def of(cls, tensors: tuple, head_size: int) -> "_Layout":
        ns = {"tensors": tensors, "head_size": head_size, "r": tensors[0] if tensors else None}
        ns.update(zip(_DECAY_AND_FRIENDS, tensors[1:]))
        C.enforce(PRETRAIN, ns)
        batch, tokens, channels = tensors[0].shape
        return cls(batch, tokens, channels // head_size, head_size)

    def heads_view(self, x: torch.Tensor) -> torch.Tensor:
        return x.view(self.batch, self.tokens, self.heads, self.head_size)

    def dense_view(self, x: torch.Tensor) -> torch.Tensor:
        return x.view(self.batch, self.tokens, self.heads * self.head_size)

    def fp32(self, *shape: int, like: torch.Tensor) -> torch.Tensor:
        return torch.empty(shape, device=like.device, dtype=torch.float32)

    def checkpoints(self, like: torch.Tensor) -> torch.Tensor:
        """State before every 16th token: [B, H, T/16, D, D]."""
        d = self.head_size
        return self.fp32(self.batch, self.heads, self.tokens // CHUNK_LEN, d, d, like=like)

    def state_dot_a(self, like: torch.Tensor) -> torch.Tensor:
        return self.fp32(self.batch, self.tokens, self.heads, self.head_size, like=like)


class _ClampwV3(torch.autograd.Function):
    """Autograd node over the two ``rwkv7_clampw_v3`` ops (forward saves the
    16-token checkpoints, backward recomputes from them)."""

    @staticmethod
    def forward(ctx, layout: _Layout, *tensors):
        split = tuple(layout.heads_view(t) for t in tensors)
        y = torch.empty_like(split[3])
        ckpt = layout.checkpoints(y)
        sda = layout.state_dot_a(y)
        torch.ops.rwkv7_clampw_v3.forward(*split, y, ckpt, sda, layout.head_size)
        ctx.layout = layout
        ctx.save_for_backward(*split, ckpt, sda)
        return layout.dense_view(y)

    @staticmethod
    def backward(ctx, dy):
        layout: _Layout = ctx.layout
        *split, ckpt, sda = ctx.saved_tensors
        grads = [torch.empty_like(t) for t in split]
        torch.ops.rwkv7_clampw_v3.backward(*split, layout.heads_view(dy.contiguous()), ckpt,
                                           sda, *grads, layout.head_size)
        return (None, *(layout.dense_view(g) for g in grads))


def pretrain_recurrent_bf16(r: torch.Tensor, w: torch.Tensor, k: torch.Tensor,
                            v: torch.Tensor, a: torch.Tensor, b: torch.Tensor, *,
                            head_size: int = 64) -> torch.Tensor:
    """clampw v3 pretraining recurrence with autograd (reference ``pretrain.py:109-126``)."""
    layout = _Layout.of((r, w, k, v, a, b), head_size)
    C.native()
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError("pretrain_recurrent_bf16 does not run under HIP graph capture: "
                           "its chunked kernels are not validated inside a captured graph")
    return _ClampwV3.apply(layout, r, w, k, v, a, b)


__all__ = ["pretrain_recurrent_bf16"]
