"""The TMix chain around WKV7 as one operator (decode and short sequences).

The reference runs three ops, each a round trip of ``[N, C]`` tensors
through HBM (composed in its ``tests/tmix/wkv7/test.py:310-414``):

1. ``infer_tmix_kk_a_gate_forward_varlen`` (``flashrwkv2/tmix/kk_a_gate``)
   writes ``new_k``, ``neg_kk = -kk`` and ``kka = kk gate``;
2. the WKV7 recurrence reads them with ``r``, the decay and ``v`` and writes
   ``y``;
3. ``infer_tmix_lnx_rkvres_xg_forward_varlen`` (``flashrwkv2/tmix/lnx_rkvres_xg``)
   reads ``y``, ``r``, ``new_k``, ``v``, ``g`` and writes the layer output.

:func:`infer_tmix_wkv7_fused_forward_varlen` computes the same chain in one
kernel that keeps every intermediate in registers (and in fp32, with no
rounding to 16 bits between the stages). The WKV7 inputs are ``k = new_k``,
``a = -kk`` and ``b = kk gate``: the RWKV-7 update
``S = diag(w) S + (kk gate)((-kk)^T S) + k v^T`` as the benchmark configs state it.
(The reference's chain test passes the two directions the other way round,
``a = kka, b = neg_kk``, to both its kernel and its oracle, so it checks the
composition rather than which ordering is RWKV-7's.)
This operator has no counterpart in the reference.
"""

from __future__ import annotations

import torch

from ... import _contract as C
from ..._contract import Each, check, is_tensor
from . import DECAY_LOGITS, RECURRENT_FP32, prepare_recurrent_metadata

_CHAIN_TOKENS = ("r", "decay_logits", "k", "v", "a12", "g")
_CHAIN_VECTORS = ("k_k", "a0", "k_a", "r_k", "ln_weight", "ln_bias")

# The recurrent family's checks with the chain's token list, then the
# producer/consumer vectors.
FUSED = (
    Each(_CHAIN_TOKENS, RECURRENT_FP32[0].rules),
    *RECURRENT_FP32[1:],
    Each(_CHAIN_VECTORS, (is_tensor(),)),
)


def _fused(ns: dict, decay_mode: int) -> torch.Tensor:
    C.enforce(FUSED, ns)
    ticket = ns["validated_metadata"]
    if ticket is None:
        ticket = prepare_recurrent_metadata(ns["cu_seqlens"], ns["state_indices"],
                                            total_tokens=ns["r"].shape[0],
                                            state_pool_size=ns["state_pool"].shape[0])
    return C.native().direct.recurrent_tmix_fused_forward(
        ns["cu_seqlens"], ns["state_indices"], ns["state_pool"],
        *(ns[n] for n in _CHAIN_TOKENS), *(ns[n] for n in _CHAIN_VECTORS),
        float(ns["scale"]), int(decay_mode), ns["decay_bias"], ticket)


def infer_tmix_wkv7_fused_forward_varlen(
    r: torch.Tensor,
    decay_logits: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    a12: torch.Tensor,
    g: torch.Tensor,
    k_k: torch.Tensor,
    a0: torch.Tensor,
    k_a: torch.Tensor,
    r_k: torch.Tensor,
    ln_weight: torch.Tensor,
    ln_bias: torch.Tensor,
    *,
    state_pool: torch.Tensor,
    cu_seqlens: torch.Tensor,
    state_indices: torch.Tensor,
    scale: float = 1.0,
    decay_bias: torch.Tensor | None = None,
    validated_metadata: object | None = None,
) -> torch.Tensor:
    """kk_a_gate -> WKV7 -> lnx_rkvres_xg in one kernel.

    Token tensors ``r, decay_logits, k, v, a12, g`` are packed ``[N, H, 64]``
    fp16/bf16 (``k`` is the raw key, ``a12`` the a-gate input, ``g`` the output
    gate); ``k_k, a0, k_a, r_k, ln_weight, ln_bias`` are ``[H*64]`` vectors of
    the same dtype. ``state_pool`` fp32 ``[slots, H, 64, 64]`` ([K,V]) is
    updated in place at ``state_indices``; metadata and tickets as for
    ``infer_recurrent_fp32io16_forward_varlen``. Returns the consumer's output
    shaped like ``v``.
    """
    return _fused(dict(locals()), DECAY_LOGITS)


def tmix_fused_internal(r, decay, k, v, a12, g, k_k, a0, k_a, r_k, ln_weight, ln_bias, *,
                        state_pool, cu_seqlens, state_indices, decay_mode, scale=1.0,
                        decay_bias=None, validated_metadata=None):
    """As :func:`infer_tmix_wkv7_fused_forward_varlen` with an explicit decay
    mode (0 logits, 1 the retention itself); parity tests and the bench."""
    ns = dict(locals())
    ns["decay_logits"] = ns.pop("decay")
    return _fused(ns, decay_mode)


__all__ = ["infer_tmix_wkv7_fused_forward_varlen"]
