"""TMix producer and consumer of the WKV7 operator (fp16 packed rows).

The producer ``infer_tmix_kk_a_gate_forward_varlen`` makes the WKV7 key and
a/b inputs; the consumer ``infer_tmix_lnx_rkvres_xg_forward_varlen`` turns
the WKV7 output into the TMix output. Both keep the reference's signatures,
keyword defaults and error contract (reference
``flashrwkv2/tmix/kk_a_gate/__init__.py:10-72`` and
``flashrwkv2/tmix/lnx_rkvres_xg/__init__.py:10-80``; importable from the
matching ``flashrwkv2.tmix`` packages). The two share one contract skeleton:
a head-size check, per-row-tensor checks, shape checks, then the
``batch_size`` / ``max_seqlen`` launch hints. The work is the gfx950 kernels
``kk_a_gate_kernel`` and ``lnx_rkvres_xg_kernel`` (``csrc/tmix_gates.hip``).
"""

from __future__ import annotations

import torch

from .. import _contract as C
from .._contract import Each, check, is_tensor

HEAD_SIZES = {64, 128, 256}


def _row_tensors(names: tuple[str, ...], anchor: str) -> Each:
    """fp16 CUDA tensors sharing the anchor's device."""
    return Each(names, (
        is_tensor(),
        check(None, C.dtype_is(torch.float16), TypeError, "{name} must have dtype torch.float16"),
        check(None, C.cuda_contiguous, ValueError, "{name} must be CUDA and contiguous"),
        check(None, C.same_device_as(anchor), ValueError, f"{{name}} must share {anchor}'s device"),
    ))


def _packed(anchor: str):
    return lambda x, ns: C.packed_rows(x, ns) and x.shape[1] % ns["head_size"] == 0


_HEAD_SIZE = check("head_size", C.one_of(HEAD_SIZES), ValueError,
                   "head_size must be one of 64, 128, or 256")
_LAUNCH_HINTS = (
    check("batch_size", C.positive_int, ValueError, "batch_size must be a positive integer"),
    check("max_seqlen", C.positive_int, ValueError, "max_seqlen must be a positive integer"),
)

# Reference ``kk_a_gate/__init__.py:24-57``.
KK_A_GATE = (
    _HEAD_SIZE,
    _row_tensors(("k", "k_k", "a0", "a12", "k_a"), "k"),
    check("k", _packed("k"), ValueError, "k must have packed shape [total_tokens,H*head_size]"),
    check(None, lambda _, ns: all(ns[n].shape == (ns["k"].shape[1],)
                                  for n in ("k_k", "a0", "k_a")), ValueError,
          "k_k, a0 and k_a must have shape [C]"),
    check("a12", C.same_shape_as("k"), ValueError, "a12 must match k's packed shape"),
    *_LAUNCH_HINTS,
)


def _channel_vector(x, ns) -> bool:
    return x.device == ns["x"].device and x.shape == (ns["x"].shape[1],)


# Reference ``lnx_rkvres_xg/__init__.py:26-68``.
LNX_RKVRES_XG = (
    _HEAD_SIZE,
    _row_tensors(("x", "r", "k", "v", "g"), "x"),
    check("x", _packed("x"), ValueError, "x must have packed shape [total_tokens,H*head_size]"),
    check(None, lambda _, ns: all(ns[n].shape == ns["x"].shape for n in ("r", "k", "v", "g")),
          ValueError, "r, k, v and g must match x's packed shape"),
    Each(("r_k", "weight", "bias"), (
        is_tensor(),
        check(None, lambda x, ns: x.dtype == torch.float16 and C.cuda_contiguous(x, ns),
              ValueError, "{name} must be contiguous CUDA float16"),
        check(None, _channel_vector, ValueError, "{name} must have shape [C] and share x's device"),
    )),
    *_LAUNCH_HINTS,
)


def _with_default_max_seqlen(ns: dict, rows: torch.Tensor) -> dict:
    # Without a hint the packed row count bounds every sequence.
    if ns["max_seqlen"] is None and isinstance(rows, torch.Tensor) and rows.ndim >= 1:
        ns["max_seqlen"] = rows.shape[0]
    return ns


def _hints(ns: dict) -> tuple[int, int, int]:
    return int(ns["head_size"]), int(ns["batch_size"]), int(ns["max_seqlen"])


def infer_tmix_kk_a_gate_forward_varlen(
    k: torch.Tensor,
    k_k: torch.Tensor,
    a0: torch.Tensor,
    a12: torch.Tensor,
    k_a: torch.Tensor,
    *,
    head_size: int = 64,
    batch_size: int = 1,
    max_seqlen: int | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``(new_k, neg_kk, kka)`` for packed fp16 rows ``[N, C]``:
    ``u = k k_k``, ``kk = u / max(|u|_head, 1e-12)``, ``gate = sigmoid(a0 + a12)``,
    ``new_k = k (gate k_a + 1 - k_a)``, ``neg_kk = -kk``, ``kka = kk gate``."""
    ns = dict(locals())
    C.enforce(KK_A_GATE[:5], ns)  # the hint default needs a checked k
    C.enforce(KK_A_GATE[5:], _with_default_max_seqlen(ns, k))
    return tuple(C.native().tmix_kk_a_gate_forward_varlen(k, k_k, a0, a12, k_a, *_hints(ns)))


def infer_tmix_lnx_rkvres_xg_forward_varlen(
    x: torch.Tensor,
    r: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    r_k: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor,
    g: torch.Tensor,
    *,
    head_size: int = 64,
    batch_size: int = 1,
    max_seqlen: int | None = None,
) -> torch.Tensor:
    """Per head of packed fp16 rows ``[N, C]``:
    ``((x - mean) / sqrt(var + 64e-5) weight + bias + (sum r k r_k) v) g``."""
    ns = dict(locals())
    C.enforce(LNX_RKVRES_XG[:5], ns)
    C.enforce(LNX_RKVRES_XG[5:], _with_default_max_seqlen(ns, x))
    return C.native().tmix_lnx_rkvres_xg_forward_varlen(x, r, k, v, r_k, weight, bias, g,
                                                        *_hints(ns))
