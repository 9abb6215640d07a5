"""WKV7 fp64 oracle -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker. The product
path (``flashrwkv_amd``) never imports it and has no CPU fallback.

Two independent restatements of the reference's naive recurrence
(``/root/reference/tests/tmix/wkv7/test.py:157-213``) live here:

* :func:`forward` / :func:`backward` call ``libwkv7_oracle.so`` (plain fp64
  loops in ``wkv7_oracle.c``), fast enough for full-length sampled heads.
* :func:`forward_einsum` is a numpy einsum restatement (per token, vectorised
  over heads), used to cross-check the C loops.
* :func:`forward_torch` is the same recurrence in torch fp32 on the CPU,
  timed as the bench's torch CPU baseline.

Decay transform: :func:`retention_from_logits` restates
``csrc/sm120/tmix/wkv7/recurrent_decay.cuh:18-22`` (``exp(-e^{-1/2} sigmoid(x))``);
its log-derivative restates ``:27-32``.

How each function is pinned (see ``tests/test_oracle.py``):

* ``retention_from_logits``: the reference's exp2 constants reproduce the
  closed form; finite differences pin the log-derivative.
* ``forward`` / ``forward_einsum``: one-step closed form, the a=b=0 gated
  linear attention closed form, the w=1, a=b=0 matmul form
  ``Y = scale * tril(R K^T) V``, the k=0 explicit transition product, joint
  linearity in (v, S0), permutation invariance of packed sequences, and
  agreement of the two independent restatements; ``forward_torch`` agrees
  with ``forward`` to fp32 rounding on equal-length and ragged batches.
* ``backward``: torch fp64 autograd through an independent per-token torch
  forward (itself checked against ``forward``), and central finite
  differences at D=4.
* ``fp16_dither``: known answers at phases 0, 1, 2, -1 and 2^31 worked out by
  hand from the definition (recurrent_decay.cuh:36-41).
* ``forward_fp16_state``: agreement with the pinned fp32-state ``forward``
  within fp16 rounding (catches a dropped term, sign or transpose); phase
  continuity (tokens split over two calls with the phase origin advanced
  by the first call's length give the same result bitwise); channel
  mapping c = h*D + key (with a = b = k = 0 the rows evolve independently,
  so H=2, D=4 must equal H=1, D=8); sensitivity to the phase origin.
* ``advance_i32`` / ``advance_i32_varlen``: the reference test's known
  answers (tests/tmix/wkv7/test.py:32-60) and int32 wrap-around.
* ``add_vec``: exact sums and round-half-to-even ties at 2048 + 1 and
  2050 + 1 (fp16 spacing 2 there).
* ``kk_a_gate``: the reference test's known answer (k = k_k = k_a = 1,
  a0 = a12 = 0, head 64: new_k = 0.5, neg_kk = -0.125, kka = 0.0625,
  tests/tmix/kk_a_gate/test.py:26-47), unit norm of kk per head, the k_a = 0
  and k_a = 1 limits (new_k = k, resp. k gate) and scale invariance of kk.
* ``lnx_rkvres_xg``: constant rows (var = 0: out = (bias + rkv v) g), a
  hand-worked two-value row, rkv by brute-force loops, per-head
  independence (heads of one row do not mix).
* ``tmix_fused``: composition of the three pinned stages; checked against
  the same stages called one after another, and against a per-token loop
  that applies the RWKV-7 update with a = -kk, b = kk gate directly.
"""

from __future__ import annotations

import ctypes
import math
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "libwkv7_oracle.so"
_LIB = None

EXP_NEG_HALF = math.exp(-0.5)


def build() -> Path:
    """Compile ``libwkv7_oracle.so`` with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def _lib():
    global _LIB
    if _LIB is None:
        if not _LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(_LIB_PATH))
        i32p = ctypes.POINTER(ctypes.c_int32)
        f64p = ctypes.POINTER(ctypes.c_double)
        lib.wkv7o_forward.argtypes = [
            ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
            i32p, i32p, i32p, i32p,
            f64p, f64p, f64p, f64p, f64p, f64p, f64p,
            ctypes.c_double, f64p, f64p, f64p, ctypes.c_int,
        ]
        lib.wkv7o_forward.restype = None
        lib.wkv7o_backward.argtypes = [
            ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
            i32p, i32p, i32p, i32p,
            f64p, f64p, f64p, f64p, f64p, f64p, f64p,
            ctypes.c_double, f64p, f64p,
            f64p, f64p, f64p, f64p, f64p, f64p, f64p, ctypes.c_int,
        ]
        lib.wkv7o_backward.restype = None
        lib.wkv7o_max_threads.argtypes = []
        lib.wkv7o_max_threads.restype = ctypes.c_int
        lib.wkv7o_retention_from_logits.argtypes = [ctypes.c_double]
        lib.wkv7o_retention_from_logits.restype = ctypes.c_double
        lib.wkv7o_retention_log_derivative.argtypes = [ctypes.c_double]
        lib.wkv7o_retention_log_derivative.restype = ctypes.c_double
        _LIB = lib
    return _LIB


def max_threads() -> int:
    return int(_lib().wkv7o_max_threads())


def _f64(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.float64))


def _i32(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.int32))


def _p(arr: np.ndarray | None, ctype):
    if arr is None:
        return ctypes.POINTER(ctype)()
    return arr.ctypes.data_as(ctypes.POINTER(ctype))


# ---------------------------------------------------------------- decay ----


def retention_from_logits(x, bias=None) -> np.ndarray:
    """``exp(-e^{-1/2} * sigmoid(x + bias))`` in fp64 (recurrent_decay.cuh:18-22)."""
    x = _f64(x)
    if bias is not None:
        x = x + _f64(bias).reshape((1,) * (x.ndim - 2) + tuple(x.shape[-2:]))
    return np.exp(-EXP_NEG_HALF / (1.0 + np.exp(-x)))


def retention_log_derivative(x, bias=None) -> np.ndarray:
    """``d log(retention) / dx = -e^{-1/2} sigma (1 - sigma)`` (recurrent_decay.cuh:27-32)."""
    x = _f64(x)
    if bias is not None:
        x = x + _f64(bias).reshape((1,) * (x.ndim - 2) + tuple(x.shape[-2:]))
    sig = 1.0 / (1.0 + np.exp(-x))
    return -EXP_NEG_HALF * sig * (1.0 - sig)


# ------------------------------------------------------------- metadata ----


def segments_from_cu_seqlens(cu_seqlens):
    """One segment per packed sequence: (seg_offsets, seg_starts, seg_ends)."""
    cu = _i32(cu_seqlens)
    count = cu.shape[0] - 1
    return (
        np.arange(count + 1, dtype=np.int32),
        np.ascontiguousarray(cu[:-1]),
        np.ascontiguousarray(cu[1:]),
    )


def chunk_metadata(lengths, chunk_size):
    """StateTune chunk metadata for packed sequences of ``lengths``.

    Mirrors the construction used by the reference's tests
    (``tests/rl_infctx/wkv7/test.py:56-80``): returns
    (sequence_chunk_offsets, chunk_token_starts, chunk_token_ends, cu_seqlens).
    """
    offsets, starts, ends, cu = [0], [], [], [0]
    start = 0
    for length in lengths:
        end = start + int(length)
        for s in range(start, end, chunk_size):
            starts.append(s)
            ends.append(min(s + chunk_size, end))
        offsets.append(len(starts))
        cu.append(end)
        start = end
    return _i32(offsets), _i32(starts), _i32(ends), _i32(cu)


# -------------------------------------------------------------- forward ----


def forward(r, w, k, v, a, b, state, *, seg_offsets, seg_starts, seg_ends,
            state_slots, scale=1.0, want_boundary=False, want_state_dot_a=False,
            num_threads=0):
    """fp64 forward over segments (C loops). ``w`` is the retention.

    ``state`` is a slot pool ``[slots,H,D,D]`` ([K,V]); a copy is updated and
    returned. Returns ``(y, state_out, boundary or None, state_dot_a or None)``.
    """
    r, w, k, v, a, b = (_f64(t) for t in (r, w, k, v, a, b))
    n, heads, d = r.shape
    state_out = _f64(state).copy()
    seg_offsets, seg_starts, seg_ends, state_slots = (
        _i32(t) for t in (seg_offsets, seg_starts, seg_ends, state_slots)
    )
    y = np.zeros((n, heads, d), dtype=np.float64)
    boundary = (
        np.zeros((seg_starts.shape[0], heads, d, d), dtype=np.float64)
        if want_boundary else None
    )
    sda = np.zeros((n, heads, d), dtype=np.float64) if want_state_dot_a else None
    f64, i32 = ctypes.c_double, ctypes.c_int32
    _lib().wkv7o_forward(
        int(seg_offsets.shape[0] - 1), heads, d,
        _p(seg_offsets, i32), _p(seg_starts, i32), _p(seg_ends, i32),
        _p(state_slots, i32), _p(state_out, f64),
        _p(r, f64), _p(w, f64), _p(k, f64), _p(v, f64), _p(a, f64), _p(b, f64),
        float(scale), _p(y, f64), _p(boundary, f64), _p(sda, f64),
        int(num_threads),
    )
    return y, state_out, boundary, sda


def forward_varlen(r, w, k, v, a, b, state_pool, cu_seqlens, state_indices,
                   scale=1.0, num_threads=0):
    """Inference varlen forward: one segment per packed sequence."""
    so, ss, se = segments_from_cu_seqlens(cu_seqlens)
    y, st, _, _ = forward(r, w, k, v, a, b, state_pool, seg_offsets=so,
                          seg_starts=ss, seg_ends=se, state_slots=state_indices,
                          scale=scale, num_threads=num_threads)
    return y, st


def backward(r, w, k, v, a, b, initial_state, *, seg_offsets, seg_starts,
             seg_ends, state_slots, scale=1.0, dy=None, dstate_final=None,
             num_threads=0):
    """fp64 adjoint of :func:`forward` (C loops, forward states recomputed).

    Returns ``dict(dr, dw, dk, dv, da, db, dstate0)`` where ``dw`` is dL/d(retention).
    """
    r, w, k, v, a, b = (_f64(t) for t in (r, w, k, v, a, b))
    n, heads, d = r.shape
    s0 = _f64(initial_state)
    seg_offsets, seg_starts, seg_ends, state_slots = (
        _i32(t) for t in (seg_offsets, seg_starts, seg_ends, state_slots)
    )
    dy = None if dy is None else _f64(dy)
    dsf = None if dstate_final is None else _f64(dstate_final)
    out = {name: np.zeros((n, heads, d)) for name in ("dr", "dw", "dk", "dv", "da", "db")}
    out["dstate0"] = np.zeros_like(s0)
    f64, i32 = ctypes.c_double, ctypes.c_int32
    _lib().wkv7o_backward(
        int(seg_offsets.shape[0] - 1), heads, d,
        _p(seg_offsets, i32), _p(seg_starts, i32), _p(seg_ends, i32),
        _p(state_slots, i32), _p(s0, f64),
        _p(r, f64), _p(w, f64), _p(k, f64), _p(v, f64), _p(a, f64), _p(b, f64),
        float(scale), _p(dy, f64), _p(dsf, f64),
        _p(out["dr"], f64), _p(out["dw"], f64), _p(out["dk"], f64),
        _p(out["dv"], f64), _p(out["da"], f64), _p(out["db"], f64),
        _p(out["dstate0"], f64), int(num_threads),
    )
    return out


def forward_einsum(r, w, k, v, a, b, state_pool, cu_seqlens, state_indices,
                   scale=1.0):
    """Independent numpy restatement of test.py:157-213 (per token, all heads)."""
    r, w, k, v, a, b = (_f64(t) for t in (r, w, k, v, a, b))
    pool = _f64(state_pool).copy()
    y = np.zeros_like(r)
    cu = [int(x) for x in np.asarray(cu_seqlens)]
    slots = [int(x) for x in np.asarray(state_indices)]
    for seq, (start, end) in enumerate(zip(cu[:-1], cu[1:])):
        s = pool[slots[seq]].copy()
        for t in range(start, end):
            sa = np.einsum("hk,hkv->hv", a[t], s)
            s = w[t][:, :, None] * s + b[t][:, :, None] * sa[:, None, :] \
                + k[t][:, :, None] * v[t][:, None, :]
            y[t] = scale * np.einsum("hk,hkv->hv", r[t], s)
        pool[slots[seq]] = s
    return y, pool


def forward_torch(r, w, k, v, a, b, state_pool, cu_seqlens, state_indices, scale=1.0):
    """torch fp32 restatement of test.py:157-213 on the CPU, per token.

    The CPU baseline's "torch" leg (not a checker): the naive recurrence in
    torch's own fp32 CPU kernels, as the reference's test runs it. Packed
    sequences of one common length advance together (one batched matmul per
    token over all sequences and heads); otherwise each sequence is stepped
    on its own. Returns (y [N,H,D], updated pool), both fp32 torch tensors.
    """
    import torch

    r, w, k, v, a, b = (torch.as_tensor(t).float() for t in (r, w, k, v, a, b))
    pool = torch.as_tensor(state_pool).float().clone()
    cu = [int(x) for x in np.asarray(cu_seqlens)]
    slots = torch.as_tensor(np.asarray(state_indices), dtype=torch.long)
    lengths = {e - s for s, e in zip(cu[:-1], cu[1:])}
    y = torch.empty_like(r)
    if len(lengths) == 1:
        t_len = lengths.pop()
        n_seq = len(cu) - 1
        view = [t.view(n_seq, t_len, *t.shape[1:]) for t in (r, w, k, v, a, b)]
        rr, ww, kk, vv, aa, bb = view
        yy = y.view(n_seq, t_len, *y.shape[1:])
        s = pool[slots]
        for t in range(t_len):
            sa = torch.matmul(aa[:, t].unsqueeze(-2), s)                  # [B,H,1,D]
            s = ww[:, t].unsqueeze(-1) * s + bb[:, t].unsqueeze(-1) * sa \
                + kk[:, t].unsqueeze(-1) * vv[:, t].unsqueeze(-2)
            yy[:, t] = scale * torch.matmul(rr[:, t].unsqueeze(-2), s).squeeze(-2)
        pool[slots] = s
        return y, pool
    for seq, (start, end) in enumerate(zip(cu[:-1], cu[1:])):
        s = pool[slots[seq]]
        for t in range(start, end):
            sa = torch.matmul(a[t].unsqueeze(-2), s)
            s = w[t].unsqueeze(-1) * s + b[t].unsqueeze(-1) * sa \
                + k[t].unsqueeze(-1) * v[t].unsqueeze(-2)
            y[t] = scale * torch.matmul(r[t].unsqueeze(-2), s).squeeze(-2)
        pool[slots[seq]] = s
    return y, pool


# ------------------------------------------------------- fp16 state -----
#
# The fp16-state (Albatross) family, restating the reference's contract oracle
# ``tests/tmix/wkv7/test.py:214-264`` and the dither of
# ``csrc/sm120/tmix/wkv7/recurrent_decay.cuh:36-46``. Arithmetic between the
# contract's fp16 rounding points (delta, state after every token, output) is
# fp64 here; the rounding points themselves are the contract.

DITHER_MULTIPLIER = 2654435769
DITHER_UNIT = 2.0 ** -41  # 4.547473508864641e-13


def fp16_dither(phase) -> np.ndarray:
    """``float32(int32(phase * 2654435769 mod 2^32)) * 2^-41`` (recurrent_decay.cuh:36-41).

    The int32 -> float32 conversion rounds to 24 bits, as the device does;
    the scaling by a power of two is exact.
    """
    p = np.asarray(phase).astype(np.int64).astype(np.uint64) & np.uint64(0xFFFFFFFF)
    with np.errstate(over="ignore"):
        bits = (p * np.uint64(DITHER_MULTIPLIER)) & np.uint64(0xFFFFFFFF)
    signed = bits.astype(np.int64) - (bits >= np.uint64(1 << 31)).astype(np.int64) * (1 << 32)
    return signed.astype(np.float32).astype(np.float64) * DITHER_UNIT


def fp16_delta(x, phase, bias=None) -> np.ndarray:
    """``fp16(retention(x + bias) - 1 + dither(phase))`` as float64 (recurrent_decay.cuh:43-46)."""
    w = retention_from_logits(x, bias)
    return (w - 1.0 + fp16_dither(phase)).astype(np.float16).astype(np.float64)


def forward_fp16_state(r, x, k, v, a, b, state_pool, elapsed_state_pool, cu_seqlens,
                       state_indices, scale=1.0, bias=None):
    """fp16-state recurrence over packed sequences (test.py:214-264).

    ``x`` are decay logits; ``state_pool`` ``[slots,H,D,D]`` ([K,V]) and the
    returned pool are float16; ``elapsed_state_pool`` ``[slots]`` int32 phase
    origins (read only). Channel ``c = h*D + key`` of token ``t`` of a
    sequence starting at ``start`` uses phase ``elapsed[slot] + c + t - start``.
    Returns ``(y float16 [N,H,D], pool float16)``.
    """
    r, x, k, v, a, b = (_f64(t) for t in (r, x, k, v, a, b))
    n, heads, d = r.shape
    pool = np.asarray(state_pool).astype(np.float16).copy()
    elapsed = np.asarray(elapsed_state_pool).astype(np.int64)
    channel = np.arange(heads * d, dtype=np.int64).reshape(heads, d)
    y = np.zeros((n, heads, d), dtype=np.float16)
    cu = [int(c) for c in np.asarray(cu_seqlens)]
    slots = [int(c) for c in np.asarray(state_indices)]
    for seq, (start, end) in enumerate(zip(cu[:-1], cu[1:])):
        slot = slots[seq]
        s = pool[slot].astype(np.float64)
        for t in range(start, end):
            delta = fp16_delta(x[t], channel + elapsed[slot] + (t - start), bias)
            sa = np.einsum("hk,hkv->hv", a[t], s)
            s = (s + s * delta[:, :, None] + b[t][:, :, None] * sa[:, None, :]
                 + k[t][:, :, None] * v[t][:, None, :])
            s = s.astype(np.float16).astype(np.float64)
            y[t] = (scale * np.einsum("hk,hkv->hv", r[t], s)).astype(np.float16)
        pool[slot] = s.astype(np.float16)
    return y, pool


def advance_i32(elapsed_state, amount) -> np.ndarray:
    """``elapsed + amount`` with int32 wrap-around (fp16 .cu:57-64)."""
    e = np.asarray(elapsed_state).astype(np.int64) + int(amount)
    return ((e + (1 << 31)) % (1 << 32) - (1 << 31)).astype(np.int32)


def advance_i32_varlen(elapsed_state_pool, cu_seqlens, state_indices) -> np.ndarray:
    """Each selected slot advanced by its sequence length (fp16 .cu:67-81)."""
    out = np.asarray(elapsed_state_pool).astype(np.int64).copy()
    cu = np.asarray(cu_seqlens).astype(np.int64)
    for seq, slot in enumerate(np.asarray(state_indices)):
        out[int(slot)] += cu[seq + 1] - cu[seq]
    return ((out + (1 << 31)) % (1 << 32) - (1 << 31)).astype(np.int32)


def add_vec(x, vec) -> np.ndarray:
    """``fp16(float32(x) + float32(vec))`` per row (fp16 .cu:85-122)."""
    x32 = np.asarray(x).astype(np.float16).astype(np.float32)
    v32 = np.asarray(vec).astype(np.float16).astype(np.float32)
    return (x32 + v32[None, :]).astype(np.float16)


# --------------------------------------------- TMix producer / consumer -----


def kk_a_gate(k, k_k, a0, a12, k_a, head_size=64):
    """The key / a-gate producer (reference kk_a_gate .cu:128-160 and
    tests/tmix/kk_a_gate/test.py:58-66), fp64 on packed ``[N, C]`` rows:
    ``u = k k_k``, ``kk = u / max(|u|_head, 1e-12)``, ``gate = sigmoid(a0 + a12)``;
    returns ``(new_k, neg_kk, kka) = (k (gate k_a + 1 - k_a), -kk, kk gate)``."""
    k, a12 = _f64(k), _f64(a12)
    n, c = k.shape
    h = c // head_size
    kr = k.reshape(n, h, head_size)
    u = kr * _f64(k_k).reshape(1, h, head_size)
    norm = np.sqrt(np.sum(u * u, axis=-1, keepdims=True))
    kk = u / np.maximum(norm, 1.0e-12)
    gate = 1.0 / (1.0 + np.exp(-(_f64(a0).reshape(1, h, head_size)
                                 + a12.reshape(n, h, head_size))))
    ka = _f64(k_a).reshape(1, h, head_size)
    new_k = kr * (gate * ka + 1.0 - ka)
    return (new_k.reshape(n, c), (-kk).reshape(n, c), (kk * gate).reshape(n, c))


def lnx_rkvres_xg(x, r, k, v, r_k, weight, bias, g, head_size=64, eps=64.0e-5):
    """The WKV7 output consumer (reference lnx_rkvres_xg .cu:56-131 and
    tests/tmix/lnx_rkvres_xg/test.py:52-64), fp64 on packed ``[N, C]`` rows:
    per head, ``((x - mean) / sqrt(var + eps) weight + bias + rkv v) g`` with the
    biased variance and ``rkv = sum_d r k r_k``."""
    x, r, k, v, g = (_f64(t) for t in (x, r, k, v, g))
    n, c = x.shape
    h = c // head_size
    shp = (n, h, head_size)
    xr = x.reshape(shp)
    mean = xr.mean(-1, keepdims=True)
    var = ((xr - mean) ** 2).mean(-1, keepdims=True)
    rkv = np.sum(r.reshape(shp) * k.reshape(shp) * _f64(r_k).reshape(1, h, head_size),
                 axis=-1, keepdims=True)
    out = ((xr - mean) / np.sqrt(var + eps) * _f64(weight).reshape(1, h, head_size)
           + _f64(bias).reshape(1, h, head_size) + rkv * v.reshape(shp)) * g.reshape(shp)
    return out.reshape(n, c)


def lnx_pretrain_forward(x, r, k, v, residual_scale, weight, bias, g, head_size=64,
                         eps=64.0e-5):
    """The consumer's training forward (reference
    csrc/sm90/tmix/lnx_rkvres_xg/pretrain_bf16_forward.cu:63-126), fp64 on
    ``[N, C]`` rows (a dense ``[B, T, C]`` is N = B T): the output of
    :func:`lnx_rkvres_xg` with ``r_k = residual_scale``, and the per-(row,
    head) ``mean`` and ``rstd = 1 / sqrt(var + eps)`` as ``[N, H]``."""
    x = _f64(x)
    n, c = x.shape
    h = c // head_size
    xr = x.reshape(n, h, head_size)
    mean = xr.mean(-1)
    var = ((xr - mean[..., None]) ** 2).mean(-1)
    out = lnx_rkvres_xg(x, r, k, v, _f64(residual_scale).reshape(-1), weight, bias, g,
                        head_size=head_size, eps=eps)
    return out, mean, 1.0 / np.sqrt(var + eps)


def lnx_pretrain_backward(dout, x, r, k, v, residual_scale, weight, bias, g,
                          head_size=64, eps=64.0e-5):
    """Gradients of :func:`lnx_pretrain_forward`'s output (reference
    csrc/sm90/tmix/lnx_rkvres_xg/pretrain_bf16_backward.cu:125-275), fp64, in
    closed form per (row, head) with gy = dout g, xhat = (x - mean) rstd,
    q = sum_d gy v, rkv = sum_d r k r_k:
    dx = rstd (gy w - mean_d(gy w) - xhat mean_d(gy w xhat)), dv = gy rkv,
    dr = q k r_k, dk = q r r_k, dg = dout (xhat w + b + rkv v), and the
    parameter gradients summed over rows: dw = sum gy xhat, db = sum gy,
    dr_k = sum q r k. Returns a dict keyed dx, dr, dk, dv, dresidual_scale
    ([H, D]), dweight, dbias ([C]), dg."""
    dout, x, r, k, v, g = (_f64(t) for t in (dout, x, r, k, v, g))
    n, c = x.shape
    h = c // head_size
    shp = (n, h, head_size)
    rk = _f64(residual_scale).reshape(1, h, head_size)
    w = _f64(weight).reshape(1, h, head_size)
    b = _f64(bias).reshape(1, h, head_size)
    xr, rr, kr, vr, gr, do = (t.reshape(shp) for t in (x, r, k, v, g, dout))
    mean = xr.mean(-1, keepdims=True)
    rstd = 1.0 / np.sqrt(((xr - mean) ** 2).mean(-1, keepdims=True) + eps)
    xhat = (xr - mean) * rstd
    gy = do * gr
    dxhat = gy * w
    dx = rstd * (dxhat - dxhat.mean(-1, keepdims=True)
                 - xhat * (dxhat * xhat).mean(-1, keepdims=True))
    rkv = np.sum(rr * kr * rk, axis=-1, keepdims=True)
    q = np.sum(gy * vr, axis=-1, keepdims=True)
    out = {
        "dx": dx, "dv": gy * rkv, "dr": q * kr * rk, "dk": q * rr * rk,
        "dg": do * (xhat * w + b + rkv * vr),
    }
    out = {key: val.reshape(n, c) for key, val in out.items()}
    out["dweight"] = np.sum(gy * xhat, axis=0).reshape(c)
    out["dbias"] = np.sum(gy, axis=0).reshape(c)
    out["dresidual_scale"] = np.sum(q * rr * kr, axis=0)
    return out


def tmix_fused(r, w, k, v, a12, g, k_k, a0, k_a, r_k, ln_weight, ln_bias, state_pool,
               cu_seqlens, state_indices, scale=1.0):
    """The fused chain, with no rounding between its stages: the producer
    (:func:`kk_a_gate`) gives the WKV7 inputs k = new_k, a = -kk and
    b = kk gate (the RWKV-7 update S += (kk gate)((-kk)^T S), as the benchmark
    configs state it), then :func:`forward_varlen` with retention ``w``, then
    the consumer (:func:`lnx_rkvres_xg`) with the producer's new_k. Token
    tensors ``[N, H, D]``, vectors ``[H*D]``; returns ``(out [N,H,D], pool)``."""
    r, w, k, v, a12, g = (_f64(t) for t in (r, w, k, v, a12, g))
    n, h, d = r.shape
    flat = lambda t: t.reshape(n, h * d)
    new_k, neg_kk, kka = kk_a_gate(flat(k), k_k, a0, flat(a12), k_a, head_size=d)
    shp = (n, h, d)
    y, pool = forward_varlen(r, w, new_k.reshape(shp), v, neg_kk.reshape(shp),
                             kka.reshape(shp), state_pool, cu_seqlens, state_indices,
                             scale=scale)
    out = lnx_rkvres_xg(flat(y), flat(r), new_k, flat(v), r_k, ln_weight, ln_bias, flat(g),
                        head_size=d)
    return out.reshape(shp), pool


# ------------------------------------------------------------- metrics -----


def max_rel_error(actual, expected) -> float:
    """Normwise max relative error ``max|x - x_ref| / max|x_ref|``."""
    actual = np.asarray(actual, dtype=np.float64)
    expected = np.asarray(expected, dtype=np.float64)
    denom = float(np.max(np.abs(expected))) if expected.size else 0.0
    if denom == 0.0:
        denom = 1.0
    return float(np.max(np.abs(actual - expected)) / denom) if expected.size else 0.0


def relative_rmse(actual, expected) -> float:
    """The reference's relative-RMSE metric (tests/tmix/wkv7/test.py:304-307)."""
    actual = np.asarray(actual, dtype=np.float64)
    expected = np.asarray(expected, dtype=np.float64)
    base = max(float(np.sqrt(np.mean(expected ** 2))), 1.0e-6)
    return float(np.sqrt(np.mean((actual - expected) ** 2)) / base)
