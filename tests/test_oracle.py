"""Pins the fp64 oracle (oracle/) before any GPU result is compared with it.

Each check is chosen so that a plausible slip in the oracle (dropped term,
wrong sign, transposed state, off-by-one in the token loop, wrong decay
constant) fails at least one of them. None of them restates the oracle's own
loop: closed forms, independent restatements, autograd and finite
differences supply the expected values.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import oracle

RNG = np.random.default_rng(1234)


def _tokens(n, h, d, *, rng=RNG, w_range=(0.3, 0.999)):
    r = rng.standard_normal((n, h, d))
    k = rng.standard_normal((n, h, d))
    v = rng.standard_normal((n, h, d))
    w = rng.uniform(*w_range, size=(n, h, d))
    kk = rng.standard_normal((n, h, d))
    kk /= np.linalg.norm(kk, axis=-1, keepdims=True)
    g = 1.0 / (1.0 + np.exp(-rng.standard_normal((n, h, d))))
    return r, w, k, v, -kk, kk * g


def _single(lengths, h=2, d=8, *, rng=RNG, state_std=0.3, slots=None, pool=None):
    n = sum(lengths)
    toks = _tokens(n, h, d, rng=rng)
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    if slots is None:
        slots = np.arange(len(lengths), dtype=np.int32)
    slots = np.asarray(slots, dtype=np.int32)
    if pool is None:
        pool = rng.standard_normal((max(slots) + 1, h, d, d)) * state_std
    return toks, cu, slots, pool


# ------------------------------------------------------------------ decay --


def test_reference_exp2_constants_restate_closed_form():
    # recurrent_decay.cuh:10-12 constants.
    assert math.isclose(-0.8750387749145276, -math.exp(-0.5) * math.log2(math.e), rel_tol=1e-15)
    assert math.isclose(-1.4426950408889634, -math.log2(math.e), rel_tol=1e-15)
    assert math.isclose(0.6065306597126334, math.exp(-0.5), rel_tol=1e-15)
    x = np.linspace(-12, 12, 97)
    exp2_form = np.exp2(-0.8750387749145276 / (1.0 + np.exp2(-1.4426950408889634 * x)))
    np.testing.assert_allclose(oracle.retention_from_logits(x.reshape(1, -1, 1)).ravel(),
                               exp2_form, rtol=1e-14)
    # Range of the logits transform: (exp(-e^{-1/2}), 1).
    assert oracle.retention_from_logits(np.array([[[-40.0]]])).item() > 0.9999999
    assert math.isclose(oracle.retention_from_logits(np.array([[[40.0]]])).item(),
                        math.exp(-math.exp(-0.5)), rel_tol=1e-12)


def test_retention_log_derivative_matches_finite_difference():
    x = np.linspace(-6, 6, 41).reshape(1, -1, 1)
    h = 1e-6
    fd = (np.log(oracle.retention_from_logits(x + h)) -
          np.log(oracle.retention_from_logits(x - h))) / (2 * h)
    np.testing.assert_allclose(oracle.retention_log_derivative(x), fd, rtol=1e-7, atol=1e-10)


def test_bias_broadcasts_per_head_feature():
    x = RNG.standard_normal((3, 2, 4))
    bias = RNG.standard_normal((2, 4))
    np.testing.assert_allclose(oracle.retention_from_logits(x, bias),
                               oracle.retention_from_logits(x + bias[None]), rtol=1e-15)


# -------------------------------------------------------- forward closed forms --


def test_one_step_closed_form_general_state():
    (r, w, k, v, a, b), cu, slots, pool = _single([1], h=3, d=6)
    scale = 0.7
    y, pool_out = oracle.forward_varlen(r, w, k, v, a, b, pool, cu, slots, scale)
    for h in range(3):
        s0 = pool[0, h]
        s1 = np.diag(w[0, h]) @ s0 + np.outer(b[0, h], a[0, h] @ s0) + np.outer(k[0, h], v[0, h])
        np.testing.assert_allclose(pool_out[0, h], s1, rtol=1e-13, atol=1e-13)
        np.testing.assert_allclose(y[0, h], scale * s1.T @ r[0, h], rtol=1e-13, atol=1e-13)


def test_zero_state_one_step_is_scaled_dot_product():
    (r, w, k, v, a, b), cu, slots, _ = _single([1], h=2, d=5)
    pool = np.zeros((1, 2, 5, 5))
    y, _ = oracle.forward_varlen(r, w, k, v, a, b, pool, cu, slots, 1.5)
    expected = 1.5 * np.einsum("hd,hd->h", r[0], k[0])[:, None] * v[0]
    np.testing.assert_allclose(y[0], expected, rtol=1e-13, atol=1e-13)


def test_unit_decay_no_delta_is_causal_linear_attention():
    t, d = 23, 7
    (r, _, k, v, _, _), cu, slots, _ = _single([t], h=1, d=d)
    w = np.ones_like(r)
    zeros = np.zeros_like(r)
    pool = np.zeros((1, 1, d, d))
    y, _ = oracle.forward_varlen(r, w, k, v, zeros, zeros, pool, cu, slots, 0.5)
    R, K, V = r[:, 0], k[:, 0], v[:, 0]
    expected = 0.5 * np.tril(R @ K.T) @ V
    np.testing.assert_allclose(y[:, 0], expected, rtol=1e-12, atol=1e-12)


def test_no_delta_is_gated_linear_attention_with_initial_state():
    t, d = 19, 6
    (r, w, k, v, _, _), cu, slots, pool = _single([t], h=1, d=d)
    zeros = np.zeros_like(r)
    y, pool_out = oracle.forward_varlen(r, w, k, v, zeros, zeros, pool, cu, slots, 1.0)
    W = w[:, 0]
    logc = np.cumsum(np.log(W), axis=0)  # log prod_{j<=t} w_j
    for tt in range(t):
        acc = (r[tt, 0] * np.exp(logc[tt])) @ pool[0, 0]
        for i in range(tt + 1):
            decay = np.exp(logc[tt] - logc[i])  # prod_{i<j<=t} w_j
            acc = acc + ((r[tt, 0] * decay) @ k[i, 0]) * v[i, 0]
        np.testing.assert_allclose(y[tt, 0], acc, rtol=1e-11, atol=1e-11)


def test_zero_key_is_product_of_transitions():
    t, d = 9, 5
    (r, w, k, v, a, b), cu, slots, pool = _single([t], h=1, d=d)
    k = np.zeros_like(k)
    _, pool_out = oracle.forward_varlen(r, w, k, v, a, b, pool, cu, slots, 1.0)
    s = pool[0, 0]
    for tt in range(t):
        m = np.diag(w[tt, 0]) + np.outer(b[tt, 0], a[tt, 0])
        s = m @ s
    np.testing.assert_allclose(pool_out[0, 0], s, rtol=1e-12, atol=1e-12)


def test_joint_linearity_in_values_and_initial_state():
    (r, w, k, v1, a, b), cu, slots, pool1 = _single([5, 11], h=2, d=6)
    v2 = RNG.standard_normal(v1.shape)
    pool2 = RNG.standard_normal(pool1.shape)
    al, be = 0.8, -1.7
    y1, s1 = oracle.forward_varlen(r, w, k, v1, a, b, pool1, cu, slots)
    y2, s2 = oracle.forward_varlen(r, w, k, v2, a, b, pool2, cu, slots)
    y3, s3 = oracle.forward_varlen(r, w, k, al * v1 + be * v2, a, b,
                                   al * pool1 + be * pool2, cu, slots)
    np.testing.assert_allclose(y3, al * y1 + be * y2, rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(s3, al * s1 + be * s2, rtol=1e-10, atol=1e-10)


def test_packing_permutation_and_slot_mapping_invariance():
    lengths = [3, 1, 7]
    (r, w, k, v, a, b), cu, _, _ = _single(lengths, h=2, d=4)
    pool = RNG.standard_normal((6, 2, 4, 4))
    slots = np.array([4, 0, 2], dtype=np.int32)
    y, out = oracle.forward_varlen(r, w, k, v, a, b, pool, cu, slots)
    order = [2, 0, 1]
    pieces = [np.arange(cu[i], cu[i + 1]) for i in order]
    idx = np.concatenate(pieces)
    cu2 = np.concatenate([[0], np.cumsum([lengths[i] for i in order])]).astype(np.int32)
    y2, out2 = oracle.forward_varlen(*(t[idx] for t in (r, w, k, v, a, b)), pool, cu2,
                                     slots[order])
    np.testing.assert_allclose(y2, y[idx], rtol=1e-13, atol=1e-13)
    np.testing.assert_allclose(out2, out, rtol=1e-13, atol=1e-13)
    untouched = [1, 3, 5]
    np.testing.assert_array_equal(out[untouched], pool[untouched])


def test_c_loops_match_independent_einsum_restatement():
    lengths = [1, 15, 16, 17, 65]
    (r, w, k, v, a, b), cu, _, _ = _single(lengths, h=2, d=16)
    pool = RNG.standard_normal((9, 2, 16, 16)) * 0.03
    slots = np.array([5, 0, 7, 2, 4], dtype=np.int32)
    y1, s1 = oracle.forward_varlen(r, w, k, v, a, b, pool, cu, slots, 0.9)
    y2, s2 = oracle.forward_einsum(r, w, k, v, a, b, pool, cu, slots, 0.9)
    np.testing.assert_allclose(y1, y2, rtol=1e-11, atol=1e-12)
    np.testing.assert_allclose(s1, s2, rtol=1e-11, atol=1e-12)


@pytest.mark.parametrize("lengths", ([1, 15, 16, 17, 65], [24, 24, 24]))
def test_torch_fp32_baseline_matches_c_loops(lengths):
    """The torch fp32 CPU baseline computes the pinned recurrence (ragged
    batches per sequence, equal lengths batched) to fp32 rounding."""
    (r, w, k, v, a, b), cu, _, _ = _single(lengths, h=2, d=16)
    pool = RNG.standard_normal((9, 2, 16, 16)) * 0.03
    slots = np.array([5, 0, 7, 2, 4][:len(lengths)], dtype=np.int32)
    y1, s1 = oracle.forward_varlen(r, w, k, v, a, b, pool, cu, slots, 0.9)
    y2, s2 = oracle.forward_torch(r, w, k, v, a, b, pool, cu, slots, 0.9)
    assert oracle.max_rel_error(y2.double().numpy(), y1) < 1e-5
    assert oracle.max_rel_error(s2.double().numpy(), s1) < 1e-5


def test_segmentation_invariance_and_boundaries():
    lengths = [37, 9]
    (r, w, k, v, a, b), _, _, _ = _single(lengths, h=2, d=8)
    s0 = RNG.standard_normal((2, 2, 8, 8)) * 0.1
    so, ss, se, cu = oracle.chunk_metadata(lengths, 8)
    y_c, st_c, boundary, sda = oracle.forward(
        r, w, k, v, a, b, s0, seg_offsets=so, seg_starts=ss, seg_ends=se,
        state_slots=np.arange(2), want_boundary=True, want_state_dot_a=True)
    y_1, st_1 = oracle.forward_varlen(r, w, k, v, a, b, s0, cu, np.arange(2))
    np.testing.assert_allclose(y_c, y_1, rtol=1e-13, atol=1e-13)
    np.testing.assert_allclose(st_c, st_1, rtol=1e-13, atol=1e-13)
    # boundary of a sequence's first chunk is S0; later ones are the state
    # after running the sequence prefix through the single-segment path.
    for seq in range(2):
        for c in range(so[seq], so[seq + 1]):
            start = ss[c]
            prefix = start - cu[seq]
            if prefix == 0:
                np.testing.assert_array_equal(boundary[c], s0[seq])
            else:
                sl = slice(cu[seq], start)
                _, st_prefix = oracle.forward_varlen(
                    *(t[sl] for t in (r, w, k, v, a, b)), s0[seq:seq + 1],
                    np.array([0, prefix], dtype=np.int32), np.zeros(1, dtype=np.int32))
                np.testing.assert_allclose(boundary[c], st_prefix[0], rtol=1e-12, atol=1e-12)
    # state_dot_a[t] = a_t^T S_{t-1}: at a sequence's first token, S_{t-1} = S0.
    for seq in range(2):
        t0 = cu[seq]
        np.testing.assert_allclose(sda[t0], np.einsum("hk,hkv->hv", a[t0], s0[seq]),
                                   rtol=1e-13, atol=1e-13)


# ---------------------------------------------------------------- backward --


def _torch_forward(r, w, k, v, a, b, s0, scale):
    """Independent per-token torch restatement for autograd (one sequence)."""
    s = s0
    ys = []
    for t in range(r.shape[0]):
        sa = torch.einsum("hk,hkv->hv", a[t], s)
        s = w[t].unsqueeze(-1) * s + b[t].unsqueeze(-1) * sa.unsqueeze(-2) \
            + k[t].unsqueeze(-1) * v[t].unsqueeze(-2)
        ys.append(scale * torch.einsum("hk,hkv->hv", r[t], s))
    return torch.stack(ys), s


def test_backward_matches_fp64_autograd():
    lengths = [13]
    (r, w, k, v, a, b), cu, slots, pool = _single(lengths, h=2, d=6)
    scale = 0.75
    dy = RNG.standard_normal(r.shape)
    dsf = RNG.standard_normal(pool.shape) * 0.1
    so, ss, se = oracle.segments_from_cu_seqlens(cu)
    grads = oracle.backward(r, w, k, v, a, b, pool, seg_offsets=so, seg_starts=ss,
                            seg_ends=se, state_slots=slots, scale=scale, dy=dy,
                            dstate_final=dsf)
    tens = [torch.tensor(x, requires_grad=True) for x in (r, w, k, v, a, b)]
    s0 = torch.tensor(pool[0], requires_grad=True)
    y_t, s_t = _torch_forward(*tens, s0, scale)
    y_o, s_o = oracle.forward_varlen(r, w, k, v, a, b, pool, cu, slots, scale)
    np.testing.assert_allclose(y_t.detach().numpy(), y_o, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(s_t.detach().numpy(), s_o[0], rtol=1e-12, atol=1e-12)
    loss = (y_t * torch.tensor(dy)).sum() + (s_t * torch.tensor(dsf[0])).sum()
    loss.backward()
    for name, t in zip(("dr", "dw", "dk", "dv", "da", "db"), tens):
        np.testing.assert_allclose(grads[name], t.grad.numpy(), rtol=1e-10, atol=1e-11,
                                   err_msg=name)
    np.testing.assert_allclose(grads["dstate0"][0], s0.grad.numpy(), rtol=1e-10, atol=1e-11)


def test_backward_central_finite_differences_tiny():
    (r, w, k, v, a, b), cu, slots, pool = _single([4, 3], h=1, d=4)
    dy = RNG.standard_normal(r.shape)
    dsf = RNG.standard_normal(pool.shape)
    so, ss, se = oracle.segments_from_cu_seqlens(cu)

    def loss(rr, ww, kk_, vv, aa, bb, p):
        y, s = oracle.forward_varlen(rr, ww, kk_, vv, aa, bb, p, cu, slots, 1.1)
        return float(np.sum(y * dy) + np.sum(s * dsf))

    grads = oracle.backward(r, w, k, v, a, b, pool, seg_offsets=so, seg_starts=ss,
                            seg_ends=se, state_slots=slots, scale=1.1, dy=dy,
                            dstate_final=dsf)
    base = [r, w, k, v, a, b, pool]
    names = ["dr", "dw", "dk", "dv", "da", "db", "dstate0"]
    eps = 1e-6
    for which, name in enumerate(names):
        arr = base[which]
        for flat in RNG.choice(arr.size, size=6, replace=False):
            idx = np.unravel_index(flat, arr.shape)
            plus = [x.copy() for x in base]
            minus = [x.copy() for x in base]
            plus[which][idx] += eps
            minus[which][idx] -= eps
            fd = (loss(*plus) - loss(*minus)) / (2 * eps)
            assert abs(fd - grads[name][idx]) <= 1e-6 * max(1.0, abs(fd)), (name, idx)


def test_metrics_are_normwise():
    ref = np.array([1.0, -4.0, 2.0])
    assert oracle.max_rel_error(ref + np.array([0.0, 0.4, 0.0]), ref) == pytest.approx(0.1)
    assert oracle.relative_rmse(ref, ref) == 0.0


# ------------------------------------------------------- fp16 state ----


def test_fp16_dither_known_answers():
    """int32(p * 2654435769 mod 2^32), rounded to float32, times 2^-41, worked by
    hand: p=1 -> -1640531527 (float32 -1640531584), p=2 -> 1013904242
    (1013904256), p=-1 -> 1640531527, p=2^31 -> -2^31."""
    phases = np.array([0, 1, 2, -1, 2**31], dtype=np.int64)
    expected = np.array([0, -1640531584, 1013904256, 1640531584, -2147483648]) * 2.0**-41
    assert np.array_equal(oracle.fp16_dither(phases), expected)
    assert np.max(np.abs(oracle.fp16_dither(np.arange(-5000, 5000)))) <= 2.0**-10


def test_fp16_delta_known_answers():
    """fp16(w - 1 + dither) at two logits with a closed-form retention, worked
    by hand. x = 30 saturates the sigmoid: w = exp(-e^-1/2) = 0.545239212;
    x = 0 halves it: w = exp(-e^-1/2 / 2) = 0.738403150. The fp16 grid on
    [-0.5, -0.25) has step 2^-12 and on [-0.25, 0) step 2^-13:
      x=30, p=0: -0.454760788 -> -1863 * 2^-12
      x=30, p=1: -0.454760788 - 7.460e-4 = -0.455506815 -> -1866 * 2^-12
      x=30, p=2: -0.454760788 + 4.611e-4 = -0.454299718 -> -1861 * 2^-12
      x=0,  p=0: -0.261596850 -> -1072 * 2^-12
      x=0,  p=1: -0.262342877 -> -1075 * 2^-12
    Flipping the dither's sign moves p=1 to -1860 * 2^-12 and p=2 to
    -1865 * 2^-12; dropping it moves both to -1863 * 2^-12."""
    x = np.array([30.0, 30.0, 30.0, 0.0, 0.0])
    phases = np.array([0, 1, 2, 0, 1], dtype=np.int64)
    expected = np.array([-1863, -1866, -1861, -1072, -1075]) * 2.0**-12
    assert np.array_equal(oracle.fp16_delta(x, phases), expected)
    # The bias is added to the logits before the sigmoid.
    assert np.array_equal(oracle.fp16_delta(x - 30.0, phases, bias=np.full(5, 30.0))[:3],
                          expected[:3])


def _fp16_case(lengths, h, d, *, seed, slots=None, pool_slots=None):
    rng = np.random.default_rng(seed)
    n = sum(lengths)
    r, _, k, v, a, b = _tokens(n, h, d, rng=rng)
    x = rng.standard_normal((n, h, d)) * 2.0
    half = [t.astype(np.float16) for t in (r * 0.3, x, k * 0.3, v * 0.3, a, b)]
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    if slots is None:
        slots = np.arange(len(lengths), dtype=np.int32)
    slots = np.asarray(slots, dtype=np.int32)
    pool_slots = pool_slots or int(slots.max()) + 1
    pool = (rng.standard_normal((pool_slots, h, d, d)) * 0.3).astype(np.float16)
    elapsed = (np.arange(pool_slots) * 11 + 3).astype(np.int32)
    bias = (rng.standard_normal((h, d)) * 0.2).astype(np.float16)
    return half, pool, elapsed, cu, slots, bias


def test_fp16_state_tracks_the_fp32_state_recurrence():
    """Same inputs through the pinned fp32-state forward: close (fp16 rounding
    and a dither of at most 2^-10 per step), but not identical."""
    half, pool, elapsed, cu, slots, bias = _fp16_case((5, 17), 2, 8, seed=31, slots=(2, 0))
    y16, pool16 = oracle.forward_fp16_state(*half, pool, elapsed, cu, slots, scale=0.7,
                                            bias=bias)
    r, x, k, v, a, b = (t.astype(np.float64) for t in half)
    w = oracle.retention_from_logits(x, bias.astype(np.float64))
    y64, pool64 = oracle.forward_varlen(r, w, k, v, a, b, pool.astype(np.float64), cu, slots,
                                        scale=0.7)
    err_y = oracle.max_rel_error(y16, y64)
    err_s = oracle.max_rel_error(pool16[[2, 0]], pool64[[2, 0]])
    assert 1e-5 < err_y < 5e-3 and 1e-5 < err_s < 5e-3, (err_y, err_s)
    assert np.array_equal(pool16[1], pool[1])


def test_fp16_state_phase_continues_across_calls():
    """Split a sequence over two calls, the second from the advanced phase
    origin and the first call's pool: bitwise the same as one call."""
    half, pool, elapsed, cu, slots, bias = _fp16_case((23,), 2, 8, seed=32)
    y, final = oracle.forward_fp16_state(*half, pool, elapsed, cu, slots, bias=bias)
    m = 9
    first = [t[:m] for t in half]
    second = [t[m:] for t in half]
    y1, mid = oracle.forward_fp16_state(*first, pool, elapsed, [0, m], slots, bias=bias)
    advanced = oracle.advance_i32_varlen(elapsed, [0, m], slots)
    y2, end = oracle.forward_fp16_state(*second, mid, advanced, [0, 23 - m], slots, bias=bias)
    assert np.array_equal(np.concatenate([y1, y2]), y) and np.array_equal(end, final)
    # The phase origin matters: one step later gives a different state.
    _, shifted = oracle.forward_fp16_state(*half, pool, elapsed + 1, cu, slots, bias=bias)
    assert not np.array_equal(shifted, final)


def test_fp16_state_channel_is_head_times_d_plus_key():
    """With a = b = k = 0 every key row evolves alone (S = fp16(S (1 + delta))),
    so H=2, D=4 equals rows h*4 + key of H=1, D=8."""
    rng = np.random.default_rng(33)
    n = 6
    x8 = (rng.standard_normal((n, 1, 8)) * 2).astype(np.float16)
    s8 = (rng.standard_normal((1, 1, 8, 8)) * 0.3).astype(np.float16)
    zeros8 = np.zeros((n, 1, 8), dtype=np.float16)
    elapsed = np.array([5], dtype=np.int32)
    cu, slots = np.array([0, n], dtype=np.int32), np.array([0], dtype=np.int32)
    _, out8 = oracle.forward_fp16_state(zeros8, x8, zeros8, zeros8, zeros8, zeros8, s8,
                                        elapsed, cu, slots)
    x4 = x8.reshape(n, 2, 4)
    s4 = np.ascontiguousarray(s8[:, 0, :, :4].reshape(1, 2, 4, 4))
    zeros4 = np.zeros((n, 2, 4), dtype=np.float16)
    _, out4 = oracle.forward_fp16_state(zeros4, x4, zeros4, zeros4, zeros4, zeros4, s4,
                                        elapsed, cu, slots)
    assert np.array_equal(out4.reshape(1, 8, 4), out8[:, 0, :, :4])
    assert not np.array_equal(out8, s8)


def test_advance_known_answers_and_wraparound():
    """Reference tests/tmix/wkv7/test.py:32-60."""
    assert oracle.advance_i32([2, 7, 11], 5).tolist() == [7, 12, 16]
    assert oracle.advance_i32_varlen([2, 5, 7, 11], [0, 2, 5], [3, 1]).tolist() == [2, 8, 7, 13]
    assert oracle.advance_i32([2**31 - 1, -(2**31)], 1).tolist() == [-(2**31), -(2**31) + 1]


def test_add_vec_exact_sums_and_ties_to_even():
    """fp16 spacing is 2 at 2048: 2048 + 1 and 2050 + 1 are ties (to even)."""
    x = np.array([[2048, 2050, 1.5, -3.0]], dtype=np.float16)
    vec = np.array([1, 1, 0.25, 3.0], dtype=np.float16)
    assert oracle.add_vec(x, vec).tolist() == [[2048.0, 2052.0, 1.75, 0.0]]


# ------------------------------------------- TMix producer / consumer -----


def test_kk_a_gate_reference_known_answer():
    # tests/tmix/kk_a_gate/test.py:26-47: k = k_k = k_a = 1, a0 = a12 = 0,
    # C = 4096, head 64 -> new_k 0.5, neg_kk -0.125 (= -1/sqrt(64)), kka 0.0625.
    n, c = 3, 4096
    new_k, neg_kk, kka = oracle.kk_a_gate(np.ones((n, c)), np.ones(c), np.zeros(c),
                                          np.zeros((n, c)), np.ones(c))
    np.testing.assert_allclose(new_k, 0.5, rtol=0, atol=1e-15)
    np.testing.assert_allclose(neg_kk, -0.125, rtol=0, atol=1e-15)
    np.testing.assert_allclose(kka, 0.0625, rtol=0, atol=1e-15)


@pytest.mark.parametrize("head_size", (64, 128, 256))
def test_kk_a_gate_unit_norm_limits_and_scale_invariance(head_size):
    rng = np.random.default_rng(5)
    n, h = 4, 2
    c = h * head_size
    k = rng.standard_normal((n, c))
    k_k = rng.standard_normal(c)
    a0 = rng.standard_normal(c)
    a12 = rng.standard_normal((n, c))
    new_k, neg_kk, kka = oracle.kk_a_gate(k, k_k, a0, a12, np.zeros(c), head_size)
    # unit norm of kk per (token, head), and kka / kk = sigmoid(a0 + a12)
    norms = np.linalg.norm(neg_kk.reshape(n, h, head_size), axis=-1)
    np.testing.assert_allclose(norms, 1.0, rtol=1e-13)
    gate = 1.0 / (1.0 + np.exp(-(a0[None, :] + a12)))
    np.testing.assert_allclose(kka, -neg_kk * gate, rtol=1e-13)
    # k_a = 0: new_k = k; k_a = 1: new_k = k * gate
    np.testing.assert_allclose(new_k, k, rtol=1e-15)
    new_k1, _, _ = oracle.kk_a_gate(k, k_k, a0, a12, np.ones(c), head_size)
    np.testing.assert_allclose(new_k1, k * gate, rtol=1e-13)
    # kk does not depend on the key's scale per head
    _, neg2, _ = oracle.kk_a_gate(3.5 * k, k_k, a0, a12, np.zeros(c), head_size)
    np.testing.assert_allclose(neg2, neg_kk, rtol=1e-13)
    # a zero key gives kk = 0 (the 1e-12 floor), not NaN
    _, neg0, _ = oracle.kk_a_gate(np.zeros((n, c)), k_k, a0, a12, np.zeros(c), head_size)
    assert np.all(neg0 == 0.0)


def test_lnx_rkvres_xg_constant_rows_hand_worked_row_and_heads():
    rng = np.random.default_rng(6)
    d, h, n = 64, 2, 3
    c = h * d
    r, k, v, g = (rng.standard_normal((n, c)) for _ in range(4))
    r_k, weight, bias = (rng.standard_normal(c) for _ in range(3))
    # rkv by explicit loops
    rkv = np.zeros((n, h))
    for t in range(n):
        for hh in range(h):
            for j in range(d):
                idx = hh * d + j
                rkv[t, hh] += r[t, idx] * k[t, idx] * r_k[idx]
    # constant x per head: var = 0, the normalised term vanishes
    x = np.repeat(rng.standard_normal((n, h)), d, axis=1)
    out = oracle.lnx_rkvres_xg(x, r, k, v, r_k, weight, bias, g).reshape(n, h, d)
    want = (bias.reshape(1, h, d) + rkv[:, :, None] * v.reshape(n, h, d)) * g.reshape(n, h, d)
    np.testing.assert_allclose(out, want, rtol=1e-12, atol=1e-12)
    # hand-worked row: x = +-1 alternating, weight 1, bias 0, r = 0, g = 1:
    # mean 0, var 1, out = x / sqrt(1 + 64e-5)
    x1 = np.tile([1.0, -1.0], c // 2)[None, :]
    out1 = oracle.lnx_rkvres_xg(x1, np.zeros((1, c)), k[:1], v[:1], r_k, np.ones(c),
                                np.zeros(c), np.ones((1, c)))
    np.testing.assert_allclose(out1, x1 / math.sqrt(1.0 + 64.0e-5), rtol=1e-14)
    # heads do not mix: changing head 1's x leaves head 0's output unchanged
    x2 = rng.standard_normal((n, c))
    o_a = oracle.lnx_rkvres_xg(x2, r, k, v, r_k, weight, bias, g)
    x3 = x2.copy()
    x3[:, d:] *= 7.0
    o_b = oracle.lnx_rkvres_xg(x3, r, k, v, r_k, weight, bias, g)
    np.testing.assert_array_equal(o_a[:, :d], o_b[:, :d])


def _lnx_case(rng, n, h, d):
    c = h * d
    x, r, k, v, g = (rng.standard_normal((n, c)) for _ in range(5))
    rs = rng.standard_normal((h, d))
    weight, bias = rng.standard_normal(c), rng.standard_normal(c)
    return [x, r, k, v, rs, weight, bias, g]


def test_lnx_pretrain_forward_statistics_and_output():
    """The training forward's output is the pinned inference consumer with
    r_k = residual_scale; mean and rstd are the row mean and
    1 / sqrt(biased var + 64e-5), checked by explicit loops."""
    rng = np.random.default_rng(11)
    n, h, d = 3, 2, 8
    args = _lnx_case(rng, n, h, d)
    out, mean, rstd = oracle.lnx_pretrain_forward(*args, head_size=d)
    x = args[0]
    for t in range(n):
        for hh in range(h):
            row = x[t, hh * d:(hh + 1) * d]
            m = sum(row) / d
            var = sum((e - m) ** 2 for e in row) / d
            assert mean[t, hh] == pytest.approx(m, rel=1e-13)
            assert rstd[t, hh] == pytest.approx(1.0 / math.sqrt(var + 64.0e-5), rel=1e-13)
    want = oracle.lnx_rkvres_xg(*args[:4], args[4].reshape(-1), *args[5:], head_size=d)
    np.testing.assert_array_equal(out, want)


def test_lnx_pretrain_backward_matches_central_differences():
    """Every gradient of the closed-form adjoint against central finite
    differences of L = sum(dout * out) through the fp64 forward (H=2, D=4)."""
    rng = np.random.default_rng(12)
    n, h, d = 3, 2, 4
    args = _lnx_case(rng, n, h, d)
    dout = rng.standard_normal((n, h * d))
    grads = oracle.lnx_pretrain_backward(dout, *args, head_size=d)
    names = ("dx", "dr", "dk", "dv", "dresidual_scale", "dweight", "dbias", "dg")

    def loss(a):
        return float(np.sum(dout * oracle.lnx_pretrain_forward(*a, head_size=d)[0]))

    eps = 1e-6
    for i, name in enumerate(names):
        base = args[i]
        fd = np.zeros_like(base)
        for idx in np.ndindex(base.shape):
            plus = [a.copy() for a in args]
            minus = [a.copy() for a in args]
            plus[i][idx] += eps
            minus[i][idx] -= eps
            fd[idx] = (loss(plus) - loss(minus)) / (2 * eps)
        np.testing.assert_allclose(grads[name], fd, rtol=1e-6, atol=1e-7, err_msg=name)


def test_lnx_pretrain_backward_matches_torch_autograd():
    """The same gradients from torch fp64 autograd through a restatement
    written with torch's own layer norm (biased var, eps 64e-5): an
    independent route to the adjoint at D = 64."""
    rng = np.random.default_rng(13)
    n, h, d = 5, 3, 64
    args = _lnx_case(rng, n, h, d)
    dout = rng.standard_normal((n, h * d))
    ts = [torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in args]
    x, r, k, v, rs, w, b, g = ts
    xn = torch.nn.functional.layer_norm(x.view(n, h, d), (d,), eps=64.0e-5)
    rkv = (r.view(n, h, d) * k.view(n, h, d) * rs.view(1, h, d)).sum(-1, keepdim=True)
    y = (xn * w.view(1, h, d) + b.view(1, h, d) + rkv * v.view(n, h, d)) * g.view(n, h, d)
    y.reshape(n, h * d).backward(torch.tensor(dout))
    grads = oracle.lnx_pretrain_backward(dout, *args, head_size=d)
    for t, name in zip(ts, ("dx", "dr", "dk", "dv", "dresidual_scale", "dweight", "dbias", "dg")):
        np.testing.assert_allclose(grads[name], t.grad.numpy(), rtol=1e-10, atol=1e-10,
                                   err_msg=name)


def test_tmix_fused_is_the_rwkv7_update_with_a_minus_kk_and_b_kk_gate():
    rng = np.random.default_rng(7)
    h, d = 2, 8
    lengths = [3, 1, 4]
    n = sum(lengths)
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    slots = np.array([2, 0, 1], dtype=np.int32)
    r, k, v, a12, g = (rng.standard_normal((n, h, d)) for _ in range(5))
    w = rng.uniform(0.4, 0.99, size=(n, h, d))
    k_k, a0, k_a, r_k, lnw, lnb = (rng.standard_normal(h * d) for _ in range(6))
    pool = rng.standard_normal((3, h, d, d)) * 0.3
    out, pool_out = oracle.tmix_fused(r, w, k, v, a12, g, k_k, a0, k_a, r_k, lnw, lnb,
                                      pool, cu, slots, scale=0.7)
    # per-token loop written from the RWKV-7 definition: kk = normalize(k k_k),
    # S = diag(w) S + (kk gate)((-kk)^T S) + k' v^T, y = scale S^T r, then
    # the per-head norm / residual / gate.
    ref_out = np.zeros((n, h, d))
    ref_pool = pool.copy()
    for s_i, (t0, t1) in enumerate(zip(cu[:-1], cu[1:])):
        st = ref_pool[slots[s_i]].copy()
        for t in range(t0, t1):
            for hh in range(h):
                sl = slice(hh * d, (hh + 1) * d)
                u = k[t, hh] * k_k[sl]
                kk = u / max(np.linalg.norm(u), 1e-12)
                gate = 1.0 / (1.0 + np.exp(-(a0[sl] + a12[t, hh])))
                kn = k[t, hh] * (gate * k_a[sl] + 1.0 - k_a[sl])
                S = st[hh]
                sa = (-kk) @ S
                S = w[t, hh][:, None] * S + np.outer(kk * gate, sa) + np.outer(kn, v[t, hh])
                st[hh] = S
                y = 0.7 * (r[t, hh] @ S)
                mu = y.mean()
                var = ((y - mu) ** 2).mean()
                rkv = np.sum(r[t, hh] * kn * r_k[sl])
                ref_out[t, hh] = ((y - mu) / math.sqrt(var + 64e-5) * lnw[sl] + lnb[sl]
                                  + rkv * v[t, hh]) * g[t, hh]
        ref_pool[slots[s_i]] = st
    np.testing.assert_allclose(out, ref_out, rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(pool_out, ref_pool, rtol=1e-10, atol=1e-10)
