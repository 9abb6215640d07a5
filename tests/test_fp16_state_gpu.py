"""fp16-state (Albatross) family on the GPU, mirroring the reference's
tests/tmix/wkv7/test.py cases for it (:31-138, :1003-1200).

Expected values: the oracle's ``forward_fp16_state`` (the reference's contract
oracle test.py:214-264 with fp64 arithmetic between the fp16 rounding points)
on the same fp16 inputs. The kernel rounds at the same points with fp32
arithmetic in between, so the two differ only where an fp32 value lies within
fp32 error of an fp16 rounding boundary (one fp16 ulp, rarely). Tolerances:
relative RMSE <= 5e-4 (the reference gates its own half2 kernels at 4e-3
against this oracle) and normwise max relative error <= 2e-3; measured worst
cases are 6e-5 and 6.4e-4. The side helpers are integer or single-rounding
work and are compared bitwise.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import flashrwkv_amd
from flashrwkv_amd import capi
from flashrwkv_amd.tmix.wkv7 import (
    infer_recurrent_add_vec_forward_varlen,
    infer_recurrent_fp16_advance_i32,
    infer_recurrent_fp16_advance_i32_varlen,
    infer_recurrent_fp16_forward_varlen,
    prepare_recurrent_metadata,
)
from oracle import oracle
from tests import parity

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
RMSE_TOL = 5e-4
MAX_TOL = 2e-3


@pytest.fixture(scope="module", autouse=True)
def _require_native():
    if flashrwkv_amd._C is None:
        pytest.fail("flashrwkv_amd native library is not built (no fallback exists)")


def _np(t):
    return t.detach().cpu().numpy()


def _case(head_size, lengths, *, num_heads=2, pool_slots=None, seed=0, bias=True):
    """Reference test.py:416-477 distributions: r 0.12, decay logits 3.5,
    k/v/a/b 0.06, pool 0.03, elapsed = 11 * slot, slots (5, 0, 7, 2, 4)."""
    g = torch.Generator().manual_seed(20260804 + head_size + seed)
    total = sum(lengths)
    shape = (total, num_heads, head_size)
    scales = (0.12, 3.5, 0.06, 0.06, 0.06, 0.06)
    tokens = [(torch.randn(shape, generator=g) * s).half() for s in scales]
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lengths)]), dtype=torch.int32)
    if len(lengths) <= 5:
        slots = torch.tensor([5, 0, 7, 2, 4][: len(lengths)], dtype=torch.int32)
    else:
        slots = torch.arange(len(lengths), dtype=torch.int32)
    pool_slots = pool_slots or max(9, len(lengths))
    pool = (torch.randn((pool_slots, num_heads, head_size, head_size), generator=g)
            * 0.03).half()
    elapsed = torch.arange(pool_slots, dtype=torch.int32) * 11
    decay_bias = (torch.randn((num_heads, head_size), generator=g) * 0.2).half() if bias else None
    return tokens, cu, slots, pool, elapsed, decay_bias


def _expected(tokens, cu, slots, pool, elapsed, decay_bias, scale=1.0):
    return oracle.forward_fp16_state(
        *(_np(t) for t in tokens), _np(pool), _np(elapsed), _np(cu), _np(slots), scale=scale,
        bias=None if decay_bias is None else _np(decay_bias))


def _check(name, actual, expected):
    actual = _np(actual).astype(np.float64)
    expected = np.asarray(expected, dtype=np.float64)
    rmse = oracle.relative_rmse(actual, expected)
    print(f"{name}: rel-rmse {rmse:.2e}")
    assert rmse <= RMSE_TOL, f"{name}: rmse {rmse:.3e}"
    # Per row (floor 1e-2) within 4e-3 and elementwise (floor 0.1) within
    # 5e-3: measured at most 1.5e-3 and 2.3e-3 (fp16 state rounding).
    parity.check(name, actual, expected, MAX_TOL, row_tol=4e-3, elem_tol=5e-3, elem_floor=0.1)


def _run(tokens, cu, slots, pool, elapsed, decay_bias, **kw):
    dev = [t.to(DEV) for t in tokens]
    state = pool.to(DEV)
    out = infer_recurrent_fp16_forward_varlen(
        *dev, state_pool=state, elapsed_state_pool=elapsed.to(DEV), cu_seqlens=cu.to(DEV),
        state_indices=slots.to(DEV), decay_bias=None if decay_bias is None else decay_bias.to(DEV),
        **kw)
    torch.cuda.synchronize()
    return out, state


# ------------------------------------------------------------ helpers ----


def test_elapsed_advance_is_in_place():
    """Reference test.py:31-35."""
    elapsed = torch.tensor([2, 7, 11], device=DEV, dtype=torch.int32)
    infer_recurrent_fp16_advance_i32(elapsed, 5)
    assert elapsed.tolist() == [7, 12, 16]
    wrap = torch.tensor([2**31 - 1], device=DEV, dtype=torch.int32)
    infer_recurrent_fp16_advance_i32(wrap, 1)
    assert wrap.tolist() == [-(2**31)]
    with pytest.raises(RuntimeError, match="out of int range"):
        infer_recurrent_fp16_advance_i32(elapsed, 2**31)


def test_elapsed_varlen_advance_updates_selected_slots():
    """Reference test.py:38-61."""
    elapsed = torch.tensor([2, 5, 7, 11], device=DEV, dtype=torch.int32)
    cu = torch.tensor([0, 2, 5], device=DEV, dtype=torch.int32)
    slots = torch.tensor([3, 1], device=DEV, dtype=torch.int32)
    ticket = prepare_recurrent_metadata(cu, slots, total_tokens=5, state_pool_size=4)
    infer_recurrent_fp16_advance_i32_varlen(elapsed, cu, slots, total_tokens=5,
                                            validated_metadata=ticket)
    torch.cuda.synchronize()
    assert elapsed.tolist() == [2, 8, 7, 13]
    # Without a ticket (device validation only), the same result.
    again = torch.tensor([2, 5, 7, 11], device=DEV, dtype=torch.int32)
    infer_recurrent_fp16_advance_i32_varlen(again, cu, slots, total_tokens=5)
    assert again.tolist() == [2, 8, 7, 13]


def test_elapsed_varlen_reuses_ticket_fail_closed():
    """Reference test.py:64-84."""
    elapsed = torch.tensor([2, 5, 7, 11], device=DEV, dtype=torch.int32)
    cu = torch.tensor([0, 2, 5], device=DEV, dtype=torch.int32)
    slots = torch.tensor([3, 1], device=DEV, dtype=torch.int32)
    ticket = prepare_recurrent_metadata(cu, slots, total_tokens=5, state_pool_size=4)
    cu[1] = 3
    before = elapsed.clone()
    with pytest.raises(RuntimeError, match="validated_metadata"):
        infer_recurrent_fp16_advance_i32_varlen(elapsed, cu, slots, total_tokens=5,
                                                validated_metadata=ticket)
    assert torch.equal(elapsed, before)


def test_elapsed_varlen_through_the_c_abi_fails_closed():
    """A non-zero status word leaves every slot untouched."""
    elapsed = torch.tensor([2, 5, 7, 11], device=DEV, dtype=torch.int32)
    cu = torch.tensor([0, 2, 5], device=DEV, dtype=torch.int32)
    slots = torch.tensor([3, 9], device=DEV, dtype=torch.int32)  # slot 9 is out of range
    status, cu_snap, slot_snap = capi.metadata_validate(cu, slots, 5, 4)
    capi.advance_i32_varlen(elapsed, cu_seqlens=cu_snap, state_indices=slot_snap,
                            metadata_status=status)
    torch.cuda.synchronize()
    assert status.item() != 0 and elapsed.tolist() == [2, 5, 7, 11]


def test_ticket_supports_same_stream_graph_replay():
    """Reference test.py:86-127: capture the advance with its ticket on one
    stream; every replay (with eager work in between) gives the same result."""
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        initial = torch.tensor([2, 5, 7, 11], device=DEV, dtype=torch.int32)
        elapsed = initial.clone()
        cu = torch.tensor([0, 2, 5], device=DEV, dtype=torch.int32)
        slots = torch.tensor([3, 1], device=DEV, dtype=torch.int32)
        ticket = prepare_recurrent_metadata(cu, slots, total_tokens=5, state_pool_size=4)
        infer_recurrent_fp16_advance_i32_varlen(elapsed, cu, slots, total_tokens=5,
                                                validated_metadata=ticket)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=stream):
        elapsed.copy_(initial)
        infer_recurrent_fp16_advance_i32_varlen(elapsed, cu, slots, total_tokens=5,
                                                validated_metadata=ticket)
    for replay in range(3):
        elapsed.fill_(-1)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert elapsed.tolist() == [2, 8, 7, 13], replay


@pytest.mark.parametrize("rows,channels", [(3, 8), (17, 4096), (5, 6), (1, 2)])
def test_add_vec_matches_fp32_add_then_round(rows, channels):
    """Reference test.py:130-138; C % 8 != 0 takes the two-element path."""
    g = torch.Generator().manual_seed(rows * 1000 + channels)
    x = torch.randn((rows, channels), generator=g).half().to(DEV)
    vec = torch.randn((channels,), generator=g).half().to(DEV)
    out = infer_recurrent_add_vec_forward_varlen(x, vec)
    assert torch.equal(out, (x.float() + vec.float()).half())
    expected = oracle.add_vec(_np(x), _np(vec))
    assert np.array_equal(_np(out).view(np.uint16), expected.view(np.uint16))


def test_add_vec_rejects_reference_invalid_shapes():
    x = torch.zeros((2, 5), device=DEV, dtype=torch.float16)
    with pytest.raises(ValueError, match="even C"):
        infer_recurrent_add_vec_forward_varlen(x, torch.zeros(5, device=DEV, dtype=torch.float16))
    x = torch.zeros((2, 4), device=DEV, dtype=torch.float16)
    with pytest.raises(ValueError, match=r"vec must have shape \[C\]"):
        infer_recurrent_add_vec_forward_varlen(x, torch.zeros(6, device=DEV, dtype=torch.float16))
    with pytest.raises(TypeError, match="float16"):
        infer_recurrent_add_vec_forward_varlen(x.float(), torch.zeros(4, device=DEV))


# ------------------------------------------------------------ forward ----


@pytest.mark.parametrize("head_size", (64, 128, 256))
@pytest.mark.parametrize("lengths", ((1,), (1, 2, 4), (8, 8)))
def test_fp16_state_family_correctness(head_size, lengths):
    """Reference test.py:1003-1076: bias on, untouched slots bitwise unchanged,
    elapsed pool read but not advanced."""
    tokens, cu, slots, pool, elapsed, bias = _case(head_size, lengths)
    y_ref, pool_ref = _expected(tokens, cu, slots, pool, elapsed, bias)
    dev_elapsed = elapsed.to(DEV)
    dev = [t.to(DEV) for t in tokens]
    state = pool.to(DEV)
    out = infer_recurrent_fp16_forward_varlen(
        *dev, state_pool=state, elapsed_state_pool=dev_elapsed, cu_seqlens=cu.to(DEV),
        state_indices=slots.to(DEV), decay_bias=bias.to(DEV))
    torch.cuda.synchronize()
    assert out.dtype == torch.float16 and state.dtype == torch.float16
    _check("output", out, y_ref)
    active = slots.long()
    _check("state", state.cpu()[active], pool_ref[_np(active)])
    untouched = [i for i in range(pool.shape[0]) if i not in set(slots.tolist())]
    assert torch.equal(state.cpu()[untouched], pool[untouched])
    assert torch.equal(dev_elapsed.cpu(), elapsed)


@pytest.mark.parametrize("lengths", ((1,), (1,) * 17, (1,) * 128, (2,) * 32, (8,), (4,) * 16))
def test_fp16_launch_shapes_cover_decode_and_short_sequences(lengths):
    """Reference test.py:1079-1131: 64 heads of 64, decode and short batches."""
    tokens, cu, slots, pool, elapsed, bias = _case(64, lengths, num_heads=64)
    y_ref, pool_ref = _expected(tokens, cu, slots, pool, elapsed, bias)
    out, state = _run(tokens, cu, slots, pool, elapsed, bias)
    _check("output", out, y_ref)
    active = slots.long()
    _check("state", state.cpu()[active], pool_ref[_np(active)])


def test_fp16_long_sequences_and_scale():
    """Sequences long enough for the token prefetch ring, with a scale."""
    tokens, cu, slots, pool, elapsed, bias = _case(64, (300, 77), num_heads=4, seed=5)
    y_ref, pool_ref = _expected(tokens, cu, slots, pool, elapsed, bias, scale=0.5)
    out, state = _run(tokens, cu, slots, pool, elapsed, bias, scale=0.5)
    _check("output", out, y_ref)
    active = slots.long()
    _check("state", state.cpu()[active], pool_ref[_np(active)])


def test_fp16_decode_long_run_in_place():
    """The fp16 decode kernel stepped 512 times in place (B=64, H=8, one token
    per sequence per call, the elapsed pool advanced after each call) against
    the oracle run over the same tokens as one 512-token sequence per sampled
    slot: every step's output and the end state."""
    print("case fp16 decode B=64 H=8, 512 in-place steps", flush=True)
    batch, heads, steps = 64, 8, 512
    sampled = (0, 29, 63)
    g = torch.Generator(device=DEV).manual_seed(20260811)
    scales = (0.12, 3.5, 0.06, 0.06, 0.06, 0.06)
    pool0 = (torch.randn((batch, heads, 64, 64), generator=g, device=DEV) * 0.03).half()
    bias = (torch.randn((heads, 64), generator=g, device=DEV) * 0.2).half()
    elapsed0 = torch.arange(batch, dtype=torch.int32, device=DEV) * 11
    state, elapsed = pool0.clone(), elapsed0.clone()
    cu = torch.arange(batch + 1, dtype=torch.int32, device=DEV)
    slots = torch.arange(batch, dtype=torch.int32, device=DEV)
    pick = torch.tensor(sampled, device=DEV)
    taken = [[] for _ in range(7)]
    for _ in range(steps):
        tokens = [(torch.randn((batch, heads, 64), generator=g, device=DEV) * s).half()
                  for s in scales]
        y = infer_recurrent_fp16_forward_varlen(
            *tokens, state_pool=state, elapsed_state_pool=elapsed, cu_seqlens=cu,
            state_indices=slots, decay_bias=bias, max_seqlen=1)
        infer_recurrent_fp16_advance_i32_varlen(elapsed, cu, slots, total_tokens=batch)
        for store, t in zip(taken, (*tokens, y)):
            store.append(t[pick])
    torch.cuda.synchronize()
    series = [torch.stack(v).cpu().numpy() for v in taken]
    assert torch.equal(elapsed.cpu(), elapsed0.cpu() + steps)
    for i, slot in enumerate(sampled):
        tokens = [s[:, i] for s in series[:6]]
        y_ref, pool_ref = oracle.forward_fp16_state(
            *tokens, _np(pool0[slot:slot + 1]), _np(elapsed0[slot:slot + 1]),
            np.array([0, steps], dtype=np.int32), np.zeros(1, dtype=np.int32),
            bias=_np(bias))
        _check(f"slot {slot} output", torch.from_numpy(series[6][:, i]), y_ref)
        _check(f"slot {slot} state", state[slot:slot + 1], pool_ref)


def test_fp16_phase_continues_across_calls_bitwise():
    """Tokens split over two calls, the elapsed pool advanced in between, give
    bitwise the one-call result (same launch shape)."""
    tokens, cu, slots, pool, elapsed, bias = _case(64, (40,), num_heads=2, seed=7)
    slot = slots.to(DEV)
    dev = [t.to(DEV) for t in tokens]
    whole_state = pool.to(DEV)
    dev_elapsed = elapsed.to(DEV)
    whole = infer_recurrent_fp16_forward_varlen(
        *dev, state_pool=whole_state, elapsed_state_pool=dev_elapsed,
        cu_seqlens=cu.to(DEV), state_indices=slot, decay_bias=bias.to(DEV))
    split_state = pool.to(DEV)
    m = 17
    parts = []
    for lo, hi in ((0, m), (m, 40)):
        cu_part = torch.tensor([0, hi - lo], device=DEV, dtype=torch.int32)
        parts.append(infer_recurrent_fp16_forward_varlen(
            *[t[lo:hi].contiguous() for t in dev], state_pool=split_state,
            elapsed_state_pool=dev_elapsed, cu_seqlens=cu_part, state_indices=slot,
            decay_bias=bias.to(DEV)))
        infer_recurrent_fp16_advance_i32_varlen(dev_elapsed, cu_part, slot,
                                                total_tokens=hi - lo)
    torch.cuda.synchronize()
    assert torch.equal(torch.cat(parts), whole)
    assert torch.equal(split_state, whole_state)
    assert dev_elapsed[slots[0].item()].item() == elapsed[slots[0].item()].item() + 40


def test_fp16_consumes_the_same_metadata_ticket_contract():
    """Reference test.py:1134-1180."""
    tokens, cu, slots, pool, elapsed, _ = _case(64, (2, 3), bias=False)
    dev = [t.to(DEV) for t in tokens]
    cu_d, slots_d, elapsed_d = cu.to(DEV), slots.to(DEV), elapsed.to(DEV)
    ticket = prepare_recurrent_metadata(cu_d, slots_d, total_tokens=5,
                                        state_pool_size=pool.shape[0])
    expected_state, observed_state = pool.to(DEV), pool.to(DEV)
    expected = infer_recurrent_fp16_forward_varlen(
        *dev, state_pool=expected_state, elapsed_state_pool=elapsed_d, cu_seqlens=cu_d,
        state_indices=slots_d)
    observed = infer_recurrent_fp16_forward_varlen(
        *dev, state_pool=observed_state, elapsed_state_pool=elapsed_d, cu_seqlens=cu_d,
        state_indices=slots_d, validated_metadata=ticket)
    torch.cuda.synchronize()
    assert torch.equal(observed, expected) and torch.equal(observed_state, expected_state)
    cu_d[1] += 1
    with pytest.raises(RuntimeError, match="version"):
        infer_recurrent_fp16_forward_varlen(
            *dev, state_pool=pool.to(DEV), elapsed_state_pool=elapsed_d, cu_seqlens=cu_d,
            state_indices=slots_d, validated_metadata=ticket)


def test_fp16_public_rejects_non_fp16_state_and_tokens():
    """Reference test.py:1183-1200."""
    tokens, cu, slots, pool, elapsed, _ = _case(64, (2,), bias=False)
    dev = [t.to(DEV) for t in tokens]
    kwargs = dict(elapsed_state_pool=elapsed.to(DEV), cu_seqlens=cu.to(DEV),
                  state_indices=slots.to(DEV))
    with pytest.raises(TypeError, match="FP16-state state_pool"):
        infer_recurrent_fp16_forward_varlen(*dev, state_pool=pool.float().to(DEV), **kwargs)
    with pytest.raises((TypeError, RuntimeError), match="float16"):
        infer_recurrent_fp16_forward_varlen(dev[0].bfloat16(), *dev[1:],
                                            state_pool=pool.to(DEV), **kwargs)
    with pytest.raises(ValueError, match="elapsed_state_pool must have shape"):
        infer_recurrent_fp16_forward_varlen(
            *dev, state_pool=pool.to(DEV), elapsed_state_pool=elapsed[:3].to(DEV),
            cu_seqlens=cu.to(DEV), state_indices=slots.to(DEV))


def test_fp16_through_the_c_abi_and_fail_closed():
    """frwkv_recurrent_fp16_forward directly; a failing status word gives NaN
    outputs and leaves the pool untouched."""
    tokens, cu, slots, pool, elapsed, bias = _case(128, (3, 6), seed=9)
    y_ref, pool_ref = _expected(tokens, cu, slots, pool, elapsed, bias, scale=1.5)
    dev = [t.to(DEV) for t in tokens]
    cu_d, slots_d = cu.to(DEV), slots.to(DEV)
    state = pool.to(DEV)
    status, cu_snap, slot_snap = capi.metadata_validate(cu_d, slots_d, 9, pool.shape[0])
    out = torch.empty_like(dev[3])
    capi.recurrent_fp16_forward(*dev, state_pool=state, elapsed_state_pool=elapsed.to(DEV),
                                cu_seqlens=cu_snap, state_indices=slot_snap,
                                metadata_status=status, output=out, scale=1.5,
                                decay_bias=bias.to(DEV).reshape(-1))
    torch.cuda.synchronize()
    _check("output", out, y_ref)
    _check("state", state.cpu()[slots.long()], pool_ref[_np(slots)])
    bad_slots = torch.tensor([5, 99], device=DEV, dtype=torch.int32)
    status, cu_snap, slot_snap = capi.metadata_validate(cu_d, bad_slots, 9, pool.shape[0])
    before = state.clone()
    capi.recurrent_fp16_forward(*dev, state_pool=state, elapsed_state_pool=elapsed.to(DEV),
                                cu_seqlens=cu_snap, state_indices=slot_snap,
                                metadata_status=status, output=out)
    torch.cuda.synchronize()
    assert status.item() != 0 and torch.isnan(out).all() and torch.equal(state, before)
