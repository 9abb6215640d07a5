"""GPU parity through the C ABI itself (ctypes, no torch operator in between).

Each entry point of include/flashrwkv_amd.h is called with raw device
pointers via flashrwkv_amd.capi and compared with the fp64 oracle
(oracle/wkv7_oracle.c, restating tests/tmix/wkv7/test.py:157-213 and
tests/tmix/wkv7/statetune/test.py:39-88 of the reference). Tolerances:
max relative error 1e-5 for fp32 tokens on the recurrent kernel, 2e-2 for
bf16 tokens and everything computed on bf16 MFMA (normwise max relative
error).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from flashrwkv_amd import capi, workloads
from oracle import oracle
from tests import parity

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda")
NAMES = ("r", "w", "k", "v", "a", "b")


@pytest.fixture(scope="module", autouse=True)
def _require_gpu():
    capi.library()
    if not torch.cuda.is_available():
        pytest.fail("a GPU is required for tests marked gpu")


def _np(t):
    return t.detach().double().cpu().numpy()


def _check(name, actual, expected, tol):
    """Normwise ``tol``; per row (floor 1e-2) and elementwise (floor 0.1)
    within 0.1 -- bf16 chunked forward and backward, measured at most 4.4e-2
    and 3.0e-2."""
    return parity.check(name, actual, expected, tol, row_tol=0.1, elem_tol=0.1,
                        elem_floor=0.1)


def _case(lengths, dtype, seed, heads=3):
    case = workloads.make_case(lengths=lengths, heads=heads, head_size=64, dtype=dtype,
                               seed=seed, state_std=0.1, pool_slots=len(lengths) + 2,
                               slots=tuple(reversed(range(2, len(lengths) + 2))))
    ref_y, ref_pool = oracle.forward_varlen(
        *(_np(case[n]) for n in NAMES), _np(case["state_pool"]),
        case["cu_seqlens"].numpy(), case["state_indices"].numpy(), scale=0.75)
    dev = {k: (v.to(DEV) if isinstance(v, torch.Tensor) else v) for k, v in case.items()}
    return case, dev, ref_y, ref_pool


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
def test_metadata_validate_then_recurrent_forward(dtype, tol):
    lengths = (1, 5, 33)
    case, dev, ref_y, ref_pool = _case(lengths, dtype, seed=41)
    n_tok = sum(lengths)
    status, cu_snap, slot_snap = capi.metadata_validate(
        dev["cu_seqlens"], dev["state_indices"], n_tok, dev["state_pool"].shape[0])
    pool = dev["state_pool"].clone()
    out = torch.empty_like(dev["v"])
    capi.recurrent_forward(*(dev[n] for n in NAMES), state_pool=pool, cu_seqlens=cu_snap,
                           state_indices=slot_snap, metadata_status=status, output=out,
                           scale=0.75, max_seqlen=max(lengths))
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    _check("y", out, ref_y, tol)
    _check("pool", pool, ref_pool, 1e-5)


@pytest.mark.parametrize("pool_dtype", (torch.float32, torch.bfloat16))
def test_chunk_forward(pool_dtype):
    lengths = (3, 64, 150)
    case, dev, ref_y, ref_pool = _case(lengths, torch.bfloat16, seed=43)
    n_tok = sum(lengths)
    status, cu_snap, slot_snap = capi.metadata_validate(
        dev["cu_seqlens"], dev["state_indices"], n_tok, dev["state_pool"].shape[0])
    pool = dev["state_pool"].to(pool_dtype)
    before = pool.clone()
    out = torch.empty_like(dev["v"])
    capi.chunk_forward(*(dev[n] for n in NAMES), state_pool=pool, cu_seqlens=cu_snap,
                       state_indices=slot_snap, metadata_status=status, output=out,
                       scale=0.75)
    torch.cuda.synchronize()
    _check("y", out, ref_y, 2e-2)
    written = case["state_indices"].tolist()
    _check("pool", pool[written], ref_pool[written], 2e-2)
    untouched = [s for s in range(pool.shape[0]) if s not in written]
    assert torch.equal(pool[untouched], before[untouched])


def test_invalid_metadata_status_gives_nan_and_keeps_pool():
    lengths = (4, 4)
    case, dev, _, _ = _case(lengths, torch.bfloat16, seed=47)
    # Duplicate slot: the device check sets a status bit, and the launch that
    # reads that status must fail closed.
    slots = torch.tensor([2, 2], dtype=torch.int32, device=DEV)
    status, cu_snap, slot_snap = capi.metadata_validate(
        dev["cu_seqlens"], slots, sum(lengths), dev["state_pool"].shape[0])
    pool = dev["state_pool"].clone()
    out = torch.zeros_like(dev["v"])
    for launch in (capi.recurrent_forward, capi.chunk_forward):
        launch(*(dev[n] for n in NAMES), state_pool=pool, cu_seqlens=cu_snap,
               state_indices=slot_snap, metadata_status=status, output=out)
        torch.cuda.synchronize()
        assert int(status.item()) & 8
        assert torch.isnan(out.float()).all()
        assert torch.equal(pool, dev["state_pool"])


def test_statetune_forward_and_backward():
    """frwkv_statetune_forward/backward with caller chunks of 100 tokens (two
    64-token pieces): the forward fills the interior buffer the backward
    reads; a second backward without it recomputes the interior states into
    its workspace and must give the same gradients bit for bit."""
    lengths = (170, 9)
    meta = oracle.chunk_metadata(lengths, 100)
    case = workloads.make_case(lengths=lengths, heads=2, head_size=64, dtype=torch.bfloat16,
                               seed=53, state_std=0.1)
    offsets, starts, ends = (torch.from_numpy(x).to(DEV) for x in meta[:3])
    toks = [case[n].to(DEV) for n in NAMES]
    n_tok, heads = sum(lengths), 2
    batch = len(lengths)
    s0 = case["state_pool"][:batch].clone()
    state = s0.to(DEV)
    out = torch.empty_like(toks[3])
    boundary = torch.empty((starts.numel(), heads, 64, 64), device=DEV)
    sda = torch.empty((n_tok, heads, 64), device=DEV)
    inner_bytes = capi.statetune_interior_bytes(64, heads, n_tok)
    assert inner_bytes == ((n_tok + 63) // 64) * heads * 64 * 64 * 4
    interior = torch.empty(inner_bytes // 4, device=DEV)
    capi.statetune_forward(*toks, sequence_chunk_offsets=offsets, chunk_token_starts=starts,
                           chunk_token_ends=ends, state=state, output=out, boundary=boundary,
                           state_dot_a=sda, interior=interior, scale=0.5)
    gen = torch.Generator().manual_seed(54)
    dy = torch.randn((n_tok, heads, 64), generator=gen).to(torch.bfloat16)
    ds = torch.randn((batch, heads, 64, 64), generator=gen) * 0.01
    assert capi.statetune_backward_workspace_bytes(64, heads, n_tok, True) == 0
    assert capi.statetune_backward_workspace_bytes(64, heads, n_tok, False) == inner_bytes
    runs = []
    for inner in (interior, None):
        grads = [torch.empty_like(t) for t in toks]
        ds0 = torch.empty((batch, heads, 64, 64), device=DEV)
        capi.statetune_backward(*toks, sequence_chunk_offsets=offsets,
                                chunk_token_starts=starts, chunk_token_ends=ends,
                                boundary=boundary, grad_output=dy.to(DEV),
                                grad_final_state=ds.to(DEV), grads=grads,
                                grad_initial_state=ds0, interior=inner, scale=0.5)
        runs.append((grads, ds0))
    torch.cuda.synchronize()
    args = [_np(case[n]) for n in NAMES]
    kw = dict(seg_offsets=meta[0], seg_starts=meta[1], seg_ends=meta[2],
              state_slots=np.arange(batch, dtype=np.int32), scale=0.5)
    y, st, bnd, ref_sda = oracle.forward(*args, _np(s0), want_boundary=True,
                                         want_state_dot_a=True, **kw)
    ref = oracle.backward(*args, _np(s0), dy=_np(dy), dstate_final=_np(ds), **kw)
    _check("y", out, y, 2e-2)
    _check("final state", state, st, 2e-2)
    _check("boundary", boundary, bnd, 2e-2)
    _check("state_dot_a", sda, ref_sda, 2e-2)
    grads, ds0 = runs[0]
    for name, g in zip(NAMES, grads):
        _check(f"d{name}", g, ref["d" + name], 2e-2)
    _check("dS0", ds0, ref["dstate0"], 2e-2)
    for name, x, y2 in zip((*NAMES, "s0"), (*runs[0][0], runs[0][1]),
                           (*runs[1][0], runs[1][1])):
        assert torch.equal(x, y2), name


@pytest.mark.parametrize("head_size", (128, 256))
def test_large_heads_backward_without_interior_recomputes_it(head_size):
    """Head sizes 128 and 256 with caller chunks longer than one 16-token
    piece: a backward without the forward's interior states recomputes them
    into its workspace (the fill-only forward) and gives the same gradients,
    bit for bit, as the backward that reads them; both match the fp64
    oracle."""
    lengths = (45, 20)
    meta = oracle.chunk_metadata(lengths, 40)
    n_tok, heads, batch, d = sum(lengths), 1, len(lengths), head_size
    case = workloads.make_case(lengths=lengths, heads=heads, head_size=d,
                               dtype=torch.bfloat16, seed=81, state_std=0.1)
    offsets, starts, ends = (torch.from_numpy(x).to(DEV) for x in meta[:3])
    toks = [case[n].to(DEV) for n in NAMES]
    s0 = case["state_pool"][:batch].clone()
    state = s0.to(DEV)
    out = torch.empty_like(toks[3])
    boundary = torch.empty((starts.numel(), heads, d, d), device=DEV)
    sda = torch.empty((n_tok, heads, d), device=DEV)
    interior = torch.empty(capi.statetune_interior_bytes(d, heads, n_tok) // 4, device=DEV)
    capi.statetune_forward(*toks, sequence_chunk_offsets=offsets, chunk_token_starts=starts,
                           chunk_token_ends=ends, state=state, output=out, boundary=boundary,
                           state_dot_a=sda, interior=interior)
    gen = torch.Generator().manual_seed(82)
    dy = torch.randn((n_tok, heads, d), generator=gen).to(torch.bfloat16)
    ds = torch.randn((batch, heads, d, d), generator=gen) * 0.01
    runs = []
    for inner in (interior, None):
        grads = [torch.empty_like(t) for t in toks]
        ds0 = torch.empty((batch, heads, d, d), device=DEV)
        capi.statetune_backward(*toks, sequence_chunk_offsets=offsets,
                                chunk_token_starts=starts, chunk_token_ends=ends,
                                boundary=boundary, grad_output=dy.to(DEV),
                                grad_final_state=ds.to(DEV), grads=grads,
                                grad_initial_state=ds0, interior=inner)
        runs.append((grads, ds0))
    torch.cuda.synchronize()
    args = [_np(case[n]) for n in NAMES]
    kw = dict(seg_offsets=meta[0], seg_starts=meta[1], seg_ends=meta[2],
              state_slots=np.arange(batch, dtype=np.int32), scale=1.0)
    ref = oracle.backward(*args, _np(s0), dy=_np(dy), dstate_final=_np(ds), **kw)
    grads, ds0 = runs[0]
    for name, g in zip(NAMES, grads):
        _check(f"d{name}", g, ref["d" + name], 2e-2)
    _check("dS0", ds0, ref["dstate0"], 2e-2)
    for name, x, y2 in zip((*NAMES, "s0"), (*runs[0][0], runs[0][1]),
                           (*runs[1][0], runs[1][1])):
        assert torch.equal(x, y2), name


@pytest.mark.parametrize("head_size", (64, 128, 256))
def test_statetune_chunk_ranges_are_clamped_to_the_tokens(head_size):
    """Chunk metadata reaching outside [0, total_tokens) runs as its clamp to
    that range (an end before the start: an empty chunk) at every head size:
    outputs, boundary states, final state and gradients equal, bit for bit,
    those of the clamped metadata."""
    lengths = (40, 24)
    n_tok, heads, batch, d = sum(lengths), 1, 2, head_size
    case = workloads.make_case(lengths=lengths, heads=heads, head_size=d,
                               dtype=torch.bfloat16, seed=71, state_std=0.1)
    toks = [case[n].to(DEV) for n in NAMES]
    offsets = torch.tensor([0, 4, 7], dtype=torch.int32, device=DEV)
    # seq 0: [-7,16) [16,32) [32,40) and an empty chunk [38,30); seq 1:
    # [40,56) [56,90) and one past the end [70,75).
    bad = ([-7, 16, 32, 38, 40, 56, 70], [16, 32, 40, 30, 56, 90, 75])
    good = ([0, 16, 32, 38, 40, 56, 64], [16, 32, 40, 38, 56, 64, 64])
    gen = torch.Generator().manual_seed(72)
    dy = torch.randn((n_tok, heads, d), generator=gen).to(torch.bfloat16).to(DEV)
    ds = (torch.randn((batch, heads, d, d), generator=gen) * 0.01).to(DEV)
    s0 = case["state_pool"][:batch].to(DEV)
    results = []
    for st, en in (bad, good):
        starts = torch.tensor(st, dtype=torch.int32, device=DEV)
        ends = torch.tensor(en, dtype=torch.int32, device=DEV)
        state = s0.clone()
        out = torch.zeros_like(toks[3])
        boundary = torch.zeros((starts.numel(), heads, d, d), device=DEV)
        sda = torch.zeros((n_tok, heads, d), device=DEV)
        interior = torch.zeros(capi.statetune_interior_bytes(d, heads, n_tok) // 4, device=DEV)
        capi.statetune_forward(*toks, sequence_chunk_offsets=offsets, chunk_token_starts=starts,
                               chunk_token_ends=ends, state=state, output=out,
                               boundary=boundary, state_dot_a=sda, interior=interior)
        grads = [torch.zeros_like(t) for t in toks]
        ds0 = torch.zeros((batch, heads, d, d), device=DEV)
        capi.statetune_backward(*toks, sequence_chunk_offsets=offsets, chunk_token_starts=starts,
                                chunk_token_ends=ends, boundary=boundary, grad_output=dy,
                                grad_final_state=ds, grads=grads, grad_initial_state=ds0,
                                interior=interior)
        torch.cuda.synchronize()
        results.append([out, state, boundary, sda, *grads, ds0])
    names = ("y", "state", "boundary", "state_dot_a", *(f"d{n}" for n in NAMES), "dS0")
    for name, x, y in zip(names, *results):
        assert torch.isfinite(x.float()).all(), name
        assert torch.equal(x, y), name


def test_statetune_backward_rejects_short_workspace():
    """Without interior states and with a workspace below the stated size
    the backward returns an argument error before launching anything."""
    lengths = (130,)
    meta = oracle.chunk_metadata(lengths, 130)
    case = workloads.make_case(lengths=lengths, heads=1, head_size=128,
                               dtype=torch.bfloat16, seed=3, state_std=0.1)
    offsets, starts, ends = (torch.from_numpy(x).to(DEV) for x in meta[:3])
    toks = [case[n].to(DEV) for n in NAMES]
    need = capi.statetune_backward_workspace_bytes(128, 1, 130, False)
    assert need == ((130 + 15) // 16) * 128 * 128 * 2  # bf16 interior states at head size 128
    grads = [torch.empty_like(t) for t in toks]
    with pytest.raises(RuntimeError, match="workspace of 256 bytes given"):
        capi.statetune_backward(*toks, sequence_chunk_offsets=offsets,
                                chunk_token_starts=starts, chunk_token_ends=ends,
                                boundary=torch.zeros((1, 1, 128, 128), device=DEV),
                                grad_output=None, grad_final_state=None, grads=grads,
                                grad_initial_state=torch.empty((1, 1, 128, 128), device=DEV),
                                work=torch.empty(256, dtype=torch.uint8, device=DEV))
