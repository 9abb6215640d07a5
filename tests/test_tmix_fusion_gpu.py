"""TMix producer (kk_a_gate), consumer (lnx_rkvres_xg) and the fused chain
on the GPU, against the fp64 oracle on the same (cast) inputs.

Cases follow the reference's own tests: tests/tmix/kk_a_gate/test.py:18-93
(the all-ones known answer at a grid-striding row count, random packed rows
for head sizes 64/128/256, shape and head-size rejection) and
tests/tmix/lnx_rkvres_xg/test.py:34-64 (random packed rows per head size).

Tolerances: the standalone kernels compute in fp32 and round each output
once to fp16, so they are held to a normwise max relative error of 2e-3
(4 fp16 ulps of the largest output; the reference uses atol = rtol = 0.04).
The fused chain runs a bf16/fp16-io recurrence with an fp32 state, as the
recurrent operator does, and is held to that operator's 2e-2 normwise
bound against the fp64 chain, and to 2e-2 against the three-kernel GPU
composition (whose intermediates are rounded to 16 bits between the stages).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import flashrwkv_amd
from flashrwkv_amd import capi
from flashrwkv_amd.tmix.kk_a_gate import infer_tmix_kk_a_gate_forward_varlen
from flashrwkv_amd.tmix.lnx_rkvres_xg import infer_tmix_lnx_rkvres_xg_forward_varlen
from flashrwkv_amd.tmix.wkv7 import (
    DECAY_LOGITS,
    DECAY_RAW_W,
    prepare_recurrent_metadata,
    recurrent_forward_internal,
)
from flashrwkv_amd.tmix.wkv7.fused import (
    infer_tmix_wkv7_fused_forward_varlen,
    tmix_fused_internal,
)
from oracle import oracle
from tests import parity

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
GATE_TOL = 2e-3
CHAIN_TOL = 2e-2


@pytest.fixture(scope="module", autouse=True)
def _require_native():
    if flashrwkv_amd._C is None:
        pytest.fail("flashrwkv_amd native library is not built (no fallback exists)")


def _np(t):
    return t.detach().double().cpu().numpy()


def _check(actual, expected, tol, label):
    """Normwise, per row (floor 1e-2) and elementwise (floor 1e-3) all within
    ``tol``: the gates and the chain round once to fp16 or bf16 at the end
    (measured elementwise at most 4.9e-4 for the gates, 3.8e-3 for the bf16
    chain, 4.1e-2 fused-vs-composition outputs at floor 1e-3, which rounds
    twice; that comparison is judged at floor 0.1)."""
    floor = 0.1 if label.startswith("fused vs composition") else 1e-3
    return parity.check(label, actual, expected, tol, row_tol=tol, elem_tol=tol,
                        elem_floor=floor)


# ------------------------------------------------------------- producer ---


def test_kk_a_gate_known_answer_over_many_rows():
    # Reference test.py:18-47 (rows 65536, C 4096): new_k 0.5, neg_kk -0.125,
    # kka 0.0625 everywhere, here across many grid-stride iterations.
    rows, c = 65536, 4096
    k = torch.ones(rows, c, device=DEV, dtype=torch.float16)
    k_k = torch.ones(c, device=DEV, dtype=torch.float16)
    a0 = torch.zeros(c, device=DEV, dtype=torch.float16)
    a12 = torch.zeros(rows, c, device=DEV, dtype=torch.float16)
    k_a = torch.ones(c, device=DEV, dtype=torch.float16)
    new_k, neg_kk, kka = infer_tmix_kk_a_gate_forward_varlen(k, k_k, a0, a12, k_a,
                                                             batch_size=256, max_seqlen=256)
    torch.cuda.synchronize()
    for out, want in ((new_k, 0.5), (neg_kk, -0.125), (kka, 0.0625)):
        assert torch.isfinite(out).all()
        assert torch.equal(out, torch.full_like(out, want))


@pytest.mark.parametrize("head_size", (64, 128, 256))
def test_kk_a_gate_matches_oracle(head_size):
    g = torch.Generator().manual_seed(17 + head_size)
    rows, heads = 37, 3
    c = heads * head_size
    k, a12 = (torch.randn(rows, c, generator=g).half() for _ in range(2))
    k_k, a0, k_a = (torch.randn(c, generator=g).half() for _ in range(3))
    outs = infer_tmix_kk_a_gate_forward_varlen(
        *(t.to(DEV) for t in (k, k_k, a0, a12, k_a)), head_size=head_size)
    torch.cuda.synchronize()
    want = oracle.kk_a_gate(_np(k), _np(k_k), _np(a0), _np(a12), _np(k_a), head_size)
    for out, ref, name in zip(outs, want, ("new_k", "neg_kk", "kka")):
        _check(out, ref, GATE_TOL, f"kk_a_gate {name} D={head_size}")


def test_kk_a_gate_rejects_bad_shapes_and_types():
    packed = torch.zeros(2, 65, device=DEV, dtype=torch.float16)
    vector = torch.zeros(65, device=DEV, dtype=torch.float16)
    with pytest.raises(ValueError, match="packed shape"):
        infer_tmix_kk_a_gate_forward_varlen(packed, vector, vector, packed, vector)
    with pytest.raises(ValueError, match="head_size"):
        infer_tmix_kk_a_gate_forward_varlen(None, None, None, None, None, head_size=32)
    k = torch.zeros(2, 64, device=DEV, dtype=torch.float16)
    v64 = torch.zeros(64, device=DEV, dtype=torch.float16)
    with pytest.raises(TypeError, match="float16"):
        infer_tmix_kk_a_gate_forward_varlen(k.float(), v64, v64, k, v64)
    with pytest.raises(ValueError, match=r"\[C\]"):
        infer_tmix_kk_a_gate_forward_varlen(k, v64[:32], v64, k, v64)
    with pytest.raises(ValueError, match="a12"):
        infer_tmix_kk_a_gate_forward_varlen(k, v64, v64, k[:1], v64)


# ------------------------------------------------------------- consumer ---


@pytest.mark.parametrize("head_size", (64, 128, 256))
def test_lnx_rkvres_xg_matches_oracle(head_size):
    g = torch.Generator().manual_seed(21 + head_size)
    rows, heads = 29, 2
    c = heads * head_size
    x, r, k, v, gate = (torch.randn(rows, c, generator=g).half() for _ in range(5))
    r_k, weight, bias = (torch.randn(c, generator=g).half() for _ in range(3))
    out = infer_tmix_lnx_rkvres_xg_forward_varlen(
        *(t.to(DEV) for t in (x, r, k, v, r_k, weight, bias, gate)), head_size=head_size)
    torch.cuda.synchronize()
    want = oracle.lnx_rkvres_xg(*(_np(t) for t in (x, r, k, v, r_k, weight, bias, gate)),
                                head_size=head_size)
    _check(out, want, GATE_TOL, f"lnx_rkvres_xg D={head_size}")


def test_lnx_rkvres_xg_rejects_bad_shapes_and_types():
    x = torch.zeros(3, 128, device=DEV, dtype=torch.float16)
    vec = torch.zeros(128, device=DEV, dtype=torch.float16)
    with pytest.raises(ValueError, match="match x"):
        infer_tmix_lnx_rkvres_xg_forward_varlen(x, x[:2], x, x, vec, vec, vec, x)
    with pytest.raises(ValueError, match=r"shape \[C\]"):
        infer_tmix_lnx_rkvres_xg_forward_varlen(x, x, x, x, vec[:64], vec, vec, x)
    with pytest.raises(TypeError, match="float16"):
        infer_tmix_lnx_rkvres_xg_forward_varlen(x.float(), x, x, x, vec, vec, vec, x)
    with pytest.raises(ValueError, match="packed shape"):
        infer_tmix_lnx_rkvres_xg_forward_varlen(x[:, :100].contiguous(), x[:, :100].contiguous(),
                                                x[:, :100].contiguous(), x[:, :100].contiguous(),
                                                vec[:100], vec[:100], vec[:100],
                                                x[:, :100].contiguous())


# ---------------------------------------------------------- fused chain ---


def _chain_case(lengths, *, heads=3, dtype=torch.bfloat16, seed=0, pool_slots=None):
    g = torch.Generator().manual_seed(20261201 + seed)
    n = sum(lengths)
    d = 64
    shp = (n, heads, d)
    r = torch.randn(shp, generator=g).to(dtype)
    k = torch.randn(shp, generator=g).to(dtype)
    v = torch.randn(shp, generator=g).to(dtype)
    a12 = torch.randn(shp, generator=g).to(dtype)
    gate = torch.sigmoid(torch.randn(shp, generator=g)).to(dtype)
    decay_logits = (torch.randn(shp, generator=g) * 2.0).to(dtype)
    c = heads * d
    k_k = (1.0 + 0.3 * torch.randn(c, generator=g)).to(dtype)
    a0 = (0.5 * torch.randn(c, generator=g)).to(dtype)
    k_a = torch.rand(c, generator=g).to(dtype)
    r_k = (0.5 * torch.randn(c, generator=g)).to(dtype)
    ln_w = (1.0 + 0.2 * torch.randn(c, generator=g)).to(dtype)
    ln_b = (0.1 * torch.randn(c, generator=g)).to(dtype)
    slots_n = pool_slots or len(lengths) + 2
    pool = torch.randn((slots_n, heads, d, d), generator=g) * 0.1
    slots = torch.randperm(slots_n, generator=g)[: len(lengths)].to(torch.int32)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lengths)]), dtype=torch.int32)
    return dict(r=r, w=decay_logits, k=k, v=v, a12=a12, g=gate, k_k=k_k, a0=a0, k_a=k_a,
                r_k=r_k, ln_w=ln_w, ln_b=ln_b, pool=pool, cu=cu, slots=slots)


def _oracle_chain(c, decay_mode, scale):
    w = _np(c["w"])
    if decay_mode == DECAY_LOGITS:
        w = oracle.retention_from_logits(w)
    return oracle.tmix_fused(*(_np(c[n]) for n in ("r",)), w,
                             *(_np(c[n]) for n in ("k", "v", "a12", "g", "k_k", "a0", "k_a",
                                                   "r_k", "ln_w", "ln_b")),
                             _np(c["pool"]), c["cu"].numpy(), c["slots"].numpy(), scale=scale)


def _run_fused(c, decay_mode, scale, *, public=False):
    d = {n: t.to(DEV) for n, t in c.items()}
    pool = d["pool"].clone()
    args = [d[n] for n in ("r", "w", "k", "v", "a12", "g", "k_k", "a0", "k_a", "r_k",
                           "ln_w", "ln_b")]
    if public:
        out = infer_tmix_wkv7_fused_forward_varlen(*args, state_pool=pool, cu_seqlens=d["cu"],
                                                   state_indices=d["slots"], scale=scale)
    else:
        out = tmix_fused_internal(*args, state_pool=pool, cu_seqlens=d["cu"],
                                  state_indices=d["slots"], decay_mode=decay_mode, scale=scale)
    torch.cuda.synchronize()
    return out, pool


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
@pytest.mark.parametrize("lengths", ([1] * 7, [1, 5, 2, 9]))
def test_fused_chain_matches_fp64_chain(dtype, lengths):
    c = _chain_case(lengths, dtype=dtype, seed=len(lengths))
    out, pool = _run_fused(c, DECAY_LOGITS, 0.8, public=True)
    want_out, want_pool = _oracle_chain(c, DECAY_LOGITS, 0.8)
    _check(out, want_out, CHAIN_TOL, f"fused out {dtype} {lengths}")
    _check(pool, want_pool, CHAIN_TOL, f"fused pool {dtype} {lengths}")
    # untouched slots stay bitwise equal
    used = set(c["slots"].tolist())
    for s in range(c["pool"].shape[0]):
        if s not in used:
            assert torch.equal(pool[s].cpu(), c["pool"][s])


def test_fused_chain_raw_retention_mode():
    c = _chain_case([2, 3], seed=11)
    c["w"] = torch.exp(-torch.exp(torch.rand(c["w"].shape) * -5.0)).to(torch.bfloat16)
    out, pool = _run_fused(c, DECAY_RAW_W, 1.0)
    want_out, want_pool = _oracle_chain(c, DECAY_RAW_W, 1.0)
    _check(out, want_out, CHAIN_TOL, "fused out raw")
    _check(pool, want_pool, CHAIN_TOL, "fused pool raw")


def test_fused_chain_matches_three_kernel_composition():
    # fp16 io (the standalone ops' dtype): kk_a_gate -> recurrent WKV7 with
    # a = -kk, b = kk gate -> lnx_rkvres_xg, each on the GPU.
    c = _chain_case([1] * 16, heads=4, dtype=torch.float16, seed=3)
    out, pool = _run_fused(c, DECAY_LOGITS, 1.0)
    d = {n: t.to(DEV) for n, t in c.items()}
    n, h, hd = d["r"].shape
    flat = lambda t: t.reshape(n, h * hd)
    new_k, neg_kk, kka = infer_tmix_kk_a_gate_forward_varlen(
        flat(d["k"]), d["k_k"], d["a0"], flat(d["a12"]), d["k_a"])
    pool3 = d["pool"].clone()
    y = recurrent_forward_internal(d["r"], d["w"], new_k.reshape(n, h, hd), d["v"],
                                   neg_kk.reshape(n, h, hd), kka.reshape(n, h, hd),
                                   state_pool=pool3, cu_seqlens=d["cu"],
                                   state_indices=d["slots"], decay_mode=DECAY_LOGITS)
    out3 = infer_tmix_lnx_rkvres_xg_forward_varlen(
        flat(y), flat(d["r"]), new_k, flat(d["v"]), d["r_k"], d["ln_w"], d["ln_b"], flat(d["g"]))
    torch.cuda.synchronize()
    _check(out, _np(out3).reshape(n, h, hd), CHAIN_TOL, "fused vs composition out")
    _check(pool, _np(pool3), CHAIN_TOL, "fused vs composition pool")


def test_fused_chain_fails_closed_and_accepts_a_ticket():
    c = _chain_case([1, 1, 1], seed=5)
    d = {n: t.to(DEV) for n, t in c.items()}
    args = [d[n] for n in ("r", "w", "k", "v", "a12", "g", "k_k", "a0", "k_a", "r_k",
                           "ln_w", "ln_b")]
    # duplicate slots through the C ABI with the device validation: NaN output,
    # pool bitwise unchanged
    bad_slots = torch.tensor([1, 1, 0], dtype=torch.int32, device=DEV)
    status, cu_snap, slot_snap = capi.metadata_validate(d["cu"], bad_slots, 3,
                                                        d["pool"].shape[0])
    pool = d["pool"].clone()
    out = torch.empty_like(d["v"])
    capi.recurrent_tmix_fused_forward(*args, state_pool=pool, cu_seqlens=cu_snap,
                                      state_indices=slot_snap, metadata_status=status,
                                      output=out)
    torch.cuda.synchronize()
    assert int(status.item()) != 0
    assert torch.isnan(out).all()
    assert torch.equal(pool, d["pool"])
    # a prepared ticket is accepted and gives the unticketed result bitwise
    ticket = prepare_recurrent_metadata(d["cu"], d["slots"], total_tokens=3,
                                        state_pool_size=d["pool"].shape[0])
    p1, p2 = d["pool"].clone(), d["pool"].clone()
    o1 = infer_tmix_wkv7_fused_forward_varlen(*args, state_pool=p1, cu_seqlens=d["cu"],
                                              state_indices=d["slots"],
                                              validated_metadata=ticket)
    o2 = infer_tmix_wkv7_fused_forward_varlen(*args, state_pool=p2, cu_seqlens=d["cu"],
                                              state_indices=d["slots"])
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(p1, p2)
