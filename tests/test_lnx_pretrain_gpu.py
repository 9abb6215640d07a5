"""GPU parity of the consumer's training form, ``pretrain_tmix_lnx_rkvres_xg_bf16``.

Expected values: the fp64 oracle (``oracle.lnx_pretrain_forward`` /
``lnx_pretrain_backward``, pinned in tests/test_oracle.py by loops, central
differences and torch fp64 autograd) fed the same bf16 inputs and the same
bf16 upstream gradient. Arithmetic is fp32 with one bf16 rounding per output
(the parameter gradients are fp32 sums over rows, rounded once), so every
output is held to 1e-2 normwise and per row; the reference's own test
(tests/tmix/lnx_rkvres_xg/test.py:69-89) only checks shapes and finiteness,
which the first case repeats with its inputs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import flashrwkv_amd
from flashrwkv_amd import capi
from flashrwkv_amd.tmix.lnx_rkvres_xg import pretrain_tmix_lnx_rkvres_xg_bf16
from oracle import oracle
from tests import parity

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
TOL = 1e-2
NAMES = ("x", "r", "k", "v", "residual_scale", "weight", "bias", "g")
GRAD_KEYS = ("dx", "dr", "dk", "dv", "dresidual_scale", "dweight", "dbias", "dg")


@pytest.fixture(scope="module", autouse=True)
def _require_native():
    if flashrwkv_amd._C is None:
        pytest.fail("flashrwkv_amd native library is not built (no fallback exists)")


def _check(name, actual, expected):
    """Normwise and per row (floor 1e-2) within 1e-2; elementwise at floor
    0.1 within 2e-2."""
    return parity.check(name, actual, expected, TOL, row_tol=TOL, elem_tol=2e-2,
                        elem_floor=0.1)


def _inputs(b, t, heads, d, seed, token_scale=0.03, gate_scale=0.1, residual_scale=0.1):
    """The reference test's recipe (tests/tmix/lnx_rkvres_xg/test.py:72-82)."""
    gen = torch.Generator().manual_seed(seed)
    c = heads * d
    toks = [(torch.randn(b, t, c, generator=gen) * token_scale).to(torch.bfloat16)
            for _ in range(4)]
    rs = (torch.randn(heads, d, generator=gen) * residual_scale).to(torch.bfloat16)
    w = torch.randn(c, generator=gen).to(torch.bfloat16)
    bias = torch.randn(c, generator=gen).to(torch.bfloat16)
    g = (torch.randn(b, t, c, generator=gen) * gate_scale).to(torch.bfloat16)
    return [*toks, rs, w, bias, g]


def _oracle(values, dy, d):
    c = values[0].shape[-1]
    flat = [v.double().numpy().reshape(-1, c) if v.dim() == 3 else v.double().numpy()
            for v in values]
    out, mean, rstd = oracle.lnx_pretrain_forward(*flat, head_size=d)
    grads = oracle.lnx_pretrain_backward(dy.double().numpy().reshape(-1, c), *flat,
                                         head_size=d)
    return out, mean, rstd, grads


@pytest.mark.parametrize("head_size", (64, 128, 256))
def test_reference_case_forward_backward(head_size):
    """The reference test's shapes and inputs (B=2, T=3, C=2D), its loss
    (mean of the squared output) for shapes and finiteness, then every output
    and gradient against the oracle with an explicit bf16 upstream gradient."""
    values = [t.to(DEV).requires_grad_() for t in _inputs(2, 3, 2, head_size, seed=23)]
    out = pretrain_tmix_lnx_rkvres_xg_bf16(*values, head_size=head_size)
    out.float().square().mean().backward()
    assert out.shape == values[0].shape and out.dtype == torch.bfloat16
    assert all(t.grad is not None and torch.isfinite(t.grad.float()).all() for t in values)
    dy = torch.randn(out.shape, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    grads = torch.autograd.grad(pretrain_tmix_lnx_rkvres_xg_bf16(*values, head_size=head_size),
                                values, dy.to(DEV))
    ref_out, _, _, ref = _oracle([v.detach().cpu() for v in values], dy, head_size)
    _check("out", out.detach().reshape(-1, out.shape[-1]), ref_out)
    for key, grad in zip(GRAD_KEYS, grads):
        want = ref[key]
        _check(key, grad.reshape(want.shape), want)


@pytest.mark.parametrize("b,t,heads,d", [(2, 512, 12, 64), (3, 100, 5, 128), (1, 70, 3, 256),
                                         (2, 65, 9, 64)])
def test_forward_statistics_and_gradients_match_oracle(b, t, heads, d):
    """Token counts that are not multiples of the backward's 64-token blocks,
    channel counts that leave the last 512-column block partial (C = 768,
    640, 576), the pretraining bench shape (2, 512, 12, 64); the saved mean
    and rstd, the output and all eight gradients against the oracle, through
    the C ABI, and the two-pass backward bitwise deterministic."""
    print(f"case B={b} T={t} H={heads} D={d}", flush=True)
    cpu = _inputs(b, t, heads, d, seed=100 + d + t, token_scale=1.0, gate_scale=1.0)
    dy = torch.randn(cpu[0].shape, generator=torch.Generator().manual_seed(7)).to(torch.bfloat16)
    values = [v.to(DEV) for v in cpu]
    c = heads * d
    out = torch.empty_like(values[0])
    mean = torch.empty((b, t, heads), device=DEV)
    rstd = torch.empty_like(mean)
    capi.lnx_pretrain_forward(*values, output=out, mean=mean, rstd=rstd, head_size=d)
    runs = []
    for _ in range(2):
        grads = [torch.empty_like(v) for v in values]
        capi.lnx_pretrain_backward(dy.to(DEV), *values, mean, rstd, grads=grads, head_size=d)
        runs.append(grads)
    torch.cuda.synchronize()
    ref_out, ref_mean, ref_rstd, ref = _oracle(cpu, dy, d)
    _check("out", out.reshape(-1, c), ref_out)
    _check("mean", mean.reshape(-1, heads), ref_mean)
    _check("rstd", rstd.reshape(-1, heads), ref_rstd)
    for key, grad in zip(GRAD_KEYS, runs[0]):
        _check(key, grad.reshape(ref[key].shape), ref[key])
    for a, e in zip(*runs):
        assert torch.equal(a, e)


def test_backward_rejects_short_workspace_before_launch():
    values = [v.to(DEV) for v in _inputs(1, 64, 2, 64, seed=3)]
    mean = torch.zeros((1, 64, 2), device=DEV)
    grads = [torch.empty_like(v) for v in values]
    need = int(capi.library().frwkv_lnx_pretrain_backward_workspace_bytes(64, 2, 64))
    assert need == 3 * 128 * 4
    with pytest.raises(RuntimeError, match="workspace of 256 bytes given"):
        capi.lnx_pretrain_backward(values[0], *values, mean, mean, grads=grads, head_size=64,
                                   work=torch.empty(256, dtype=torch.uint8, device=DEV))
