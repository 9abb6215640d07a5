"""Pretraining (clampw v3) operator: GPU parity and the reference's contract.

Expected values: the fp64 oracle (oracle/wkv7_oracle.c, restating the
reference's clampw recurrence tests/tmix/wkv7/pretrain/test.py:49-70: S0 = 0,
retention exp(-e^{-1/2} sigmoid(w))), fed the same bf16 inputs. The oracle's
forward over 16-token segments gives the boundary states every 16 tokens
and a^T S_{t-1}; its adjoint gives every gradient (dL/dw scaled by
w d(log w)/dx for the logits). Tolerance: normwise max relative error 2e-2
(bf16 operands on MFMA, fp32 accumulation and state). Cases follow the
reference test's shapes, plus lengths that are not multiples of 64.
"""

from __future__ import annotations

import inspect

import numpy as np
import pytest
import torch

import flashrwkv_amd
from flashrwkv_amd import capi
from flashrwkv_amd.tmix.wkv7 import pretrain_recurrent_bf16
from oracle import oracle
from tests import parity

TOL = 2e-2
NAMES = ("r", "w", "k", "v", "a", "b")


def test_public_contract_matches_clampw_v3():
    """Reference test.py:83-90 (signature and exports); runs without a GPU."""
    signature = inspect.signature(pretrain_recurrent_bf16)
    assert tuple(signature.parameters) == ("r", "w", "k", "v", "a", "b", "head_size")
    assert signature.parameters["head_size"].default == 64
    assert flashrwkv_amd.pretrain_recurrent_bf16 is pretrain_recurrent_bf16
    assert "pretrain_recurrent_bf16" in flashrwkv_amd.__all__
    assert not hasattr(flashrwkv_amd, "pretrain_recurrent_fp32io16")
    if flashrwkv_amd._C is not None:
        assert hasattr(torch.ops.rwkv7_clampw_v3, "forward")
        assert hasattr(torch.ops.rwkv7_clampw_v3, "backward")


def _case(batch, tokens, heads, *, scale=0.05, seed=20260806, d=64):
    """Reference test.py:31-46: six N(0, 1) * scale bf16 tensors [B,T,H*D]."""
    g = torch.Generator().manual_seed(seed + batch + tokens + heads)
    shape = (batch, tokens, heads * d)
    return [(torch.randn(shape, generator=g) * scale).to(torch.bfloat16) for _ in range(6)]


def _np(t):
    return t.detach().double().cpu().numpy()


def _check(name, actual, expected, tol=TOL):
    """Normwise ``tol``; per row (floor 1e-2) within 0.5 and elementwise
    (floor 0.1) within 0.2 (measured at most 0.29 and 0.11). These cases'
    a and b are independent N(0, s^2) vectors (the reference test's recipe),
    not RWKV-7's a = -kk, b = kk g with |kk| = 1: at s = 0.3, |a||b| is about
    6, the chunk form's (I - Lab)^-1 has entries far above 1 and amplifies
    the bf16 rounding of its operands, so low-norm rows carry relative errors
    that the normalised inputs of the other tests (about 1e-2) do not."""
    return parity.check(name, actual, expected, tol, row_tol=0.5, elem_tol=0.2,
                        elem_floor=0.1)


def _oracle(values, dy, batch, tokens, heads, d=64):
    """fp64 forward (16-token segments) and adjoint of the clampw recurrence."""
    packed = [_np(t).reshape(batch * tokens, heads, d) for t in values]
    x = packed[1]
    w = oracle.retention_from_logits(x)
    args = [packed[0], w, *packed[2:]]
    s0 = np.zeros((batch, heads, d, d))
    slots = np.arange(batch, dtype=np.int32)
    meta16 = oracle.chunk_metadata([tokens] * batch, 16)
    y, _, bnd, sda = oracle.forward(*args, s0, seg_offsets=meta16[0], seg_starts=meta16[1],
                                    seg_ends=meta16[2], state_slots=slots,
                                    want_boundary=True, want_state_dot_a=True)
    grads = None
    if dy is not None:
        meta = oracle.chunk_metadata([tokens] * batch, 64)
        grads = oracle.backward(*args, s0, seg_offsets=meta[0], seg_starts=meta[1],
                                seg_ends=meta[2], state_slots=slots,
                                dy=_np(dy).reshape(batch * tokens, heads, d))
        grads["dw"] = grads["dw"] * w * oracle.retention_log_derivative(x)
    return y, bnd, sda, grads


@pytest.mark.gpu
@pytest.mark.parametrize("batch,tokens,heads", [(1, 16, 1), (2, 32, 2), (2, 144, 3),
                                                (1, 256, 2)])
def test_forward_matches_clampw_recurrence(batch, tokens, heads):
    values = _case(batch, tokens, heads)
    dev = [t.cuda() for t in values]
    out = pretrain_recurrent_bf16(*dev)
    torch.cuda.synchronize()
    assert out.shape == dev[0].shape and out.dtype == torch.bfloat16
    y_ref, _, _, _ = _oracle(values, None, batch, tokens, heads)
    _check("y", out.reshape(batch * tokens, heads, 64), y_ref)
    # Bitwise determinism (reference test.py:104).
    assert torch.equal(out, pretrain_recurrent_bf16(*dev))


@pytest.mark.gpu
@pytest.mark.parametrize("batch,tokens,heads", [(1, 64, 1), (2, 208, 2)])
def test_op_boundary_every_16_tokens_and_state_dot_a(batch, tokens, heads):
    """torch.ops.rwkv7_clampw_v3.forward's s ([B,H,T/16,D,D]: the state before
    token 16 i) and sa ([B,T,H,D]: a_t^T S_{t-1})."""
    values = _case(batch, tokens, heads, scale=0.3, seed=11)
    dev = [t.cuda().view(batch, tokens, heads, 64) for t in values]
    y = torch.empty_like(dev[3])
    s = torch.empty((batch, heads, tokens // 16, 64, 64), device="cuda")
    sa = torch.empty((batch, tokens, heads, 64), device="cuda")
    torch.ops.rwkv7_clampw_v3.forward(*dev, y, s, sa, 64)
    torch.cuda.synchronize()
    y_ref, bnd_ref, sda_ref, _ = _oracle(values, None, batch, tokens, heads)
    _check("y", y.reshape(batch * tokens, heads, 64), y_ref)
    _check("s", s.permute(0, 2, 1, 3, 4).reshape(-1, heads, 64, 64), bnd_ref)
    _check("sa", sa.reshape(batch * tokens, heads, 64), sda_ref)


@pytest.mark.gpu
@pytest.mark.parametrize("batch,tokens,heads", [(1, 16, 1), (2, 144, 2)])
def test_backward_matches_clampw_recurrence(batch, tokens, heads):
    """Reference test.py:107-129, against the fp64 adjoint."""
    values = _case(batch, tokens, heads, scale=0.3, seed=17)
    leaves = [t.cuda().requires_grad_(True) for t in values]
    out = pretrain_recurrent_bf16(*leaves)
    g = torch.Generator().manual_seed(5)
    dy = torch.randn(out.shape, generator=g).to(torch.bfloat16)
    out.backward(dy.cuda())
    torch.cuda.synchronize()
    _, _, _, grads = _oracle(values, dy, batch, tokens, heads)
    for name, leaf in zip(NAMES, leaves):
        assert torch.isfinite(leaf.grad.float()).all()
        _check(f"d{name}", leaf.grad.reshape(batch * tokens, heads, 64), grads["d" + name])


@pytest.mark.gpu
def test_c_abi_pretrain_forward_backward():
    """The same path straight through the C ABI (frwkv_pretrain_forward/backward)."""
    batch, tokens, heads = 1, 80, 2
    values = _case(batch, tokens, heads, scale=0.3, seed=23)
    dev = [t.cuda().view(batch, tokens, heads, 64) for t in values]
    y = torch.empty_like(dev[3])
    s = torch.empty((batch, heads, tokens // 16, 64, 64), device="cuda")
    sa = torch.empty((batch, tokens, heads, 64), device="cuda")
    capi.pretrain_forward(*dev, output=y, boundary=s, state_dot_a=sa)
    g = torch.Generator().manual_seed(9)
    dy = torch.randn(y.shape, generator=g).to(torch.bfloat16)
    grads = [torch.empty_like(t) for t in dev]
    capi.pretrain_backward(*dev, grad_output=dy.cuda(), boundary=s, grads=grads)
    torch.cuda.synchronize()
    y_ref, _, _, ref = _oracle(values, dy.view(batch, tokens, heads * 64), batch, tokens,
                               heads)
    _check("y", y.reshape(-1, heads, 64), y_ref)
    for name, grad in zip(NAMES, grads):
        _check(f"d{name}", grad.reshape(-1, heads, 64), ref["d" + name])


@pytest.mark.gpu
def test_invalid_input_contract_is_rejected():
    """Reference test.py:147-166 (same error types and messages)."""
    valid = [t.cuda() for t in _case(1, 16, 1)]
    with pytest.raises(TypeError, match="bfloat16"):
        pretrain_recurrent_bf16(valid[0].float(), *valid[1:])
    with pytest.raises(ValueError, match="T must be divisible"):
        pretrain_recurrent_bf16(*[t[:, :15].contiguous() for t in valid])
    with pytest.raises(ValueError, match="C must be divisible"):
        pretrain_recurrent_bf16(*[t[:, :, :63].contiguous() for t in valid])
    with pytest.raises(ValueError, match="must match r shape"):
        pretrain_recurrent_bf16(valid[0], valid[1][:, :, :32].contiguous(), *valid[2:])
    with pytest.raises(ValueError, match="contiguous CUDA"):
        pretrain_recurrent_bf16(valid[0].transpose(1, 2), *valid[1:])
    with pytest.raises(ValueError, match="contiguous CUDA"):
        pretrain_recurrent_bf16(*[t.cpu() for t in valid])
    # The input's last dimension must be a multiple of head_size.
    with pytest.raises(ValueError, match="C must be divisible"):
        pretrain_recurrent_bf16(*valid, head_size=128)


# ---------------------------------------------------------------- head sizes 128 and 256 ----
# Head size 128 trains with the bf16 MFMA forward and backward over 16-token
# pieces, head size 256 with the per-token fp32 kernels. Same oracle; bf16
# inputs, fp32 state, bf16 outputs and gradients.

# Input scale of the head-size-128 cases. Their inputs are six independent
# N(0, s^2) vectors (not RWKV-7's a = -kk, b = kk g with |kk| = 1); at
# 128 features |a||b| is about 128 s^2, and the piece's (I - Lab)^-1 then
# amplifies the bf16 rounding of the MFMA operands. Measured normwise
# errors with the MFMA forward and backward: s = 0.2, 3.9e-3 .. 9.3e-3 for
# the gradients and at most 7.5e-3 for y, the 16-token states and a^T S;
# s = 0.3, 9.8e-3 .. 1.1e-1. The cases below run at 0.2 within the 2e-2
# bound (the reference test's own scale is 0.05,
# tests/tmix/wkv7/pretrain/test.py:30-46, with elementwise rtol 0.08 for
# the gradients, test.py:143-144); test_head128_ill_conditioned_inputs
# keeps s = 0.3 finite and within normwise 0.15.
HEAD128_SCALE = 0.2


@pytest.mark.gpu
@pytest.mark.parametrize("head_size", (128, 256))
@pytest.mark.parametrize("batch,tokens,heads", [(1, 16, 1), (2, 48, 2)])
def test_generalized_forward_backward_matches_recurrence(head_size, batch, tokens, heads):
    """Reference test.py:131-145 (head sizes 128 and 256), against the fp64
    forward and adjoint."""
    scale = HEAD128_SCALE if head_size == 128 else 0.3
    values = _case(batch, tokens, heads, scale=scale, seed=29, d=head_size)
    leaves = [t.cuda().requires_grad_(True) for t in values]
    out = pretrain_recurrent_bf16(*leaves, head_size=head_size)
    g = torch.Generator().manual_seed(31)
    dy = torch.randn(out.shape, generator=g).to(torch.bfloat16)
    out.backward(dy.cuda())
    torch.cuda.synchronize()
    y_ref, _, _, grads = _oracle(values, dy, batch, tokens, heads, d=head_size)
    _check("y", out.reshape(batch * tokens, heads, head_size), y_ref)
    for name, leaf in zip(NAMES, leaves):
        assert torch.isfinite(leaf.grad.float()).all()
        _check(f"d{name}", leaf.grad.reshape(batch * tokens, heads, head_size),
               grads["d" + name])
    # Forward bitwise determinism (reference test.py:104).
    again = pretrain_recurrent_bf16(*[t.detach() for t in leaves], head_size=head_size)
    assert torch.equal(out.detach(), again)


@pytest.mark.gpu
@pytest.mark.parametrize("head_size", (128, 256))
def test_op_boundary_and_state_dot_a_large_heads(head_size):
    """The op's s (state before every 16th token) and sa at head sizes 128/256,
    and the C ABI backward with the gradients of every input."""
    batch, tokens, heads = 2, 64, 1
    scale = HEAD128_SCALE if head_size == 128 else 0.3
    values = _case(batch, tokens, heads, scale=scale, seed=37, d=head_size)
    dev = [t.cuda().view(batch, tokens, heads, head_size) for t in values]
    y = torch.empty_like(dev[3])
    s = torch.empty((batch, heads, tokens // 16, head_size, head_size), device="cuda")
    sa = torch.empty((batch, tokens, heads, head_size), device="cuda")
    torch.ops.rwkv7_clampw_v3.forward(*dev, y, s, sa, head_size)
    g = torch.Generator().manual_seed(41)
    dy = torch.randn(y.shape, generator=g).to(torch.bfloat16)
    grads = [torch.empty_like(t) for t in dev]
    capi.pretrain_backward(*dev, grad_output=dy.cuda(), boundary=s, grads=grads)
    torch.cuda.synchronize()
    y_ref, bnd_ref, sda_ref, ref = _oracle(values, dy.view(batch, tokens, heads * head_size),
                                           batch, tokens, heads, d=head_size)
    _check("y", y.reshape(-1, heads, head_size), y_ref)
    _check("s", s.permute(0, 2, 1, 3, 4).reshape(-1, heads, head_size, head_size), bnd_ref)
    _check("sa", sa.reshape(-1, heads, head_size), sda_ref)
    for name, grad in zip(NAMES, grads):
        _check(f"d{name}", grad.reshape(-1, heads, head_size), ref["d" + name])


@pytest.mark.gpu
@pytest.mark.parametrize("seed", (29, 37))
def test_head128_ill_conditioned_inputs(seed):
    """Head size 128 at the input scale 0.3 (six times the reference test's):
    |a||b| is about 11, and the chunk form's (I - Lab)^-1 amplifies the bf16
    rounding of its operands in the forward's 16-token states (normwise
    error 9e-3 .. 4.5e-2) and in the backward. The bf16 MFMA forward and
    backward stay finite and within normwise 0.15; measured 9.8e-3 .. 1.1e-1
    (dw at seed 37, of which 5.4e-2 remains when the backward starts from
    exact states)."""
    batch, tokens, heads, d = 2, 64, 1, 128
    values = _case(batch, tokens, heads, scale=0.3, seed=seed, d=d)
    leaves = [t.cuda().requires_grad_(True) for t in values]
    out = pretrain_recurrent_bf16(*leaves, head_size=d)
    g = torch.Generator().manual_seed(41)
    dy = torch.randn(out.shape, generator=g).to(torch.bfloat16)
    out.backward(dy.cuda())
    torch.cuda.synchronize()
    _, _, _, grads = _oracle(values, dy, batch, tokens, heads, d=d)
    for name, leaf in zip(NAMES, leaves):
        assert torch.isfinite(leaf.grad.float()).all()
        err = parity.normwise(leaf.grad.reshape(batch * tokens, heads, d), grads["d" + name])
        assert err <= 0.15, (name, err)
