"""CPU tests of the public Python layer: the ``flashrwkv2`` import path, the
reference signatures, the argument contracts (types, messages and order,
which all run before any launch) and the chunk-list builders."""

from __future__ import annotations

import inspect

import numpy as np
import pytest
import torch

import flashrwkv2
import flashrwkv_amd
from flashrwkv_amd.rl_infctx.wkv7 import chunk_lists

_REQ = inspect.Parameter.empty

# Public signatures of the reference (positional names, keyword-only names
# with defaults; `_REQ` = required), read from the reference's Python sources:
# tmix/wkv7/__init__.py, chunk.py, statetune.py, pretrain.py,
# rl_infctx/wkv7/__init__.py, tmix/kk_a_gate, tmix/lnx_rkvres_xg.
_TOKENS = ["r", "decay_logits", "k", "v", "a", "b"]
REFERENCE_SIGNATURES = {
    "flashrwkv2.tmix.wkv7.prepare_recurrent_metadata": (
        ["cu_seqlens", "state_indices"],
        [("total_tokens", _REQ), ("state_pool_size", _REQ), ("max_seqlen", None)]),
    "flashrwkv2.tmix.wkv7.infer_recurrent_fp32io16_forward_varlen": (
        _TOKENS,
        [("state_pool", _REQ), ("cu_seqlens", _REQ), ("state_indices", _REQ), ("scale", 1.0),
         ("decay_bias", None), ("max_seqlen", None), ("validated_metadata", None)]),
    "flashrwkv2.tmix.wkv7.infer_recurrent_fp16_forward_varlen": (
        _TOKENS,
        [("state_pool", _REQ), ("elapsed_state_pool", _REQ), ("cu_seqlens", _REQ),
         ("state_indices", _REQ), ("scale", 1.0), ("decay_bias", None), ("max_seqlen", None),
         ("validated_metadata", None)]),
    "flashrwkv2.tmix.wkv7.infer_recurrent_fp16_advance_i32": (["elapsed_state", "amount"], []),
    "flashrwkv2.tmix.wkv7.infer_recurrent_fp16_advance_i32_varlen": (
        ["elapsed_state_pool", "cu_seqlens", "state_indices"],
        [("total_tokens", _REQ), ("validated_metadata", None)]),
    "flashrwkv2.tmix.wkv7.infer_recurrent_add_vec_forward_varlen": (["x", "vec"], []),
    "flashrwkv2.tmix.wkv7.chunk.infer_chunk_bf16_forward_varlen": (
        _TOKENS,
        [("state_pool", _REQ), ("cu_seqlens", _REQ), ("state_indices", _REQ),
         ("chunk_size", 16), ("max_seqlen", None), ("scale", 1.0), ("decay_bias", None),
         ("validated_metadata", None)]),
    "flashrwkv2.tmix.wkv7.statetune.statetune_recurrent_fp32io16": (
        ["initial_state", "sequence_chunk_offsets", "chunk_token_starts", "chunk_token_ends",
         *_TOKENS], [("scale", 1.0)]),
    "flashrwkv2.tmix.wkv7.pretrain.pretrain_recurrent_bf16": (
        ["r", "w", "k", "v", "a", "b"], [("head_size", 64)]),
    "flashrwkv2.rl_infctx.wkv7.rl_infctx_chunk_fp32io16": (
        _TOKENS,
        [("state_pool", None), ("cu_seqlens", _REQ), ("state_indices", None),
         ("chunk_size", 16), ("strategy", "recompute"), ("scale", 1.0), ("decay_bias", None)]),
    "flashrwkv2.tmix.kk_a_gate.infer_tmix_kk_a_gate_forward_varlen": (
        ["k", "k_k", "a0", "a12", "k_a"],
        [("head_size", 64), ("batch_size", 1), ("max_seqlen", None)]),
    "flashrwkv2.tmix.lnx_rkvres_xg.infer_tmix_lnx_rkvres_xg_forward_varlen": (
        ["x", "r", "k", "v", "r_k", "weight", "bias", "g"],
        [("head_size", 64), ("batch_size", 1), ("max_seqlen", None)]),
    "flashrwkv2.tmix.lnx_rkvres_xg.pretrain_tmix_lnx_rkvres_xg_bf16": (
        ["x", "r", "k", "v", "residual_scale", "weight", "bias", "g"], [("head_size", 64)]),
    "flashrwkv2.tmix.lnx_rkvres_xg.pretrain.pretrain_tmix_lnx_rkvres_xg_bf16": (
        ["x", "r", "k", "v", "residual_scale", "weight", "bias", "g"], [("head_size", 64)]),
    "flashrwkv2.pretrain_tmix_lnx_rkvres_xg_bf16": (
        ["x", "r", "k", "v", "residual_scale", "weight", "bias", "g"], [("head_size", 64)]),
}


def _resolve(path: str):
    module_path, name = path.rsplit(".", 1)
    module = __import__(module_path, fromlist=[name])
    return getattr(module, name)


@pytest.mark.parametrize("path", sorted(REFERENCE_SIGNATURES))
def test_reference_import_paths_and_signatures(path):
    fn = _resolve(path)
    positional, keywords = REFERENCE_SIGNATURES[path]
    params = list(inspect.signature(fn).parameters.values())
    pos = [p.name for p in params if p.kind == p.POSITIONAL_OR_KEYWORD]
    kw = [(p.name, p.default) for p in params if p.kind == p.KEYWORD_ONLY]
    assert pos == positional
    assert kw == keywords


def test_flashrwkv2_modules_are_the_build_modules():
    import flashrwkv2.rl_infctx.wkv7 as rl
    import flashrwkv2.tmix.wkv7 as wkv7
    import flashrwkv2.tmix.wkv7.chunk as chunk
    import flashrwkv2.tmix.wkv7.pretrain as pretrain
    import flashrwkv2.tmix.wkv7.statetune as statetune
    import flashrwkv_amd.tmix.wkv7 as impl

    assert wkv7 is impl
    assert chunk.infer_chunk_bf16_forward_varlen is impl.infer_chunk_bf16_forward_varlen
    assert statetune.statetune_recurrent_fp32io16 is flashrwkv2.statetune_recurrent_fp32io16
    assert pretrain.pretrain_recurrent_bf16 is flashrwkv2.pretrain_recurrent_bf16
    assert rl.rl_infctx_chunk_fp32io16 is flashrwkv2.rl_infctx_chunk_fp32io16
    assert flashrwkv2._C is flashrwkv_amd._C
    for name in flashrwkv2.__all__:
        assert callable(getattr(flashrwkv2, name))


def test_native_namespace_and_ticket_method_names():
    if flashrwkv_amd._C is None:
        pytest.skip("native libraries not built")
    import sys

    assert sys.modules["flashrwkv2._C"] is flashrwkv_amd._C
    ops = torch.ops.flashrwkv2
    for name in ("prepare_recurrent_metadata", "recurrent_fp32_from_decay_logits",
                 "infer_chunk_bf16_forward_varlen", "statetune_recurrent_fp32io16_forward",
                 "statetune_recurrent_fp32io16_backward", "rl_infctx_chunk_fp32io16_forward",
                 "recurrent_fp16_from_decay_logits"):
        assert hasattr(ops, name)
    schema = str(ops.prepare_recurrent_metadata.default._schema)
    assert "torch.classes.flashrwkv2.MetadataTicket" in schema
    assert hasattr(torch.ops.rwkv7_clampw_v3, "forward")
    methods = {str(s).split("(")[0] for s in torch._C._jit_get_custom_class_schemas()
               if "classes.flashrwkv2.MetadataTicket _0" in str(s)}
    for method in ("_check_compatible", "_status", "_max_seqlen", "_query_start_loc_snapshot",
                   "_state_indices_snapshot", "check_compatible", "max_seqlen"):
        assert method in methods, method


# ------------------------------------------------------------- contracts --
def _tokens(n=4, h=2, d=64, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(0)
    return [torch.randn(n, h, d, generator=g).to(dtype) for _ in range(6)]


def _meta():
    return torch.tensor([0, 4], dtype=torch.int32), torch.tensor([0], dtype=torch.int32)


def test_recurrent_contract_order():
    from flashrwkv2.tmix.wkv7 import infer_recurrent_fp32io16_forward_varlen as fwd

    r, w, k, v, a, b = _tokens()
    cu, si = _meta()
    pool = torch.zeros(1, 2, 64, 64)
    kw = dict(state_pool=pool, cu_seqlens=cu, state_indices=si)
    with pytest.raises(TypeError, match="^r must be a torch.Tensor$"):
        fwd(None, w, k, v, a, b, **kw)
    with pytest.raises(ValueError, match=r"^k must have packed shape \[total_tokens,H,D\]$"):
        fwd(r, w, k[0], v, a, b, **kw)
    with pytest.raises(ValueError, match="^decay_logits must be contiguous$"):
        fwd(r, w.transpose(0, 1), k, v, a, b, **kw)
    # tokens are checked before the pool, the pool before the metadata
    with pytest.raises(TypeError, match="^b must be a torch.Tensor$"):
        fwd(r, w, k, v, a, 1.0, state_pool=None, cu_seqlens=None, state_indices=si)
    with pytest.raises(TypeError, match="^state_pool must be a torch.Tensor$"):
        fwd(r, w, k, v, a, b, state_pool=None, cu_seqlens=None, state_indices=si)
    with pytest.raises(ValueError, match="^state_pool must be contiguous$"):
        fwd(r, w, k, v, a, b, **{**kw, "state_pool": pool.transpose(2, 3)})
    with pytest.raises(TypeError, match="^state_pool must have dtype float32$"):
        fwd(r, w, k, v, a, b, **{**kw, "state_pool": pool.half()})
    with pytest.raises(TypeError, match="^cu_seqlens must be a torch.Tensor$"):
        fwd(r, w, k, v, a, b, **{**kw, "cu_seqlens": [0, 4]})
    with pytest.raises(ValueError, match="^cu_seqlens must be one-dimensional$"):
        fwd(r, w, k, v, a, b, **{**kw, "cu_seqlens": cu[None]})
    with pytest.raises(TypeError, match="^state_indices must be a torch.Tensor$"):
        fwd(r, w, k, v, a, b, **{**kw, "state_indices": 0})


def test_fp16_and_helper_contracts():
    from flashrwkv2.tmix.wkv7 import (
        infer_recurrent_add_vec_forward_varlen,
        infer_recurrent_fp16_advance_i32,
        infer_recurrent_fp16_advance_i32_varlen,
        infer_recurrent_fp16_forward_varlen,
    )

    r, w, k, v, a, b = _tokens(dtype=torch.float16)
    cu, si = _meta()
    pool = torch.zeros(1, 2, 64, 64, dtype=torch.float16)
    elapsed = torch.zeros(1, dtype=torch.int32)
    kw = dict(state_pool=pool, elapsed_state_pool=elapsed, cu_seqlens=cu, state_indices=si)
    with pytest.raises(TypeError, match="^FP16-state state_pool must have dtype float16$"):
        infer_recurrent_fp16_forward_varlen(r, w, k, v, a, b, **{**kw, "state_pool": pool.float()})
    with pytest.raises(TypeError, match="^elapsed_state_pool must have dtype torch.int32$"):
        infer_recurrent_fp16_forward_varlen(r, w, k, v, a, b,
                                            **{**kw, "elapsed_state_pool": elapsed.long()})
    with pytest.raises(ValueError, match="^elapsed_state_pool must be contiguous CUDA int32$"):
        infer_recurrent_fp16_forward_varlen(r, w, k, v, a, b, **kw)
    with pytest.raises(TypeError, match="^elapsed_state must be a torch.Tensor$"):
        infer_recurrent_fp16_advance_i32([1], 1)
    with pytest.raises(TypeError, match="^elapsed_state must have dtype torch.int32$"):
        infer_recurrent_fp16_advance_i32(elapsed.float(), 1)
    with pytest.raises(ValueError, match="^elapsed_state must be contiguous CUDA int32$"):
        infer_recurrent_fp16_advance_i32(elapsed, 1)
    with pytest.raises(ValueError, match="^elapsed_state_pool must be non-empty contiguous"):
        infer_recurrent_fp16_advance_i32_varlen(elapsed, cu, si, total_tokens=4)
    with pytest.raises(TypeError, match="^x must be a torch.Tensor$"):
        infer_recurrent_add_vec_forward_varlen(None, None)
    with pytest.raises(TypeError, match="^x must have dtype torch.float16$"):
        infer_recurrent_add_vec_forward_varlen(torch.zeros(2, 4), torch.zeros(4))
    with pytest.raises(ValueError, match="^x must be contiguous CUDA float16$"):
        infer_recurrent_add_vec_forward_varlen(torch.zeros(2, 4, dtype=torch.float16),
                                               torch.zeros(4))


def test_chunk_contract_order():
    from flashrwkv2.tmix.wkv7.chunk import infer_chunk_bf16_forward_varlen as chunk

    r, w, k, v, a, b = _tokens()
    cu, si = _meta()
    kw = dict(state_pool=torch.zeros(1, 2, 64, 64, dtype=torch.bfloat16), cu_seqlens=cu,
              state_indices=si)
    with pytest.raises(TypeError, match="^chunk_size must be an integer$"):
        chunk(r, w, k, v, a, b, **kw, chunk_size=True)
    with pytest.raises(ValueError, match="^chunk_size must be positive$"):
        chunk(r, w, k, v, a, b, **kw, chunk_size=0)
    with pytest.raises(ValueError, match="^scale must be finite$"):
        chunk(r, w, k, v, a, b, **kw, scale=float("nan"))
    with pytest.raises(TypeError, match="^r must be a torch.Tensor$"):
        chunk(None, w, k, v, a, b, **kw)
    with pytest.raises(ValueError, match="^r must be contiguous CUDA bfloat16$"):
        chunk(r, w, k, v, a, b, **kw)


def test_statetune_contract_order():
    from flashrwkv2.tmix.wkv7.statetune import statetune_recurrent_fp32io16 as st

    r, w, k, v, a, b = _tokens()
    offs = torch.tensor([0, 1], dtype=torch.int32)
    starts = torch.tensor([0], dtype=torch.int32)
    ends = torch.tensor([4], dtype=torch.int32)
    s0 = torch.zeros(1, 2, 64, 64)
    with pytest.raises(TypeError, match="^state must be a torch.Tensor$"):
        st(None, offs, starts, ends, r, w, k, v, a, b)
    with pytest.raises(ValueError, match="^state must be contiguous CUDA$"):
        st(s0, offs, starts, ends, r, w, k, v, a, b)


def test_pretrain_contract_order():
    from flashrwkv2.tmix.wkv7.pretrain import pretrain_recurrent_bf16 as pre

    x = torch.zeros(1, 16, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="^head_size must be one of 64, 128, or 256$"):
        pre(x, x, x, x, x, x, head_size=32)
    with pytest.raises(TypeError, match="^r must be a torch.Tensor$"):
        pre(None, x, x, x, x, x)
    with pytest.raises(ValueError, match=r"^r must have shape \[B,T,C\] with nonzero dimensions$"):
        pre(x[0], x, x, x, x, x)
    with pytest.raises(TypeError, match="^r must be bfloat16$"):
        pre(x.float(), x, x, x, x, x)
    with pytest.raises(ValueError, match="^r must be contiguous CUDA$"):
        pre(x, x, x, x, x, x)


def test_rl_and_gate_contract_order():
    from flashrwkv2.rl_infctx.wkv7 import rl_infctx_chunk_fp32io16 as rl
    from flashrwkv2.tmix.kk_a_gate import infer_tmix_kk_a_gate_forward_varlen as gate
    from flashrwkv2.tmix.lnx_rkvres_xg import infer_tmix_lnx_rkvres_xg_forward_varlen as lnx

    r, w, k, v, a, b = _tokens()
    cu, _ = _meta()
    with pytest.raises(ValueError, match="^chunk_size must be one of 16, 32, or 64$"):
        rl(r, w, k, v, a, b, cu_seqlens=cu, chunk_size=8)
    with pytest.raises(ValueError, match="^strategy must be 'materialized' or 'recompute'$"):
        rl(r, w, k, v, a, b, cu_seqlens=cu, strategy="other")
    with pytest.raises(ValueError, match="^r must be contiguous CUDA$"):
        rl(r, w, k, v, a, b, cu_seqlens=cu)
    x = torch.zeros(4, 128, dtype=torch.float16)
    c = torch.zeros(128, dtype=torch.float16)
    with pytest.raises(ValueError, match="^head_size must be one of 64, 128, or 256$"):
        gate(x, c, c, x, c, head_size=32)
    with pytest.raises(TypeError, match="^k must have dtype torch.float16$"):
        gate(x.float(), c.float(), c, x, c)
    with pytest.raises(ValueError, match="^k must be CUDA and contiguous$"):
        gate(x, c, c, x, c)
    with pytest.raises(TypeError, match="^x must be a torch.Tensor$"):
        lnx(None, x, x, x, c, c, c, x)
    with pytest.raises(TypeError, match="^x must have dtype torch.float16$"):
        lnx(x.float(), x, x, x, c, c, c, None)


# ---------------------------------------------------------- chunk lists --
def _chunk_lists_loop(offsets, chunk_size):
    """Per-token walk: a new chunk opens at a sequence start and every
    chunk_size tokens after it."""
    seq_offsets, starts, ends = [0], [], []
    for s in range(len(offsets) - 1):
        for t in range(offsets[s], offsets[s + 1]):
            if (t - offsets[s]) % chunk_size == 0:
                starts.append(t)
                ends.append(t)
            ends[-1] = t + 1
        seq_offsets.append(len(starts))
    return seq_offsets, starts, ends


@pytest.mark.parametrize("chunk_size", [16, 32, 64])
def test_rl_chunk_lists_match_a_token_walk(chunk_size):
    rng = np.random.default_rng(chunk_size)
    lengths = rng.integers(1, 300, size=23)
    lengths[:4] = [1, chunk_size, chunk_size + 1, 2 * chunk_size]
    offsets = np.concatenate([[0], np.cumsum(lengths)])
    got = chunk_lists(offsets, chunk_size)
    want = _chunk_lists_loop(offsets.tolist(), chunk_size)
    for g, w in zip(got, want):
        assert g.tolist() == w


def test_lnx_pretrain_contract_rejects_before_launch():
    """Reference ``tmix/lnx_rkvres_xg/pretrain.py:9-30``: head size, then per
    tensor its type and dtype/device/contiguity, then token shapes,
    residual_scale and weight/bias shapes, all before any launch (CPU tensors
    fail at the dtype/device check)."""
    from flashrwkv2.tmix.lnx_rkvres_xg import pretrain_tmix_lnx_rkvres_xg_bf16 as fn

    x = torch.zeros((1, 2, 64), dtype=torch.bfloat16)
    args = [x] * 4 + [torch.zeros((1, 64), dtype=torch.bfloat16),
                      torch.zeros(64, dtype=torch.bfloat16), torch.zeros(64, dtype=torch.bfloat16),
                      x]
    with pytest.raises(ValueError, match="head_size must be one of 64, 128, or 256"):
        fn(*args, head_size=32)
    with pytest.raises(TypeError, match="x must be a torch.Tensor"):
        fn(None, *args[1:])
    # Each tensor is type-checked and then dtype/device-checked before the
    # next one, so a CPU x fails before a non-tensor r is looked at.
    with pytest.raises(ValueError, match="x must be contiguous CUDA bfloat16"):
        fn(x, [1], *args[2:])
    with pytest.raises(ValueError, match="x must be contiguous CUDA bfloat16"):
        fn(*args)
