"""``flashrwkv2`` import path for the MI355X-native WKV7 operators.

Reference callers import the WKV7 family as ``flashrwkv2.*`` and the native
module as ``flashrwkv2._C`` (reference ``flashrwkv2/__init__.py:1-12,
86-96``; ``flashrwkv2/tmix/wkv7/__init__.py:8-17``). This package makes
those module paths resolve to this build's modules: each name below is the
very module object of ``flashrwkv_amd`` registered under its reference path,
so ``import flashrwkv2.tmix.wkv7.chunk`` and ``flashrwkv_amd.tmix.wkv7.chunk``
are one module. Only the WKV7 path and its producer/consumer are provided;
the reference's other operator families are not part of this build.
``_C`` is ``None`` when the native libraries are not built, as in the
reference, and every operator then raises RuntimeError.
"""

import importlib as _importlib
import sys as _sys

import flashrwkv_amd as _impl

# reference module path -> module of this build
_MODULES = {
    "tmix": "flashrwkv_amd.tmix",
    "tmix.wkv7": "flashrwkv_amd.tmix.wkv7",
    "tmix.wkv7.chunk": "flashrwkv_amd.tmix.wkv7.chunk",
    "tmix.wkv7.statetune": "flashrwkv_amd.tmix.wkv7.statetune",
    "tmix.wkv7.pretrain": "flashrwkv_amd.tmix.wkv7.pretrain",
    "tmix.kk_a_gate": "flashrwkv_amd.tmix.kk_a_gate",
    "tmix.lnx_rkvres_xg": "flashrwkv_amd.tmix.lnx_rkvres_xg",
    "tmix.lnx_rkvres_xg.pretrain": "flashrwkv_amd.tmix.lnx_rkvres_xg.pretrain",
    "rl_infctx": "flashrwkv_amd.rl_infctx",
    "rl_infctx.wkv7": "flashrwkv_amd.rl_infctx.wkv7",
}
for _path, _target in _MODULES.items():
    _module = _importlib.import_module(_target)
    _sys.modules[f"{__name__}.{_path}"] = _module
    if "." not in _path:
        globals()[_path] = _module

_C = _impl._C
if _C is not None:
    _sys.modules[f"{__name__}._C"] = _C

from flashrwkv_amd import (  # noqa: E402
    infer_chunk_bf16_forward_varlen,
    infer_recurrent_add_vec_forward_varlen,
    infer_recurrent_fp16_advance_i32,
    infer_recurrent_fp16_advance_i32_varlen,
    infer_recurrent_fp16_forward_varlen,
    infer_recurrent_fp32io16_forward_varlen,
    prepare_recurrent_metadata,
    pretrain_recurrent_bf16,
    statetune_recurrent_fp32io16,
)
from flashrwkv_amd.rl_infctx.wkv7 import (  # noqa: E402
    rl_infctx_chunk_fp32io16,
    rl_infctx_chunk_fp32io16_factor_recompute,
)
from flashrwkv_amd.tmix.gates import (  # noqa: E402
    infer_tmix_kk_a_gate_forward_varlen,
    infer_tmix_lnx_rkvres_xg_forward_varlen,
)
from flashrwkv_amd.tmix.lnx_rkvres_xg.pretrain import (  # noqa: E402
    pretrain_tmix_lnx_rkvres_xg_bf16,
)

__all__ = [
    "infer_chunk_bf16_forward_varlen",
    "infer_recurrent_add_vec_forward_varlen",
    "infer_recurrent_fp16_advance_i32",
    "infer_recurrent_fp16_advance_i32_varlen",
    "infer_recurrent_fp16_forward_varlen",
    "infer_recurrent_fp32io16_forward_varlen",
    "infer_tmix_kk_a_gate_forward_varlen",
    "infer_tmix_lnx_rkvres_xg_forward_varlen",
    "prepare_recurrent_metadata",
    "pretrain_recurrent_bf16",
    "pretrain_tmix_lnx_rkvres_xg_bf16",
    "rl_infctx_chunk_fp32io16",
    "rl_infctx_chunk_fp32io16_factor_recompute",
    "statetune_recurrent_fp32io16",
]

__version__ = _impl.__version__
