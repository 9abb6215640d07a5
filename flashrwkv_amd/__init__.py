"""flashrwkv_amd: MI355X-native WKV7 operators behind the flashrwkv2 WKV7 API.

Public names mirror ``flashrwkv2.__all__``'s WKV7 entries
(reference ``flashrwkv2/__init__.py:86-96``). ``_C`` is the native facade;
it is ``None`` when the in-tree libraries are not built, in which case every
operator raises RuntimeError (there is no fallback path).
"""

import torch as _torch  # noqa: F401  (load PyTorch before the native binding)

try:
    from . import _C
except ImportError:
    _C = None

from .tmix.wkv7 import (
    infer_chunk_bf16_forward_varlen,
    infer_recurrent_add_vec_forward_varlen,
    infer_recurrent_fp16_advance_i32,
    infer_recurrent_fp16_advance_i32_varlen,
    infer_recurrent_fp16_forward_varlen,
    infer_recurrent_fp32io16_forward_varlen,
    prepare_recurrent_metadata,
    pretrain_recurrent_bf16,
)
from .tmix.wkv7.statetune import statetune_recurrent_fp32io16

__all__ = [
    "infer_chunk_bf16_forward_varlen",
    "infer_recurrent_add_vec_forward_varlen",
    "infer_recurrent_fp16_advance_i32",
    "infer_recurrent_fp16_advance_i32_varlen",
    "infer_recurrent_fp16_forward_varlen",
    "infer_recurrent_fp32io16_forward_varlen",
    "prepare_recurrent_metadata",
    "pretrain_recurrent_bf16",
    "statetune_recurrent_fp32io16",
]

__version__ = "0.1.0"
