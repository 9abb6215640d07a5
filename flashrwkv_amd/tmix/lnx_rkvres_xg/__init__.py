"""``flashrwkv2.tmix.lnx_rkvres_xg``: the TMix consumer of the WKV7 output.

The inference op is defined in :mod:`flashrwkv_amd.tmix.gates` together with
the producer; the bf16 training form (forward and backward) in
:mod:`.pretrain`, exported here as in the reference
(``flashrwkv2/tmix/lnx_rkvres_xg/__init__.py:87-89``).
"""

from ..gates import infer_tmix_lnx_rkvres_xg_forward_varlen
from .pretrain import pretrain_tmix_lnx_rkvres_xg_bf16

__all__ = ["infer_tmix_lnx_rkvres_xg_forward_varlen", "pretrain_tmix_lnx_rkvres_xg_bf16"]
