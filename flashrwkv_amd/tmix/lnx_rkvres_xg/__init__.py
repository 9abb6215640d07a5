"""``flashrwkv2.tmix.lnx_rkvres_xg``: the TMix consumer of the WKV7 output.

Defined in :mod:`flashrwkv_amd.tmix.gates` together with the producer. The
reference's bf16 pretraining variant of this op is not part of the WKV7 path
and is not rebuilt.
"""

from ..gates import infer_tmix_lnx_rkvres_xg_forward_varlen

__all__ = ["infer_tmix_lnx_rkvres_xg_forward_varlen"]
