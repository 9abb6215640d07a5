"""``flashrwkv2.tmix.kk_a_gate``: the TMix producer of the WKV7 inputs.

Defined in :mod:`flashrwkv_amd.tmix.gates` together with the consumer.
"""

from ..gates import infer_tmix_kk_a_gate_forward_varlen

__all__ = ["infer_tmix_kk_a_gate_forward_varlen"]
