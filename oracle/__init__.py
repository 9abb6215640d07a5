"""fp64 CPU oracle for the WKV7 hot path -- TEST INFRASTRUCTURE ONLY.

Importable only from tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg. The product package flashrwkv_amd never imports it.
"""
