"""CPU checks of the matrix benchmark's helpers (bench.py --workload matrix).

The matrix gate compares the GPU output with ``fp32_gate_reference``, an
fp32 torch restatement of the decay-logits recurrence; here that reference is
itself checked against the fp64 oracle on ragged sequences with permuted
slots, and the percentile statistic against hand-computed values.
"""

from __future__ import annotations

import numpy as np
import torch

import bench
from oracle import oracle


def test_percentile_matches_linear_interpolation():
    assert bench.percentile([1.0, 2.0, 3.0, 4.0], 0.5) == 2.5
    assert abs(bench.percentile([5.0, 1.0, 3.0], 0.1) - 1.4) < 1e-12
    assert bench.percentile([2.0], 0.9) == 2.0
    assert bench.percentile([3.0, 1.0, 2.0], 1.0) == 3.0


def test_gate_reference_matches_fp64_oracle():
    g = torch.Generator().manual_seed(3)
    lengths = (3, 1, 5, 2)
    n, heads, d = sum(lengths), 2, 64

    def rnd(scale):
        return (torch.randn((n, heads, d), generator=g) * scale).to(torch.bfloat16)

    r, x, k, v, a, b = rnd(0.15), rnd(4.0), rnd(0.08), rnd(0.08), rnd(0.08), rnd(0.08)
    cu = torch.tensor(np.cumsum((0,) + lengths), dtype=torch.int32)
    slots = torch.tensor([3, 0, 5, 1], dtype=torch.int32)
    pool = torch.randn((6, heads, d, d), generator=g) * 0.02
    bias = (torch.randn((heads, d), generator=g) * 0.25).to(torch.bfloat16)
    y, new_pool = bench.fp32_gate_reference(r, x, k, v, a, b, pool, cu, slots, bias=bias,
                                            scale=0.5)
    w = oracle.retention_from_logits(x.double().numpy(), bias.double().numpy())
    y_ref, pool_ref = oracle.forward_varlen(
        r.double().numpy(), w, k.double().numpy(), v.double().numpy(), a.double().numpy(),
        b.double().numpy(), pool.double().numpy(), cu.numpy(), slots.numpy(), scale=0.5)
    assert oracle.relative_rmse(y.double().numpy(), y_ref) < 1e-5
    assert oracle.relative_rmse(new_pool.double().numpy(), pool_ref) < 1e-5
    # Unused slots are copied unchanged.
    for i in (2, 4):
        assert torch.equal(new_pool[i], pool[i])


def test_relative_rmse_definition():
    e = torch.tensor([3.0, 4.0])
    assert bench.relative_rmse(e, e) == 0.0
    assert abs(bench.relative_rmse(e + 1.0, e) - 1.0 / np.sqrt(12.5)) < 1e-6


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU; --gpus N > 1 exits with status 2 and a JSON
    message, before anything touches a device."""
    import json
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    proc = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"],
                          capture_output=True, text=True, timeout=120)
    assert proc.returncode == 2
    line = json.loads(proc.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"]
