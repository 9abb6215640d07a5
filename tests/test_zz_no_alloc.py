"""The allocation-free StateTune backward (frwkv_statetune_backward_noalloc)
against frwkv_statetune_backward with a caller workspace, through the C ABI.

Both run the same kernels, the variant with its workspace in the library's
static per-device scratch; two calls in a row, the second smaller, must each
equal the workspace entry bit for bit (the second call finds the first one's
data in the scratch). Cases that need the scratch: head size 64 without the
forward's interior states and chunks longer than a piece (the interior states
are recomputed into it), and head size 256 (fp32 gradient slices).
"""

from __future__ import annotations

import os
import subprocess
import sys

import numpy as np
import pytest
import torch

from flashrwkv_amd import capi, workloads
from oracle import oracle

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda")
REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NAMES = ("r", "w", "k", "v", "a", "b")


@pytest.fixture(scope="module", autouse=True)
def _require_gpu():
    capi.library()
    if not torch.cuda.is_available():
        pytest.fail("a GPU is required for tests marked gpu")


def _case(lengths, chunk, heads, head_size, seed):
    meta = oracle.chunk_metadata(lengths, chunk)
    case = workloads.make_case(lengths=lengths, heads=heads, head_size=head_size,
                               dtype=torch.bfloat16, seed=seed, state_std=0.1)
    offsets, starts, ends = (torch.from_numpy(x).to(DEV) for x in meta[:3])
    toks = [case[n].to(DEV) for n in NAMES]
    n_tok = sum(lengths)
    batch = len(lengths)
    state = case["state_pool"][:batch].to(DEV).clone()
    out = torch.empty_like(toks[3])
    boundary = torch.empty((starts.numel(), heads, head_size, head_size), device=DEV)
    sda = torch.empty((n_tok, heads, head_size), device=DEV)
    capi.statetune_forward(*toks, sequence_chunk_offsets=offsets, chunk_token_starts=starts,
                           chunk_token_ends=ends, state=state, output=out, boundary=boundary,
                           state_dot_a=sda, scale=0.5)
    g = torch.Generator().manual_seed(seed + 1)
    dy = torch.randn((n_tok, heads, head_size), generator=g).to(torch.bfloat16).to(DEV)
    ds = (torch.randn((batch, heads, head_size, head_size), generator=g) * 0.01).to(DEV)
    meta_dev = dict(sequence_chunk_offsets=offsets, chunk_token_starts=starts,
                    chunk_token_ends=ends)
    return toks, meta_dev, boundary, dy, ds


def _backward(entry, toks, meta, boundary, dy, ds, **extra):
    grads = [torch.empty_like(t) for t in toks]
    ds0 = torch.empty_like(ds)
    entry(*toks, **meta, boundary=boundary, grad_output=dy, grad_final_state=ds, grads=grads,
          grad_initial_state=ds0, scale=0.5, **extra)
    return grads + [ds0]


@pytest.mark.parametrize("head_size,first,second", [
    (64, ((300, 90), 160, 2), ((150,), 100, 1)),
    (128, ((40, 9), 32, 2), ((20,), 18, 1)),
    (256, ((40, 9), 16, 2), ((20,), 8, 1)),
])
def test_noalloc_backward_matches_workspace_entry_twice(head_size, first, second):
    for call, (lengths, chunk, heads) in enumerate((first, second)):
        print(f"call {call}: head_size {head_size} lengths {lengths} chunk {chunk} "
              f"heads {heads}", flush=True)
        n_tok = sum(lengths)
        need = capi.statetune_backward_workspace_bytes(head_size, heads, n_tok, False)
        assert 0 < need <= capi.NOALLOC_SCRATCH_BYTES
        toks, meta, boundary, dy, ds = _case(lengths, chunk, heads, head_size, seed=500 + call)
        expected = _backward(capi.statetune_backward, toks, meta, boundary, dy, ds)
        actual = _backward(capi.statetune_backward_noalloc, toks, meta, boundary, dy, ds)
        torch.cuda.synchronize()
        for name, x, e in zip((*NAMES, "s0"), actual, expected):
            assert torch.isfinite(x.float()).all(), (call, name)
            assert torch.equal(x, e), (call, name)


def test_noalloc_backward_rejects_oversized_workspace_before_launch():
    """Head size 256 with 4096 tokens needs more than the static scratch: the
    call returns an argument error and leaves every output untouched."""
    n_tok, heads, d = 4096, 1, 256
    need = capi.statetune_backward_workspace_bytes(d, heads, n_tok, True)
    assert need > capi.NOALLOC_SCRATCH_BYTES
    toks = [torch.zeros((n_tok, heads, d), dtype=torch.bfloat16, device=DEV)
            for _ in NAMES]
    meta = dict(sequence_chunk_offsets=torch.tensor([0, 1], dtype=torch.int32, device=DEV),
                chunk_token_starts=torch.tensor([0], dtype=torch.int32, device=DEV),
                chunk_token_ends=torch.tensor([n_tok], dtype=torch.int32, device=DEV))
    grads = [torch.full_like(t, 7.0) for t in toks]
    ds0 = torch.full((1, heads, d, d), 7.0, device=DEV)
    with pytest.raises(RuntimeError, match="needs .* bytes of scratch"):
        capi.statetune_backward_noalloc(
            *toks, **meta, boundary=torch.zeros((1, heads, d, d), device=DEV),
            grad_output=None, grad_final_state=None, grads=grads, grad_initial_state=ds0,
            interior=torch.zeros((n_tok // 16, heads, d, d), device=DEV))
    torch.cuda.synchronize()
    assert all(bool((g == 7.0).all()) for g in grads) and bool((ds0 == 7.0).all())


_RESIDENCY_CHILD = """
import sys
import torch
sys.path.insert(0, {repo!r})
from flashrwkv_amd import capi
from tests.test_zz_no_alloc import _backward, _case
toks, meta, boundary, dy, ds = _case((300, 90), 160, 2, 64, seed=700)
for _ in range(2):
    _backward(capi.statetune_backward, toks, meta, boundary, dy, ds)
torch.cuda.synchronize()
free_before = torch.cuda.mem_get_info()[0]
_backward(capi.statetune_backward_noalloc, toks, meta, boundary, dy, ds)
torch.cuda.synchronize()
free_after = torch.cuda.mem_get_info()[0]
print("scratch-residency", free_before - free_after, flush=True)
"""


def test_scratch_becomes_resident_at_the_first_noalloc_call():
    """The static scratch sits in a code object of its own, which HIP loads on
    a device at the first use of one of its symbols: a process that runs the
    library's other kernels holds none of it, and the first call of the
    allocation-free entry makes it resident. Checked in a fresh process (the
    array of this one may be loaded already) from the device's free memory."""
    print("child process: workspace backward twice, then the noalloc entry", flush=True)
    proc = subprocess.run([sys.executable, "-c", _RESIDENCY_CHILD.format(repo=REPO)],
                          cwd=REPO, capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stdout[-2000:] + proc.stderr[-2000:]
    line = [x for x in proc.stdout.splitlines() if x.startswith("scratch-residency")][-1]
    grown = int(line.split()[1])
    print(f"device memory taken by the first noalloc call: {grown} bytes", flush=True)
    assert grown >= capi.NOALLOC_SCRATCH_BYTES
    assert grown < capi.NOALLOC_SCRATCH_BYTES + (64 << 20)
