"""WKV7 benchmark on one MI355X (driver contract: one JSON line on stdout).

Default workload (benchmark config 1): batched decode, B=256 sequences, H=40
heads, D=64, T=1 per step, bf16 token io, fp32 state pool [256,40,64,64]
updated in place, S0 ~ N(0, 0.1), retention w = exp(-exp(u)), u ~ U(-5,0)
(raw-retention mode). One step = one launch over the whole batch.

Cache-cold measurement: the 167.8 MB pool fits MI355X's 256 MB Infinity
Cache, so consecutive in-place steps on one pool can read state from the
cache. The timed loop therefore rotates over 4 pool replicas (671 MB) and 8
token sets; step i uses replica i % 4, which keeps every step's state traffic
on HBM. The in-place single-pool rate is reported beside it.

Steps are replayed from HIP graphs (64 consecutive steps, eight times the
8-step rotation, captured as one graph, and one graph for a remainder), so
host launch overhead is not on the timed path. HIP events on
the launch stream bracket the timed region; the average launch duration is
elapsed / steps.

The default run (--workload all) adds a "chunked_prefill" object measuring
benchmark config 3 (chunked prefill, B=16, T=4096, H=32) against the bf16 MFMA
roofline (--workload prefill makes that the headline line instead), and the
other legs: fp16-state and fused decode, config 4 training, config 2, config 0,
clampw-v3 pretraining and StateTune at head sizes 128 and 256.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0
BF16_PEAK_TFLOPS = 2516.6

# rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, mean KiB per dispatch of each
# kernel at its bench workload (the traffic summaries under profiles/ give the
# runs and their commands). Calibration: a 256 MiB device copy (--workload copy) reads
# FETCH_SIZE 131084.4 KiB and WRITE_SIZE 262144.0 KiB per dispatch, so fetched
# bytes are FETCH_SIZE * 1024 * (262144 / 131084.4) and written bytes
# WRITE_SIZE * 1024.
_COPY_KIB = 262144.0
_COPY_FETCH_KIB = 131084.4
_COPY_WRITE_KIB = 262144.0
PMC_KIB = {  # kernel -> (FETCH_SIZE, WRITE_SIZE)
    "recurrent_fp32_kernel<64,64,64,Bf16,kRawW>": (85811.4, 165205.5),
    "chunk_fwd_kernel<Bf16,kRawW,float>": (790660.5, 270353.9),
    "chunk_fwd_kernel<Bf16,kRawW,float>/statetune": (790712.8, 1318935.6),
    "chunk_fwd_kernel<Bf16,kRawW,float>/precise": (395420.7, 135168.0),
    "chunk_bwd_kernel<Bf16,kRawW>": (1184971.4, 1581074.2),
    "recurrent_fp16_decode_kernel": (44876.3, 83232.4),
}

# The kernel sources PMC_KIB was measured on: sha256 over these files, in
# order (the build script carries the compile flags). When the tree's sources
# differ, the constants describe other kernels and pmc_traffic reports None
# instead of a stale figure. Restamped once without a new measurement: a
# host-only change to chunk_fwd.hip (the interior-state byte count) whose
# gfx950 assembly was compared equal to the measured one except for the
# compilation-unit id.
PMC_SOURCES = ("flashrwkv_amd/csrc/recurrent.hip", "flashrwkv_amd/csrc/chunk_fwd.hip",
               "flashrwkv_amd/csrc/chunk_bwd.hip", "flashrwkv_amd/csrc/chunk_common.h",
               "flashrwkv_amd/csrc/wkv7_device.h", "flashrwkv_amd/csrc/wkv7_mfma.h",
               "flashrwkv_amd/_build.py")
PMC_SOURCES_SHA = "bba890fa1207aef767566d53c84f672dc60e779206bd164f67bc08a235499919"


def kernel_sources_sha() -> str:
    import hashlib

    h = hashlib.sha256()
    for rel in PMC_SOURCES:
        h.update((ROOT / rel).read_bytes())
    return h.hexdigest()


def pmc_traffic(kernel: str) -> int | None:
    """Measured HBM bytes per dispatch of ``kernel`` (calibrated counters), or
    None when the kernel sources changed since the measurement."""
    if kernel not in PMC_KIB or kernel_sources_sha() != PMC_SOURCES_SHA:
        return None
    fetch, write = PMC_KIB[kernel]
    return int(round(fetch * 1024 * _COPY_KIB / _COPY_FETCH_KIB
                     + write * 1024 * _COPY_KIB / _COPY_WRITE_KIB))


# MFMA busy share per SIMD of the chunked kernels on the same sources
# (SQ_VALU_MFMA_BUSY_CYCLES / 1024 SIMDs over SQ_BUSY_CU_CYCLES / 256 CUs, in
# %), from the counter passes of the bench workloads.
PMC_MFMA_BUSY_PCT = {
    "chunk_fwd_kernel<Bf16,kRawW,float>": 21.4,
    "chunk_fwd_kernel<Bf16,kRawW,float>/varlen": 21.0,
    "chunk_fwd_kernel<Bf16,kRawW,float>/statetune": 15.5,
    "chunk_fwd_kernel<Bf16,kRawW,float>/precise": 14.8,
    "chunk_bwd_kernel<Bf16,kRawW>": 13.1,
}


def pmc_mfma_busy(kernel: str) -> float | None:
    """Measured MFMA busy % per SIMD of ``kernel``, or None when the kernel
    sources changed since the measurement."""
    if kernel not in PMC_MFMA_BUSY_PCT or kernel_sources_sha() != PMC_SOURCES_SHA:
        return None
    return PMC_MFMA_BUSY_PCT[kernel]


def _sum_or_none(*xs):
    return None if any(x is None for x in xs) else sum(xs)


METRIC = "WKV7 tokens/s + % roofline (HBM GB/s decode, MFMA TFLOP/s chunked), h32d64"


def _parse():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=1000)
    p.add_argument("--warmup", type=int, default=50)
    p.add_argument("--workload", default="all",
                   choices=("all", "decode", "decode_fp16", "decode_fused", "prefill", "training",
                            "recurrent_long", "copy", "matrix", "training_large", "config0",
                            "pretrain"),
                   help="all: decode headline line plus the prefill, training and "
                        "long-sequence legs; matrix: the reference operator benchmark's "
                        "case matrix with its correctness gate")
    p.add_argument("--prefill-steps", type=int, default=20)
    p.add_argument("--training-steps", type=int, default=10)
    p.add_argument("--cpu-seconds", type=float, default=8.0,
                   help="bound on the CPU-baseline sample (0 disables it)")
    p.add_argument("--matrix-dtype", default="bfloat16", choices=("bfloat16", "float16"))
    p.add_argument("--matrix-stress", action="store_true", help="add the stress cases")
    p.add_argument("--matrix-warmup", type=int, default=5)
    p.add_argument("--matrix-samples", type=int, default=30)
    p.add_argument("--matrix-sample-iters", type=int, default=4)
    p.add_argument("--matrix-seed", type=int, default=20260804)
    return p.parse_args()


def decode_bytes_per_step(batch: int, heads: int, d: int = 64, io_bytes: int = 2,
                          state_bytes: int = 4) -> int:
    """Algorithmic HBM bytes of one decode launch.

    Per (sequence, head): state read + write 2*D*D*state_bytes, six token rows
    (r, w, k, v, a, b) 6*D*io_bytes, one output row D*io_bytes.
    """
    per_unit = 2 * d * d * state_bytes + 7 * d * io_bytes
    return batch * heads * per_unit


def cpu_baseline_decode(batch, heads, seconds):
    """Times the fp64 C oracle (the restated reference recurrence) on host cores."""
    import numpy as np
    import torch

    from flashrwkv_amd import workloads
    from oracle import oracle

    cores = len(os.sched_getaffinity(0))
    case = workloads.make_case(lengths=[1] * batch, heads=heads, head_size=64,
                               dtype=torch.bfloat16, seed=99, state_std=0.1)
    args = [case[n].double().numpy() for n in ("r", "w", "k", "v", "a", "b")]
    pool = case["state_pool"].double().numpy()
    cu = case["cu_seqlens"].numpy()
    slots = case["state_indices"].numpy()
    oracle.forward_varlen(*args, pool, cu, slots, num_threads=cores)  # warm-up
    steps = 0
    t0 = time.perf_counter()
    while True:
        _, pool = oracle.forward_varlen(*args, pool, cu, slots, num_threads=cores)
        steps += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= seconds:
            break
    return {
        "value": steps * batch / elapsed,
        "unit": "tokens/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{steps} decode steps of B={batch}, H={heads}, D=64 through the fp64 C "
                  f"oracle (oracle/wkv7_oracle.c), OpenMP over (sequence, head), "
                  f"{elapsed:.1f} s",
    }


def cpu_baseline_decode_fp16(batch, heads, seconds, sample=32):
    """Times the fp16-state oracle (oracle.forward_fp16_state: fp64 arithmetic
    with the contract's fp16 rounding points, one numpy loop per sequence, one
    thread) on decode steps of ``sample`` sequences; sequences are independent,
    so tokens/s does not depend on how many a step holds."""
    import numpy as np
    import torch

    from flashrwkv_amd import workloads
    from oracle import oracle

    case = workloads.make_case(lengths=[1] * sample, heads=heads, head_size=64,
                               dtype=torch.float16, seed=99, state_std=0.1)
    args = [case[n].double().numpy() for n in ("r", "w", "k", "v", "a", "b")]
    args[1] = np.random.default_rng(1).standard_normal(args[1].shape) * 3.5  # decay logits
    pool = case["state_pool"].numpy().astype(np.float16)
    elapsed_pool = np.arange(pool.shape[0], dtype=np.int32) * 11
    cu = case["cu_seqlens"].numpy()
    slots = case["state_indices"].numpy()
    steps = 0
    t0 = time.perf_counter()
    while True:
        _, pool = oracle.forward_fp16_state(*args, pool, elapsed_pool, cu, slots)
        steps += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= seconds:
            break
    return {
        "value": steps * sample / elapsed,
        "unit": "tokens/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{steps} decode steps of {sample} sequences (of B={batch}), H={heads}, D=64 "
                  f"through the fp16-state oracle (numpy, one thread), {elapsed:.1f} s",
    }


def cpu_baseline_tmix_chain(batch, heads, seconds, sample=64):
    """Times the fp64 chain oracle (oracle.tmix_fused: kk_a_gate in numpy, the
    recurrence in the C oracle over every core, lnx_rkvres_xg in numpy) on
    decode steps of ``sample`` sequences."""
    import numpy as np

    from oracle import oracle

    cores = len(os.sched_getaffinity(0))
    rng = np.random.default_rng(3)
    d = 64
    shape = (sample, heads, d)
    r, k, v, a12 = (rng.standard_normal(shape) for _ in range(4))
    w = np.exp(-np.exp(rng.uniform(-5.0, 0.0, shape)))
    g = 1.0 / (1.0 + np.exp(-rng.standard_normal(shape)))
    vec = lambda: rng.standard_normal(heads * d) * 0.1
    k_k, a0, k_a, r_k, ln_w, ln_b = vec(), vec(), vec(), vec(), 1.0 + vec(), vec()
    pool = rng.standard_normal((sample, heads, d, d)) * 0.1
    cu = np.arange(sample + 1, dtype=np.int32)
    slots = np.arange(sample, dtype=np.int32)
    steps = 0
    t0 = time.perf_counter()
    while True:
        _, pool = oracle.tmix_fused(r, w, k, v, a12, g, k_k, a0, k_a, r_k, ln_w, ln_b, pool,
                                    cu, slots)
        steps += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= seconds:
            break
    return {
        "value": steps * sample / elapsed,
        "unit": "tokens/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{steps} decode steps of {sample} sequences (of B={batch}), H={heads}, D=64 "
                  f"through the fp64 chain oracle (gates in numpy, the recurrence in the C "
                  f"oracle with OpenMP over (sequence, head)), {elapsed:.1f} s",
    }


def cpu_baseline_torch(lengths, heads, seconds, *, seed=97, u_low=-5.0, heads_total=None,
                       backward=False, dtype=None):
    """The torch fp32 restatement of the naive recurrence (oracle.forward_torch)
    on the host CPU, timed once with every available core and once with
    torch.set_num_threads(1): 1 warm-up, then repeats until ``seconds`` pass
    (at least 3). tokens/s counts token-heads / heads_total (heads are
    independent, so a head sample scales exactly). ``backward``: each repeat
    also runs torch autograd back to every input and S0 (dy ~ N(0,1))."""
    import torch

    from flashrwkv_amd import workloads
    from oracle import oracle

    cores = len(os.sched_getaffinity(0))
    heads_total = heads if heads_total is None else heads_total
    case = workloads.make_case(lengths=lengths, heads=heads, head_size=64,
                               dtype=dtype or torch.bfloat16, seed=seed, state_std=0.1,
                               u_low=u_low)
    args = [case[n].float().requires_grad_(backward) for n in ("r", "w", "k", "v", "a", "b")]
    pool = case["state_pool"].float().requires_grad_(backward)
    cu, slots = case["cu_seqlens"].numpy(), case["state_indices"].numpy()
    tokens = sum(lengths)
    dy = torch.randn(args[0].shape, generator=torch.Generator().manual_seed(seed))
    before = torch.get_num_threads()
    out = {"kind": "port", "unit": "train tokens/s" if backward else "tokens/s",
           "cpu_count": os.cpu_count(), "affinity_cores": cores,
           "sample": f"oracle.forward_torch (torch fp32, per token"
                     f"{', + autograd backward' if backward else ''}) on {len(lengths)} "
                     f"sequence(s) x {heads} heads, {tokens} tokens per repeat"}

    def once():
        y, _ = oracle.forward_torch(*args, pool, cu, slots)
        if backward:
            y.backward(dy)

    try:
        for label, threads in (("all_cores", cores), ("one_thread", 1)):
            torch.set_num_threads(threads)
            once()
            reps, t0 = 0, time.perf_counter()
            while True:
                once()
                reps += 1
                elapsed = time.perf_counter() - t0
                if reps >= 3 and elapsed >= seconds:
                    break
            out[label] = {"value": round(reps * tokens * heads / heads_total / elapsed, 1),
                          "threads": torch.get_num_threads(),
                          "wall_s": round(elapsed, 2), "repeats": reps}
    finally:
        torch.set_num_threads(before)
    return out


def cpu_baseline_gate(cores):
    """The reference bench's correctness gate (benchmarks/tmix/wkv7/bench.py:374-501),
    run beside the CPU baseline with the same fp64 oracle as the checker.

    Inputs follow the reference bench's recipe (bench.py:309-371) at config 1's
    decode shape: B=256, H=40, D=64, T=1, bf16, r*0.15, decay logits*4.0,
    k/v/a/b*0.08, a pool of B+4 slots ~ N(0, 0.02), state_indices reversed.
    The public entry (decay logits) runs twice from the same state; the gate
    checks relative RMSE of output and written state against the oracle
    (limit 0.002, the fp32io16_recurrent entry of
    tests/fixtures/tolerances-v1.json), bitwise-untouched unused slots,
    bitwise determinism and finiteness."""
    import numpy as np
    import torch

    import flashrwkv_amd
    from oracle import oracle

    batch, heads, d = 256, 40, 64
    dev = torch.device("cuda:0")
    gen = torch.Generator().manual_seed(20260811)
    shape = (batch, heads, d)

    def rnd(scale):
        return (torch.randn(shape, generator=gen) * scale).to(torch.bfloat16)

    r, x, k, v, a, b = rnd(0.15), rnd(4.0), rnd(0.08), rnd(0.08), rnd(0.08), rnd(0.08)
    pool = torch.randn((batch + 4, heads, d, d), generator=gen) * 0.02
    cu = torch.arange(batch + 1, dtype=torch.int32)
    slots = torch.arange(batch - 1, -1, -1, dtype=torch.int32)
    dv = {n: t.to(dev) for n, t in (("r", r), ("x", x), ("k", k), ("v", v), ("a", a),
                                    ("b", b), ("cu", cu), ("slots", slots))}
    ticket = flashrwkv_amd.prepare_recurrent_metadata(
        dv["cu"], dv["slots"], total_tokens=batch, state_pool_size=batch + 4)
    runs = []
    for _ in range(2):
        state = pool.to(dev)
        out = flashrwkv_amd.infer_recurrent_fp32io16_forward_varlen(
            dv["r"], dv["x"], dv["k"], dv["v"], dv["a"], dv["b"], state_pool=state,
            cu_seqlens=dv["cu"], state_indices=dv["slots"], validated_metadata=ticket)
        torch.cuda.synchronize()
        runs.append((out.cpu(), state.cpu()))
    (out, state), (out2, state2) = runs
    w = oracle.retention_from_logits(x.double().numpy())
    y_ref, pool_ref = oracle.forward_varlen(
        r.double().numpy(), w, k.double().numpy(), v.double().numpy(), a.double().numpy(),
        b.double().numpy(), pool.double().numpy(), cu.numpy(), slots.numpy(),
        num_threads=cores)
    active = slots.long().numpy()
    untouched = [i for i in range(batch + 4) if i not in set(active.tolist())]
    out_rmse = oracle.relative_rmse(out.double().numpy(), y_ref)
    state_rmse = oracle.relative_rmse(state.double().numpy()[active], pool_ref[active])
    limit = 0.002
    gate = {
        "output_relative_rmse": out_rmse,
        "state_relative_rmse": state_rmse,
        "limit_relative_rmse": limit,
        "untouched_slots": bool(torch.equal(state[untouched], pool[untouched])),
        "deterministic": bool(torch.equal(out, out2) and torch.equal(state, state2)),
        "finite": bool(torch.isfinite(out.float()).all() and torch.isfinite(state).all()),
        "inputs": "reference bench recipe at B=256, H=40, D=64, bf16, public decay-logits entry",
    }
    gate["passed"] = bool(gate["finite"] and gate["untouched_slots"] and gate["deterministic"]
                          and out_rmse <= limit and state_rmse <= limit
                          and np.isfinite(out_rmse) and np.isfinite(state_rmse))
    return gate


def bench_decode(args, fp16_state=False):
    """Config 1 decode. ``fp16_state``: the fp16-state family instead (fp16
    tokens with decay logits, fp16 pool, phase origins), same shape."""
    import torch

    import flashrwkv_amd
    from flashrwkv_amd import workloads
    from flashrwkv_amd.tmix.wkv7 import DECAY_RAW_W, prepare_recurrent_metadata

    if flashrwkv_amd._C is None:
        raise SystemExit("flashrwkv_amd native library is not built")
    ops = flashrwkv_amd._C.ops
    dev = torch.device("cuda:0")
    batch, heads, d = 256, 40, 64
    # Enough replicas that the rotation (>= 671 MB) exceeds the 256 MB cache.
    n_pools, n_tokens = (8, 8) if fp16_state else (4, 8)
    state_dtype = torch.float16 if fp16_state else torch.float32
    io_dtype = torch.float16 if fp16_state else torch.bfloat16

    gen = torch.Generator(device=dev).manual_seed(20260805)
    pools = [(torch.randn((batch, heads, d, d), generator=gen, device=dev) * 0.1)
             .to(state_dtype) for _ in range(n_pools)]
    token_sets = [workloads.make_tokens(batch, heads, d, dtype=io_dtype,
                                       seed=20260805 + i, device=dev)
                  for i in range(n_tokens)]
    if fp16_state:
        # Decay logits (the family's only decay form), reference test scale.
        # k scaled down so that 1000+ in-place steps stay inside fp16 range.
        for t in token_sets:
            t["w"] = (torch.randn((batch, heads, d), generator=gen, device=dev) * 3.5).half()
            t["k"] = (t["k"].float() * 0.05).half()
    elapsed = torch.arange(batch, device=dev, dtype=torch.int32) * 11
    outputs = [torch.empty((batch, heads, d), device=dev, dtype=io_dtype)
               for _ in range(n_tokens)]
    cu = torch.arange(batch + 1, device=dev, dtype=torch.int32)
    slots = torch.arange(batch, device=dev, dtype=torch.int32)

    stream = torch.cuda.Stream(device=dev)
    # Inputs were made on the default stream: order the side stream after them.
    stream.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(stream):
        ticket = prepare_recurrent_metadata(cu, slots, total_tokens=batch,
                                            state_pool_size=batch, max_seqlen=1)

        def step(i, pool=None):
            t = token_sets[i % n_tokens]
            target = pools[i % n_pools] if pool is None else pool
            if fp16_state:
                ops.recurrent_fp16_from_decay_logits(
                    cu, slots, elapsed, target, t["r"], t["w"], t["k"], t["v"], t["a"],
                    t["b"], outputs[i % n_tokens], 1.0, None, ticket, 1)
            else:
                ops.recurrent_fp32_forward_internal(
                    cu, slots, target, t["r"], t["w"], t["k"], t["v"], t["a"], t["b"],
                    outputs[i % n_tokens], 1.0, DECAY_RAW_W, None, ticket, 1)

        for i in range(8):
            step(i)
        stream.synchronize()
        rotation = 8  # lcm(n_pools, n_tokens)
        # Steps are replayed as HIP graphs of 64 consecutive steps (8 rotations)
        # plus one graph for the remainder: graph launches then cost about
        # 0.01 us per step instead of 0.5-0.7 us with 8-step graphs.
        cycle = 8 * rotation

        def capture(count, pool=None):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                for i in range(count):
                    step(i, pool)
            return g

        def graphs(pool=None):
            # Every graph a run replays, captured before any timing.
            sizes = {cycle} | {n % cycle for n in (args.warmup, args.steps)} - {0}
            return {n: capture(n, pool) for n in sorted(sizes)}

        def run_steps(g, count):
            # Graph positions restart at 0 and cycle is a multiple of the
            # rotation, so step i still uses pool i % n_pools, tokens i % 8.
            for _ in range(count // cycle):
                g[cycle].replay()
            if count % cycle:
                g[count % cycle].replay()

        def timed(g):
            run_steps(g, args.warmup)
            stream.synchronize()
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            wall0 = time.perf_counter()
            start.record(stream)
            run_steps(g, args.steps)
            end.record(stream)
            end.synchronize()
            torch.cuda.synchronize()
            return start.elapsed_time(end) / args.steps, time.perf_counter() - wall0

        # Cache-cold: step i uses pool replica i % n_pools and token set i % 8.
        cold_ms, wall = timed(graphs())
        # In-place: one pool, the literal "consecutive steps" of the config.
        inplace_ms, _ = timed(graphs(pools[0]))

    nbytes = decode_bytes_per_step(batch, heads, d, state_bytes=2 if fp16_state else 4)
    achieved = nbytes / (cold_ms * 1e-3) / 1e9
    tok_s = batch / (cold_ms * 1e-3)
    if fp16_state:
        kernel = "recurrent_fp16_decode_kernel"
        return {
            "workload": f"wkv7_decode_fp16_state: B=256, H=40, D=64, T=1 per step, fp16 io, "
                        f"fp16 state pool in place, decay logits, {n_pools} rotating pool "
                        "replicas (cache-cold), HIP graphs of 64 steps",
            "ms_per_step": round(cold_ms, 6),
            "tokens_per_s": round(tok_s, 1),
            "roofline": {
                "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                "traffic": pmc_traffic(kernel),
                "kernel": kernel, "algorithmic_bytes_per_launch": nbytes,
            },
            "inplace_single_pool": {
                "ms_per_step": round(inplace_ms, 6),
                "tokens_per_s": round(batch / (inplace_ms * 1e-3), 1),
                "achieved_GBps": round(nbytes / (inplace_ms * 1e-3) / 1e9, 1),
            },
            **({"cpu_baseline": cpu_baseline_decode_fp16(batch, heads, args.cpu_seconds / 2)}
               if args.cpu_seconds > 0 else {}),
        }
    line = {
        "metric": METRIC,
        "value": round(tok_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(cold_ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded; benchmark config 1 distributions)",
        "config": {
            "workload": "wkv7_decode_cfg1: B=256, H=40, D=64, T=1 per step, bf16 io, "
                        "fp32 state pool in place, raw retention, 4 rotating pool "
                        "replicas (cache-cold), HIP graphs of 64 steps",
            "batch": batch, "heads": heads, "head_size": d, "io_dtype": "bf16",
            "state_dtype": "fp32", "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": pmc_traffic("recurrent_fp32_kernel<64,64,64,Bf16,kRawW>"),
            "kernel": "recurrent_fp32_kernel<64,64,64,Bf16,kRawW>",
            "algorithmic_bytes_per_launch": nbytes,
        },
        "inplace_single_pool": {
            "ms_per_step": round(inplace_ms, 6),
            "tokens_per_s": round(batch / (inplace_ms * 1e-3), 1),
            "achieved_GBps": round(nbytes / (inplace_ms * 1e-3) / 1e9, 1),
        },
        "wall_s_timed_region": round(wall, 4),
    }
    if args.cpu_seconds > 0:
        line["cpu_baseline"] = cpu_baseline_decode(batch, heads, args.cpu_seconds)
        line["cpu_baseline"]["torch_fp32"] = cpu_baseline_torch(
            [1] * batch, heads, args.cpu_seconds / 2)
        line["gate"] = cpu_baseline_gate(line["cpu_baseline"]["cores"])
    return line


def chunk_flops(chunk: int = 64, d: int = 64) -> int:
    """Algorithmic FLOPs of one (64-token chunk, head) of the chunked forward.

    18 C^2 D (four C x C x D triangle products and four C x C x D
    applications) + 8 C D^2 (two C x D x D state products, two D x C x D state
    updates) + C^3 / 3 (triangular inverse).
    """
    return 18 * chunk * chunk * d + 8 * chunk * d * d + chunk ** 3 // 3


def cpu_baseline_prefill(t_len, heads_total, seconds, *, lengths=None, u_low=-8.0, seed=98):
    """fp64 C oracle on a bounded sample: whole (sequence, head) recurrences,
    one sequence of ``t_len`` tokens, or the packed sequences ``lengths``
    (the oracle loops over them one by one)."""
    import numpy as np
    import torch

    from flashrwkv_amd import workloads
    from oracle import oracle

    cores = len(os.sched_getaffinity(0))
    sample_heads = max(1, cores)
    lengths = [t_len] if lengths is None else list(lengths)
    t_len = sum(lengths)
    case = workloads.make_case(lengths=lengths, heads=sample_heads, head_size=64,
                               dtype=torch.bfloat16, seed=seed, state_std=0.0, u_low=u_low)
    args = [case[n].double().numpy() for n in ("r", "w", "k", "v", "a", "b")]
    pool = np.zeros((len(lengths), sample_heads, 64, 64))
    cu = case["cu_seqlens"].numpy()
    slots = case["state_indices"].numpy()
    reps = 0
    t0 = time.perf_counter()
    while True:
        oracle.forward_varlen(*args, pool, cu, slots, num_threads=cores)
        reps += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= seconds:
            break
    token_heads_per_s = reps * t_len * sample_heads / elapsed
    return {
        "value": token_heads_per_s / heads_total,
        "unit": "tokens/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{reps} x ({len(lengths)} sequence(s) of {t_len} tokens in all x "
                  f"{sample_heads} heads) through the fp64 C oracle, OpenMP over heads, "
                  f"{elapsed:.1f} s; token-heads/s divided by H={heads_total} (heads are "
                  f"independent)",
    }


def bench_decode_fused(args):
    """The TMix chain around decode at config 1's shape (B=256, H=40, D=64, one
    token per step, fp16 io, fp32 pool, decay logits, 4 rotating pool
    replicas): the fused kernel (producer + WKV7 step + consumer) against the
    same chain as three kernels (kk_a_gate, the recurrent op, lnx_rkvres_xg).
    Both run from HIP graphs of 8 steps with a prepared ticket."""
    import torch

    import flashrwkv_amd
    from flashrwkv_amd.tmix.wkv7 import DECAY_LOGITS, prepare_recurrent_metadata

    ops = flashrwkv_amd._C.ops
    dev = torch.device("cuda:0")
    batch, heads, d = 256, 40, 64
    c = heads * d
    n_pools, n_tokens = 4, 8
    gen = torch.Generator(device=dev).manual_seed(20260811)
    f16 = torch.float16

    def randn(*shape, s=1.0):
        return torch.randn(shape, generator=gen, device=dev) * s

    pools = [randn(batch, heads, d, d, s=0.1) for _ in range(n_pools)]
    tokens = [{"r": randn(batch, heads, d).to(f16), "w": randn(batch, heads, d, s=2.0).to(f16),
               "k": randn(batch, heads, d).to(f16), "v": randn(batch, heads, d).to(f16),
               "a12": randn(batch, heads, d).to(f16),
               "g": torch.sigmoid(randn(batch, heads, d)).to(f16)} for _ in range(n_tokens)]
    vec = {"k_k": (1.0 + randn(c, s=0.3)).to(f16), "a0": randn(c, s=0.5).to(f16),
           "k_a": torch.rand(c, generator=gen, device=dev).to(f16),
           "r_k": randn(c, s=0.5).to(f16), "ln_w": (1.0 + randn(c, s=0.2)).to(f16),
           "ln_b": randn(c, s=0.1).to(f16)}
    cu = torch.arange(batch + 1, device=dev, dtype=torch.int32)
    slots = torch.arange(batch, device=dev, dtype=torch.int32)
    stream = torch.cuda.Stream(device=dev)
    stream.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(stream):
        ticket = prepare_recurrent_metadata(cu, slots, total_tokens=batch,
                                            state_pool_size=batch, max_seqlen=1)

        def fused(i):
            t = tokens[i % n_tokens]
            ops.recurrent_tmix_fused_forward(
                cu, slots, pools[i % n_pools], t["r"], t["w"], t["k"], t["v"], t["a12"], t["g"],
                vec["k_k"], vec["a0"], vec["k_a"], vec["r_k"], vec["ln_w"], vec["ln_b"], 1.0,
                DECAY_LOGITS, None, ticket)

        y_bufs = [torch.empty((batch, heads, d), device=dev, dtype=f16) for _ in range(n_tokens)]

        def chain(i):
            t = tokens[i % n_tokens]
            flat = lambda x: x.reshape(batch, c)
            new_k, neg_kk, kka = ops.tmix_kk_a_gate_forward_varlen(
                flat(t["k"]), vec["k_k"], vec["a0"], flat(t["a12"]), vec["k_a"], 64, batch, 1)
            y = y_bufs[i % n_tokens]
            ops.recurrent_fp32_from_decay_logits(
                cu, slots, pools[i % n_pools], t["r"], t["w"], new_k.reshape(batch, heads, d),
                t["v"], neg_kk.reshape(batch, heads, d), kka.reshape(batch, heads, d), y, 1.0,
                None, ticket, 1)
            ops.tmix_lnx_rkvres_xg_forward_varlen(
                flat(y), flat(t["r"]), new_k, flat(t["v"]), vec["r_k"], vec["ln_w"],
                vec["ln_b"], flat(t["g"]), 64, batch, 1)

        def graph_ms(step):
            for i in range(8):
                step(i)
            stream.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                for i in range(8):
                    step(i)
            reps = max(1, args.steps // 8)
            for _ in range(max(1, args.warmup // 8)):
                g.replay()
            stream.synchronize()
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record(stream)
            for _ in range(reps):
                g.replay()
            end.record(stream)
            end.synchronize()
            return start.elapsed_time(end) / (8 * reps)

        fused_ms = graph_ms(fused)
        chain_ms = graph_ms(chain)
    units = batch * heads
    fused_bytes = units * (2 * d * d * 4 + 7 * d * 2)
    # kk_a_gate: read k, a12, write 3; WKV: 6 reads + y; lnx: 5 reads + out.
    chain_bytes = units * (2 * d * d * 4 + (5 + 7 + 6) * d * 2)
    gbps = fused_bytes / (fused_ms * 1e-3) / 1e9
    return {
        "workload": "tmix_chain_decode: kk_a_gate -> WKV7 step -> lnx_rkvres_xg at B=256, "
                    "H=40, D=64, T=1 per step, fp16 io, fp32 state pool, decay logits, "
                    f"{n_pools} rotating pool replicas",
        "fused": {"ms_per_step": round(fused_ms, 6),
                  "tokens_per_s": round(batch / (fused_ms * 1e-3), 1),
                  "kernel": "recurrent_tmix_fused_kernel<F16,kLogits>",
                  "roofline": {"bound": "hbm", "achieved": round(gbps, 1),
                               "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                               "frac": round(gbps / HBM_PEAK_GBPS, 4),
                               "algorithmic_bytes_per_launch": fused_bytes}},
        "three_kernel_chain": {"ms_per_step": round(chain_ms, 6),
                               "tokens_per_s": round(batch / (chain_ms * 1e-3), 1),
                               "algorithmic_bytes_per_step": chain_bytes},
        "speedup": round(chain_ms / fused_ms, 3),
        **({"cpu_baseline": cpu_baseline_tmix_chain(batch, heads, args.cpu_seconds / 2)}
           if args.cpu_seconds > 0 else {}),
    }


def _kernel_ms(fn, steps, stream, warmup=2):
    """Mean ms per call of ``fn`` (kernel launches only, no host work in the
    loop), timed with HIP events on ``stream``, the stream fn launches on."""
    import torch

    with torch.cuda.stream(stream):
        for _ in range(warmup):
            fn()
        stream.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(steps):
            fn()
        end.record(stream)
        end.synchronize()
    return start.elapsed_time(end) / steps


def bench_prefill(args):
    """benchmark config 3: chunked prefill, B=16, T=4096, H=32, D=64, bf16 io,
    raw retention u ~ U(-8, 0), fp32 state pool updated in place."""
    import torch

    import flashrwkv_amd
    from flashrwkv_amd import workloads
    from flashrwkv_amd.tmix.wkv7 import DECAY_RAW_W

    if flashrwkv_amd._C is None:
        raise SystemExit("flashrwkv_amd native library is not built")
    ops = flashrwkv_amd._C.ops
    dev = torch.device("cuda:0")
    batch, t_len, heads, d = 16, 4096, 32, 64
    n_tok = batch * t_len
    tok = workloads.make_tokens(n_tok, heads, d, dtype=torch.bfloat16, seed=20260807,
                                device=dev, u_low=-8.0)
    pool = torch.zeros((batch, heads, d, d), device=dev)
    cu = torch.arange(0, n_tok + 1, t_len, device=dev, dtype=torch.int32)
    slots = torch.arange(batch, device=dev, dtype=torch.int32)
    stream = torch.cuda.Stream(device=dev)
    # Inputs were made on the default stream: order the side stream after them.
    stream.wait_stream(torch.cuda.current_stream(dev))

    def step():
        ops.chunk_forward_internal(tok["r"], tok["w"], tok["k"], tok["v"], tok["a"],
                                   tok["b"], pool, cu, slots, 1.0, DECAY_RAW_W, None)

    with torch.cuda.stream(stream):
        for _ in range(3):
            step()
        stream.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(args.prefill_steps):
            step()
        end.record(stream)
        end.synchronize()
    ms = start.elapsed_time(end) / args.prefill_steps
    # The kernel alone: the op above validates the metadata on every call
    # (two small kernels); through the C ABI the validated snapshot is reused.
    from flashrwkv_amd import capi
    status, cu_snap, slot_snap = capi.metadata_validate(cu, slots, n_tok, batch)
    out_t = torch.empty_like(tok["v"])
    kernel_ms = _kernel_ms(lambda: capi.chunk_forward(
        tok["r"], tok["w"], tok["k"], tok["v"], tok["a"], tok["b"], state_pool=pool,
        cu_seqlens=cu_snap, state_indices=slot_snap, metadata_status=status, output=out_t,
        decay_mode=DECAY_RAW_W), args.prefill_steps, stream)
    chunk_heads = batch * heads * (t_len // 64)
    flops = chunk_heads * chunk_flops()
    nbytes = n_tok * heads * 7 * d * 2 + 2 * batch * heads * d * d * 4
    tflops = flops / (kernel_ms * 1e-3) / 1e12
    gbps = nbytes / (kernel_ms * 1e-3) / 1e9
    attainable = min(BF16_PEAK_TFLOPS, flops / nbytes * HBM_PEAK_GBPS / 1e3)
    out = {
        "workload": "wkv7_chunked_prefill_cfg3: B=16, T=4096, H=32, D=64, bf16 io, chunk 64, "
                    "raw retention u~U(-8,0), fp32 state pool",
        "ms_per_step": round(ms, 4),
        "tokens_per_s": round(n_tok / (ms * 1e-3), 1),
        "kernel_ms": round(kernel_ms, 4),
        "kernel_tokens_per_s": round(n_tok / (kernel_ms * 1e-3), 1),
        "timing": "ms_per_step: the op per call (metadata validation + kernel); kernel_ms "
                  "and the roofline: the kernel alone through the C ABI",
        "steps": args.prefill_steps,
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2),
                     "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / BF16_PEAK_TFLOPS, 4),
                     "frac_of_attainable": round(tflops / attainable, 4),
                     "attainable": round(attainable, 1),
                     "traffic": pmc_traffic("chunk_fwd_kernel<Bf16,kRawW,float>"),
                     "mfma_busy_pct": pmc_mfma_busy("chunk_fwd_kernel<Bf16,kRawW,float>"),
                     "kernel": "chunk_fwd_kernel<Bf16,kRawW,float>",
                     "algorithmic_flops_per_launch": flops},
        "hbm": {"achieved_GBps": round(gbps, 1), "peak": HBM_PEAK_GBPS,
                "frac": round(gbps / HBM_PEAK_GBPS, 4),
                "algorithmic_bytes_per_launch": nbytes},
    }
    if args.cpu_seconds > 0:
        out["cpu_baseline"] = cpu_baseline_prefill(t_len, heads, args.cpu_seconds)
        out["cpu_baseline"]["torch_fp32"] = cpu_baseline_torch(
            [t_len], 8, args.cpu_seconds / 2, seed=98, u_low=-8.0, heads_total=heads)
    return out


def bench_prefill_varlen(args):
    """benchmark config 3, varlen batch: 64 packed sequences with lengths
    uniform in [128, 4096] (seeded), H=32, D=64, bf16 io, u ~ U(-8, 0), fp32
    pool. Algorithmic FLOPs count each sequence's chunks at their real length
    (a partial last chunk of c tokens costs chunk_flops(c))."""
    import torch

    import flashrwkv_amd
    from flashrwkv_amd import workloads
    from flashrwkv_amd.tmix.wkv7 import DECAY_RAW_W

    ops = flashrwkv_amd._C.ops
    dev = torch.device("cuda:0")
    heads, d = 32, 64
    lengths = workloads.varlen_lengths()
    n_tok = sum(lengths)
    tok = workloads.make_tokens(n_tok, heads, d, dtype=torch.bfloat16, seed=20260810,
                                device=dev, u_low=-8.0)
    offsets = [0]
    for length in lengths:
        offsets.append(offsets[-1] + length)
    cu = torch.tensor(offsets, device=dev, dtype=torch.int32)
    batch = len(lengths)
    slots = torch.arange(batch, device=dev, dtype=torch.int32)
    pool = torch.zeros((batch, heads, d, d), device=dev)
    stream = torch.cuda.Stream(device=dev)
    # Inputs were made on the default stream: order the side stream after them.
    stream.wait_stream(torch.cuda.current_stream(dev))

    def step():
        ops.chunk_forward_internal(tok["r"], tok["w"], tok["k"], tok["v"], tok["a"],
                                   tok["b"], pool, cu, slots, 1.0, DECAY_RAW_W, None)

    with torch.cuda.stream(stream):
        for _ in range(3):
            step()
        stream.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(args.prefill_steps):
            step()
        end.record(stream)
        end.synchronize()
    ms = start.elapsed_time(end) / args.prefill_steps
    from flashrwkv_amd import capi
    status, cu_snap, slot_snap = capi.metadata_validate(cu, slots, n_tok, batch)
    out_t = torch.empty_like(tok["v"])
    kernel_ms = _kernel_ms(lambda: capi.chunk_forward(
        tok["r"], tok["w"], tok["k"], tok["v"], tok["a"], tok["b"], state_pool=pool,
        cu_seqlens=cu_snap, state_indices=slot_snap, metadata_status=status, output=out_t,
        decay_mode=DECAY_RAW_W), args.prefill_steps, stream)
    flops = heads * sum((length // 64) * chunk_flops() + chunk_flops(length % 64)
                        for length in lengths)
    nbytes = n_tok * heads * 7 * d * 2 + 2 * batch * heads * d * d * 4
    tflops = flops / (kernel_ms * 1e-3) / 1e12
    gbps = nbytes / (kernel_ms * 1e-3) / 1e9
    out = {
        "workload": f"wkv7_chunked_prefill_cfg3_varlen: {batch} sequences, lengths "
                    f"U[128,4096] (seeded; N={n_tok}), H=32, D=64, bf16 io, u~U(-8,0), "
                    "fp32 pool",
        "ms_per_step": round(ms, 4),
        "tokens_per_s": round(n_tok / (ms * 1e-3), 1),
        "kernel_ms": round(kernel_ms, 4),
        "achieved_TFLOPs": round(tflops, 2),
        "mfma_frac": round(tflops / BF16_PEAK_TFLOPS, 4),
        "mfma_busy_pct": pmc_mfma_busy("chunk_fwd_kernel<Bf16,kRawW,float>/varlen"),
        "achieved_GBps": round(gbps, 1),
        "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4),
        "algorithmic_flops": flops,
        "algorithmic_bytes": nbytes,
    }
    if args.cpu_seconds > 0:
        # The batch's first sequences, whole, as the oracle loops over them
        # (the C oracle one by one; the torch restatement over the packed run).
        sample = lengths[:4]
        out["cpu_baseline"] = cpu_baseline_prefill(0, heads, args.cpu_seconds, lengths=sample,
                                                   seed=20260810)
        out["cpu_baseline"]["torch_fp32"] = cpu_baseline_torch(
            sample, 8, args.cpu_seconds / 2, seed=20260810, u_low=-8.0, heads_total=heads)
    return out


def bench_training(args):
    """benchmark config 4: chunked forward + backward (StateTune), B=8, T=4096,
    H=64, D=64, chunk 64, bf16 io, raw retention, S0 ~ N(0, 0.1), dY ~ N(0, 1),
    dS_T ~ N(0, 0.01). One step = autograd forward + backward."""
    import torch

    import flashrwkv_amd
    from flashrwkv_amd import workloads
    from flashrwkv_amd.tmix.wkv7.statetune import statetune_recurrent_internal

    if flashrwkv_amd._C is None:
        raise SystemExit("flashrwkv_amd native library is not built")
    dev = torch.device("cuda:0")
    batch, t_len, heads, d = 8, 4096, 64, 64
    n_tok = batch * t_len
    tok = workloads.make_tokens(n_tok, heads, d, dtype=torch.bfloat16, seed=20260808,
                                device=dev)
    leaves = [tok[n].requires_grad_(True) for n in ("r", "w", "k", "v", "a", "b")]
    gen = torch.Generator(device=dev).manual_seed(20260809)
    s0 = (torch.randn((batch, heads, d, d), generator=gen, device=dev) * 0.1).requires_grad_(True)
    dy = torch.randn((n_tok, heads, d), generator=gen, device=dev).to(torch.bfloat16)
    ds = torch.randn((batch, heads, d, d), generator=gen, device=dev) * 0.01
    offsets = torch.arange(0, batch + 1, device=dev, dtype=torch.int32) * (t_len // 64)
    starts = torch.arange(0, n_tok, 64, device=dev, dtype=torch.int32)
    ends = starts + 64

    def step():
        for t in (*leaves, s0):
            t.grad = None  # fresh gradients each step, as after optimizer.zero_grad()
        y, st, _, _ = statetune_recurrent_internal(s0, offsets, starts, ends, *leaves)
        torch.autograd.backward([y, st], [dy, ds])

    for _ in range(2):
        step()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.training_steps):
        step()
    end.record()
    end.synchronize()
    ms = start.elapsed_time(end) / args.training_steps
    # The two kernels alone through the C ABI (the autograd step above also
    # clones S0, allocates outputs and gradients and splits no chunks here).
    from flashrwkv_amd import capi
    stream = torch.cuda.Stream(device=dev)
    stream.wait_stream(torch.cuda.current_stream(dev))
    raw = [t.detach() for t in leaves]
    st_k = s0.detach().clone()
    y_k = torch.empty_like(raw[3])
    bnd = torch.empty((batch * (t_len // 64), heads, d, d), device=dev)
    sda = torch.empty((n_tok, heads, d), device=dev)
    grads_k = [torch.empty_like(t) for t in raw]
    ds0_k = torch.empty_like(ds)
    # 64-token chunks have no interior piece starts; the buffer is passed as
    # the autograd path passes it.
    inner = torch.empty(capi.statetune_interior_bytes(d, heads, n_tok) // 4, device=dev)
    fwd_ms = _kernel_ms(lambda: capi.statetune_forward(
        *raw, sequence_chunk_offsets=offsets, chunk_token_starts=starts,
        chunk_token_ends=ends, state=st_k, output=y_k, boundary=bnd, state_dot_a=sda,
        interior=inner), args.training_steps, stream)
    bwd_ms = _kernel_ms(lambda: capi.statetune_backward(
        *raw, sequence_chunk_offsets=offsets, chunk_token_starts=starts,
        chunk_token_ends=ends, boundary=bnd, grad_output=dy, grad_final_state=ds,
        grads=grads_k, grad_initial_state=ds0_k, interior=inner), args.training_steps, stream)
    kernel_ms = fwd_ms + bwd_ms
    chunk_heads = batch * heads * (t_len // 64)
    flops = 3 * chunk_heads * chunk_flops()
    tok_bytes = n_tok * heads * d * 2
    state_bytes = batch * heads * d * d * 4
    boundary_bytes = chunk_heads * d * d * 4
    # forward: 6 token reads, y write, boundary and state_dot_a writes, S0/S_T;
    # backward: 6 token reads + dY, boundary read, 6 gradient writes, dS_T/dS0.
    nbytes = (6 + 1) * tok_bytes + 2 * boundary_bytes + 2 * state_bytes \
        + 7 * tok_bytes + boundary_bytes + 6 * tok_bytes + 2 * state_bytes
    tflops = flops / (kernel_ms * 1e-3) / 1e12
    gbps = nbytes / (kernel_ms * 1e-3) / 1e9
    out = {
        "workload": "wkv7_training_cfg4: chunked forward + backward (StateTune), B=8, T=4096, "
                    "H=64, D=64, chunk 64, bf16 io, raw retention, fp32 state and boundaries",
        "ms_per_step": round(ms, 4),
        "train_tokens_per_s": round(n_tok / (ms * 1e-3), 1),
        "kernel_ms": {"forward": round(fwd_ms, 4), "backward": round(bwd_ms, 4)},
        "timing": "ms_per_step: autograd forward + backward; kernel_ms and the roofline: "
                  "the two kernels alone through the C ABI",
        "steps": args.training_steps,
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / BF16_PEAK_TFLOPS, 4),
                     "algorithmic_flops_per_step": flops,
                     "traffic": _sum_or_none(pmc_traffic("chunk_fwd_kernel<Bf16,kRawW,float>/statetune"),
                                             pmc_traffic("chunk_bwd_kernel<Bf16,kRawW>")),
                     "mfma_busy_pct": {
                         "forward": pmc_mfma_busy("chunk_fwd_kernel<Bf16,kRawW,float>/statetune"),
                         "backward": pmc_mfma_busy("chunk_bwd_kernel<Bf16,kRawW>")},
                     "kernel": "chunk_fwd_kernel<Bf16,kRawW,float> + chunk_bwd_kernel<Bf16,kRawW>"},
        "hbm": {"achieved_GBps": round(gbps, 1), "peak": HBM_PEAK_GBPS,
                "frac": round(gbps / HBM_PEAK_GBPS, 4), "algorithmic_bytes_per_step": nbytes},
    }
    if args.cpu_seconds > 0:
        out["cpu_baseline"] = cpu_baseline_training(t_len, heads, args.cpu_seconds)
        out["cpu_baseline"]["torch_fp32"] = cpu_baseline_torch(
            [t_len], 4, args.cpu_seconds / 2, heads_total=heads, backward=True)
    return out


def cpu_baseline_training(t_len, heads_total, seconds, head_size=64):
    """fp64 C oracle forward + adjoint on a bounded sample of whole (sequence,
    head) recurrences (heads are independent, so the rate scales exactly; the
    per-token work does not depend on the sequence length, so a shorter
    sample sequence measures the same rate)."""
    import numpy as np
    import torch

    from flashrwkv_amd import workloads
    from oracle import oracle

    cores = len(os.sched_getaffinity(0))
    sample_heads = max(1, cores)
    case = workloads.make_case(lengths=[t_len], heads=sample_heads, head_size=head_size,
                               dtype=torch.bfloat16, seed=97, state_std=0.1)
    args = [case[n].double().numpy() for n in ("r", "w", "k", "v", "a", "b")]
    s0 = case["state_pool"].double().numpy()
    so, ss, se = oracle.segments_from_cu_seqlens(case["cu_seqlens"].numpy())
    slots = np.zeros(1, dtype=np.int32)
    dy = np.random.default_rng(0).standard_normal(args[0].shape)
    reps = 0
    t0 = time.perf_counter()
    while True:
        oracle.forward(*args, s0, seg_offsets=so, seg_starts=ss, seg_ends=se,
                       state_slots=slots, num_threads=cores)
        oracle.backward(*args, s0, seg_offsets=so, seg_starts=ss, seg_ends=se,
                        state_slots=slots, dy=dy, num_threads=cores)
        reps += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= seconds:
            break
    return {
        "value": reps * t_len * sample_heads / elapsed / heads_total,
        "unit": "train tokens/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{reps} x (1 sequence x {sample_heads} heads x T={t_len}, D={head_size}) "
                  f"forward + adjoint through the fp64 C oracle, OpenMP over heads, "
                  f"{elapsed:.1f} s; token-heads/s divided by H={heads_total}",
    }


def bench_training_large(args):
    """StateTune at head sizes 128 (bf16 MFMA over 16-token pieces) and 256
    (the per-token fp32 training kernels): B=8, T=4096, C=H*D=4096, bf16 io, raw retention, S0 ~ N(0, 0.1),
    dY ~ N(0, 1), dS_T ~ N(0, 0.01), caller chunks of 64 tokens (split into
    16-token kernel chunks by the wrapper). One step = autograd forward +
    backward. No benchmark config uses these head sizes; this leg records their
    cost beside config 4's D=64 step."""
    import torch

    import flashrwkv_amd
    from flashrwkv_amd import workloads
    from flashrwkv_amd.tmix.wkv7.statetune import statetune_recurrent_internal

    if flashrwkv_amd._C is None:
        raise SystemExit("flashrwkv_amd native library is not built")
    dev = torch.device("cuda:0")
    out = {}
    for d in (128, 256):
        batch, t_len, heads = 8, 4096, 4096 // d
        n_tok = batch * t_len
        tok = workloads.make_tokens(n_tok, heads, d, dtype=torch.bfloat16, seed=20260812 + d,
                                    device=dev)
        leaves = [tok[n].requires_grad_(True) for n in ("r", "w", "k", "v", "a", "b")]
        gen = torch.Generator(device=dev).manual_seed(20260813 + d)
        s0 = (torch.randn((batch, heads, d, d), generator=gen, device=dev) * 0.1
              ).requires_grad_(True)
        dy = torch.randn((n_tok, heads, d), generator=gen, device=dev).to(torch.bfloat16)
        ds = torch.randn((batch, heads, d, d), generator=gen, device=dev) * 0.01
        offsets = torch.arange(0, batch + 1, device=dev, dtype=torch.int32) * (t_len // 64)
        starts = torch.arange(0, n_tok, 64, device=dev, dtype=torch.int32)
        ends = starts + 64

        def step():
            for t in (*leaves, s0):
                t.grad = None
            y, st, _, _ = statetune_recurrent_internal(s0, offsets, starts, ends, *leaves)
            torch.autograd.backward([y, st], [dy, ds])

        step()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        steps = max(1, args.training_steps // 5)
        e0.record()
        for _ in range(steps):
            step()
        e1.record()
        e1.synchronize()
        ms = e0.elapsed_time(e1) / steps
        out[f"d{d}"] = {"workload": f"StateTune B=8, T=4096, H={heads}, D={d}, bf16, raw "
                                    f"retention, 64-token caller chunks",
                        "steps": steps, "ms_per_step": round(ms, 3),
                        "train_tokens_per_s": round(n_tok / (ms * 1e-3), 1)}
        if args.cpu_seconds > 0:
            out[f"d{d}"]["cpu_baseline"] = cpu_baseline_training(
                512, heads, args.cpu_seconds / 4, head_size=d)
        del tok, leaves, s0, dy, ds
        torch.cuda.empty_cache()
    return out


def bench_config0(args):
    """benchmark config 0, the reference's CPU-runnable case: fp32 io, B=1,
    T=64, H=32, D=64, S0 = 0, raw retention. fp32 tokens always run the
    per-token fp32 kernel (four waves per (sequence, head), 32 units), so the
    call is bound by its 64 dependent steps, not by bandwidth: the figures are
    microseconds per call and tokens/s; the HBM line only states the rate the
    call's 4.72 MB reach. kernel_us: 50 calls captured in one HIP graph and
    replayed (no host launch cost); op_us: the public-op path per eager call
    with a prepared ticket."""
    import torch

    import flashrwkv_amd
    from flashrwkv_amd import capi, workloads
    from flashrwkv_amd.tmix.wkv7 import DECAY_RAW_W, prepare_recurrent_metadata

    if flashrwkv_amd._C is None:
        raise SystemExit("flashrwkv_amd native library is not built")
    ops = flashrwkv_amd._C.ops
    dev = torch.device("cuda:0")
    t_len, heads, d = 64, 32, 64
    case = workloads.make_case(lengths=[t_len], heads=heads, head_size=d, dtype=torch.float32,
                               seed=20260804, state_std=0.0)
    tok = {n: case[n].to(dev) for n in ("r", "w", "k", "v", "a", "b")}
    cu, slots = case["cu_seqlens"].to(dev), case["state_indices"].to(dev)
    pool = torch.zeros((1, heads, d, d), device=dev)
    out_t = torch.empty_like(tok["v"])
    status, cu_snap, slot_snap = capi.metadata_validate(cu, slots, t_len, 1)
    stream = torch.cuda.Stream(device=dev)
    stream.wait_stream(torch.cuda.current_stream(dev))
    per_graph, replays = 50, 20

    def call():
        capi.recurrent_forward(tok["r"], tok["w"], tok["k"], tok["v"], tok["a"], tok["b"],
                               state_pool=pool, cu_seqlens=cu_snap, state_indices=slot_snap,
                               metadata_status=status, output=out_t, max_seqlen=t_len)

    with torch.cuda.stream(stream):
        call()
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for _ in range(per_graph):
                call()
        graph.replay()
        stream.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(replays):
            graph.replay()
        e1.record(stream)
        e1.synchronize()
    kernel_ms = e0.elapsed_time(e1) / (per_graph * replays)
    with torch.cuda.stream(stream):
        ticket = prepare_recurrent_metadata(cu, slots, total_tokens=t_len, state_pool_size=1,
                                            max_seqlen=t_len)
        op_ms = _kernel_ms(lambda: ops.recurrent_fp32_forward_internal(
            cu, slots, pool, tok["r"], tok["w"], tok["k"], tok["v"], tok["a"], tok["b"],
            out_t, 1.0, DECAY_RAW_W, None, ticket, t_len), 200, stream)
    nbytes = t_len * heads * 7 * d * 4 + 2 * heads * d * d * 4
    flops = 9 * d * d * t_len * heads
    gbps = nbytes / (kernel_ms * 1e-3) / 1e9
    out = {
        "workload": "wkv7_recurrent_cfg0: fp32 io, B=1, T=64, H=32, D=64, S0=0, raw retention "
                    "(per-token fp32 kernel)",
        "kernel_us": round(kernel_ms * 1e3, 2),
        "op_us": round(op_ms * 1e3, 2),
        "tokens_per_s": round(t_len / (kernel_ms * 1e-3), 1),
        "bound": "latency (64 dependent steps per (sequence, head); 32 units)",
        "hbm": {"achieved_GBps": round(gbps, 1), "peak": HBM_PEAK_GBPS,
                "frac": round(gbps / HBM_PEAK_GBPS, 4), "algorithmic_bytes_per_call": nbytes},
        "algorithmic_flops_per_call": flops,
        "timing": "kernel_us: 50 calls in one HIP graph, replayed 20 times, HIP events on "
                  "the launch stream; op_us: the internal op with a prepared ticket, eager",
    }
    if args.cpu_seconds > 0:
        tb = cpu_baseline_torch([t_len], heads, args.cpu_seconds / 2, seed=20260804,
                                heads_total=heads, dtype=torch.float32)
        out["cpu_baseline"] = {
            "value": tb["all_cores"]["value"], "unit": "tokens/s",
            "cores": tb["all_cores"]["threads"], "kind": "port",
            "sample": tb["sample"] + " (fp32 tokens), every core",
            "one_thread": tb["one_thread"],
            "fp64_c_oracle": cpu_baseline_prefill(t_len, heads, args.cpu_seconds / 2,
                                                  u_low=-5.0, seed=20260804),
        }
    return out


def bench_pretrain(args):
    """clampw-v3 pretraining at the reference pretraining bench's shape
    (benchmarks/tmix/wkv7/pretrain/bench.py:16-63): B=2, T=512, H=12, D=64,
    dense bf16 [B,T,C] inputs N(0,1) * 0.05 (w as decay logits), dY ~ N(0,1);
    one step = pretrain_recurrent_bf16 forward + torch.autograd.grad to all
    six inputs, as that bench times it (5 warm-up steps). The shape has 192
    chunk-heads for 256 CUs, so the step is bound by the chunk recurrence's
    latency, not by bandwidth or the matrix cores."""
    import torch

    import flashrwkv_amd
    from flashrwkv_amd import capi
    from flashrwkv_amd.tmix.wkv7 import pretrain_recurrent_bf16

    if flashrwkv_amd._C is None:
        raise SystemExit("flashrwkv_amd native library is not built")
    dev = torch.device("cuda:0")
    batch, t_len, heads, d = 2, 512, 12, 64
    shape = (batch, t_len, heads * d)
    gen = torch.Generator(device=dev).manual_seed(20260806)
    values = tuple((torch.randn(shape, generator=gen, device=dev) * 0.05).to(torch.bfloat16)
                   .requires_grad_() for _ in range(6))
    grad_output = torch.randn(shape, generator=gen, device=dev).to(torch.bfloat16)

    def step():
        y = pretrain_recurrent_bf16(*values)
        torch.autograd.grad(y, values, grad_output)

    for _ in range(5):
        step()
    torch.cuda.synchronize()
    iters = max(10, 5 * args.training_steps)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        step()
    e1.record()
    e1.synchronize()
    ms = e0.elapsed_time(e1) / iters
    # The two kernels alone through the C ABI.
    stream = torch.cuda.Stream(device=dev)
    stream.wait_stream(torch.cuda.current_stream(dev))
    split = [v.detach().view(batch, t_len, heads, d) for v in values]
    y_k = torch.empty_like(split[3])
    bnd = torch.empty((batch, heads, t_len // 16, d, d), device=dev)
    sda = torch.empty((batch, t_len, heads, d), device=dev, dtype=torch.float32)
    grads = [torch.empty_like(t) for t in split]
    dy = grad_output.view(batch, t_len, heads, d)
    fwd_ms = _kernel_ms(lambda: capi.pretrain_forward(*split, output=y_k, boundary=bnd,
                                                      state_dot_a=sda), iters, stream)
    bwd_ms = _kernel_ms(lambda: capi.pretrain_backward(*split, grad_output=dy, boundary=bnd,
                                                       grads=grads), iters, stream)
    chunk_heads = batch * heads * (t_len // 64)
    flops = 3 * chunk_heads * chunk_flops()
    tflops = flops / ((fwd_ms + bwd_ms) * 1e-3) / 1e12
    out = {
        "workload": "clampw-v3 pretraining, reference bench shape: B=2, T=512, H=12, D=64, "
                    "bf16, decay logits, S0=0",
        "ms_per_step": round(ms, 4),
        "train_tokens_per_s": round(batch * t_len / (ms * 1e-3), 1),
        "kernel_ms": {"forward": round(fwd_ms, 4), "backward": round(bwd_ms, 4)},
        "achieved_TFLOPs": round(tflops, 3),
        "mfma_frac": round(tflops / BF16_PEAK_TFLOPS, 5),
        "algorithmic_flops_per_step": flops,
        "bound": "latency (192 chunk-heads, 8 chunks each, on 256 CUs)",
        "timing": "ms_per_step: autograd forward + torch.autograd.grad, as the reference "
                  "bench; kernel_ms: the two kernels alone through the C ABI",
        "iterations": iters,
    }
    if args.cpu_seconds > 0:
        tb = cpu_baseline_torch([t_len] * batch, heads, args.cpu_seconds / 2, seed=20260806,
                                heads_total=heads, backward=True)
        out["cpu_baseline"] = {
            "value": tb["all_cores"]["value"], "unit": "train tokens/s",
            "cores": tb["all_cores"]["threads"], "kind": "port",
            "sample": tb["sample"] + ", every core (RWKV-7 input distributions and raw "
                      "retention: the same arithmetic as the logits form)",
            "one_thread": tb["one_thread"],
            "fp64_c_oracle": cpu_baseline_training(t_len, heads, args.cpu_seconds / 2),
        }
    return out


def bench_copy(args):
    """A plain device copy of known size: the calibration run for the
    FETCH_SIZE / WRITE_SIZE counters (bytes per dispatch vs counter KiB)."""
    import torch

    n = 256 * 1024 * 1024 // 4  # 256 MiB of fp32
    src = torch.rand(n, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    return {"workload": "copy_calibration", "bytes_read": n * 4, "bytes_written": n * 4,
            "dispatches": 5}


def bench_recurrent_long(args):
    """benchmark config 2: B=8, T=4096, H=32, D=64, bf16 io, fp32 state, S0 = 0:
    the recurrent operator (max_seqlen known, so its split-precision chunk
    kernel), the operator's fp32 per-token kernel (max_seqlen unknown) and
    the plain bf16 chunk operator."""
    import torch

    import flashrwkv_amd
    from flashrwkv_amd import workloads
    from flashrwkv_amd.tmix.wkv7 import DECAY_RAW_W, prepare_recurrent_metadata

    if flashrwkv_amd._C is None:
        raise SystemExit("flashrwkv_amd native library is not built")
    ops = flashrwkv_amd._C.ops
    dev = torch.device("cuda:0")
    batch, t_len, heads, d = 8, 4096, 32, 64
    n_tok = batch * t_len
    tok = workloads.make_tokens(n_tok, heads, d, dtype=torch.bfloat16, seed=20260806,
                                device=dev)
    cu = torch.arange(0, n_tok + 1, t_len, device=dev, dtype=torch.int32)
    slots = torch.arange(batch, device=dev, dtype=torch.int32)
    pool = torch.zeros((batch, heads, d, d), device=dev)
    out = torch.empty((n_tok, heads, d), device=dev, dtype=torch.bfloat16)
    args_tok = (tok["r"], tok["w"], tok["k"], tok["v"], tok["a"], tok["b"])

    def timed(fn, reps):
        fn()
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            fn()
        end.record()
        end.synchronize()
        return start.elapsed_time(end) / reps

    # The operator with a validated-metadata ticket (no per-call validation
    # launch), as a serving loop calls it.
    ticket = prepare_recurrent_metadata(cu, slots, total_tokens=n_tok, state_pool_size=batch,
                                        max_seqlen=t_len)
    op_ms = timed(lambda: ops.recurrent_fp32_forward_internal(
        cu, slots, pool, *args_tok, out, 1.0, DECAY_RAW_W, None, ticket, t_len), 10)
    token_ms = timed(lambda: ops.recurrent_fp32_forward_internal(
        cu, slots, pool, *args_tok, out, 1.0, DECAY_RAW_W, None, None, -1), 3)
    chunk_ms = timed(lambda: ops.chunk_forward_internal(
        *args_tok, pool, cu, slots, 1.0, DECAY_RAW_W, None), 10)
    nbytes = n_tok * heads * 7 * d * 2 + 2 * batch * heads * d * d * 4

    def leg(ms, what):
        return {"ms": round(ms, 4), "kernel": what,
                "tokens_per_s": round(n_tok / (ms * 1e-3), 1),
                "achieved_GBps": round(nbytes / (ms * 1e-3) / 1e9, 1)}

    op = leg(op_ms, "chunk_fwd_kernel, split-bf16 products")
    kernel = "chunk_fwd_kernel<Bf16,kRawW,float>/precise"
    op["roofline"] = {
        "bound": "hbm", "achieved": op["achieved_GBps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
        "frac": round(op["achieved_GBps"] / HBM_PEAK_GBPS, 4), "traffic": pmc_traffic(kernel),
        "mfma_busy_pct": pmc_mfma_busy(kernel),
        "kernel": kernel, "algorithmic_bytes_per_launch": nbytes,
    }
    out = {
        "workload": "wkv7_recurrent_long_cfg2: B=8, T=4096, H=32, D=64, bf16 io, fp32 state",
        "recurrent_op": op,
        "per_token_kernel": leg(token_ms, "recurrent_fp32_kernel"),
        "bf16_chunk_op": leg(chunk_ms, "chunk_fwd_kernel, bf16 products"),
        "algorithmic_bytes": nbytes,
    }
    if args.cpu_seconds > 0:
        out["cpu_baseline"] = cpu_baseline_prefill(t_len, heads, args.cpu_seconds, u_low=-5.0,
                                                   seed=20260806)
        out["cpu_baseline"]["torch_fp32"] = cpu_baseline_torch(
            [t_len], 8, args.cpu_seconds / 2, seed=20260806, heads_total=heads)
    return out


# The reference operator benchmark's case matrix (benchmarks/tmix/wkv7/bench.py:132-172):
# 21 (B, T) cases, operator shapes h32/h40/h64 at D=64, and the stress cases.
MATRIX_BT = ((1, 1), (1, 2), (1, 4), (1, 8), (1, 16), (1, 32), (1, 64), (1, 128), (1, 256),
             (2, 1), (4, 1), (8, 1), (16, 1), (32, 1), (64, 1), (128, 1), (256, 1),
             (2, 2), (4, 4), (8, 8), (16, 16))
MATRIX_SHAPES = {"h32d64": 32, "h40d64": 40, "h64d64": 64}
MATRIX_STRESS = {
    "stress_decode_b320_t1": (1,) * 320,
    "stress_decode_b2048_t1": (1,) * 2048,
    "stress_equal_b320_t16": (16,) * 320,
    "stress_ragged_b320_t1_to_t16": tuple(range(1, 17)) * 20,
    "stress_ragged_long_b32": (1, 4, 8, 16, 32, 64, 96, 128) * 4,
    "stress_ragged_skew_b32": (128,) + (1,) * 31,
}
# fp32io16_recurrent relative-RMSE limits (reference tests/fixtures/tolerances-v1.json:8-11).
MATRIX_RMSE_LIMIT = 0.002


def percentile(values, q):
    """Linear-interpolated percentile of ``values`` at ``q`` in [0, 1]
    (the reference bench's statistic, bench.py:581-592)."""
    if not values or not 0.0 <= q <= 1.0:
        raise ValueError("percentile needs samples and q in [0, 1]")
    ordered = sorted(values)
    pos = (len(ordered) - 1) * q
    lo, hi = int(pos // 1), int(-(-pos // 1))
    return ordered[lo] + (ordered[hi] - ordered[lo]) * (pos - lo)


def relative_rmse(actual, expected):
    """rmse(actual - expected) / max(rmse(expected), 1e-6), in fp32."""
    diff = actual.float() - expected.float()
    base = expected.float().square().mean().sqrt().clamp_min(1e-6)
    return float((diff.square().mean().sqrt() / base).item())


def fp32_gate_reference(r, x, k, v, a, b, pool, cu, slots, bias=None, scale=1.0):
    """fp32 torch restatement of the decay-logits recurrence for the matrix
    gate, on the tokens' device: one step per token position, batched over the
    sequences still running (elementwise products and sums, no batched GEMM).
    Returns (output fp32 [N,H,D], updated copy of the pool)."""
    import torch

    lengths = (cu[1:] - cu[:-1]).tolist()
    starts = cu[:-1].long()
    slot_idx = slots.long()
    state = pool.float().index_select(0, slot_idx).clone()
    out = torch.empty(r.shape, device=r.device, dtype=torch.float32)
    h, d = r.shape[1], r.shape[2]
    bias_f = None if bias is None else bias.float().reshape(h, d)
    len_t = torch.tensor(lengths, device=r.device)
    for t in range(max(lengths)):
        act = torch.nonzero(len_t > t).flatten()
        tok = starts.index_select(0, act) + t
        xs = x.index_select(0, tok).float()
        if bias_f is not None:
            xs = xs + bias_f
        w = torch.exp(-0.6065306597126334 * torch.sigmoid(xs))
        s = state.index_select(0, act)
        sa = (a.index_select(0, tok).float().unsqueeze(-1) * s).sum(dim=2)
        s = (w.unsqueeze(-1) * s + b.index_select(0, tok).float().unsqueeze(-1) * sa.unsqueeze(2)
             + k.index_select(0, tok).float().unsqueeze(-1) * v.index_select(0, tok).float()
             .unsqueeze(2))
        state.index_copy_(0, act, s)
        out.index_copy_(0, tok, scale * (r.index_select(0, tok).float().unsqueeze(-1) * s)
                        .sum(dim=2))
    new_pool = pool.float().clone()
    new_pool.index_copy_(0, slot_idx, state)
    return out, new_pool


def bench_matrix(args):
    """The reference operator benchmark (benchmarks/tmix/wkv7/bench.py) on this
    build: for every case of the (B, T) matrix (plus the stress cases with
    --matrix-stress) and operator shape, the reference's input recipe
    (bench.py:309-371: r*0.15, decay logits*4.0, k/v/a/b*0.08, a pool of B+4
    slots ~ N(0, 0.02), state_indices reversed, seed + case index), its
    correctness gate (bench.py:374-501: relative RMSE of output and written
    state <= 0.002 against an fp32 recurrence, untouched slots bitwise equal,
    a second launch bitwise equal, finite values) and its timing (bench.py:
    542-578: warm-up, then samples of consecutive in-place launches, each
    sample from a reset pool, timed with events; p10/p50/p90 and tok_s_p50).
    Launches go through recurrent_fp32_from_decay_logits with a validated
    ticket, as the reference's timed boundary does. Each row adds the HBM
    rate of the algorithmic bytes at p50."""
    import torch

    import flashrwkv_amd

    if flashrwkv_amd._C is None:
        raise SystemExit("flashrwkv_amd native library is not built")
    ops = flashrwkv_amd._C.ops
    dev = torch.device("cuda:0")
    dtype = {"bfloat16": torch.bfloat16, "float16": torch.float16}[args.matrix_dtype]
    cases = [(f"{bsz}x{t}", (t,) * bsz) for bsz, t in MATRIX_BT]
    if args.matrix_stress:
        cases += list(MATRIX_STRESS.items())
    rows = []
    for shape_name, heads in MATRIX_SHAPES.items():
        d = 64
        for index, (label, lengths) in enumerate(cases):
            bsz, n_tok = len(lengths), sum(lengths)
            gen = torch.Generator(device=dev).manual_seed(args.matrix_seed + index)

            def rnd(scale):
                return (torch.randn((n_tok, heads, d), device=dev, generator=gen) * scale).to(
                    dtype)

            r, x, k, v, a, b = rnd(0.15), rnd(4.0), rnd(0.08), rnd(0.08), rnd(0.08), rnd(0.08)
            offsets = [0]
            for length in lengths:
                offsets.append(offsets[-1] + length)
            cu = torch.tensor(offsets, device=dev, dtype=torch.int32)
            slots = torch.arange(bsz - 1, -1, -1, device=dev, dtype=torch.int32)
            pool = torch.randn((bsz + 4, heads, d, d), device=dev, generator=gen) * 0.02
            ticket = flashrwkv_amd.prepare_recurrent_metadata(
                cu, slots, total_tokens=n_tok, state_pool_size=bsz + 4)
            # Correctness gate.
            y_ref, pool_ref = fp32_gate_reference(r, x, k, v, a, b, pool, cu, slots)
            outs = []
            for _ in range(2):
                st = pool.clone()
                y = flashrwkv_amd.infer_recurrent_fp32io16_forward_varlen(
                    r, x, k, v, a, b, state_pool=st, cu_seqlens=cu, state_indices=slots,
                    validated_metadata=ticket)
                outs.append((y, st))
            torch.cuda.synchronize()
            (y, st), (y2, st2) = outs
            act = slots.long()
            unused = torch.tensor([i for i in range(bsz + 4) if i not in set(act.tolist())],
                                  device=dev, dtype=torch.long)
            gate = {
                "output_relative_rmse": relative_rmse(y, y_ref),
                "state_relative_rmse": relative_rmse(st.index_select(0, act),
                                                     pool_ref.index_select(0, act)),
                "untouched_slots": bool(torch.equal(st.index_select(0, unused),
                                                    pool.index_select(0, unused))),
                "deterministic": bool(torch.equal(y, y2) and torch.equal(st, st2)),
                "finite": bool(torch.isfinite(y.float()).all()
                               and torch.isfinite(st.index_select(0, act)).all()),
            }
            gate["passed"] = bool(gate["finite"] and gate["untouched_slots"]
                                  and gate["deterministic"]
                                  and gate["output_relative_rmse"] <= MATRIX_RMSE_LIMIT
                                  and gate["state_relative_rmse"] <= MATRIX_RMSE_LIMIT)
            # The operator's kernel for this call (its rule in frwkv_recurrent_forward:
            # bf16 tokens at head size 64 with max_seqlen >= 64 take the split-bf16
            # chunk kernel).
            chunked = args.matrix_dtype == "bfloat16" and max(lengths) >= 64
            row = {"operator_shape": shape_name, "case": label, "B": bsz,
                   "T": lengths[0] if len(set(lengths)) == 1 else None,
                   "max_seqlen": max(lengths),
                   "kernel": "chunk_fwd_kernel (split-bf16)" if chunked
                   else "recurrent_fp32_kernel",
                   "total_tokens": n_tok, "dtype": args.matrix_dtype, "correctness": gate}
            if gate["passed"]:
                out = torch.empty_like(v)
                state = pool.clone()

                def launch():
                    ops.recurrent_fp32_from_decay_logits(cu, slots, state, r, x, k, v, a, b,
                                                         out, 1.0, None, ticket, -1)

                for _ in range(args.matrix_warmup):
                    state.copy_(pool)
                    for _ in range(args.matrix_sample_iters):
                        launch()
                torch.cuda.synchronize()
                samples = []
                for _ in range(args.matrix_samples):
                    state.copy_(pool)
                    e0 = torch.cuda.Event(enable_timing=True)
                    e1 = torch.cuda.Event(enable_timing=True)
                    e0.record()
                    for _ in range(args.matrix_sample_iters):
                        launch()
                    e1.record()
                    e1.synchronize()
                    samples.append(e0.elapsed_time(e1) / args.matrix_sample_iters)
                p50 = percentile(samples, 0.5)
                nbytes = bsz * heads * 2 * d * d * 4 + n_tok * heads * 7 * d * 2
                row["timing"] = {
                    "p10_ms": round(percentile(samples, 0.1), 6), "p50_ms": round(p50, 6),
                    "p90_ms": round(percentile(samples, 0.9), 6),
                    "tok_s_p50": round(n_tok * 1000.0 / p50, 3),
                    "hbm_GBps_p50": round(nbytes / (p50 * 1e-3) / 1e9, 1),
                    "algorithmic_bytes": nbytes,
                }
                print(f"RESULT operator_shape={shape_name} case={label} dtype={args.matrix_dtype} "
                      f"correctness=passed p10_ms={row['timing']['p10_ms']:.6f} "
                      f"p50_ms={p50:.6f} p90_ms={row['timing']['p90_ms']:.6f} "
                      f"tok_s_p50={row['timing']['tok_s_p50']:.3f}", file=sys.stderr,
                      flush=True)
            else:
                row["failure"] = "correctness gate failed"
                print(f"RESULT operator_shape={shape_name} case={label} correctness=failed",
                      file=sys.stderr, flush=True)
            rows.append(row)
    return {"workload": "reference operator benchmark matrix (recurrent_fp32_from_decay_logits)",
            "warmup": args.matrix_warmup, "samples": args.matrix_samples,
            "sample_iters": args.matrix_sample_iters, "seed": args.matrix_seed,
            "rmse_limit": MATRIX_RMSE_LIMIT, "all_passed": all(r["correctness"]["passed"]
                                                                 for r in rows),
            "rows": rows}


def _progress(leg: str) -> None:
    """One line per finished leg on stderr (stdout carries only the JSON line)."""
    print(f"[bench] {leg} done", file=sys.stderr, flush=True)


def main():
    args = _parse()
    if args.gpus != 1:
        print(json.dumps({"error": f"--gpus {args.gpus}: this build measures one GPU only. "
                          "Every (sequence, head) recurrence is independent, so N GPUs "
                          "would each run the one-GPU kernels on their share of sequences "
                          "or heads with no communication; no multi-GPU run is made."}))
        raise SystemExit(2)
    if args.workload == "prefill":
        pre = bench_prefill(args)
        line = {
            "metric": METRIC, "value": pre["tokens_per_s"], "unit": "tokens/s",
            "n_gpus": 1, "steps": args.prefill_steps, "warmup": 3,
            "ms_per_step": pre["ms_per_step"], "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (seeded; benchmark config 3 distributions)",
            "config": {"workload": pre["workload"], "parallelism": "single GPU"},
            "roofline": pre["roofline"], "hbm": pre["hbm"],
        }
        if "cpu_baseline" in pre:
            line["cpu_baseline"] = pre["cpu_baseline"]
        line["varlen"] = bench_prefill_varlen(args)
    elif args.workload == "training":
        line = {"metric": METRIC, "training": bench_training(args)}
    elif args.workload == "copy":
        line = {"metric": METRIC, "copy": bench_copy(args)}
    elif args.workload == "recurrent_long":
        line = {"metric": METRIC, "recurrent_long": bench_recurrent_long(args)}
    elif args.workload == "decode_fp16":
        line = {"metric": METRIC, "decode_fp16_state": bench_decode(args, fp16_state=True)}
    elif args.workload == "decode_fused":
        line = {"metric": METRIC, "decode_tmix_fused": bench_decode_fused(args)}
    elif args.workload == "matrix":
        line = {"metric": METRIC, "matrix": bench_matrix(args)}
    elif args.workload == "training_large":
        line = {"metric": METRIC, "training_large_heads": bench_training_large(args)}
    elif args.workload == "config0":
        line = {"metric": METRIC, "recurrent_cfg0": bench_config0(args)}
    elif args.workload == "pretrain":
        line = {"metric": METRIC, "pretrain_clampw": bench_pretrain(args)}
    else:
        line = bench_decode(args)
        _progress("decode")
        if args.workload == "all":
            legs = (("decode_fp16_state", lambda: bench_decode(args, fp16_state=True)),
                    ("decode_tmix_fused", lambda: bench_decode_fused(args)),
                    ("chunked_prefill", lambda: bench_prefill(args)),
                    ("varlen", lambda: bench_prefill_varlen(args)),
                    ("training", lambda: bench_training(args)),
                    ("recurrent_long", lambda: bench_recurrent_long(args)),
                    ("recurrent_cfg0", lambda: bench_config0(args)),
                    ("pretrain_clampw", lambda: bench_pretrain(args)),
                    ("training_large_heads", lambda: bench_training_large(args)))
            for name, leg in legs:
                if name == "varlen":
                    line["chunked_prefill"]["varlen"] = leg()
                else:
                    line[name] = leg()
                _progress(name)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
