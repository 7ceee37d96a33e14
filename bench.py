"""Benchmark: one full Muon optimizer.step() on the Llama-3-8B-shaped parameter set.

Workload: 32 layers x {q, o 4096x4096; k, v 1024x4096;
gate, up 14336x4096; down 4096x14336} bf16 parameters (6.98e9 values) with fp32
momentum, synthetic gradients g = diag(exp(z)) Z (z ~ N(0,1) per row, Z ~ N(0,1)),
Polar Express 5 steps, cautious weight decay 0.1, Nesterov 0.95, foreach batching by
shape. A step is one optimizer.step() over the whole set; inputs are resident in HBM.

Prints one JSON line: value = orthogonalization TFLOP/s of the whole step
(symmetric-minimal FLOPs 3 m^2 n + m^3 per matrix per iteration / step time),
ms_per_step = Muon step time, plus the roofline of the dominant kernel (the B X GEMM)
from hipEvent timing of every launch, per-kernel breakdowns, and the CPU baseline
(the oracle's per-parameter loop on a bounded sample, on this host's cores).

The K timed steps run without per-launch events (the step as a caller runs it); K more
steps with the library's per-launch hipEvent brackets on give the per-kernel breakdown and
the roofline, and their step time is printed beside (breakdown_ms_per_step).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
       [--config llama|gpt2|moe|moe_flat|plumbing] [--lp 8bit|4bit|fp8 [--block-size N|tensor]]
       [--no-cpu-baseline] | --reference-suite | --blas-ceiling | --calibrate-copy
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "dtensor-muon_amd"))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E

CONFIGS = {
    # name: (layers, [(rows, cols, per-layer count)], workload label)
    "llama": (32, [(4096, 4096, 2), (1024, 4096, 2), (14336, 4096, 2), (4096, 14336, 1)],
              "Llama-3-8B-shaped: 32 x {q,o 4096x4096; k,v 1024x4096; gate,up 14336x4096; down 4096x14336}"),
    "gpt2": (12, [(768, 2304, 1), (768, 768, 1), (768, 3072, 1), (3072, 768, 1)],
             "GPT-2-small-shaped: 12 x {768x2304, 768x768, 768x3072, 3072x768}"),
    "moe": (16, [(64 * 1408, 2048, 0)], "MoE: 16 x {gate, up (64,1408,2048), down (64,2048,1408)}"),
    # the same tensors with flatten=True: each becomes one (64, 2883584) matrix
    "moe_flat": (16, [(64 * 1408, 2048, 0)],
                 "MoE, flatten=True: 16 x {gate, up (64,1408,2048), down (64,2048,1408)} as (64, 2883584)"),
    # one fp32 parameter, Newton-Schulz, per-parameter driver
    "plumbing": (1, [(256, 512, 1)], "plumbing: one fp32 256x512 parameter, Newton-Schulz, foreach=False"),
}


def _shapes(config: str):
    layers, per_layer, _ = CONFIGS[config]
    if config in ("moe", "moe_flat"):
        return [(64, 1408, 2048)] * (2 * layers) + [(64, 2048, 1408)] * layers
    out = []
    for _ in range(layers):
        for r, c, n in per_layer:
            out += [(r, c)] * n
    return out


def orth_flops(shape, steps: int) -> float:
    """Symmetric-minimal FLOPs of the iteration for one tensor: per matrix and step
    m(m+1) n [X X^T] + m(m+1) m [A A] + 2 m^2 n [B X]."""
    nb = 1
    for d in shape[:-2]:
        nb *= d
    m, n = min(shape[-2:]), max(shape[-2:])
    return nb * steps * (m * (m + 1) * n + m * (m + 1) * m + 2 * m * m * n)


def _config_hparams(config: str) -> tuple[str, "torch.dtype"]:
    """(strategy, param dtype) of a workload: Newton-Schulz for the plumbing check and the
    MoE set (BASELINE.json configs 1 and 4), Polar Express otherwise; fp32 params for the
    plumbing check, bf16 otherwise."""
    import torch

    strategy = "newton_schulz" if config in ("moe", "moe_flat", "plumbing") else "polar_express"
    return strategy, (torch.float32 if config == "plumbing" else torch.bfloat16)


def cpu_baseline(config: str = "llama", min_seconds: float = 10.0) -> dict:
    """The reference's per-parameter loop restated on the CPU (oracle.muon_ref: the
    foreach=False driver, MuonBaseline.update, the eager bf16 loop of the workload's
    strategy), with the workload's param dtype, cautious wd 0.1 and Nesterov 0.95.

    Small workloads (plumbing, GPT-2: at most 64 matrices) are stepped whole: one warm-up
    step, then steps until min_seconds (at least 3), median step time. Larger ones are
    sampled: one matrix of each distinct shape, whole passes over the shapes until
    min_seconds (10-30 s of CPU work on the bench host), and the full step extrapolated
    from each shape's median time times its count. Reported as orthogonalization TFLOP/s
    of the measured steps (their symmetric-minimal FLOPs over their summed time)."""
    import statistics

    import torch

    from oracle import muon_ref

    strategy, pdtype = _config_hparams(config)
    threads = len(os.sched_getaffinity(0))
    threads = min(threads, int(os.environ.get("OMP_NUM_THREADS", threads)))
    torch.set_num_threads(threads)
    gen = torch.Generator().manual_seed(0)
    shapes = _shapes(config)
    counts: dict[tuple, int] = {}
    for s in shapes:  # a stacked (experts, rows, cols) tensor counts as its matrices
        key = tuple(s[-2:])
        counts[key] = counts.get(key, 0) + math.prod(s[:-2])
    hp = dict(lr=1e-3, wd=0.1, use_cautious_wd=True, momentum=0.95, nesterov=True,
              strategy=strategy)

    def grad_like(shape):
        z = torch.randn(*shape[:-1], 1, generator=gen)
        return (torch.randn(shape, generator=gen) * torch.exp(z)).to(pdtype)

    try:
        cpu = open("/proc/cpuinfo").read().split("model name")[1].split("\n")[0].strip(" :\t")
    except Exception:
        cpu = "unknown"
    direct = sum(counts.values()) <= 64
    if direct:
        params = [torch.randn(s, generator=gen).to(pdtype) for s in shapes]
        grads = [grad_like(s) for s in shapes]
        ref = muon_ref.MuonRef(params, **hp)
        ref.step(grads)  # warm-up (state allocation, first-call costs)
        times = []
        while len(times) < 3 or (sum(times) < min_seconds and len(times) < 20000):
            t0 = time.perf_counter()
            ref.step(grads)
            times.append(time.perf_counter() - t0)
        med = statistics.median(times)
        flops = sum(orth_flops(s, 5) for s in shapes)
        return {
            "value": round(flops / med / 1e12, 6),
            "unit": "TFLOP/s",
            "cores": threads,
            "kind": "port",
            "sample": (f"oracle per-parameter Muon step (eager bf16 {strategy} 5, cautious wd, "
                       f"Nesterov, {str(pdtype).replace('torch.', '')} params) over the whole "
                       f"set of {len(shapes)} tensors: median of {len(times)} steps after one "
                       f"warm-up ({sum(times):.1f} s); CPU: {cpu}"),
            "ms_per_step": round(med * 1e3, 3),
        }
    warm = torch.randn(256, 512, generator=gen).to(pdtype)
    muon_ref.MuonRef([warm], **hp).step([warm.clone()])
    cases = []
    for shape in counts:
        p = torch.randn(shape, generator=gen).to(pdtype)
        cases.append((shape, muon_ref.MuonRef([p], **hp), grad_like(shape)))
    # Whole passes over the distinct shapes until at least min_seconds of CPU work.
    per_shape = {shape: [] for shape in counts}
    total_s, total_flops, passes = 0.0, 0.0, 0
    while passes < 1 or (total_s < min_seconds and passes < 10):
        for shape, ref, g in cases:
            t0 = time.perf_counter()
            ref.step([g])
            dt = time.perf_counter() - t0
            per_shape[shape].append(dt)
            total_s += dt
            total_flops += orth_flops(shape, 5)
        passes += 1
    full_s, parts = 0.0, []
    for shape, count in counts.items():
        med = statistics.median(per_shape[shape])
        full_s += med * count
        parts.append(f"{'x'.join(map(str, shape))}: {med * 1e3:.0f} ms")
    return {
        "value": round(total_flops / total_s / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle per-parameter Muon step (eager bf16 {strategy} 5, cautious wd, "
                   f"Nesterov, {str(pdtype).replace('torch.', '')} params) on one matrix of each "
                   f"distinct shape, {passes} passes ({'; '.join(parts)} median per step; "
                   f"{total_s:.1f} s); CPU: {cpu}"),
        "extrapolated_ms_per_step": round(full_s * 1e3, 1),
    }


def _median_ms(fn, reps: int = 50, warmup: int = 5, flush=None) -> float:
    """Median of `reps` timings of fn() with hipEvents on the current stream, the way the
    reference's harness times (triton.testing.do_bench, return_mode="median"): the
    caches are flushed by a 512 MB fill before every timed call (larger than the MI355X's
    256 MB last-level cache)."""
    import statistics

    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    samples = []
    for _ in range(reps):
        if flush is not None:
            flush.zero_()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        fn()
        e1.record()
        e1.synchronize()
        samples.append(e0.elapsed_time(e1))
    return statistics.median(samples)


def reference_suite(dev) -> dict:
    """The reference's own published single-device benchmarks (benchmark/RESULTS.md:18-37),
    on this GPU and this library, timed as the reference times them (median, caches
    flushed):

    * Gram of a (32, 2048, 1024) bf16 batch (bench_kernels.py:22-72): muonium_amd's
      `gram` next to hipBLASLt's dense x @ x^T (x^T made contiguous beforehand);
    * Newton-Schulz and Polar Express loops, 5 steps on (32, 2048, 1024) bf16
      (bench_kernels.py:75-132): `ns_loop` / `pe_loop`;
    * one optimizer.step() on the _QUICK set (bench_optim.py:28-33, 137-179): 16 fp32
      matrices, 4 each of 512x512, 512x1536, 512x2048, 2048x512, use_cautious_wd=False,
      lr 1e-3, wd 0.1, momentum 0.95, Nesterov, 5 steps; the grads are refilled inside the
      timed call as the reference's _step_fn does; per-parameter and foreach drivers,
      both strategies.

    The reference's numbers are from an NVIDIA RTX PRO 6000 Blackwell Max-Q (CUDA 13.0,
    PyTorch 2.12.1), not from an MI355X; they are reported beside ours, not divided."""
    import torch

    from muonium_amd import Muon
    from muonium_amd.kernels.gram import gram
    from muonium_amd.orthogonalize.newton_schulz import ns_loop
    from muonium_amd.orthogonalize.polar_express import pe_loop

    flush = torch.empty(512 << 20, dtype=torch.uint8, device=dev)
    out = {}
    gen = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(32, 2048, 1024, device=dev, generator=gen).bfloat16()
    xt = x.mT.contiguous()
    t_ours = _median_ms(lambda: gram(x), flush=flush)
    t_blas = _median_ms(lambda: torch.bmm(x, xt), flush=flush)
    sym = 32 * 2048 * 2049 * 1024  # upper triangle, symmetric-minimal
    out["gram_32x2048x1024_bf16"] = {
        "ms": round(t_ours, 4), "tflops_symmetric_minimal": round(sym / t_ours / 1e9, 1),
        "hipblaslt_dense_ms": round(t_blas, 4),
        "reference_ms": {"triton_gram": 0.6077, "torch_x_xT": 1.1234},
    }
    loop_flops = 32 * 5 * (1024 * 1025 * 2048 + 1024 * 1025 * 1024 + 2 * 1024 * 1024 * 2048)
    for name, fn, ref_ms in (("ns_loop", ns_loop, {"eager": 12.7727, "compiled": 10.1110,
                                                   "triton": 9.3620}),
                             ("pe_loop", pe_loop, {"eager": 12.7811, "compiled": 10.1018,
                                                   "triton": 9.3657})):
        t = _median_ms(lambda: fn(x, 5), flush=flush)
        out[f"{name}_5steps_32x2048x1024_bf16"] = {
            "ms": round(t, 4), "tflops_symmetric_minimal": round(loop_flops / t / 1e9, 1),
            "reference_ms": ref_ms,
        }
    del x, xt
    shapes = [(512, 512)] * 4 + [(512, 1536)] * 4 + [(512, 2048)] * 4 + [(2048, 512)] * 4
    ref_step = {("newton_schulz", False): 9.3614, ("polar_express", False): 9.5561,
                ("newton_schulz", True): 2.4483, ("polar_express", True): 2.6481}
    for (strategy, foreach), ref_ms in ref_step.items():
        g1 = torch.Generator(device=dev).manual_seed(1)
        g0 = torch.Generator(device=dev).manual_seed(0)
        params = [torch.nn.Parameter(torch.randn(*s, device=dev, generator=g1)) for s in shapes]
        grads = [torch.randn(*s, device=dev, generator=g0) for s in shapes]
        opt = Muon(params, foreach=foreach, lr=1e-3, wd=0.1, momentum=0.95, nesterov=True,
                   ns_steps=5, use_cautious_wd=False, orthogonalization_strategy=strategy)

        def step():
            for p, g in zip(params, grads):
                p.grad = g.clone()
            opt.step()

        t = _median_ms(step, flush=flush)
        key = f"quick_step_{'foreach' if foreach else 'per_param'}_{strategy}"
        out[key] = {"ms": round(t, 4), "reference_ms": ref_ms}
        del opt, params, grads
    torch.cuda.empty_cache()
    return {"reference_suite": "benchmark/RESULTS.md:18-37 workloads on MI355X",
            "reference_hardware": "NVIDIA RTX PRO 6000 Blackwell Max-Q, CUDA 13.0, PyTorch 2.12.1",
            "results": out}


def blas_ceiling(config: str, dev, reps: int = 3) -> dict:
    """Library reference for the orthogonalization: per bucket of the workload, the three
    products of one iteration with torch.bmm (hipBLASLt, dense: X X^T and A A computed in
    full) on random bf16 operands. Reports each product's dense TFLOP/s and the time the
    library would take for the workload's 5 iterations, next to the symmetric-minimal
    FLOPs the step is credited with."""
    import torch

    counts: dict[tuple, int] = {}
    for s in _shapes(config):
        key = (min(s[-2:]), max(s[-2:]))
        counts[key] = counts.get(key, 0) + math.prod(s[:-2])
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        ev0.record()
        for _ in range(reps):
            fn()
        ev1.record()
        torch.cuda.synchronize()
        return ev0.elapsed_time(ev1) / reps

    out, total_ms, total_flops = {}, 0.0, 0.0
    gen = torch.Generator(device=dev).manual_seed(0)
    for (m, n), count in counts.items():
        X = torch.randn(count, m, n, device=dev, generator=gen).bfloat16()
        XT = X.transpose(1, 2).contiguous()  # transposed operands made contiguous
        A = torch.randn(count, m, m, device=dev, generator=gen).bfloat16()
        t_xx = timed(lambda: torch.bmm(X, XT))
        t_aa = timed(lambda: torch.bmm(A, A))
        t_bx = timed(lambda: torch.bmm(A, X))
        d = 2.0 * count
        out[f"{m}x{n}x{count}"] = {
            "xxT_ms": round(t_xx, 3), "xxT_tflops": round(d * m * m * n / t_xx / 1e9, 1),
            "aa_ms": round(t_aa, 3), "aa_tflops": round(d * m * m * m / t_aa / 1e9, 1),
            "bx_ms": round(t_bx, 3), "bx_tflops": round(d * m * m * n / t_bx / 1e9, 1),
        }
        total_ms += 5 * (t_xx + t_aa + t_bx)
        total_flops += 5 * count * (m * (m + 1) * n + m * (m + 1) * m + 2 * m * m * n)
        del X, XT, A
        torch.cuda.empty_cache()
    return {"blas_ceiling": "torch.bmm (hipBLASLt), bf16, dense products", "config": config,
            "buckets": out, "orth_ms_per_step": round(total_ms, 3),
            "orth_tflops_symmetric_minimal": round(total_flops / (total_ms * 1e-3) / 1e12, 1)}


def hbm_ceiling(dev, reps: int = 5) -> dict:
    """Library reference for the update passes: torch's own streaming kernels on 2 GiB bf16
    buffers (far above the 256 MB Infinity Cache) at several read:write mixes, the median of
    `reps` timed calls each, as bytes moved per second."""
    import torch

    n = 1 << 30
    gen = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(n, device=dev, dtype=torch.bfloat16, generator=gen)
    y = torch.randn(n, device=dev, dtype=torch.bfloat16, generator=gen)
    z = torch.empty_like(x)
    cases = {
        "read (x.sum())": (lambda: x.sum(), 2 * n),
        "write (z.fill_)": (lambda: z.fill_(1.0), 2 * n),
        "copy 1R:1W (z.copy_(x))": (lambda: z.copy_(x), 4 * n),
        "add 2R:1W (torch.add(x, y, out=z))": (lambda: torch.add(x, y, out=z), 6 * n),
    }
    out = {}
    for name, (fn, nbytes) in cases.items():
        fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(reps):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1))
        ms = sorted(ts)[len(ts) // 2]
        out[name] = {"ms": round(ms, 4), "bytes": nbytes,
                     "tbs": round(nbytes / (ms * 1e-3) / 1e12, 3)}
    return {"hbm_ceiling": "torch streaming kernels, bf16, 2 GiB buffers", "results": out}


def _measured_traffic(kernels, config: str, lp):
    """HBM bytes per dispatch of `kernels` (one name, or several that serve one product:
    their dispatch-weighted mean over those the profile saw) from the committed rocprofv3
    PMC summary (FETCH_SIZE + WRITE_SIZE, each scaled by a 1 GiB copy), for the workload
    it was measured on; None elsewhere."""
    files = {"llama": "muon_step_llama3_8b_traffic.json", "moe_flat": "muon_step_moe_flat_traffic.json"}
    if config not in files or lp:
        return None, None
    if isinstance(kernels, str):
        kernels = [kernels]
    path = os.path.join(ROOT, "profiles", files[config])
    try:
        with open(path) as f:
            data = json.load(f)
        seen = [data["kernels"][k] for k in kernels if k in data["kernels"]]
        n = sum(int(k["dispatches"]) for k in seen)
        if n == 0:
            return None, None
        traffic = sum(k["traffic_bytes"] * int(k["dispatches"]) for k in seen) / n
        return int(round(traffic)), os.path.relpath(path, ROOT)
    except (OSError, KeyError, ValueError, TypeError):
        return None, None


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", default="llama", choices=sorted(CONFIGS))
    ap.add_argument("--lp", default=None, choices=["8bit", "4bit", "fp8"])
    ap.add_argument("--block-size", default=None,
                    help="MuonLP block size (default 256, 4-bit 128), or 'tensor' for one "
                         "scale per tensor")
    ap.add_argument("--strategy", default=None)
    ap.add_argument("--algorithm", default="muon", choices=["muon", "normuon"],
                    help="the param group's algorithm (normuon: per-row variance state and "
                         "its post-pass)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a 1 GiB device-to-device copy 5 times (PMC calibration)")
    ap.add_argument("--hbm-ceiling", action="store_true",
                    help="only time torch's streaming kernels (read, write, copy, add) on 2 GiB "
                         "buffers as a reference for the update passes")
    ap.add_argument("--blas-ceiling", action="store_true",
                    help="only time the iteration's three products per bucket with torch.bmm "
                         "(hipBLASLt) as a library reference")
    ap.add_argument("--products", default=None, choices=["q", "kv", "gate", "down"],
                    help="only run the iteration's products on --count random bf16 matrices of "
                         "one Llama bucket's shape (one Newton-Schulz step, twice; for "
                         "profiling the product kernels)")
    ap.add_argument("--count", type=int, default=32)
    ap.add_argument("--reference-suite", action="store_true",
                    help="only run the reference's own published single-device benchmarks "
                         "(Gram, NS/PE loops, the 16-matrix step) and print their times")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build targets one GPU (no collectives); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    import torch

    from muonium_amd import Muon, _lib
    from muonium_amd.optim import Muon4bit, Muon8bit, MuonFp8

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.calibrate_copy:
        # A plain copy of known size: FETCH_SIZE / WRITE_SIZE of these dispatches give
        # the counters' scale against exactly 1 GiB read and 1 GiB written.
        src = torch.empty(1 << 29, dtype=torch.bfloat16, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": src.numel() * 2, "dispatches": 5}))
        return
    if args.hbm_ceiling:
        print(json.dumps(hbm_ceiling(dev)), flush=True)
        return
    if args.blas_ceiling:
        print(json.dumps(blas_ceiling(args.config, dev)), flush=True)
        return
    if args.reference_suite:
        print(json.dumps(reference_suite(dev)), flush=True)
        return
    if args.products:
        from muonium_amd import _ops

        shape = {"q": (4096, 4096), "kv": (1024, 4096), "gate": (14336, 4096),
                 "down": (4096, 14336)}[args.products]
        gen = torch.Generator(device=dev).manual_seed(0)
        xs = [torch.randn(shape, device=dev, generator=gen).bfloat16() for _ in range(args.count)]
        for _ in range(2):
            _ops.orthogonalize(xs, [(3.4445, -4.7750, 2.0315)], prescale=1.0, eps=1e-7,
                               iter_dtype=torch.bfloat16, out_dtype=torch.bfloat16)
        torch.cuda.synchronize()
        print(json.dumps({"products": args.products, "shape": shape, "count": args.count}))
        return
    shapes = _shapes(args.config)
    strategy, pdtype = _config_hparams(args.config)
    strategy = args.strategy or strategy
    flatten = args.config == "moe_flat"
    print(f"[bench] config={args.config} tensors={len(shapes)} strategy={strategy} "
          f"lp={args.lp}", file=sys.stderr, flush=True)

    gen = torch.Generator(device=dev).manual_seed(0)
    params = []
    for s in shapes:
        p = torch.empty(s, dtype=pdtype, device=dev)
        p.normal_(0.0, 0.02, generator=gen)
        q = torch.nn.Parameter(p)
        rows = s[-2]
        z = torch.randn(*s[:-2], rows, 1, device=dev, generator=gen)
        g = torch.randn(s, device=dev, generator=gen) * torch.exp(z)
        q.grad = g.to(pdtype)
        del g, z
        params.append(q)
    numel = sum(p.numel() for p in params)
    kw = dict(lr=1e-3, wd=0.1, use_cautious_wd=True, momentum=0.95, nesterov=True, ns_steps=5,
              orthogonalization_strategy=strategy)
    groups = [{"params": params, "flatten": flatten}]  # flatten is a group key
    if args.algorithm != "muon":
        groups[0]["algorithm"] = args.algorithm
    if args.lp:
        cls = {"8bit": Muon8bit, "4bit": Muon4bit, "fp8": MuonFp8}[args.lp]
        if args.block_size == "tensor":
            block = None  # one scale per tensor
        else:
            block = int(args.block_size or {"8bit": 256, "4bit": 128, "fp8": 256}[args.lp])
        opt = cls(groups, foreach=True, block_size=block, **kw)
    else:
        opt = Muon(groups, foreach=args.config != "plumbing", **kw)
    # Every step starts from the same synthetic gradients, as in training, where backward
    # writes fresh gradients before each step. The foreach update adds the momentum into
    # the gradients in place (Nesterov, muon.py:107-108), so stepping on without a refill
    # grows them about 2.5x per step until, after about 37 steps, the fp32 sum of squares
    # of a 4096 x 4096 matrix overflows and the iteration runs on zeros (measured 10%
    # faster). The refill is a device copy between steps, outside the timed intervals.
    grads = [p.grad for p in params]
    grads0 = [g.clone() for g in grads]

    def refill():
        torch._foreach_copy_(grads, grads0)

    torch.cuda.synchronize()
    print(f"[bench] params={numel / 1e9:.3f}e9, warmup {args.warmup}", file=sys.stderr, flush=True)

    for i in range(args.warmup):
        refill()
        opt.step()
        torch.cuda.synchronize()
        print(f"[bench] warmup step {i} done", file=sys.stderr, flush=True)

    def timed_steps(bracketed: bool):
        """K steps between a synchronize on each side, each step between its own pair of
        events (no synchronization inside; the gradient refill before a step lies outside
        its pair): (mean ms per step, median ms per step, wall s). With `bracketed` every
        library launch also records its own hipEvent pair."""
        _lib.timing_enable(bracketed)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in range(args.steps)]
        for e0, e1 in evs:
            refill()
            e0.record()
            opt.step()
            e1.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        step_ms = sorted(e0.elapsed_time(e1) for e0, e1 in evs)
        mean = sum(step_ms) / args.steps
        med = step_ms[len(step_ms) // 2] if len(step_ms) % 2 else \
            0.5 * (step_ms[len(step_ms) // 2 - 1] + step_ms[len(step_ms) // 2])
        return mean, med, wall

    # the timed region: the step as a caller runs it, no per-launch events
    ms_per_step, median_ms, wall = timed_steps(False)
    print(f"[bench] {args.steps} steps: {ms_per_step:.2f} ms/step (wall {wall:.2f}s)",
          file=sys.stderr, flush=True)
    # the breakdown region: the same K steps with every launch bracketed
    brk_ms, _, _ = timed_steps(True)
    kern = _lib.timing_read()
    _lib.timing_enable(False)
    print(f"[bench] {args.steps} bracketed steps: {brk_ms:.2f} ms/step", file=sys.stderr, flush=True)

    # the matrices the iteration sees: flatten=True collapses (e, r, c) to (e, r * c)
    orth_shapes = [(s[0], math.prod(s[1:])) if flatten and len(s) > 2 else s for s in shapes]
    flops_step = sum(orth_flops(s, 5) for s in orth_shapes)
    value = flops_step / (ms_per_step * 1e-3) / 1e12
    # the last B X of each plain-Muon bucket carries the apply (the post-pass fused into its
    # epilogue, gemm_bx_apply): its whole time is counted as orthogonalization time
    orth_ms = sum(kern[k][0] for k in ("syrk_xx", "syrk_aa", "gemm_bx", "gemm_bx_apply")) / args.steps
    apply_fused = kern["gemm_bx_apply"][1] > 0
    kernels = {}
    for k, (ms, n, work) in kern.items():
        if n == 0:
            continue
        entry = {"ms_per_step": round(ms / args.steps, 3), "launches_per_step": n // args.steps,
                 "avg_launch_ms": round(ms / n, 4)}
        if k in ("syrk_xx", "syrk_aa", "gemm_bx", "gemm_bx_apply"):
            tf = work / (ms * 1e-3) / 1e12
            entry.update(tflops=round(tf, 1), frac=round(tf / PEAK_BF16_TFLOPS, 4))
            if k == "gemm_bx_apply":
                # the same product plus the apply: each parameter element read and written
                entry.update(apply_param_bytes_per_elem=2 * pdtype.itemsize)
        elif k in ("prepass", "postpass", "lp_prepass"):
            gbs = work / (ms * 1e-3) / 1e9
            entry.update(gbs=round(gbs, 1), frac=round(gbs / PEAK_HBM_GBS, 4),
                         bytes_per_elem=round(work / (numel * args.steps), 3))
            if k == "prepass" and work > 12.5 * numel * args.steps:
                # the pre-pass also writes the Nesterov g' back into the gradients (2 B per
                # bf16 value, the foreach driver's in-place update); without that write it
                # moves 12 B per value (g 2 + m 4 in, m 4 + X 2 out)
                gbs12 = 12.0 * numel * args.steps / (ms * 1e-3) / 1e9
                entry.update(gbs_12B=round(gbs12, 1), frac_12B=round(gbs12 / PEAK_HBM_GBS, 4))
        kernels[k] = entry

    gms, gn, gwork = kern["gemm_bx"]
    avg_ms = gms / max(gn, 1)
    if all(min(s[-2:]) <= 64 for s in orth_shapes) and pdtype == torch.bfloat16:
        # iterates of at most 64 rows run in short.hip: the B X launch streams X in and X'
        # out (bf16, 4 m n bytes per matrix), HBM-bound; it also forms the next Gram
        # partials from registers. With the apply fused, the last of the 5 iterations is the
        # gemm_bx_apply launch (X and the parameters in, the parameters out)
        plain_iters = 5 - (1 if apply_fused else 0)
        bx_bytes = sum(plain_iters * 4 * (math.prod(s[:-2]) if len(s) > 2 else 1) * min(s[-2:])
                       * max(s[-2:]) for s in orth_shapes) * args.steps / max(gn, 1)
        achieved = bx_bytes / (avg_ms * 1e-3) / 1e9
        traffic, traffic_src = _measured_traffic("short_bx_kernel<-1>", args.config, args.lp)
        if apply_fused:
            ams, an, _ = kern["gemm_bx_apply"]
            abytes = (2 + 2 * pdtype.itemsize) * numel * args.steps
            kernels["gemm_bx_apply"].update(
                bytes_per_elem=2 + 2 * pdtype.itemsize,
                gbs=round(abytes / (ams * 1e-3) / 1e9, 1),
                gbs_frac=round(abytes / (ams * 1e-3) / 1e9 / PEAK_HBM_GBS, 4))
        roofline = {
            "bound": "hbm",
            "kernel": "short_bx_kernel<-1> (X' = a X + B X, 64-row iterate)",
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_src,
            "avg_launch_ms": round(avg_ms, 4),
            "bytes_per_launch": bx_bytes,
        }
    else:
        achieved = (gwork / max(gn, 1)) / (avg_ms * 1e-3) / 1e12
        # the optimizer iterates in bf16 whatever the params' dtype (zeropower casts to
        # bf16, orthogonalize.py:101-102), so fp32 params (plumbing) run this kernel too
        # two kernels serve this product: gemm_bf16_nn16_kernel for K >= 768 (its plain
        # instantiation <0, 0>; the <1|2, 1> ones carry the fused apply, timed apart as
        # gemm_bx_apply) and gemm_bf16_nn4_kernel below; the launch brackets time whichever ran
        knames = ["gemm_bf16_nn16_kernel<0, 0>", "gemm_bf16_nn4_kernel"]
        peak = PEAK_BF16_TFLOPS
        traffic, traffic_src = _measured_traffic(knames, args.config, args.lp)
        roofline = {
            "bound": "mfma",
            "kernel": "gemm_bf16_nn16_kernel<0, 0> (K >= 768) / gemm_bf16_nn4_kernel "
                      "(X' = a X + B X)",
            "achieved": round(achieved, 1),
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": round(achieved / peak, 4),
            "traffic": traffic,
            "traffic_source": traffic_src,
            "avg_launch_ms": round(avg_ms, 4),
            "flop_per_launch": gwork / max(gn, 1),
        }
    upd_ms = sum(kern[k][0] for k in ("prepass", "postpass", "lp_prepass")) / args.steps
    upd_bytes = sum(kern[k][2] for k in ("prepass", "postpass", "lp_prepass")) / args.steps
    # the passes' bytes without the pre-pass's write-back of g' into the gradients: 18 B
    # per bf16 value with fp32 momentum (pre 12 + post 6)
    upd_bytes18 = (18.0 * numel if (not args.lp and pdtype == torch.bfloat16 and not apply_fused)
                   else None)
    # with the apply fused, the update kernels are the pre-pass alone: 12 B per value
    # without the write-back of g' into the gradients
    upd_bytes12 = 12.0 * numel if (apply_fused and not args.lp and pdtype == torch.bfloat16) else None

    cpu = None
    # the oracle's per-parameter loop restates the per-matrix problem; it is not run for
    # the flatten=True workload (a different matrix per tensor)
    if not args.no_cpu_baseline and args.config != "moe_flat":
        print("[bench] cpu baseline ...", file=sys.stderr, flush=True)
        cpu = cpu_baseline(args.config)

    _, _, label = CONFIGS[args.config]
    line = {
        "metric": "Muon step ms + orthogonalization TFLOP/s, Llama-3-8B-shaped params, 1 GPU",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "median_ms_per_step": round(median_ms, 3),
        "breakdown_ms_per_step": round(brk_ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32" if pdtype == torch.float32 else "bf16",
        "data": "synthetic (seeded N(0,1) gradients with per-row log-normal scales; random-init bf16 params)",
        "config": {
            "workload": label + (f"; MuonLP {args.lp}, block {block or 'per tensor'}"
                                 if args.lp else "") + ("; NorMuon" if args.algorithm == "normuon" else ""),
            "algorithm": args.algorithm,
            "params": numel,
            "strategy": strategy,
            "ns_steps": 5,
            "foreach": args.config != "plumbing",
            "momentum_dtype": (args.lp or "fp32"),
            "orth_tflop_per_step": round(flops_step / 1e12, 3),
        },
        "orth_kernel_ms_per_step": round(orth_ms, 3),
        "orth_kernel_tflops": round(flops_step / (orth_ms * 1e-3) / 1e12, 1) if orth_ms else None,
        "update_kernel_ms_per_step": round(upd_ms, 3),
        "update_kernel_gbs": round(upd_bytes / (upd_ms * 1e-3) / 1e9, 1) if upd_ms else None,
        "update_kernel_bytes_per_elem": round(upd_bytes / numel, 3),
        "update_kernel_gbs_18B": (round(upd_bytes18 / (upd_ms * 1e-3) / 1e9, 1)
                                  if upd_ms and upd_bytes18 else None),
        "update_kernel_gbs_12B": (round(upd_bytes12 / (upd_ms * 1e-3) / 1e9, 1)
                                  if upd_ms and upd_bytes12 else None),
        "update_apply_fused_into": "gemm_bx_apply" if apply_fused else None,
        "kernels": kernels,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
