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

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config llama|gpt2|moe]
       [--lp 8bit|4bit|fp8] [--no-cpu-baseline]
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


def cpu_baseline(config: str = "llama", min_seconds: float = 10.0) -> dict:
    """The reference's per-parameter loop restated on the CPU (oracle.muon_ref), on a
    bounded sample: steps of ONE matrix of each distinct shape of the workload (bf16
    Polar Express 5, cautious wd, Nesterov), whole passes over the shapes until at
    least min_seconds (10-30 s of CPU work on the bench host). Reported
    as the sample's orthogonalization TFLOP/s, plus the full-step time extrapolated
    by weighting each shape's time with its count in the workload."""
    import torch

    from oracle import muon_ref

    threads = len(os.sched_getaffinity(0))
    threads = min(threads, int(os.environ.get("OMP_NUM_THREADS", threads)))
    torch.set_num_threads(threads)
    gen = torch.Generator().manual_seed(0)
    shapes = _shapes(config)
    counts: dict[tuple, int] = {}
    for s in shapes:  # a stacked (experts, rows, cols) tensor counts as its matrices
        key = tuple(s[-2:])
        counts[key] = counts.get(key, 0) + math.prod(s[:-2])
    warm = torch.randn(256, 512, generator=gen).bfloat16()
    muon_ref.MuonRef([warm], lr=1e-3, wd=0.1, strategy="polar_express").step([warm.clone()])
    cases = []
    for shape in counts:
        p = torch.randn(shape, generator=gen).bfloat16()
        z = torch.randn(*shape[:-1], 1, generator=gen)
        g = (torch.randn(shape, generator=gen) * torch.exp(z)).bfloat16()
        cases.append((shape, muon_ref.MuonRef([p], lr=1e-3, wd=0.1, strategy="polar_express"), g))
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
        mean = sum(per_shape[shape]) / len(per_shape[shape])
        full_s += mean * count
        parts.append(f"{'x'.join(map(str, shape))}: {mean * 1e3:.0f} ms")
    try:
        cpu = open("/proc/cpuinfo").read().split("model name")[1].split("\n")[0].strip(" :\t")
    except Exception:
        cpu = "unknown"
    return {
        "value": round(total_flops / total_s / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle per-parameter Muon step (bf16 Polar Express 5, cautious wd, "
                   f"Nesterov) on one bf16 matrix of each distinct shape, {passes} passes "
                   f"({'; '.join(parts)} mean per step; {total_s:.1f} s); CPU: {cpu}"),
        "extrapolated_ms_per_step": round(full_s * 1e3, 1),
    }


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


def _measured_traffic(kernel: str, config: str, lp):
    """HBM bytes per dispatch of `kernel` from the committed rocprofv3 PMC summary
    (FETCH_SIZE + WRITE_SIZE, each scaled by a 1 GiB copy), for the workload it was
    measured on; None elsewhere."""
    files = {"llama": "muon_step_llama3_8b_traffic.json", "moe_flat": "muon_step_moe_flat_traffic.json"}
    if config not in files or lp:
        return None, None
    path = os.path.join(ROOT, "profiles", files[config])
    try:
        with open(path) as f:
            data = json.load(f)
        return data["kernels"][kernel]["traffic_bytes"], os.path.relpath(path, ROOT)
    except (OSError, KeyError, ValueError):
        return None, None


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", default="llama", choices=sorted(CONFIGS))
    ap.add_argument("--lp", default=None, choices=["8bit", "4bit", "fp8"])
    ap.add_argument("--block-size", type=int, default=None)
    ap.add_argument("--strategy", default=None)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a 1 GiB device-to-device copy 5 times (PMC calibration)")
    ap.add_argument("--blas-ceiling", action="store_true",
                    help="only time the iteration's three products per bucket with torch.bmm "
                         "(hipBLASLt) as a library reference")
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
    if args.blas_ceiling:
        print(json.dumps(blas_ceiling(args.config, dev)), flush=True)
        return
    shapes = _shapes(args.config)
    strategy = args.strategy or ("newton_schulz" if args.config in ("moe", "moe_flat", "plumbing")
                                 else "polar_express")
    flatten = args.config == "moe_flat"
    pdtype = torch.float32 if args.config == "plumbing" else torch.bfloat16
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
    if args.lp:
        cls = {"8bit": Muon8bit, "4bit": Muon4bit, "fp8": MuonFp8}[args.lp]
        block = args.block_size or {"8bit": 256, "4bit": 128, "fp8": 256}[args.lp]
        opt = cls(groups, foreach=True, block_size=block, **kw)
    else:
        opt = Muon(groups, foreach=args.config != "plumbing", **kw)
    torch.cuda.synchronize()
    print(f"[bench] params={numel / 1e9:.3f}e9, warmup {args.warmup}", file=sys.stderr, flush=True)

    for i in range(args.warmup):
        opt.step()
        torch.cuda.synchronize()
        print(f"[bench] warmup step {i} done", file=sys.stderr, flush=True)

    _lib.timing_enable(True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record()
    for i in range(args.steps):
        opt.step()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kern = _lib.timing_read()
    _lib.timing_enable(False)
    ms_per_step = ev0.elapsed_time(ev1) / args.steps
    print(f"[bench] {args.steps} steps: {ms_per_step:.2f} ms/step (wall {wall:.2f}s)",
          file=sys.stderr, flush=True)

    # the matrices the iteration sees: flatten=True collapses (e, r, c) to (e, r * c)
    orth_shapes = [(s[0], math.prod(s[1:])) if flatten and len(s) > 2 else s for s in shapes]
    flops_step = sum(orth_flops(s, 5) for s in orth_shapes)
    value = flops_step / (ms_per_step * 1e-3) / 1e12
    orth_ms = sum(kern[k][0] for k in ("syrk_xx", "syrk_aa", "gemm_bx")) / args.steps
    kernels = {}
    for k, (ms, n, work) in kern.items():
        if n == 0:
            continue
        entry = {"ms_per_step": round(ms / args.steps, 3), "launches_per_step": n // args.steps,
                 "avg_launch_ms": round(ms / n, 4)}
        if k in ("syrk_xx", "syrk_aa", "gemm_bx"):
            tf = work / (ms * 1e-3) / 1e12
            entry.update(tflops=round(tf, 1), frac=round(tf / PEAK_BF16_TFLOPS, 4))
        elif k in ("prepass", "postpass", "lp_prepass"):
            gbs = work / (ms * 1e-3) / 1e9
            entry.update(gbs=round(gbs, 1), frac=round(gbs / PEAK_HBM_GBS, 4))
        kernels[k] = entry

    gms, gn, gwork = kern["gemm_bx"]
    avg_ms = gms / max(gn, 1)
    if all(min(s[-2:]) <= 64 for s in orth_shapes) and pdtype == torch.bfloat16:
        # iterates of at most 64 rows run in short.hip: the B X launch streams X in and X'
        # out (bf16, 4 m n bytes per matrix), HBM-bound; it also forms the next Gram
        # partials from registers
        bx_bytes = sum(5 * 4 * (math.prod(s[:-2]) if len(s) > 2 else 1) * min(s[-2:]) * max(s[-2:])
                       for s in orth_shapes) * args.steps / max(gn, 1)
        achieved = bx_bytes / (avg_ms * 1e-3) / 1e9
        traffic, traffic_src = _measured_traffic("short_bx_kernel", args.config, args.lp)
        roofline = {
            "bound": "hbm",
            "kernel": "short_bx_kernel (X' = a X + B X, 64-row iterate)",
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
        traffic, traffic_src = _measured_traffic("gemm_bf16_nn4_kernel", args.config, args.lp)
        roofline = {
            "bound": "mfma",
            "kernel": "gemm_bf16_nn4_kernel (X' = a X + B X)",
            "achieved": round(achieved, 1),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": traffic,
            "traffic_source": traffic_src,
            "avg_launch_ms": round(avg_ms, 4),
            "flop_per_launch": gwork / max(gn, 1),
        }
    upd_ms = sum(kern[k][0] for k in ("prepass", "postpass", "lp_prepass")) / args.steps
    upd_bytes = sum(kern[k][2] for k in ("prepass", "postpass", "lp_prepass")) / args.steps

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
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) gradients with per-row log-normal scales; random-init bf16 params)",
        "config": {
            "workload": label + (f"; MuonLP {args.lp}" if args.lp else ""),
            "params": numel,
            "strategy": strategy,
            "ns_steps": 5,
            "foreach": True,
            "momentum_dtype": (args.lp or "fp32"),
            "orth_tflop_per_step": round(flops_step / 1e12, 3),
        },
        "orth_kernel_ms_per_step": round(orth_ms, 3),
        "orth_kernel_tflops": round(flops_step / (orth_ms * 1e-3) / 1e12, 1) if orth_ms else None,
        "update_kernel_ms_per_step": round(upd_ms, 3),
        "update_kernel_gbs": round(upd_bytes / (upd_ms * 1e-3) / 1e9, 1) if upd_ms else None,
        "kernels": kernels,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
