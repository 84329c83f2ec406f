#!/usr/bin/env python3
"""Benchmark of the gfx950 attention path at the Chronos-2 time-attention shape.

A step is one batched attention call over the whole synthetic batch (B=64 series x 12 heads,
L=577 tokens, D=64, f32, RoPE, left-padding key mask, scale 1/8) with every input already resident
in HBM. Prints one JSON line with whole-job TFLOP/s, the roofline of the kernel (achieved
algorithmic TFLOP/s over the kernel's event-timed average duration vs the f32 matrix peak), the
series-forecasts/sec of one call, and the CPU baseline: the C restatement of the reference's CPU
attention (oracle/, `kind: port`) timed on this host's cores over the same inputs.

    python bench.py [--steps K] [--warmup W] [--workload chronos2|bolt]
    python bench.py --copy-mib N    # plain N MiB device copy: calibrates the HBM byte counters
"""
import argparse
import json
import os
import pathlib
import sys
import time

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "tsfm-zig_amd"))
sys.path.insert(0, str(ROOT / "tests"))

METRIC = "attention TFLOP/s + % MFMA peak; series-forecasts/sec at Chronos-2 shape"


def cpu_threads() -> int:
    # The GPU box grants 16 CPUs per GPU whatever nproc reports.
    return max(1, min(16, os.cpu_count() or 1))


def oracle_path() -> pathlib.Path:
    flags = pathlib.Path("/proc/cpuinfo").read_text() if pathlib.Path("/proc/cpuinfo").exists() else ""
    lib16 = ROOT / "oracle" / "liboracle_l16.so"
    return lib16 if (" avx512f" in flags and lib16.exists()) else ROOT / "oracle" / "liboracle_l8.so"


def traffic_for(workload: str):
    p = ROOT / "profiles" / "traffic.json"
    if p.exists():
        return json.loads(p.read_text()).get(workload)
    return None


def run_chronos2(args, torch, ta, workloads):
    w = workloads.chronos2()
    a = w.arrays
    dev = {n: torch.from_numpy(np.ascontiguousarray(a[n])).cuda() for n in ("q", "k", "v", "key_valid", "rope_cos", "rope_sin")}
    o = torch.empty_like(dev["q"])
    stream = torch.cuda.current_stream()
    all_valid = bool(a["key_valid"].all())

    def step():
        rc = ta.chronos2_time_attention(dev["q"], dev["k"], dev["v"], o, dev["rope_cos"], dev["rope_sin"],
                                        dev["key_valid"], all_valid, w.B, w.n_q, w.H * 64, w.H, 64, scale=w.scale,
                                        stream=stream)
        if rc != ta.OK:
            raise RuntimeError(f"tsfm_attn_fwd returned {rc}: {ta.last_error()}")

    config = {"workload": w.name, "B": w.B, "H": w.H, "L": w.n_q, "D": 64, "mask": "keys_additive", "rope": True,
              "scale": w.scale, "layout": "(B, L, H*D) f32"}

    def cpu_leg(n_series):
        import _oracle

        orc = _oracle.Oracle(oracle_path())
        B = n_series
        q = np.ascontiguousarray(a["q"][:B]).ravel().copy()
        k = np.ascontiguousarray(a["k"][:B]).ravel().copy()
        v = np.ascontiguousarray(a["v"][:B]).ravel()
        kv = np.ascontiguousarray(a["key_valid"][:B]).ravel()
        d = w.H * 64
        out = np.zeros(B * w.n_q * d, np.float32)
        t0 = time.perf_counter()
        # The reference path this call replaces: serial RoPE loop, then forRange(b*nh, TimeJob.attend).
        orc.chronos2_rope(q, k, a["rope_cos"], a["rope_sin"], B * w.n_q, w.n_q, d, w.H, 64)
        orc.chronos2_time_attention(cpu_threads(), q, k, v, out, kv, bool(kv.all()), B, w.n_q, d, w.H, 64, w.scale)
        dt = time.perf_counter() - t0
        return dt, out.reshape(B, w.n_q, d), orc.lanes

    return w, step, o, config, cpu_leg


def run_bolt(args, torch, ta, workloads):
    w = workloads.bolt()
    a = w.arrays
    L = w.n_q
    buckets = np.zeros(2 * L - 1, np.int32)
    ta.load().tsfm_t5_bucket_table(buckets.ctypes.data, L, L, 32, 128)
    dev = {n: torch.from_numpy(np.ascontiguousarray(x)).cuda() for n, x in
           dict(q=a["q"], k=a["k"], v=a["v"], key_valid=a["key_valid"], rel_table=a["rel_table"], buckets=buckets).items()}
    o = torch.empty_like(dev["q"])
    stream = torch.cuda.current_stream()
    all_valid = bool(a["key_valid"].all())

    def step():
        rc = ta.bolt_self_attention(dev["q"], dev["k"], dev["v"], o, dev["rel_table"], dev["buckets"], dev["key_valid"],
                                    all_valid, w.B, L, w.H * 64, w.H, 64, 32, stream=stream)
        if rc != ta.OK:
            raise RuntimeError(f"tsfm_attn_fwd returned {rc}: {ta.last_error()}")

    config = {"workload": w.name, "B": w.B, "H": w.H, "L": L, "D": 64, "mask": "keys_additive", "bias": "t5 32/128",
              "scale": 1.0, "layout": "(B, L, H*D) f32"}

    def cpu_leg(n_series):
        import _oracle

        orc = _oracle.Oracle(oracle_path())
        B = n_series
        q = np.ascontiguousarray(a["q"][:B]).ravel()
        k = np.ascontiguousarray(a["k"][:B]).ravel()
        v = np.ascontiguousarray(a["v"][:B]).ravel()
        kv = np.ascontiguousarray(a["key_valid"][:B]).ravel()
        d = w.H * 64
        out = np.zeros(B * L * d, np.float32)
        t0 = time.perf_counter()
        bias = orc.position_bias(a["rel_table"], L, w.H, 32, 128)
        orc.bolt_self_attention(cpu_threads(), q, k, v, out, bias, kv, bool(kv.all()), B, L, d, w.H, 64)
        dt = time.perf_counter() - t0
        return dt, out.reshape(B, L, d), orc.lanes

    return w, step, o, config, cpu_leg


WORKLOADS = {"chronos2": run_chronos2, "bolt": run_bolt}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="chronos2", choices=sorted(WORKLOADS))
    ap.add_argument("--cpu-series", type=int, default=None, help="series in the CPU-baseline sample")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline (profiling runs)")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="only run a plain device copy of this many MiB, 3 times (counter calibration)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build measures one GPU (the attention path shards by series with no exchange); "
              f"--gpus {args.gpus} / WORLD_SIZE {world} is not run", file=sys.stderr)
        return 2

    import torch
    import tsfm_attn as ta
    from tsfm_attn import workloads

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    if args.copy_mib:
        n = args.copy_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_each_way": n * 4, "launches": 3}), flush=True)
        return 0
    if not ta.available():
        print(f"bench.py: libtsfm_attn unavailable: {ta.last_error()}", file=sys.stderr)
        return 1

    w, step, o, config, cpu_leg = WORKLOADS[args.workload](args, torch, ta, workloads)
    stream = torch.cuda.current_stream()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # One event pair per launch, recorded on the stream the kernel runs on (the same per-dispatch
    # duration rocprofv3 --kernel-trace reports); wall time around the whole loop gives `value`.
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    t0 = time.perf_counter()
    for i in range(args.steps):
        starts[i].record(stream)
        step()
        ends[i].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kernel_ms = sum(a.elapsed_time(b) for a, b in zip(starts, ends)) / args.steps
    ms_per_step = wall * 1e3 / args.steps

    achieved = w.flops / (kernel_ms * 1e-3) / 1e12
    peak = workloads.MI355X_PEAK["f32_mfma_tflops"]
    value = w.flops / (ms_per_step * 1e-3) / 1e12
    line = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": config,
        "mfma_peak_frac": round(value / peak, 4),
        "series_forecasts_per_s": round(w.B / (ms_per_step * 1e-3), 1),
        "series_forecasts_per_s_all_layers": round(w.B / (ms_per_step * 1e-3 * w.meta["num_layers"]), 1),
        "num_layers": w.meta["num_layers"],
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 3),
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": round(achieved / peak, 4),
            "traffic": traffic_for(w.name),
            "algorithmic_flops": w.flops,
            "algorithmic_bytes": w.bytes,
            "kernel_ms": round(kernel_ms, 4),
        },
        "cpu_baseline": None,
    }

    if not args.no_cpu:
        n_series = args.cpu_series or w.B
        dt, want, lanes = cpu_leg(n_series)
        got = o.cpu().numpy()[:n_series]
        import _ref

        sample_flops = w.flops * n_series / w.B
        line["cpu_baseline"] = {
            "value": round(sample_flops / dt / 1e12, 5),
            "unit": "TFLOP/s",
            "cores": cpu_threads(),
            "kind": "port",
            "sample": f"{n_series} of {w.B} series x {w.H} heads, same inputs; C restatement of the reference CPU "
                      f"path ({lanes} f32 lanes), {dt:.2f} s",
            "series_forecasts_per_s": round(n_series / dt, 2),
            "gpu_speedup": round((dt / n_series) / (ms_per_step * 1e-3 / w.B), 1),
        }
        line["parity_max_scaled_err"] = float(f"{_ref.scaled_err(got, want):.3e}")

    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
