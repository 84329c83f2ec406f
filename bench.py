#!/usr/bin/env python3
"""Benchmark of the gfx950 attention path.

Headline workload (the metric's): Chronos-2 time attention, B=64 series x 12 heads, L=577 tokens,
D=64, f32, RoPE, left-padding key mask, scale 1/8. A step is one batched attention call over the
whole synthetic batch with every input already resident in HBM. Prints one JSON line with
whole-job TFLOP/s, the roofline of the dominant kernel (algorithmic work over its HIP-event-timed
mean launch duration, against the MI355X peak that bounds it) and the CPU baseline: the C
restatement of the reference's CPU attention (oracle/, `kind: port`) timed on this host's cores
over a sample of the same inputs, with the parity of the timed output against it.

The default run adds `other_configs`, each measured the same way (timed steps, roofline, CPU
baseline, parity and the reference-derived parity bar): 1 = bolt_forecast, 2 = bolt, 4 = decode,
5 = prefill, 3-e2e = chronos2_forecast, whose whole forecasts per second are the line's
`series_forecasts_per_s` (the attention call alone gives `attention_series_per_s`), and 4-e2e =
timestral_forecast, the whole Timestral forecast at the decode shape with and without its cache.
`--workload X` measures X alone.

Other workloads (parity-test shapes, measured the same way):
  bolt     Chronos-Bolt-base encoder self-attention, B=256 H=12 L=129, f32, T5 bias, no scale
  prefill  Timestral-shaped causal prefill, f16, B=32 rows H=16 L=2048, 10 % rows key-padded
  decode   Timestral-shaped KV-cached block decode, bf16, B=128 H=16, prefix 256 + 8 x 32;
           a step rewinds the cache to the prefix and runs 8 x (append 32, attend 32)
  variate  Timestral variate attention at the prefill shape, f32: 8 series x 4 variates (target,
           past, 2 known) over L=2048 slots, H=16, covariate firewalls, key padding, sigmoid gate
  proj     the Chronos-2 q/k/v projections with RoPE epilogue at the attention's shape, f32:
           64 x 577 tokens, d_model 768, three (768, 768) weights
  bolt_forward  the Chronos-Bolt-small model forward at the end-to-end configuration (16 series,
           32 patches + REG, d_model 512, 6 + 6 layers, 9 quantiles x 64), f32, random-init weights
  bolt_forecast  the whole Chronos-Bolt-small forecast at the end-to-end configuration: 16 series
           x 512 raw steps (sinusoid + trend + noise, 2 % NaN) in, 9 quantiles x 64 steps out; the
           instance norm, patching and inverse norm run on the device around bolt_forward
  timestral_forecast  the whole Timestral forecast at the decode shape (d_model 1024, 16 heads, 4
           layers): 128 series x 4096 steps in, 8 decode blocks of 32 patches (4096 steps) out, with
           the K/V cache; the same forecast re-encoding every block (the reference's decode) is
           timed beside it (`reencode`, `cache_speedup`)
  chronos2_forecast  the whole Chronos-2-base forecast at the attention's shape: 64 series x 8192
           raw steps in (512 patches + REG + 64 future = 577 tokens), 21 quantiles x 1024 steps out
  encoder  the Chronos-2 encoder stack at the Chronos-2-base size (12 layers, d_model 768, 12 heads,
           d_ff 3072) over 64 series x 577 tokens, f32, random-init weights; the roofline is over
           the whole stack (every launch but the row norms runs on the f32 matrix cores)

    python bench.py [--steps K] [--warmup W] [--no-cpu]
                    [--workload chronos2|bolt|prefill|decode|variate|proj|encoder|bolt_forward|bolt_forecast|
                     chronos2_forecast|timestral_forecast]
    python bench.py --copy-mib N    # plain N MiB device copy: calibrates the HBM byte counters
"""
import argparse
import ctypes
import json
import os
import pathlib
import sys
import time
from dataclasses import dataclass
from typing import Callable, Optional

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "tsfm-zig_amd"))
sys.path.insert(0, str(ROOT / "tests"))

METRIC = "attention TFLOP/s + % MFMA peak; series-forecasts/sec at Chronos-2 shape"


GPU_HOST_CPU_SHARE = 16  # host CPUs a one-GPU job is granted on the GPU hosts, whatever nproc shows


def _cgroup_cpu_quota():
    """CPUs allowed by the cgroup v2 (cpu.max) or v1 (cfs quota) limit, or None when unlimited."""
    try:
        quota, period = pathlib.Path("/sys/fs/cgroup/cpu.max").read_text().split()[:2]
        if quota != "max":
            return max(1, int(int(quota) // int(period)))
        return None
    except (OSError, ValueError):
        pass
    try:
        q = int(pathlib.Path("/sys/fs/cgroup/cpu/cpu.cfs_quota_us").read_text())
        p = int(pathlib.Path("/sys/fs/cgroup/cpu/cpu.cfs_period_us").read_text())
        return max(1, q // p) if q > 0 else None
    except (OSError, ValueError):
        return None


def cpu_thread_limits() -> dict:
    """The host logical cores this process may use, and where each limit comes from."""
    lim = {"affinity": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)}
    quota = _cgroup_cpu_quota()
    if quota is not None:
        lim["cgroup_quota"] = quota
    lim["gpu_host_share"] = GPU_HOST_CPU_SHARE
    return lim


def cpu_threads() -> int:
    """Threads of the CPU baseline: the logical cores in this process's affinity mask, capped by a
    cgroup CPU quota and by the one-GPU job's share of the host."""
    return max(1, min(cpu_thread_limits().values()))


def oracle_path() -> pathlib.Path:
    """The oracle build with the f32 lane count the reference picks on this host (nn.lanes)."""
    info = pathlib.Path("/proc/cpuinfo")
    flags = info.read_text() if info.exists() else ""
    lib16 = ROOT / "oracle" / "liboracle_l16.so"
    return lib16 if (" avx512f" in flags and lib16.exists()) else ROOT / "oracle" / "liboracle_l8.so"


def traffic_for(workload: str):
    """Measured HBM bytes per launch of the dominant kernel (rocprofv3 FETCH_SIZE/WRITE_SIZE,
    calibrated against a plain copy), or None when not measured for this workload."""
    p = ROOT / "profiles" / "traffic.json"
    if p.exists():
        return json.loads(p.read_text()).get(workload)
    return None


@dataclass
class Bench:
    w: object                          # tsfm_attn.workloads.Workload
    step: Callable[[], None]
    output: Callable[[], np.ndarray]   # f32 numpy of the step's result, for the parity check
    cpu_leg: Callable[[int], tuple]    # n_series -> (seconds, expected output, lanes)
    config: dict
    dtype: str
    bound: str                         # "mfma" or "hbm"
    peak: float
    unit: str
    cpu_default: int                   # series in the default CPU sample
    # For a step of several launches: the mean duration (ms) of the dominant kernel over the
    # timed steps, from events the step recorded around it; None = the step is one launch.
    kernel_ms: Optional[Callable[[], float]] = None
    kernel_work: Optional[float] = None  # algorithmic work per dominant launch (bound's unit)
    # The dominant matrix work is f32 arithmetic run on the bf16 matrix cores as a three-way split
    # (six bf16 products per f32 product): the line then also reports that pipe's own ceiling.
    x3: bool = False


def _check(ta, rc):
    if rc != ta.OK:
        raise RuntimeError(f"tsfm_attn returned {rc}: {ta.last_error()}")


def _orc(lib=None):
    import _oracle

    return _oracle.Oracle(lib or oracle_path())


def run_chronos2(torch, ta, workloads, peak):
    w = workloads.chronos2()
    a = w.arrays
    dev = {n: torch.from_numpy(np.ascontiguousarray(a[n])).cuda() for n in ("q", "k", "v", "key_valid", "rope_cos", "rope_sin")}
    o = torch.empty_like(dev["q"])
    all_valid = bool(a["key_valid"].all())
    d = w.H * 64

    def step():
        _check(ta, ta.chronos2_time_attention(dev["q"], dev["k"], dev["v"], o, dev["rope_cos"], dev["rope_sin"],
                                              dev["key_valid"], all_valid, w.B, w.n_q, d, w.H, 64, scale=w.scale))

    def cpu_leg(B, lib=None):
        orc = _orc(lib)
        q = np.ascontiguousarray(a["q"][:B]).ravel().copy()
        k = np.ascontiguousarray(a["k"][:B]).ravel().copy()
        v = np.ascontiguousarray(a["v"][:B]).ravel()
        kv = np.ascontiguousarray(a["key_valid"][:B]).ravel()
        out = np.zeros(B * w.n_q * d, np.float32)
        t0 = time.perf_counter()
        # The reference path this call replaces: serial RoPE loop, then forRange(b*nh, TimeJob.attend).
        orc.chronos2_rope(q, k, a["rope_cos"], a["rope_sin"], B * w.n_q, w.n_q, d, w.H, 64)
        orc.chronos2_time_attention(cpu_threads(), q, k, v, out, kv, bool(kv.all()), B, w.n_q, d, w.H, 64, w.scale)
        return time.perf_counter() - t0, out.reshape(B, w.n_q, d), orc.lanes

    config = {"workload": w.name, "B": w.B, "H": w.H, "L": w.n_q, "D": 64, "mask": "keys_additive", "rope": True,
              "scale": w.scale, "layout": "(B, L, H*D) f32"}
    return Bench(w, step, lambda: o.cpu().numpy(), cpu_leg, config, "f32", "mfma", peak["f32_mfma_tflops"],
                 "TFLOP/s", w.B, x3=True)


def run_bolt(torch, ta, workloads, peak):
    w = workloads.bolt()
    a = w.arrays
    L, d = w.n_q, w.H * 64
    buckets = np.zeros(2 * L - 1, np.int32)
    _check(ta, ta.load().tsfm_t5_bucket_table(buckets.ctypes.data, L, L, 32, 128))
    dev = {n: torch.from_numpy(np.ascontiguousarray(x)).cuda() for n, x in
           dict(q=a["q"], k=a["k"], v=a["v"], key_valid=a["key_valid"], rel_table=a["rel_table"], buckets=buckets).items()}
    o = torch.empty_like(dev["q"])
    all_valid = bool(a["key_valid"].all())

    def step():
        _check(ta, ta.bolt_self_attention(dev["q"], dev["k"], dev["v"], o, dev["rel_table"], dev["buckets"],
                                          dev["key_valid"], all_valid, w.B, L, d, w.H, 64, 32))

    def cpu_leg(B, lib=None):
        orc = _orc(lib)
        q = np.ascontiguousarray(a["q"][:B]).ravel()
        k = np.ascontiguousarray(a["k"][:B]).ravel()
        v = np.ascontiguousarray(a["v"][:B]).ravel()
        kv = np.ascontiguousarray(a["key_valid"][:B]).ravel()
        out = np.zeros(B * L * d, np.float32)
        t0 = time.perf_counter()
        bias = orc.position_bias(a["rel_table"], L, w.H, 32, 128)
        orc.bolt_self_attention(cpu_threads(), q, k, v, out, bias, kv, bool(kv.all()), B, L, d, w.H, 64)
        return time.perf_counter() - t0, out.reshape(B, L, d), orc.lanes

    config = {"workload": w.name, "B": w.B, "H": w.H, "L": L, "D": 64, "mask": "keys_additive", "bias": "t5 32/128",
              "scale": 1.0, "layout": "(B, L, H*D) f32"}
    return Bench(w, step, lambda: o.cpu().numpy(), cpu_leg, config, "f32", "mfma", peak["f32_mfma_tflops"],
                 "TFLOP/s", w.B, x3=True)


def run_prefill(torch, ta, workloads, peak):
    w = workloads.timestral_prefill()
    a = w.arrays
    row = w.H * 64
    dev = {n: torch.from_numpy(np.ascontiguousarray(a[n])).to(torch.float16).cuda() for n in ("q", "k", "v")}
    kvd = torch.from_numpy(np.ascontiguousarray(a["key_valid"])).cuda()
    o = torch.empty_like(dev["q"])
    mask = ta.Mask.pick(True, bool(a["key_valid"].all()), False)  # per chunk, as the reference decides
    args = ta.make_args(q=dev["q"], k=dev["k"], v=dev["v"], o=o, mask=mask, batch=w.B, heads=w.H, n_q=w.n_q,
                        n_k=w.n_k, q_tok=row, q_batch=w.n_q * row, k_tok=row, k_batch=w.n_k * row, v_tok=row,
                        v_batch=w.n_k * row, o_tok=row, o_batch=w.n_q * row, scale=w.scale, key_valid=kvd,
                        kv_batch=w.n_k)

    def step():
        _check(ta, ta.fwd(args))

    def cpu_leg(B, lib=None):
        orc = _orc(lib)
        r = lambda x: np.ascontiguousarray(x[:B]).astype(np.float16).astype(np.float32)
        q, k, v = r(a["q"]), r(a["k"]), r(a["v"])
        kv = np.ascontiguousarray(a["key_valid"][:B])
        out = np.zeros((B, w.n_q, row), np.float32)
        t0 = time.perf_counter()
        orc.batched_self_attend(cpu_threads(), int(mask), q, row, w.n_q * row, k, row, w.n_k * row, v, row,
                                w.n_k * row, out, row, w.n_q * row, kv, w.n_k, None, B, w.H, w.n_q, 64, w.scale)
        return time.perf_counter() - t0, out, orc.lanes

    config = {"workload": w.name, "B": w.B, "H": w.H, "L": w.n_q, "D": 64, "mask": mask.name.lower(),
              "padded_rows": int(a["padded_rows"].sum()), "scale": w.scale, "layout": "(B, L, H*D) f16"}
    return Bench(w, step, lambda: o.float().cpu().numpy(), cpu_leg, config, "f16", "mfma", peak["f16_mfma_tflops"],
                 "TFLOP/s", 8)


def run_decode(torch, ta, workloads, peak):
    w = workloads.timestral_decode()
    a = w.arrays
    P, nb, blk = w.meta["prefix"], w.meta["blocks"], w.meta["block"]
    row, T = w.H * 64, P + nb * blk
    dev = {n: torch.from_numpy(np.ascontiguousarray(a[n])).to(torch.bfloat16).cuda() for n in ("q", "k", "v")}
    out = torch.zeros((w.B, nb * blk, row), dtype=torch.bfloat16, device="cuda")
    cache = ta.KvCache(ta.DTYPE_BF16, w.B, w.H, T)
    cache.append(dev["k"], dev["v"], P, row, T * row, row, T * row)
    stream = torch.cuda.current_stream()
    events = []  # (start, end) around the 8 decode-block launches of each timed step
    pool = []    # event pairs made (and recorded once) before the timed steps
    # The block views, made once: the host issues a launch in a few microseconds, ahead of the
    # GPU, so the event pair around a step's launches brackets the kernels and not the host's Python.
    views = [(dev["k"][:, P + i * blk:], dev["v"][:, P + i * blk:], dev["q"][:, P + i * blk:], out[:, i * blk:])
             for i in range(nb)]

    def prepare(steps):
        while len(pool) < steps:
            pair = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            pair[0].record(stream)
            pair[1].record(stream)
            pool.append(pair)
        torch.cuda.synchronize()

    def step(record=True):
        cache.truncate(P)  # host-side length only
        if record:
            e0, e1 = pool[len(events)]
            e0.record(stream)
        for i in range(nb):
            kb, vb, qb, ob = views[i]
            # One launch per block: the block's K/V into the cache, then its 32 queries over it.
            cache.append_attend(kb, vb, qb, ob, blk, w.scale, row, T * row, row, T * row, row, T * row, row,
                                nb * blk * row, stream)
        if record:
            e1.record(stream)
            events.append((e0, e1))

    def kernel_ms():
        # Per launch: the 8 back-to-back launches of a step between one event pair (the gaps between
        # them included), so no event sits between two launches.
        return sum(a0.elapsed_time(a1) for a0, a1 in events) / (len(events) * nb)

    def cpu_leg(B, lib=None):
        orc = _orc(lib)
        r = lambda x: np.ascontiguousarray(x[:B]).astype(np.float32)
        bf = lambda x: torch.from_numpy(r(x)).to(torch.bfloat16).float().numpy()
        q, k, v = bf(a["q"]), bf(a["k"]), bf(a["v"])
        want = np.zeros((B, nb * blk, row), np.float32)
        full = np.zeros((B, T, row), np.float32)
        t0 = time.perf_counter()
        # The reference's way (src/timestral/forecaster.zig:466-561): every block re-encodes the whole
        # grown context, i.e. causal selfAttend over P + 32(i+1) tokens; block i's rows are its output.
        for i in range(nb):
            n = P + (i + 1) * blk
            orc.batched_self_attend(cpu_threads(), 2, q, row, T * row, k, row, T * row, v, row, T * row, full, row,
                                    T * row, None, 0, None, B, w.H, n, 64, w.scale)
            want[:, i * blk:(i + 1) * blk] = full[:, n - blk:n]
        return time.perf_counter() - t0, want, orc.lanes

    # Work of the decode-block kernel (kv_attend<bf16, append>), per launch, averaged over the 8
    # blocks: the cache's K/V read (the keys before the block), the block's new K/V read once and
    # written into the cache, q read, o written, in bytes.
    bytes_per_attend = w.B * w.H * sum((P + i * blk) * 64 * 2 * 2 + 2 * blk * 64 * 2 + 2 * blk * 64 * 2 * 2
                                       for i in range(nb)) / nb
    config = {"workload": w.name, "B": w.B, "H": w.H, "D": 64, "prefix": P, "blocks": nb, "block": blk,
              "mask": "causal", "scale": w.scale, "layout": "(B, T, H*D) bf16; cache K [B][H][cap][64], V chunked"}
    b = Bench(w, lambda: step(True), lambda: out.float().cpu().numpy(), cpu_leg, config, "bf16", "hbm",
              peak["hbm_gbps"], "GB/s", 8, kernel_ms, bytes_per_attend / 1e9)
    b.warm = lambda: step(False)
    b.reset_events = events.clear
    b.prepare = prepare
    return b


def run_variate(torch, ta, workloads, peak):
    w = workloads.timestral_variate()
    a = w.arrays
    G, V, L, H = w.meta["groups"], w.meta["vall"], w.meta["L"], w.H
    d = H * 64
    dev = {n: torch.from_numpy(np.ascontiguousarray(a[n])).cuda() for n in ("qkv", "gate", "key_valid")}
    o = torch.empty((G * V, L, d), dtype=torch.float32, device="cuda")
    roles = [int(r) for r in a["roles"]]

    def step():
        _check(ta, ta.timestral_variate_attention(dev["qkv"], o, dev["key_valid"], roles, True, G, V, L, 0, d, H, 64,
                                                  gate=dev["gate"]))

    def cpu_leg(n, lib=None):
        orc = _orc(lib)
        qkv = np.ascontiguousarray(a["qkv"][: n * V])
        gate = np.ascontiguousarray(a["gate"][: n * V])
        kv = np.ascontiguousarray(a["key_valid"][: n * V])
        want = np.zeros((n * V, L, d), np.float32)
        t0 = time.perf_counter()
        orc.timestral_variate_attention(cpu_threads(), qkv, want, kv, a["roles"], True, n, V, L, 0, d, H, 64)
        orc.mul_sigmoid(want, want, gate)
        return time.perf_counter() - t0, want.reshape(n, V, L, d), orc.lanes

    config = {"workload": w.name, "series": G, "variates": V, "H": H, "L": L, "D": 64, "roles": "target,past,known,known",
              "covariates": True, "gate": "sigmoid", "layout": "qkv (rows, L, 3d) permuted, o and gate (rows, L, d) f32"}
    return Bench(w, step, lambda: o.cpu().numpy().reshape(G, V, L, d), cpu_leg, config, "f32", "hbm",
                 peak["hbm_gbps"], "GB/s", 1)


def run_proj(torch, ta, workloads, peak):
    w = workloads.chronos2_projection()
    a = w.arrays
    d, L, M = w.meta["d_model"], w.n_q, w.meta["tokens"]
    dev = {n: torch.from_numpy(np.ascontiguousarray(a[n])).cuda() for n in ("x", "wq", "wk", "wv", "rope_cos", "rope_sin")}
    outs = [torch.empty((M, d), dtype=torch.float32, device="cuda") for _ in range(3)]

    def step():
        _check(ta, ta.chronos2_qkv_projection(dev["x"], dev["wq"], dev["wk"], dev["wv"], *outs, dev["rope_cos"],
                                              dev["rope_sin"], w.B, L, d, w.H, 64))

    def output():
        return torch.stack(outs).reshape(3, w.B, L, d).permute(1, 0, 2, 3).cpu().numpy()

    def cpu_leg(B, lib=None):
        orc = _orc(lib)
        x = np.ascontiguousarray(a["x"][: B * L])
        ys = [np.zeros((B * L, d), np.float32) for _ in range(3)]
        t0 = time.perf_counter()
        # The reference path this call replaces: three nn.linear calls, then the serial RoPE loop.
        for y, wt in zip(ys, (a["wq"], a["wk"], a["wv"])):
            orc.linear(cpu_threads(), y, x, B * L, wt, d, d)
        orc.chronos2_rope(ys[0], ys[1], a["rope_cos"], a["rope_sin"], B * L, L, d, w.H, 64)
        return time.perf_counter() - t0, np.stack(ys).reshape(3, B, L, d).transpose(1, 0, 2, 3), orc.lanes

    config = {"workload": w.name, "B": w.B, "L": L, "d_model": d, "H": w.H, "outputs": "q,k,v", "rope": True,
              "layout": "x (B*L, d), W (d, d) x3, q/k/v (B*L, d) f32"}
    return Bench(w, step, output, cpu_leg, config, "f32", "mfma", peak["f32_mfma_tflops"], "TFLOP/s", 16, x3=True)


def run_encoder(torch, ta, workloads, peak):
    w = workloads.chronos2_encoder()
    a, m = w.arrays, w.meta
    d, L, F = m["d_model"], w.n_q, m["d_ff"]
    cu = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()
    dev = {n: cu(a[n]) for n in ("x", "key_valid", "rope_cos", "rope_sin", "final_norm")}
    layers = [{k: cu(v) for k, v in ly.items()} for ly in m["layers"]]
    x = torch.empty_like(dev["x"])
    all_valid = bool(a["key_valid"].all())

    def step():
        x.copy_(dev["x"])  # the stack runs in place: each step starts from the same embedded tokens
        _check(ta, ta.chronos2_encode(x, dev["key_valid"], dev["rope_cos"], dev["rope_sin"], layers, dev["final_norm"],
                                      w.B, L, d, w.H, F, m["eps"], keys_all_valid=all_valid, scale=1.0))

    def cpu_leg(B, lib=None):
        orc = _orc(lib)
        out = np.ascontiguousarray(a["x"][: B * L]).copy()
        kv = np.ascontiguousarray(a["key_valid"][:B]).ravel().copy()
        t0 = time.perf_counter()
        orc.chronos2_encode(cpu_threads(), out, kv, B, L, d, w.H, 64, F, m["layers"], a["final_norm"], m["eps"],
                            a["rope_cos"], a["rope_sin"], 1.0)
        return time.perf_counter() - t0, out.reshape(B, L, d), orc.lanes

    config = {"workload": w.name, "B": w.B, "L": L, "d_model": d, "H": w.H, "d_ff": F, "layers": m["n_layers"],
              "mask": "keys_additive", "rope": True, "scale": 1.0, "weights": "random-init f32"}
    b = Bench(w, step, lambda: x.cpu().numpy().reshape(w.B, L, d), cpu_leg, config, "f32", "mfma",
              peak["f32_mfma_tflops"], "TFLOP/s", 1, x3=True)
    return b


def run_bolt_forward(torch, ta, workloads, peak):
    w = workloads.bolt_forward()
    a, m = w.arrays, w.meta
    cu = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()
    dev = {n: cu(v) for n, v in a.items()}
    enc = [{k: cu(v) for k, v in ly.items()} for ly in m["enc"]]
    dec = [{k: cu(v) for k, v in ly.items()} for ly in m["dec"]]
    ie, oe = ({k: cu(v) for k, v in b.items()} for b in (m["ie"], m["oe"]))
    raw = torch.empty((w.B, m["out"]), dtype=torch.float32, device="cuda")
    all_valid = bool(a["patch_valid"].all())
    d, F, npch = m["d_model"], m["d_ff"], m["n_patch"]

    # The argument block is built once, as a caller holding a loaded model does.
    args = ta.bolt_forward_args(enc, dec, dev["feats"], dev["patch_valid"], dev["reg"], dev["dec_start"],
                         dev["rel_table"], dev["enc_final_norm"], dev["dec_final_norm"], ie, oe, raw, w.B, npch, d, w.H,
                         64, F, m["eps"], m["buckets"], m["max_distance"], all_valid, True, None)
    fn = ta.load().tsfm_bolt_forward

    def step():
        _check(ta, fn(ctypes.byref(args)))

    def cpu_leg(B, lib=None):
        orc = _orc(lib)
        want = np.zeros((B, m["out"]), np.float32)
        t0 = time.perf_counter()
        orc.bolt_model_forward(cpu_threads(), want, np.ascontiguousarray(a["feats"][: B * npch]),
                               np.ascontiguousarray(a["patch_valid"][:B]), a["reg"], a["dec_start"], a["rel_table"],
                               m["buckets"], m["max_distance"], B, npch, d, w.H, 64, F, m["enc"], a["enc_final_norm"],
                               m["dec"], a["dec_final_norm"], m["eps"], m["ie"], m["oe"])
        return time.perf_counter() - t0, want, orc.lanes

    config = {"workload": w.name, "series": w.B, "patches": npch, "reg": True, "d_model": d, "H": w.H, "d_ff": F,
              "layers": "6 enc + 6 dec", "head": f"{m['out']} (9 quantiles x 64)", "weights": "random-init f32"}
    return Bench(w, step, lambda: raw.cpu().numpy(), cpu_leg, config, "f32", "mfma", peak["f32_mfma_tflops"],
                 "TFLOP/s", w.B)


def run_bolt_forecast(torch, ta, workloads, peak):
    import shutil
    import tempfile

    from tsfm_attn import checkpoint

    w = workloads.bolt_forward()
    a, m = w.arrays, w.meta
    d, F, length, P = m["d_model"], m["d_ff"], a["ctx"].shape[1], m["out"] // 9
    levels = np.linspace(0.1, 0.9, 9).astype(np.float32)
    host = dict(reg=a["reg"], dec_start=a["dec_start"], rel_table=a["rel_table"], enc_final_norm=a["enc_final_norm"],
                dec_final_norm=a["dec_final_norm"], enc=m["enc"], dec=m["dec"], ie=m["ie"], oe=m["oe"])
    # The random-init checkpoint is written as config.json + model.safetensors and read back the way
    # a caller loads a local model directory; the forecast then runs from the loaded weights.
    ckpt = tempfile.mkdtemp(prefix="bolt_small_")
    cfg = checkpoint.bolt_config_dict(d_model=d, d_ff=F, num_heads=w.H, num_layers=len(m["enc"]),
                                      num_decoder_layers=len(m["dec"]), context_length=2048, patch=16,
                                      prediction_length=P, quantiles=levels.tolist(), eps=m["eps"],
                                      buckets=m["buckets"], max_distance=m["max_distance"])
    checkpoint.write_bolt_checkpoint(ckpt, cfg, host)
    fc = checkpoint.load_bolt(ckpt)
    shutil.rmtree(ckpt, ignore_errors=True)  # the weights are on the device now
    ctx_dev = torch.from_numpy(np.ascontiguousarray(a["ctx"])).cuda()
    out = torch.empty((w.B, P, 9), dtype=torch.float32, device="cuda")
    # The argument block (about 130 weight pointers) is built once, as a caller holding a loaded
    # model does; each step is one forecaster.forecast call (tsfm_bolt_forecast_horizon).
    args = fc.forecast_args(out, ctx_dev, P)
    fn = ta.load().tsfm_bolt_forecast_horizon

    def step():
        _check(ta, fn(ctypes.byref(args)))

    orc_w = dict(host, d_model=d, heads=w.H, d_ff=F, eps=m["eps"], buckets=m["buckets"], max_distance=m["max_distance"])

    def cpu_leg(B, lib=None):
        orc = _orc(lib)
        ctx = np.ascontiguousarray(a["ctx"][:B])
        t0 = time.perf_counter()
        want = orc.bolt_forecast_horizon(cpu_threads(), ctx, P, orc_w, P, 2048, levels)
        return time.perf_counter() - t0, want, orc.lanes

    config = {"workload": "bolt_small_forecast", "series": w.B, "context": length, "horizon": P,
              "missing": "2 %", "d_model": d, "H": w.H, "d_ff": F, "layers": "6 enc + 6 dec",
              "head": f"{m['out']} (9 quantiles x {P})", "weights": "random-init f32, local config.json + model.safetensors",
              "input": "sinusoid (period 24, amplitude 10) + trend + N(0,1), seed 0"}
    return Bench(w, step, lambda: out.cpu().numpy(), cpu_leg, config, "f32", "mfma", peak["f32_mfma_tflops"],
                 "TFLOP/s", w.B)


def run_chronos2_forecast(torch, ta, workloads, peak):
    w = workloads.chronos2_forecast()
    a, m = w.arrays, w.meta
    cu = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()
    dev = {n: cu(v) for n, v in a.items()}
    layers = [{k: cu(v) for k, v in ly.items()} for ly in m["layers"]]
    ie, oe = ({k: cu(v) for k, v in b.items()} for b in (m["ie"], m["oe"]))
    d, F, T, hz, q = m["d_model"], m["d_ff"], m["context"], m["horizon"], m["quantiles"]
    out = torch.empty((w.B, hz, q), dtype=torch.float32, device="cuda")
    # The argument block (about 140 weight pointers) is built once, as a caller holding a loaded
    # model does; each step is one tsfm_chronos2_forecast call.
    args = ta.chronos2_forecast_args(out, dev["ctx"], T, hz, dev["reg"], dev["rope_cos"], dev["rope_sin"], layers,
                                     dev["final_norm"], ie, oe, w.B, d, w.H, F, m["eps"], time_scale=m["time_scale"],
                                     arcsinh=True)
    fn = ta.load().tsfm_chronos2_forecast

    def step():
        _check(ta, fn(ctypes.byref(args)))

    def cpu_leg(B, lib=None):
        orc = _orc(lib)
        want = np.zeros((B, hz, q), np.float32)
        ctx = np.ascontiguousarray(a["ctx"][:B])
        t0 = time.perf_counter()
        orc.chronos2_forecast(cpu_threads(), want, ctx, T, 0, T, B, m["patch"], hz, m["time_scale"], True, a["reg"], d,
                              w.H, 64, F, m["layers"], a["final_norm"], m["eps"], a["rope_cos"], a["rope_sin"], 1.0,
                              m["ie"], m["oe"])
        return time.perf_counter() - t0, want, orc.lanes

    config = {"workload": "chronos2_base_forecast", "series": w.B, "context": T, "horizon": hz, "quantiles": q,
              "tokens": w.n_q, "d_model": d, "H": w.H, "d_ff": F, "layers": m["n_layers"], "asinh": True,
              "missing": "oldest 0-25 % + 2 %", "weights": "random-init f32",
              "input": "sinusoid (period 24, amplitude 10) + trend + N(0,1)"}
    return Bench(w, step, lambda: out.cpu().numpy(), cpu_leg, config, "f32", "mfma", peak["f32_mfma_tflops"],
                 "TFLOP/s", 1, x3=True)


def run_timestral_forecast(torch, ta, workloads, peak):
    w = workloads.timestral_forecast()
    a, m = w.arrays, w.meta
    model = m["model"]
    cu = lambda x: None if x is None else torch.from_numpy(np.ascontiguousarray(x)).cuda()
    dm = dict(model)
    dm["patch_proj"] = {k: cu(v) for k, v in model["patch_proj"].items()}
    dm["head"] = {k: cu(v) for k, v in model["head"].items()}
    dm["forecast_query"], dm["out_norm"] = cu(model["forecast_query"]), cu(model["out_norm"])
    dm["layers"] = [dict(attns=[{k: (cu(v) if isinstance(v, np.ndarray) else v) for k, v in at.items()}
                                for at in ly["attns"]], mlp_norm=cu(ly["mlp_norm"]), w12=cu(ly["w12"]), w3=cu(ly["w3"]))
                    for ly in model["layers"]]
    x, obs = cu(a["inputs"]), cu(a["observed"])
    T, hz, q = m["context"], m["horizon"], model["q"]
    outs = {c: torch.empty((w.B, 1, hz, q), dtype=torch.float32, device="cuda") for c in (True, False)}
    # Argument blocks built once, as a caller holding a loaded model does; a step is one
    # forecaster.forecast call with the K/V cache (blocks after the first run only their new
    # patches and decoder tokens). The same call without the cache re-encodes the grown context
    # every block, as the reference's blockDecode does (src/timestral/forecaster.zig:466-561).
    args = {c: ta.timestral_forecast_args(outs[c], x, obs, dm, w.B, 1, T, hz, per_shot=m["per_shot"], kv_cache=c)
            for c in (True, False)}
    fn = ta.load().tsfm_timestral_forecast

    def step(cached=True):
        _check(ta, fn(ctypes.byref(args[cached])))

    def cpu_leg(B, lib=None):
        orc = _orc(lib)
        t0 = time.perf_counter()
        rc, want = orc.timestral_forecast(cpu_threads(), model, a["inputs"][:B], a["observed"][:B], B, 1, T, hz, 0,
                                          m["per_shot"])
        if rc != 0:
            raise RuntimeError(f"oracle timestral_forecast returned {rc}")
        return time.perf_counter() - t0, want, orc.lanes

    def reencode(steps):
        """The uncached forecast (the reference's re-encoding decode) timed over `steps` calls."""
        step(False)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            step(False)
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / steps
        gap = float(((outs[True] - outs[False]).abs() / outs[False].abs().clamp(min=1)).max())
        return {"ms_per_step": round(ms, 3), "value": round(m["reencode_flops"] / (ms * 1e-3) / 1e12, 3),
                "unit": "TFLOP/s", "flops": m["reencode_flops"], "steps": steps,
                "series_forecasts_per_s": round(w.B / (ms * 1e-3), 2), "cached_vs_reencoded_max_scaled_diff": gap}

    config = {"workload": "timestral_forecast", "series": w.B, "variates": 1, "context": T, "horizon": hz,
              "per_shot_patches": m["per_shot"], "blocks": m["blocks"], "patch": model["ps"], "d_model": m["d_model"],
              "H": w.H, "mlp_hidden": m["hid"], "layers": m["schedule"], "quantiles": q, "asinh": True,
              "symmetric_averaging": True, "kv_cache": True, "missing": "oldest 0-25 % + 2 %",
              "weights": "random-init f32", "input": "sinusoid (period 24, amplitude 10) + trend + N(0,1)"}
    b = Bench(w, step, lambda: outs[True].cpu().numpy(), cpu_leg, config, "f32", "mfma", peak["f32_mfma_tflops"],
              "TFLOP/s", 1, x3=True)
    b.cpu_flops = m["reencode_flops"]  # the CPU leg runs the reference's re-encoding decode
    b.extra = reencode
    return b


WORKLOADS = {"chronos2": run_chronos2, "bolt": run_bolt, "prefill": run_prefill, "decode": run_decode,
             "variate": run_variate, "proj": run_proj, "encoder": run_encoder, "bolt_forward": run_bolt_forward,
             "bolt_forecast": run_bolt_forecast, "chronos2_forecast": run_chronos2_forecast,
             "timestral_forecast": run_timestral_forecast}
# The default run: the headline (the Chronos-2 time attention, the metric's shape) and, beside it,
# every other synthetic shape of the benchmark plus the whole Chronos-2 forecast at the headline's
# shape (the metric's series-forecasts/sec).
OTHER_CONFIGS = [("1", "bolt_forecast"), ("2", "bolt"), ("4", "decode"), ("5", "prefill"),
                 ("3-e2e", "chronos2_forecast"), ("4-e2e", "timestral_forecast")]
SPINUP_S = 0.25  # untimed load before the timed region, after the --warmup steps
CPU_SAMPLE_S = 10.0  # timed CPU work in the cpu_baseline leg (the sample is repeated up to this)


def _other_lane_lib():
    """The oracle build with the other f32 lane count (the reference on the other kind of host)."""
    here = oracle_path()
    other = ROOT / "oracle" / ("liboracle_l8.so" if here.name == "liboracle_l16.so" else "liboracle_l16.so")
    if other.name == "liboracle_l16.so":
        info = pathlib.Path("/proc/cpuinfo")
        if not (info.exists() and " avx512f" in info.read_text()):
            return None  # this host cannot run the 16-lane build
    return other if other.exists() else None


def measure(torch, bench, steps: int, warmup: int, do_cpu: bool) -> dict:
    """Time `steps` steps of one workload (after `warmup` steps and SPINUP_S of untimed load, between
    two full synchronisations), then its CPU baseline and parity. Returns the JSON fields."""
    import _ref
    from tsfm_attn import workloads

    w = bench.w
    stream = torch.cuda.current_stream()
    warm = getattr(bench, "warm", bench.step)
    for _ in range(warmup):
        warm()
    torch.cuda.synchronize()
    # The engine clock ramps up over the first milliseconds of load: keep warming (untimed) until
    # the GPU has been busy for SPINUP_S, so the timed steps do not start on a cold clock.
    t_warm = time.perf_counter()
    while time.perf_counter() - t_warm < SPINUP_S:
        for _ in range(8):
            warm()
        torch.cuda.synchronize()
    reset = getattr(bench, "reset_events", None)
    if reset is not None:
        reset()
    prepare = getattr(bench, "prepare", None)  # untimed set-up the timed steps use (event pools)
    if prepare is not None:
        prepare(steps)
    # Timed region: the steps between two full synchronisations. One event pair on the stream the
    # kernels run on brackets all the steps (no event between two steps' launches), so a
    # single-launch step's figure is the per-dispatch duration rocprofv3 --kernel-trace reports
    # plus the GPU's gap between two launches; a multi-launch step records its dominant kernel
    # itself.
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    for i in range(steps):
        bench.step()
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / steps
    step_ms = start.elapsed_time(end) / steps
    if bench.kernel_ms is not None:
        kernel_ms = bench.kernel_ms()
        work = bench.kernel_work
    else:
        kernel_ms = step_ms
        work = w.flops / 1e12 if bench.bound == "mfma" else w.bytes / 1e9
    achieved = work / (kernel_ms * 1e-3)
    flop_peak = workloads.MI355X_PEAK["f32_mfma_tflops" if bench.dtype == "f32" else "f16_mfma_tflops"]
    value = w.flops / (ms_per_step * 1e-3) / 1e12
    out = {
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "ms_per_step": round(ms_per_step, 4),
        "dtype": bench.dtype,
        "config": bench.config,
        "mfma_peak_frac": round(value / flop_peak, 4),
        "roofline": {
            "bound": bench.bound,
            "achieved": round(achieved, 3),
            "peak": bench.peak,
            "unit": bench.unit,
            "frac": round(achieved / bench.peak, 4),
            "traffic": traffic_for(w.name),
            # algorithmic work of one dominant-kernel launch, the numerator of `achieved`
            "work_per_launch": work * (1e12 if bench.bound == "mfma" else 1e9),
            "work_unit": "FLOP" if bench.bound == "mfma" else "B",
            "kernel_ms": round(kernel_ms, 4),
            "step_flops": w.flops,
            "step_bytes": w.bytes,
        },
        "cpu_baseline": None,
    }
    if bench.x3:
        # f32 products as six bf16 products each on v_mfma_f32_{32x32x16,16x16x32}_bf16: the pipe's
        # f32-equivalent ceiling is the bf16 dense peak / 6 (above the f32 matrix peak of `peak`).
        pipe_peak = workloads.MI355X_PEAK["bf16_mfma_tflops"] / 6
        out["roofline"]["bf16x3_pipe"] = {
            "bf16_products_per_f32_product": 6,
            "peak_f32_equiv": round(pipe_peak, 1),
            "frac": round(achieved / pipe_peak, 4),
        }
    extra = getattr(bench, "extra", None)
    if extra is not None:  # a second timing beside the step (the Timestral forecast without its cache)
        out["reencode"] = extra(min(steps, 3))
        out["cache_speedup"] = round(out["reencode"]["ms_per_step"] / ms_per_step, 2)
    if not do_cpu:
        return out
    n_series = min(w.B, bench.cpu_default)
    # The sample is run again until about CPU_SAMPLE_S seconds of CPU work have been timed.
    dt, want, lanes = bench.cpu_leg(n_series)
    passes = 1
    while dt < CPU_SAMPLE_S and passes < 200:
        dt += bench.cpu_leg(n_series)[0]
        passes += 1
    got = bench.output()[:n_series]
    sample_flops = getattr(bench, "cpu_flops", w.flops) * n_series / w.B * passes
    out["cpu_baseline"] = {
        "value": round(sample_flops / dt / 1e12, 5),
        "unit": "TFLOP/s",
        "cores": cpu_threads(),
        "kind": "port",
        "sample": f"{n_series} of {w.B} series (rows), same inputs, {passes} passes in {dt:.1f} s; C restatement of "
                  f"the reference CPU path ({lanes} f32 lanes, {cpu_threads()} threads; limits "
                  f"{cpu_thread_limits()})",
        "series_forecasts_per_s": round(n_series * passes / dt, 2),
        "gpu_speedup": round((dt / (n_series * passes)) / (ms_per_step * 1e-3 / w.B), 1),
    }
    err = _ref.scaled_err(got, want)
    out["parity_max_scaled_err"] = float(f"{err:.3e}")
    if bench.dtype == "f32":
        # The f32 bar derived from the reference itself: its own 8-lane vs 16-lane spread on this
        # sample (tests/_ref.py reference_bar), never tighter than 1e-5.
        other = _other_lane_lib()
        if other is not None:
            want_other = bench.cpu_leg(n_series, str(other))[1]
            pair = (want_other, want) if lanes == 16 else (want, want_other)
            bar, spread, _ = _ref.reference_bar(*pair)
            out["parity_bar"] = float(f"{bar:.3e}")
            out["parity_cross_host_spread"] = float(f"{spread:.3e}")
            if lanes != 16:  # compare with the 16-lane build, as the tests do
                out["parity_max_scaled_err"] = float(f"{_ref.scaled_err(got, want_other):.3e}")
    else:
        out["parity_bar"] = 1e-2
    out["parity_ok"] = out["parity_max_scaled_err"] <= out.get("parity_bar", 1e-5)
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default=None, choices=sorted(WORKLOADS),
                    help="measure only this workload (default: the headline plus every other shape)")
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

    name = args.workload or "chronos2"
    bench = WORKLOADS[name](torch, ta, workloads, workloads.MI355X_PEAK)
    w = bench.w
    t_run = time.perf_counter()
    head = measure(torch, bench, args.steps, args.warmup, not args.no_cpu)
    print(f"bench.py: {name} measured ({time.perf_counter() - t_run:.0f} s)", file=sys.stderr, flush=True)
    del bench
    line = {
        "metric": METRIC,
        "value": head["value"],
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": head["dtype"],
        "data": "synthetic",
        "config": head["config"],
        "mfma_peak_frac": head["mfma_peak_frac"],
        # one attention call over the batch: series whose attention one call finishes per second
        "attention_series_per_s": round(w.B / (head["ms_per_step"] * 1e-3), 1),
        "roofline": head["roofline"],
        "cpu_baseline": head["cpu_baseline"],
    }
    for k in ("parity_max_scaled_err", "parity_bar", "parity_cross_host_spread", "parity_ok", "reencode",
              "cache_speedup"):
        if k in head:
            line[k] = head[k]
    if w.meta.get("num_layers"):
        line["num_layers"] = w.meta["num_layers"]
    if args.workload is None:
        others = {}
        for cfg, wl in OTHER_CONFIGS:
            b = WORKLOADS[wl](torch, ta, workloads, workloads.MI355X_PEAK)
            r = measure(torch, b, args.steps, args.warmup, not args.no_cpu)
            r["workload"] = wl
            r["series_forecasts_per_s"] = round(b.w.B / (r["ms_per_step"] * 1e-3), 2)
            others[cfg] = r
            print(f"bench.py: {wl} measured ({time.perf_counter() - t_run:.0f} s)", file=sys.stderr, flush=True)
            del b
            torch.cuda.empty_cache()
        line["other_configs"] = others
        # The metric's series-forecasts/sec at the Chronos-2 shape: whole forecasts (64 series x 8192
        # steps in, 21 quantiles x 1024 steps out, every layer) per second.
        line["series_forecasts_per_s"] = others["3-e2e"]["series_forecasts_per_s"]
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
