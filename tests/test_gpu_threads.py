"""The library's threading contract, through the C ABI with concurrent callers.

The reference enters its backend from several pool threads at once (par.forRange workers,
src/core/par.zig:13-28; per-thread stream and scratch, src/platform/cuda/gemm.c:171-227). Here:
several host threads call at the same time (ctypes releases the GIL for the call) and every result
must have the bits of the same call made alone; two threads queue split products on one shared
stream (the null stream) and must not share partial-sum buffers; a thread that exits releases its
buffers while the library keeps working for the others.
"""
import threading

import numpy as np
import pytest

import _ref

pytestmark = pytest.mark.gpu


def _attn_case(seed, B=3, H=2, n=150):
    rng = np.random.default_rng(seed)
    d = H * 64
    q, k, v = (rng.standard_normal((B, n, d)).astype(np.float32) for _ in range(3))
    kv = _ref.left_pad_valid(rng, B, n, n // 4)
    return q, k, v, kv, B, H, n, d


def _attn_host(ta, case):
    q, k, v, kv, B, H, n, d = case
    o = np.zeros_like(q)
    rc = ta.fwd(ta.make_args(q=q, k=k, v=v, o=o, mask=ta.Mask.KEYS_ADDITIVE, batch=B, heads=H, n_q=n, n_k=n,
                             q_tok=d, q_batch=n * d, k_tok=d, k_batch=n * d, v_tok=d, v_batch=n * d, o_tok=d,
                             o_batch=n * d, scale=0.125, key_valid=kv, kv_batch=n))
    assert rc == ta.OK, ta.last_error()
    return o


def _run_threads(fns):
    """Start every fn at the same moment; re-raise the first failure."""
    start = threading.Barrier(len(fns))
    errors = []

    def wrap(fn):
        try:
            start.wait()
            fn()
        except BaseException as e:  # noqa: BLE001 - reported below
            errors.append(e)

    threads = [threading.Thread(target=wrap, args=(fn,)) for fn in fns]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    if errors:
        raise errors[0]


def test_concurrent_host_pointer_calls_match_serial_bits(ta, gpu_ready):
    """Four threads, each its own inputs, host pointers (each thread's own stream and staging
    buffer), five calls each at the same time: every output equals the serial call's bits."""
    cases = [_attn_case(100 + i) for i in range(4)]
    serial = [_attn_host(ta, c) for c in cases]
    got = [[None] * 5 for _ in cases]

    def worker(i):
        def run():
            for r in range(5):
                got[i][r] = _attn_host(ta, cases[i])
        return run

    _run_threads([worker(i) for i in range(len(cases))])
    for i, want in enumerate(serial):
        for r in range(5):
            assert np.array_equal(got[i][r], want), (i, r)


def _proj_case(torch, seed, tokens=48, d=256, nh=4):
    rng = np.random.default_rng(seed)
    inner = nh * 64
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    x = cu(rng.standard_normal((tokens, d)).astype(np.float32))
    ws = [cu((rng.standard_normal((inner, d)) / np.sqrt(d)).astype(np.float32)) for _ in range(3)]
    outs = [torch.zeros((tokens, inner), dtype=torch.float32, device="cuda") for _ in range(3)]
    return x, ws, outs, tokens, d, nh


def _proj_run(ta, c, stream):
    x, ws, outs, tokens, d, nh = c
    rc = ta.bolt_qkv_projection(x, *ws, *outs, 1, tokens, d, nh, 64, stream=stream)
    assert rc == ta.OK, ta.last_error()


def test_two_threads_share_the_null_stream(ta, gpu_ready):
    """Split products (48 tokens: a reduction split over workgroups, then a fixed-order sum of the
    partials) queued by two threads on the one null stream, interleaved: each thread's partials are
    its own, so every result has the bits of the product run alone."""
    import torch

    cases = [_proj_case(torch, 7 + i) for i in range(2)]
    want = []
    for c in cases:
        _proj_run(ta, c, 0)
        torch.cuda.synchronize()
        want.append([o.cpu().numpy().copy() for o in c[2]])
    bad = []

    def worker(i):
        def run():
            for _ in range(20):
                _proj_run(ta, cases[i], 0)
                torch.cuda.synchronize()
                for o, w in zip(cases[i][2], want[i]):
                    if not np.array_equal(o.cpu().numpy(), w):
                        bad.append(i)
        return run

    _run_threads([worker(0), worker(1)])
    assert not bad, bad


def test_thread_exit_releases_and_library_keeps_working(ta, gpu_ready):
    """A thread that makes device-pointer split products on two streams and host-pointer calls,
    then exits (its stream, staging buffer and partial-sum buffers are released); the main thread's
    next calls give the same bits as before."""
    import torch

    c = _proj_case(torch, 3)
    case = _attn_case(5)
    _proj_run(ta, c, 0)
    torch.cuda.synchronize()
    want_p = [o.cpu().numpy().copy() for o in c[2]]
    want_a = _attn_host(ta, case)
    side = torch.cuda.Stream()

    def visitor():
        _proj_run(ta, c, 0)
        _proj_run(ta, c, side.cuda_stream)
        _attn_host(ta, case)

    t = threading.Thread(target=visitor)
    t.start()
    t.join()
    torch.cuda.synchronize()
    _proj_run(ta, c, 0)
    torch.cuda.synchronize()
    assert all(np.array_equal(o.cpu().numpy(), w) for o, w in zip(c[2], want_p))
    assert np.array_equal(_attn_host(ta, case), want_a)


def test_fused_row_norm_equals_the_separate_launch(ta, gpu_ready):
    """The Chronos-Bolt forward normalises the rows of each split residual product inside the
    product's reduce, and (at most 16 series) its decoder's 16-row products normalise their input
    rows as they load them; TSFM_UNFUSED_NORM=1 queues every product and nn.rmsNorm as separate
    launches instead. The forward's output has the same bits either way."""
    import os

    import torch

    from tsfm_attn import workloads

    w = workloads.bolt_forward(B=4, n_layers=2)
    a, m = w.arrays, w.meta
    cu = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()
    dev = {n: cu(v) for n, v in a.items()}
    enc = [{k: cu(v) for k, v in ly.items()} for ly in m["enc"]]
    dec = [{k: cu(v) for k, v in ly.items()} for ly in m["dec"]]
    ie, oe = ({k: cu(v) for k, v in b.items()} for b in (m["ie"], m["oe"]))

    def run():
        raw = torch.zeros((w.B, m["out"]), dtype=torch.float32, device="cuda")
        rc = ta.bolt_forward(raw, dev["feats"], dev["patch_valid"], dev["reg"], dev["dec_start"], dev["rel_table"],
                             enc, dev["enc_final_norm"], dec, dev["dec_final_norm"], ie, oe, w.B, m["n_patch"],
                             m["d_model"], w.H, m["d_ff"], m["eps"], keys_all_valid=bool(a["patch_valid"].all()))
        assert rc == ta.OK, ta.last_error()
        torch.cuda.synchronize()
        return raw.cpu().numpy()

    fused = run()
    os.environ["TSFM_UNFUSED_NORM"] = "1"
    try:
        separate = run()
    finally:
        del os.environ["TSFM_UNFUSED_NORM"]
    assert np.array_equal(fused, separate)
