"""GPU parity of the f32 attention path against the CPU oracle, through the C ABI.

Bar: scaled error max|gpu - oracle| / max(|oracle|, 1) <= 1e-5 (the f32 tolerance), every mask,
ragged sizes (1, 15, 16, 17, 65, 129, 577), host and device pointers, the family call sites at
their full shapes, padding between heads left untouched (src/core/gpu_test.zig:30-34), and
bit-identical results across repeats and batch compositions.
"""
import numpy as np
import pytest

import _ref
from _oracle import ORC_FULL

pytestmark = pytest.mark.gpu

TOL = 1e-5
THREADS = 16


def _torch():
    import torch

    return torch


def run_generic(ta, mask, q, k, v, key_valid, B, H, n_q, n_k, scale, o_tok=None, device=False, **extra):
    """q (B, n_q, H*64), k/v (B, n_k, H*64) numpy f32; returns o (B, n_q, o_tok)."""
    row = H * 64
    o_tok = o_tok or row
    o = np.full((B, n_q, o_tok), -12345.0, np.float32)
    kw = dict(mask=mask, batch=B, heads=H, n_q=n_q, n_k=n_k, q_tok=row, q_batch=n_q * row, k_tok=row,
              k_batch=n_k * row, v_tok=row, v_batch=n_k * row, o_tok=o_tok, o_batch=n_q * o_tok, scale=scale,
              key_valid=key_valid, kv_batch=key_valid.shape[1] if key_valid is not None else 0, **extra)
    if device:
        torch = _torch()
        dev = {n: torch.from_numpy(np.ascontiguousarray(x)).cuda() for n, x in
               dict(q=q, k=k, v=v, o=o).items()}
        for name in ("key_valid", "rope_cos", "rope_sin", "rel_table", "rel_bucket", "bias"):
            if kw.get(name) is not None:
                kw[name] = torch.from_numpy(np.ascontiguousarray(kw[name])).cuda()
        ta.fwd_checked(ta.make_args(q=dev["q"], k=dev["k"], v=dev["v"], o=dev["o"], **kw))
        torch.cuda.synchronize()
        return dev["o"].cpu().numpy()
    ta.fwd_checked(ta.make_args(q=q, k=k, v=v, o=o, **kw))
    return o


def oracle_generic(orc, mask, q, k, v, key_valid, B, H, n, scale):
    row = H * 64
    o = np.zeros((B, n, row), np.float32)
    orc.batched_self_attend(THREADS, mask, q, row, n * row, k, row, n * row, v, row, n * row, o, row, n * row,
                            key_valid, n if key_valid is not None else 0, None, B, H, n, 64, scale)
    return o


def _inputs(seed, B, H, n_q, n_k):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, n_q, H * 64), dtype=np.float32)
    k = rng.standard_normal((B, n_k, H * 64), dtype=np.float32)
    v = rng.standard_normal((B, n_k, H * 64), dtype=np.float32)
    kv = (rng.random((B, n_k)) > 0.3).astype(np.uint8)
    kv[:, -1] = 1
    return q, k, v, kv


@pytest.mark.parametrize("mask", [0, 1, 2, 3, 4])
@pytest.mark.parametrize("n", [1, 15, 16, 17, 65, 129, 144, 145, 200, 400])
def test_masks_match_oracle(ta, orc, gpu_ready, mask, n):
    B, H = 2, 3
    q, k, v, kv = _inputs(100 + n + 7 * mask, B, H, n, n)
    got = run_generic(ta, mask, q, k, v, kv, B, H, n, n, 0.125)
    want = oracle_generic(orc, mask, q, k, v, kv, B, H, n, 0.125)
    assert _ref.scaled_err(got, want) <= TOL


@pytest.mark.parametrize("mask", [0, 1, 2, 3, 4])
@pytest.mark.parametrize("n", [161, 257])
def test_single_trailing_query_and_key_match_oracle(ta, orc, gpu_ready, mask, n):
    """n = 32k + 1 with one workgroup per (series, head) in the bf16x3 kernel: the last query runs on
    the VALU at the end of the workgroup (each wave a slice of its keys, merged through LDS), and for
    the non-causal masks the last key runs on the VALU after the 32-key chunks."""
    B, H = 2, 3
    q, k, v, kv = _inputs(300 + n + 7 * mask, B, H, n, n)
    got = run_generic(ta, mask, q, k, v, kv, B, H, n, n, 0.125)
    want = oracle_generic(orc, mask, q, k, v, kv, B, H, n, 0.125)
    assert _ref.scaled_err(got, want) <= TOL


@pytest.mark.parametrize("mask", [1, 3])
def test_single_trailing_query_with_dense_bias(ta, orc, gpu_ready, mask):
    B, H, n = 2, 2, 161
    q, k, v, kv = _inputs(60 + mask, B, H, n, n)
    bias = np.random.default_rng(61).standard_normal((H, n, n)).astype(np.float32)
    got = run_generic(ta, mask, q, k, v, kv, B, H, n, n, 0.125, bias=bias, bias_head=n * n, bias_row=n)
    row = H * 64
    want = np.zeros((B, n, row), np.float32)
    orc.batched_self_attend(THREADS, mask, q, row, n * row, k, row, n * row, v, row, n * row, want, row, n * row, kv,
                            n, bias, B, H, n, 64, 0.125)
    assert _ref.scaled_err(got, want) <= TOL


def test_single_trailing_query_all_invalid_row_is_uniform(ta, orc, gpu_ready):
    """A row whose keys are all invalid (additive -FLT_MAX) keeps the reference's uniform weights in
    the single-query VALU pass and the last-key pass as in the chunks."""
    B, H, n = 2, 2, 161
    q, k, v, kv = _inputs(13, B, H, n, n)
    kv[0, :] = 0
    got = run_generic(ta, 1, q, k, v, kv, B, H, n, n, 1.0)
    want = oracle_generic(orc, 1, q, k, v, kv, B, H, n, 1.0)
    assert _ref.scaled_err(got, want) <= TOL


def test_decoder_single_trailing_query_matches_float64(ta, gpu_ready):
    """DECODER rows of 33 queries over 183 keys: the bf16x3 kernel with the last query on the VALU."""
    B, H, ne, h, l = 2, 2, 150, 33, 140
    sl = ne + h
    q, k, v, _ = _inputs(19, B, H, h, sl)
    rng = np.random.default_rng(20)
    kv = (rng.random((B, ne)) > 0.25).astype(np.uint8)
    got = run_generic(ta, 5, q, k, v, kv, B, H, h, sl, 0.125, q_pos0=ne, ctx_keys=l, chain_start=ne)
    for b in range(B):
        allowed = _ref.allowed_matrix(5, h, sl, kv[b], q_pos0=ne, ctx_keys=l, chain_start=ne)
        for hh in range(H):
            sel = slice(hh * 64, hh * 64 + 64)
            want = _ref.naive_attend(q[b, :, sel], k[b, :, sel], v[b, :, sel], allowed, 0.125)
            assert _ref.scaled_err(got[b, :, sel], want) <= TOL


@pytest.mark.parametrize("mask", [1, 3])
@pytest.mark.parametrize("n", [17, 145, 577])
def test_dense_bias_matches_oracle(ta, orc, gpu_ready, mask, n):
    """A dense additive bias [H, n, n] (the reference's bias argument of selfAttend). n = 16k + 1
    leaves one query in the last 16-query block of a workgroup: the single-query VALU path, in the
    LDS-resident kernel (17) and in the streaming one (145, 577)."""
    B, H = 2, 2
    q, k, v, kv = _inputs(40 + n + mask, B, H, n, n)
    bias = np.random.default_rng(41 + n).standard_normal((H, n, n)).astype(np.float32)
    got = run_generic(ta, mask, q, k, v, kv, B, H, n, n, 0.125, bias=bias, bias_head=n * n, bias_row=n)
    row = H * 64
    want = np.zeros((B, n, row), np.float32)
    orc.batched_self_attend(THREADS, mask, q, row, n * row, k, row, n * row, v, row, n * row, want, row, n * row, kv,
                            n, bias, B, H, n, 64, 0.125)
    assert _ref.scaled_err(got, want) <= TOL


@pytest.mark.parametrize("mask", [0, 1, 3])
def test_device_pointers_match_host_pointers(ta, gpu_ready, mask):
    B, H, n = 3, 2, 97
    q, k, v, kv = _inputs(7, B, H, n, n)
    host = run_generic(ta, mask, q, k, v, kv, B, H, n, n, 0.125)
    dev = run_generic(ta, mask, q, k, v, kv, B, H, n, n, 0.125, device=True)
    assert np.array_equal(host, dev)


@pytest.mark.parametrize("device", [False, True])
def test_padding_between_rows_is_untouched(ta, orc, gpu_ready, device):
    """o with a token stride wider than H*D: the gap keeps its sentinel (gpu_test.zig:30-34)."""
    B, H, n = 2, 2, 37
    q, k, v, kv = _inputs(8, B, H, n, n)
    got = run_generic(ta, 1, q, k, v, kv, B, H, n, n, 0.125, o_tok=H * 64 + 12, device=device)
    assert np.all(got[:, :, H * 64:] == -12345.0)
    want = oracle_generic(orc, 1, q, k, v, kv, B, H, n, 0.125)
    assert _ref.scaled_err(got[:, :, : H * 64], want) <= TOL


def test_decoder_mask_matches_float64(ta, gpu_ready):
    """DECODER rows: h queries at [ne, ne+h) over ctx keys [0, l) that are valid plus the chain."""
    B, H, ne, h, l = 3, 2, 40, 9, 34
    sl = ne + h
    q, k, v, _ = _inputs(9, B, H, h, sl)
    rng = np.random.default_rng(10)
    kv = (rng.random((B, ne)) > 0.25).astype(np.uint8)
    got = run_generic(ta, 5, q, k, v, kv, B, H, h, sl, 0.125, q_pos0=ne, ctx_keys=l, chain_start=ne)
    for b in range(B):
        allowed = _ref.allowed_matrix(5, h, sl, kv[b], q_pos0=ne, ctx_keys=l, chain_start=ne)
        for hh in range(H):
            sel = slice(hh * 64, hh * 64 + 64)
            want = _ref.naive_attend(q[b, :, sel], k[b, :, sel], v[b, :, sel], allowed, 0.125)
            assert _ref.scaled_err(got[b, :, sel], want) <= TOL


def test_causal_with_query_offset_matches_concatenated_rows(ta, orc, gpu_ready):
    """Queries [P, P+n) of causal attention over n_k = P + n keys equal rows [P, P+n) of the full
    causal selfAttend (the KV-cache identity)."""
    B, H, P, n = 2, 2, 70, 33
    q, k, v, _ = _inputs(11, B, H, P + n, P + n)
    full = oracle_generic(orc, 2, q, k, v, None, B, H, P + n, 0.125)
    got = run_generic(ta, 2, np.ascontiguousarray(q[:, P:]), k, v, None, B, H, n, P + n, 0.125, q_pos0=P)
    assert _ref.scaled_err(got, full[:, P:]) <= TOL


@pytest.mark.parametrize("n_q,n_k", [(300, 100), (145, 144), (20, 144), (1, 577)])
def test_rectangular_full_mask_matches_float64(ta, gpu_ready, n_q, n_k):
    """n_q != n_k (several query tiles over one short key row; one query over a long one),
    against float64, so both the LDS-resident (n_k <= 144) and the streaming kernel are covered."""
    B, H = 2, 2
    q, k, v, _ = _inputs(17 + n_q, B, H, n_q, n_k)
    got = run_generic(ta, 0, q, k, v, None, B, H, n_q, n_k, 0.125)
    for b in range(B):
        allowed = np.ones((n_q, n_k), bool)
        for hh in range(H):
            sel = slice(hh * 64, hh * 64 + 64)
            want = _ref.naive_attend(q[b, :, sel], k[b, :, sel], v[b, :, sel], allowed, 0.125)
            assert _ref.scaled_err(got[b, :, sel], want) <= TOL


def test_keys_additive_all_invalid_row_is_uniform(ta, orc, gpu_ready):
    B, H, n = 2, 1, 40
    q, k, v, kv = _inputs(12, B, H, n, n)
    kv[0, :] = 0
    got = run_generic(ta, 1, q, k, v, kv, B, H, n, n, 1.0)
    want = oracle_generic(orc, 1, q, k, v, kv, B, H, n, 1.0)
    assert _ref.scaled_err(got, want) <= TOL
    np.testing.assert_allclose(got[0], np.tile(v[0].mean(axis=0), (n, 1)), atol=1e-5)


# ---- family call sites -------------------------------------------------------------------------


def _c2_oracle(orc, w, B):
    """Oracle output plus the RoPE'd q and k it attended over (for the float64 reference)."""
    q = np.ascontiguousarray(w.arrays["q"][:B]).ravel().copy()
    k = np.ascontiguousarray(w.arrays["k"][:B]).ravel().copy()
    v = np.ascontiguousarray(w.arrays["v"][:B]).ravel()
    kv = np.ascontiguousarray(w.arrays["key_valid"][:B])
    d = w.H * 64
    orc.chronos2_rope(q, k, w.arrays["rope_cos"], w.arrays["rope_sin"], B * w.n_q, w.n_q, d, w.H, 64)
    o = np.zeros(B * w.n_q * d, np.float32)
    orc.chronos2_time_attention(THREADS, q, k, v, o, kv.ravel(), bool(kv.all()), B, w.n_q, d, w.H, 64, w.scale)
    shape = (B, w.n_q, d)
    return o.reshape(shape), q.reshape(shape), k.reshape(shape)


# Scale-1.0 parity. With q, k ~ N(0, 1) and D = 64 unscaled, logits have standard deviation 8 and
# the softmax amplifies last-bit differences of the 64-term dot products: the reference's own
# output moves by ~1.2e-5 between its 8-lane (AVX2) and 16-lane (AVX-512) builds on these inputs.
# The bar is _ref.reference_bar: twice the larger of that cross-host spread and the reference's
# distance from float64 (at least 1e-5), against the 16-lane build; the GPU must also be no further
# from float64 than the reference's worse build. At scale 1/8 (the benchmarked shape) the spread
# is far below 1e-5 and the bar is the 1e-5 parity target.


@pytest.mark.parametrize("scale", [0.125, 1.0])
def test_chronos2_time_attention_full_shape(ta, orc, orc16, gpu_ready, scale):
    """Chronos-2 time attention at B=64, H=12, L=577 (RoPE, left-padding mask), scale 1/sqrt(64)
    as benchmarked and 1.0 as the model calls it (src/chronos2/model.zig:306)."""
    from tsfm_attn import workloads

    w = workloads.chronos2(scale=scale)
    a = w.arrays
    o = np.zeros_like(a["q"])
    rc = ta.chronos2_time_attention(a["q"], a["k"], a["v"], o, a["rope_cos"], a["rope_sin"], a["key_valid"],
                                    bool(a["key_valid"].all()), w.B, w.n_q, w.H * 64, w.H, 64, scale=scale)
    assert rc == ta.OK, ta.last_error()
    want16, q_rot, k_rot = _c2_oracle(orc16, w, w.B)
    want8, _, _ = _c2_oracle(orc, w, w.B)
    if scale != 1.0:
        _ref.assert_within_reference_bar(o, want8, want16)
        return
    # float64 attention over the first 16 series
    gpu_f64, o8_f64, o16_f64 = _ref.f64_errors([o, want8, want16], q_rot, k_rot, a["v"], a["key_valid"], 16, w.H,
                                               w.n_q, scale)
    bar = max(_ref.reference_bar(want8, want16)[0], 2.0 * max(o8_f64, o16_f64))
    assert _ref.scaled_err(o, want16) <= bar
    assert gpu_f64 <= max(o8_f64, o16_f64), (gpu_f64, o8_f64, o16_f64)


def test_chronos2_time_attention_back_to_back_launches_agree(ta, gpu_ready):
    """The benchmarked Chronos-2 launch (B=64, H=12, L=577, RoPE, left padding) six times back to
    back on one stream, no synchronisation in between: the same bits every time (the kernel is
    deterministic, so a staged chunk read before every wave's copy landed shows up)."""
    import torch
    from tsfm_attn import workloads

    w = workloads.chronos2(scale=0.125)
    a = w.arrays
    dev = {n: torch.from_numpy(np.ascontiguousarray(a[n])).cuda() for n in ("q", "k", "v", "rope_cos", "rope_sin",
                                                                            "key_valid")}
    outs = [torch.full_like(dev["q"], -7.0) for _ in range(6)]
    for o in outs:
        assert ta.chronos2_time_attention(dev["q"], dev["k"], dev["v"], o, dev["rope_cos"], dev["rope_sin"],
                                          dev["key_valid"], bool(a["key_valid"].all()), w.B, w.n_q, w.H * 64, w.H,
                                          64, scale=0.125) == ta.OK, ta.last_error()
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o.view(torch.int32), outs[0].view(torch.int32))


def test_bolt_self_attention_full_shape(ta, orc, orc16, gpu_ready):
    """Chronos-Bolt-base encoder self-attention at B=256, H=12, L=129 with the T5 bias built on the
    device from the (32, 12) table, against the oracle's positionBias + SelfJob (scale 1.0: the
    reference-derived bar above)."""
    from tsfm_attn import workloads

    w = workloads.bolt()
    a = w.arrays
    L, H, d = w.n_q, w.H, w.H * 64
    buckets = np.zeros(2 * L - 1, np.int32)
    assert ta.load().tsfm_t5_bucket_table(buckets.ctypes.data, L, L, 32, 128) == ta.OK
    o = np.zeros_like(a["q"])
    rc = ta.bolt_self_attention(a["q"], a["k"], a["v"], o, a["rel_table"], buckets, a["key_valid"],
                                bool(a["key_valid"].all()), w.B, L, d, H, 64, 32)
    assert rc == ta.OK, ta.last_error()
    bias = orc16.position_bias(a["rel_table"], L, H, 32, 128)
    outs = []
    for o_ in (orc, orc16):
        want = np.zeros_like(a["q"])
        o_.bolt_self_attention(THREADS, a["q"], a["k"], a["v"], want, bias, a["key_valid"],
                               bool(a["key_valid"].all()), w.B, L, d, H, 64)
        outs.append(want)
    want8, want16 = outs
    gpu_f64, o8_f64, o16_f64 = _ref.f64_errors([o, want8, want16], a["q"], a["k"], a["v"], a["key_valid"], w.B, H, L,
                                               1.0, bias.reshape(H, L, L))
    bar = max(_ref.reference_bar(want8, want16)[0], 2.0 * max(o8_f64, o16_f64))
    assert _ref.scaled_err(o, want16) <= bar
    assert gpu_f64 <= max(o8_f64, o16_f64), (gpu_f64, o8_f64, o16_f64)
    # The dense-bias path (positionBias materialised by the caller) gives the same result.
    o2 = np.zeros_like(a["q"])
    ta.fwd_checked(ta.make_args(q=a["q"], k=a["k"], v=a["v"], o=o2, mask=ta.Mask.KEYS_ADDITIVE, batch=w.B, heads=H,
                                n_q=L, n_k=L, q_tok=d, q_batch=L * d, k_tok=d, k_batch=L * d, v_tok=d, v_batch=L * d,
                                o_tok=d, o_batch=L * d, scale=1.0, key_valid=a["key_valid"], kv_batch=L, bias=bias,
                                bias_head=L * L, bias_row=L))
    assert np.array_equal(o, o2)


def test_bolt_self_attention_back_to_back_launches_agree(ta, gpu_ready):
    """The benchmarked Chronos-Bolt-base launch (B=256, H=12, L=129: the single query 128 on the
    VALU before the blocks, with the second LDS stage as its scratch) six times back to back on one
    stream, no synchronisation in between: the same bits every time."""
    import torch
    from tsfm_attn import workloads

    w = workloads.bolt()
    a = w.arrays
    L, H, d = w.n_q, w.H, w.H * 64
    buckets = np.zeros(2 * L - 1, np.int32)
    assert ta.load().tsfm_t5_bucket_table(buckets.ctypes.data, L, L, 32, 128) == ta.OK
    dev = {n: torch.from_numpy(np.ascontiguousarray(a[n])).cuda() for n in ("q", "k", "v", "rel_table", "key_valid")}
    db = torch.from_numpy(buckets).cuda()
    outs = [torch.full_like(dev["q"], -7.0) for _ in range(6)]
    for o in outs:
        assert ta.bolt_self_attention(dev["q"], dev["k"], dev["v"], o, dev["rel_table"], db, dev["key_valid"],
                                      bool(a["key_valid"].all()), w.B, L, d, H, 64, 32) == ta.OK, ta.last_error()
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o.view(torch.int32), outs[0].view(torch.int32))


def test_bolt_cross_attention(ta, orc, gpu_ready):
    rng = np.random.default_rng(13)
    nb, seq, nh = 16, 33, 8
    inner = nh * 64
    q = rng.standard_normal(nb * inner).astype(np.float32)
    k = rng.standard_normal(nb * seq * inner).astype(np.float32)
    v = rng.standard_normal(nb * seq * inner).astype(np.float32)
    kv = _ref.left_pad_valid(rng, nb, seq, 10, tail_valid=1)
    o = np.zeros(nb * inner, np.float32)
    assert ta.bolt_cross_attention(q, k, v, o, kv, nb, seq, inner, nh, 64) == ta.OK, ta.last_error()
    want = np.zeros_like(o)
    orc.bolt_cross_attention(THREADS, q, k, v, want, kv.ravel(), nb, seq, inner, nh, 64)
    assert _ref.scaled_err(o, want) <= TOL


@pytest.mark.parametrize("all_valid", [True, False])
def test_timestral_time_attention_f32(ta, orc, gpu_ready, all_valid):
    """Timestral TimeJob (encoder rows causal / bidirectional for known-future rows, decoder rows
    block-causal) with per-group partial RoPE, in the fused (token, qkv, head, hd) layout."""
    rng = np.random.default_rng(14 + all_valid)
    rows, vall, ne, l, h, nh = 6, 3, 48, 40, 16, 4
    d, sl, hd = nh * 64, ne + h, 64
    qkv = rng.standard_normal(rows * sl * 3 * d).astype(np.float32)
    kv = np.ones((rows, ne), np.uint8) if all_valid else _ref.left_pad_valid(rng, rows, ne, 12)
    bidir = np.array([0, 0, 1, 0, 1, 1], np.uint8)
    first_obs = [0, 5]
    cos_t, sin_t = _ref.timestral_rope_tables(rows // vall, ne, l, h, hd, hd // 2, 10000.0, first_obs)
    o = np.zeros(rows * sl * d, np.float32)
    rc = ta.timestral_time_attention(qkv, o, cos_t, sin_t, kv, all_valid, bidir, rows, vall, ne, l, h, d, nh, hd)
    assert rc == ta.OK, ta.last_error()
    want = np.zeros_like(o)
    roped = qkv.copy()
    orc.timestral_rope(THREADS, roped, cos_t, sin_t, rows, sl, vall, d, nh, hd)
    orc.timestral_time_attention(THREADS, roped, want, kv.ravel(), all_valid, bidir, rows, ne, l, h, d, nh, hd)
    assert _ref.scaled_err(o, want) <= TOL


# ---- determinism -------------------------------------------------------------------------------


def test_repeatable_and_batch_independent(ta, gpu_ready):
    """Same bits on a repeat, and a (series, head) gives the same bits whatever else is in the batch."""
    B, H, n = 8, 3, 150
    q, k, v, kv = _inputs(15, B, H, n, n)
    a = run_generic(ta, 1, q, k, v, kv, B, H, n, n, 0.125)
    b = run_generic(ta, 1, q, k, v, kv, B, H, n, n, 0.125)
    assert np.array_equal(a, b)
    one = run_generic(ta, 1, np.ascontiguousarray(q[5:6]), np.ascontiguousarray(k[5:6]),
                      np.ascontiguousarray(v[5:6]), np.ascontiguousarray(kv[5:6]), 1, H, n, n, 0.125)
    assert np.array_equal(one[0], a[5])
