"""GPU parity of the fused Q/K/V(/gate) projection with RoPE epilogue (tsfm_qkv_project) against
the oracle's nn.linear (src/core/nn.zig:262-293) followed by the family RoPE loops
(src/chronos2/model.zig:236-245, src/timestral/model.zig:558-577), through the C ABI.

Bar: scaled error max|gpu - oracle| / max(|oracle|, 1) <= 1e-5 (the f32 tolerance). Covered: the
Chronos-2 layout (three weights, one RoPE table), the Timestral layout (the permuted fused weight,
interleaved qkv output, per-group tables with partial RoPE and negative positions, the gate),
Chronos-Bolt (no RoPE), token counts that leave a partial 128-token tile, head counts whose
columns leave a partial 128-column tile, d_in != heads * 64, padded strides (padding untouched),
host and device pointers, and the argument checks.
"""
import numpy as np
import pytest

import _ref

pytestmark = pytest.mark.gpu

TOL = 1e-5
THREADS = 16


def _weights(rng, n, d_in, count):
    return [(rng.standard_normal((n, d_in)) / np.sqrt(d_in)).astype(np.float32) for _ in range(count)]


def _linear(orc, x, w):
    y = np.zeros((x.shape[0], w.shape[0]), np.float32)
    orc.linear(THREADS, y, np.ascontiguousarray(x), x.shape[0], np.ascontiguousarray(w), w.shape[0], x.shape[1])
    return y


def _chronos2_oracle(orc, x, wq, wk, wv, cos_t, sin_t, b, seq, d, nh):
    q, k, v = (_linear(orc, x, w) for w in (wq, wk, wv))
    orc.chronos2_rope(q, k, cos_t, sin_t, b * seq, seq, d, nh, 64)
    return q, k, v


@pytest.mark.parametrize("b,seq", [(2, 77), (1, 128), (3, 200)])
def test_chronos2_projection_matches_oracle(ta, orc, gpu_ready, b, seq):
    d, nh = 768, 12
    rng = np.random.default_rng(b * 1000 + seq)
    x = rng.standard_normal((b * seq, d)).astype(np.float32)
    wq, wk, wv = _weights(rng, d, d, 3)
    cos_t, sin_t = orc.chronos2_rope_tables(seq, 64, 10000.0)
    q, k, v = (np.full((b * seq, d), -3.0, np.float32) for _ in range(3))
    rc = ta.chronos2_qkv_projection(x, wq, wk, wv, q, k, v, cos_t, sin_t, b, seq, d, nh, 64)
    assert rc == ta.OK, ta.last_error()
    want = _chronos2_oracle(orc, x, wq, wk, wv, cos_t, sin_t, b, seq, d, nh)
    for got, ref in zip((q, k, v), want):
        assert _ref.scaled_err(got, ref) <= TOL


def test_tile_shapes_give_the_same_bits(ta, orc, gpu_ready):
    """34 series of 128 tokens, 2304 output columns: 34 x 18 = 612 tiles of 128 x 128, more than two
    per CU of a 256-CU device with a last round under half full, so the first 28 token tiles take
    128 x 128 tiles and the rest 64 x 64 ones. One series alone (18 tiles) runs all in 64 x 64 tiles:
    the blocked accumulation makes its rows the same bits in either launch."""
    b, seq, d, nh = 34, 128, 768, 12
    rng = np.random.default_rng(34)
    x = rng.standard_normal((b * seq, d)).astype(np.float32)
    wq, wk, wv = _weights(rng, d, d, 3)
    cos_t, sin_t = orc.chronos2_rope_tables(seq, 64, 10000.0)
    full = [np.full((b * seq, d), -3.0, np.float32) for _ in range(3)]
    rc = ta.chronos2_qkv_projection(x, wq, wk, wv, *full, cos_t, sin_t, b, seq, d, nh, 64)
    assert rc == ta.OK, ta.last_error()
    want = _chronos2_oracle(orc, x, wq, wk, wv, cos_t, sin_t, b, seq, d, nh)
    for got, ref in zip(full, want):
        assert _ref.scaled_err(got, ref) <= TOL
    for s in (0, 20, b - 1):
        rows = slice(s * seq, (s + 1) * seq)
        one = [np.full((seq, d), -3.0, np.float32) for _ in range(3)]
        rc = ta.chronos2_qkv_projection(np.ascontiguousarray(x[rows]), wq, wk, wv, *one, cos_t, sin_t, 1, seq, d,
                                        nh, 64)
        assert rc == ta.OK, ta.last_error()
        for got, ref in zip(one, full):
            np.testing.assert_array_equal(got, ref[rows])


def test_chronos2_projection_device_pointers(ta, orc, gpu_ready):
    import torch

    b, seq, d, nh = 4, 145, 768, 12
    rng = np.random.default_rng(7)
    x = rng.standard_normal((b * seq, d)).astype(np.float32)
    wq, wk, wv = _weights(rng, d, d, 3)
    cos_t, sin_t = orc.chronos2_rope_tables(seq, 64, 10000.0)
    dev = [torch.from_numpy(a).cuda() for a in (x, wq, wk, wv, cos_t, sin_t)]
    outs = [torch.full((b * seq, d), -3.0, device="cuda") for _ in range(3)]
    rc = ta.chronos2_qkv_projection(dev[0], dev[1], dev[2], dev[3], *outs, dev[4], dev[5], b, seq, d, nh, 64)
    assert rc == ta.OK, ta.last_error()
    torch.cuda.synchronize()
    want = _chronos2_oracle(orc, x, wq, wk, wv, cos_t, sin_t, b, seq, d, nh)
    for got, ref in zip(outs, want):
        assert _ref.scaled_err(got.cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("gated", [False, True])
def test_timestral_projection_matches_oracle(ta, orc, gpu_ready, gated):
    """Fused permuted weight into the interleaved (token, qkv, head, hd) buffer, per-group RoPE
    tables (partial RoPE: rope_dim = hd / 2; positions relative to the first observed patch, so
    negative for early tokens), and the gate projection."""
    groups, vall, ne, l, h, nh = 2, 3, 30, 24, 8, 4
    d, sl, rows = nh * 64, ne + h, groups * vall
    rng = np.random.default_rng(40 + gated)
    x = rng.standard_normal((rows * sl, d)).astype(np.float32)
    w_qkv = (rng.standard_normal((3 * d, d)) / np.sqrt(d)).astype(np.float32)
    w_gate = (rng.standard_normal((d, d)) / np.sqrt(d)).astype(np.float32) if gated else None
    cos_t, sin_t = _ref.timestral_rope_tables(groups, ne, l, h, 64, 32, 10000.0, [5, 0])
    qkv = np.full((rows * sl, 3 * d), -3.0, np.float32)
    gate = np.full((rows * sl, d), -3.0, np.float32) if gated else None
    rc = ta.timestral_qkv_projection(x, w_qkv, qkv, cos_t, sin_t, rows, vall, sl, d, nh, 64, w_gate=w_gate,
                                     gate=gate)
    assert rc == ta.OK, ta.last_error()
    want = _linear(orc, x, w_qkv)
    orc.timestral_rope(THREADS, want, cos_t, sin_t, rows, sl, vall, d, nh, 64)
    assert _ref.scaled_err(qkv, want) <= TOL
    if gated:
        assert _ref.scaled_err(gate, _linear(orc, x, w_gate)) <= TOL


@pytest.mark.parametrize("nh,d_in,tokens", [(3, 96, 200), (1, 32, 5), (5, 160, 129), (12, 768, 1), (2, 48, 77), (1, 16, 3),
                                           (8, 512, 528), (2, 256, 40), (3, 512, 16), (8, 2048, 16), (1, 2048, 7)])
def test_bolt_projection_odd_shapes(ta, orc, gpu_ready, nh, d_in, tokens):
    """No RoPE (Chronos-Bolt); d_in != heads * 64; column counts 3 * nh * 64 that end in half a
    128-column tile; token counts that end in a partial 128-token tile. Two shapes have few output
    tiles and a long reduction, so the three outputs are computed as split partials summed by the
    reduce kernel: the Chronos-Bolt-small encoder's 528 tokens x 512, 40 tokens x 256, and 16 or 7
    tokens over d_in 2048 (the Chronos-Bolt-small decoder's second feed-forward product). Other
    products of at most 16 tokens take the 16-token kernel, whose sixteen waves split the
    reduction inside one workgroup: 1, 3, 5 and 16 tokens, d_in from 16 (one wave with work) to
    768."""
    inner = nh * 64
    rng = np.random.default_rng(nh * 7 + d_in + tokens)
    x = rng.standard_normal((tokens, d_in)).astype(np.float32)
    ws = _weights(rng, inner, d_in, 3)
    outs = [np.full((tokens, inner), -3.0, np.float32) for _ in range(3)]
    rc = ta.bolt_qkv_projection(x, *ws, *outs, 1, tokens, d_in, nh, 64)
    assert rc == ta.OK, ta.last_error()
    for got, w in zip(outs, ws):
        assert _ref.scaled_err(got, _linear(orc, x, w)) <= TOL


def test_padded_strides_leave_padding_untouched(ta, orc, gpu_ready):
    """x_tok > d_in and q/k/v token strides > heads * 64: only each token's own columns are written
    (src/core/gpu_test.zig:30-34 guards the same for the reference's GEMM)."""
    b, seq, d_in, nh = 2, 50, 128, 2
    width, x_tok, y_tok = nh * 64, 132, 200
    rng = np.random.default_rng(9)
    xp = rng.standard_normal((b * seq, x_tok)).astype(np.float32)
    wq, wk, wv = _weights(rng, width, d_in, 3)
    cos_t, sin_t = orc.chronos2_rope_tables(seq, 64, 10000.0)
    outs = [np.full((b * seq, y_tok), -5.0, np.float32) for _ in range(3)]
    a = ta.ProjArgs(dtype=ta.DTYPE_F32, batch=b, seq=seq, d_in=d_in, heads=nh, head_dim=64, flags=0, rope_half=32,
                    x=xp.ctypes.data, x_tok=x_tok, w_q=wq.ctypes.data, w_k=wk.ctypes.data, w_v=wv.ctypes.data,
                    q=outs[0].ctypes.data, q_tok=y_tok, k=outs[1].ctypes.data, k_tok=y_tok, v=outs[2].ctypes.data,
                    v_tok=y_tok, rope_cos=cos_t.ctypes.data, rope_sin=sin_t.ctypes.data)
    assert ta.qkv_project(a) == ta.OK, ta.last_error()
    x = np.ascontiguousarray(xp[:, :d_in])
    q, k, v = (_linear(orc, x, w) for w in (wq, wk, wv))
    qf = np.zeros((b * seq, width), np.float32)
    kf = np.zeros_like(qf)
    qf[:], kf[:] = q, k
    orc.chronos2_rope(qf, kf, cos_t, sin_t, b * seq, seq, width, nh, 64)
    for got, ref in zip(outs, (qf, kf, v)):
        assert _ref.scaled_err(got[:, :width], ref) <= TOL
        assert np.all(got[:, width:] == -5.0)


@pytest.mark.parametrize("out", ["float16", "bfloat16"])
@pytest.mark.parametrize("device", [False, True])
def test_half_outputs_round_the_f32_result(ta, orc, gpu_ready, out, device):
    """q/k/v/gate emitted in bf16 or f16 for the half-precision attention: the f32 result rounded
    once. The bound is the rounding itself (half an ulp: 2^-11 relative for f16, 2^-8 for bf16)
    plus the f32 product's own difference from the oracle."""
    import torch

    groups, vall, ne, l, h, nh = 2, 2, 40, 32, 8, 3
    d, sl, rows = nh * 64, ne + h, groups * vall
    rng = np.random.default_rng(60 + device)
    x = rng.standard_normal((rows * sl, d)).astype(np.float32)
    w_qkv = (rng.standard_normal((3 * d, d)) / np.sqrt(d)).astype(np.float32)
    w_gate = (rng.standard_normal((d, d)) / np.sqrt(d)).astype(np.float32)
    cos_t, sin_t = _ref.timestral_rope_tables(groups, ne, l, h, 64, 32, 10000.0, [3, 0])
    dt = getattr(torch, out)
    qkv = torch.full((rows * sl, 3 * d), -3.0, dtype=dt)
    gate = torch.full((rows * sl, d), -3.0, dtype=dt)
    args = [x, w_qkv, qkv, cos_t, sin_t]
    if device:
        args = [torch.from_numpy(a).cuda() if isinstance(a, np.ndarray) else a.cuda() for a in args]
        wg, gt = torch.from_numpy(w_gate).cuda(), gate.cuda()
    else:
        wg, gt = w_gate, gate
    rc = ta.timestral_qkv_projection(*args, rows, vall, sl, d, nh, 64, w_gate=wg, gate=gt)
    assert rc == ta.OK, ta.last_error()
    if device:
        torch.cuda.synchronize()
        qkv, gate = args[2].cpu(), gt.cpu()
    want = _linear(orc, x, w_qkv)
    orc.timestral_rope(THREADS, want, cos_t, sin_t, rows, sl, vall, d, nh, 64)
    rel = 2.0 ** -11 if out == "float16" else 2.0 ** -8
    for got, ref in ((qkv, want), (gate, _linear(orc, x, w_gate))):
        g = got.float().numpy()
        assert np.all(np.abs(g - ref) <= rel * np.abs(ref) + 1e-5 * np.maximum(np.abs(ref), 1.0))
        # and it is the rounding of a value within the f32 bar of the oracle
        assert _ref.scaled_err(g, torch.from_numpy(ref).to(dt).float().numpy()) <= 2 * rel


# ---- the reference backend's GEMM seam: tsfm_sgemm_nt / tsfm_weight_register ---------------------


@pytest.mark.parametrize("m,n,k,pad", [(37, 36, 48, 0), (300, 128, 160, 4), (129, 2304, 768, 0), (5, 4, 16, 8)])
def test_sgemm_nt_matches_oracle_gemm_nt(ta, orc, gpu_ready, m, n, k, pad):
    """cuda_sgemm_nt's contract (src/platform/cuda/gemm.c:316-322): C = alpha A B^T with leading
    dimensions; only the n columns of each C row are written. Against the oracle's gemmNT."""
    rng = np.random.default_rng(m + n + k)
    lda, ldb, ldc = k + pad, k + 2 * pad, n + pad
    a = rng.standard_normal(m * lda).astype(np.float32)
    b = rng.standard_normal(n * ldb).astype(np.float32)
    c = np.full(m * ldc, -9.0, np.float32)
    assert ta.sgemm_nt(m, n, k, 0.7, a, lda, b, ldb, c, ldc) == ta.OK, ta.last_error()
    want = np.zeros(m * ldc, np.float32)
    orc.gemm_nt(want, ldc, a, lda, b, ldb, m, n, k, 0.7)
    got, ref = c.reshape(m, ldc)[:, :n], want.reshape(m, ldc)[:, :n]
    assert np.all(c.reshape(m, ldc)[:, n:] == -9.0)
    # Unnormalised N(0, 1) operands: any f32 summation order is off the exact product by up to
    # k * 2^-24 * sum|a_i b_i| (the textbook bound); the oracle's order and the matrix cores' differ,
    # so both are held to that bound against float64 rather than to each other.
    A = a.reshape(m, lda)[:, :k].astype(np.float64)
    B = b.reshape(n, ldb)[:, :k].astype(np.float64)
    exact = 0.7 * A @ B.T
    bound = k * 2.0 ** -24 * 0.7 * (np.abs(A) @ np.abs(B).T) + 1e-30
    assert np.all(np.abs(got - exact) <= bound)
    assert np.all(np.abs(ref - exact) <= bound)
    # and no further from float64 than a few times the oracle (one accumulator per output against
    # the oracle's sixteen lane sums and a tree)
    assert np.abs(got - exact).max() <= 8 * np.abs(ref - exact).max() + 1e-7


@pytest.mark.parametrize("m,n,k,pad", [(1, 4, 16, 0), (33, 64, 64, 4), (129, 100, 512, 8), (577, 768, 768, 0),
                                       (200, 2304, 96, 12)])
def test_sgemm_nn_matches_oracle_gemm_nn(ta, orc, gpu_ready, m, n, k, pad):
    """cuda_sgemm_nn's contract (src/platform/cuda/gemm.c:324-330): C = A B with B row-major [k][ldb]
    (ldb any >= n, here also odd); only the n columns of each C row are written. Against the
    oracle's gemmNN and float64, the same bars as the transposed product."""
    rng = np.random.default_rng(7 * m + n + k)
    lda, ldb, ldc = k + pad, n + pad + 1, n + pad
    a = rng.standard_normal(m * lda).astype(np.float32)
    b = rng.standard_normal(k * ldb).astype(np.float32)
    c = np.full(m * ldc, -9.0, np.float32)
    assert ta.sgemm_nn(m, n, k, a, lda, b, ldb, c, ldc) == ta.OK, ta.last_error()
    want = np.zeros(m * ldc, np.float32)
    orc.gemm_nn(want, ldc, a, lda, b, ldb, m, n, k)
    got, ref = c.reshape(m, ldc)[:, :n], want.reshape(m, ldc)[:, :n]
    assert np.all(c.reshape(m, ldc)[:, n:] == -9.0)
    A = a.reshape(m, lda)[:, :k].astype(np.float64)
    B = b.reshape(k, ldb)[:, :n].astype(np.float64)
    exact = A @ B
    bound = k * 2.0 ** -24 * (np.abs(A) @ np.abs(B)) + 1e-30
    assert np.all(np.abs(got - exact) <= bound)
    assert np.all(np.abs(ref - exact) <= bound)
    assert np.abs(got - exact).max() <= 8 * np.abs(ref - exact).max() + 1e-7


def test_sgemm_nn_registered_weight_gives_the_uploaded_bits(ta, gpu_ready):
    """B registered once (Weight.handle) gives the same bits as B uploaded with the call, and a
    permutation matrix as B picks columns of A exactly (a transposed B would apply the inverse)."""
    rng = np.random.default_rng(11)
    m, n, k = 70, 48, 48
    a = rng.standard_normal((m, k)).astype(np.float32)
    perm = rng.permutation(n)
    b = np.zeros((k, n), np.float32)
    b[perm, np.arange(n)] = 1.0  # column j of A B is column perm[j] of A
    h = ta.weight_register(b)
    assert h is not None, ta.last_error()
    try:
        c1 = np.zeros((m, n), np.float32)
        c2 = np.zeros((m, n), np.float32)
        assert ta.sgemm_nn(m, n, k, a, k, b, n, c1, n, b_buf=h) == ta.OK, ta.last_error()
        assert ta.sgemm_nn(m, n, k, a, k, b, n, c2, n) == ta.OK, ta.last_error()
    finally:
        ta.weight_release(h)
    assert np.array_equal(c1, c2)
    assert np.array_equal(c1, a[:, perm])


def test_registered_weight_linear_matches_oracle(ta, orc, gpu_ready):
    """nn.linear with a registered weight (Weight.handle, src/core/nn.zig:276-283): the same result
    as with the weight uploaded per call, and as the oracle's linear."""
    rows, inp, out = 150, 768, 3072
    rng = np.random.default_rng(5)
    x = rng.standard_normal((rows, inp)).astype(np.float32)
    w = (rng.standard_normal((out, inp)) / np.sqrt(inp)).astype(np.float32)
    h = ta.weight_register(w)
    assert h is not None, ta.last_error()
    try:
        y1 = np.zeros((rows, out), np.float32)
        y2 = np.zeros((rows, out), np.float32)
        assert ta.linear(y1, x, rows, w, out, inp, w_buf=h) == ta.OK, ta.last_error()
        assert ta.linear(y2, x, rows, w, out, inp) == ta.OK, ta.last_error()
    finally:
        ta.weight_release(h)
    assert np.array_equal(y1, y2)
    assert _ref.scaled_err(y1, _linear(orc, x, w)) <= TOL


def test_presplit_operands_give_the_same_bits(ta, orc, gpu_ready):
    """A product of at least 2^30 multiply-adds through tsfm_qkv_project splits x and the weights
    into bf16 parts once (its operand workspace) and reads them with DMA; tsfm_qkv_project_noalloc
    has no such workspace and splits its tiles as it loads them. Same split, same products in the
    same order: bit-identical q/k/v, both within the bar of the oracle."""
    import torch

    b, seq, d, nh = 8, 577, 768, 12
    tokens, inner = b * seq, nh * 64
    assert tokens * 3 * inner * d >= 1 << 30
    rng = np.random.default_rng(577)
    x = rng.standard_normal((tokens, d)).astype(np.float32)
    ws = _weights(rng, inner, d, 3)
    cos_t, sin_t = orc.chronos2_rope_tables(seq, 64, 10000.0)
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    dx, dw, dc, ds = cu(x), [cu(w) for w in ws], cu(cos_t), cu(sin_t)

    def run(fn):
        outs = [torch.full((tokens, inner), -3.0, device="cuda") for _ in range(3)]
        a = ta.ProjArgs(dtype=ta.DTYPE_F32, out_dtype=ta.DTYPE_F32, batch=b, seq=seq, d_in=d, heads=nh, head_dim=64,
                        flags=ta.DEVICE_PTRS, rope_half=32, rope_rows_per_table=0, rope_row0=0, rope_table_stride=0,
                        x=dx.data_ptr(), x_tok=d, w_q=dw[0].data_ptr(), w_k=dw[1].data_ptr(), w_v=dw[2].data_ptr(),
                        w_gate=None, q=outs[0].data_ptr(), q_tok=inner, k=outs[1].data_ptr(), k_tok=inner,
                        v=outs[2].data_ptr(), v_tok=inner, gate=None, gate_tok=0, rope_cos=dc.data_ptr(),
                        rope_sin=ds.data_ptr(), stream=0)
        assert fn(a) == ta.OK, ta.last_error()
        torch.cuda.synchronize()
        return [o.cpu().numpy() for o in outs]

    pre, own = run(ta.qkv_project), run(ta.qkv_project_noalloc)
    want = _chronos2_oracle(orc, x, *ws, cos_t, sin_t, b, seq, d, nh)
    for got, alt, ref in zip(pre, own, want):
        np.testing.assert_array_equal(got, alt)
        assert _ref.scaled_err(got, ref) <= TOL


def test_presplit_product_back_to_back_launches_agree(ta, gpu_ready):
    """The benchmarked q/k/v projection (64 x 577 tokens, d 768, RoPE: 256 x 128 tiles staged by
    DMA in two LDS stages, then the rows past them) four times back to back on one stream, no
    synchronisation in between: the same bits every time (a stage read before its copies landed
    would show up)."""
    import torch

    b, seq, d, nh = 64, 577, 768, 12
    tokens, inner = b * seq, nh * 64
    rng = np.random.default_rng(64577)
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    dx = cu(rng.standard_normal((tokens, d)).astype(np.float32))
    dw = [cu(w) for w in _weights(rng, inner, d, 3)]
    cos_t = np.cos(np.outer(np.arange(seq), 10000.0 ** (-np.arange(32) / 32))).astype(np.float32)
    sin_t = np.sin(np.outer(np.arange(seq), 10000.0 ** (-np.arange(32) / 32))).astype(np.float32)
    dc, ds = cu(cos_t), cu(sin_t)
    runs = []
    for _ in range(4):
        outs = [torch.full((tokens, inner), -3.0, device="cuda") for _ in range(3)]
        a = ta.ProjArgs(dtype=ta.DTYPE_F32, out_dtype=ta.DTYPE_F32, batch=b, seq=seq, d_in=d, heads=nh, head_dim=64,
                        flags=ta.DEVICE_PTRS, rope_half=32, rope_rows_per_table=0, rope_row0=0, rope_table_stride=0,
                        x=dx.data_ptr(), x_tok=d, w_q=dw[0].data_ptr(), w_k=dw[1].data_ptr(), w_v=dw[2].data_ptr(),
                        w_gate=None, q=outs[0].data_ptr(), q_tok=inner, k=outs[1].data_ptr(), k_tok=inner,
                        v=outs[2].data_ptr(), v_tok=inner, gate=None, gate_tok=0, rope_cos=dc.data_ptr(),
                        rope_sin=ds.data_ptr(), stream=0)
        assert ta.qkv_project(a) == ta.OK, ta.last_error()
        runs.append(outs)
    torch.cuda.synchronize()
    for outs in runs[1:]:
        for got, first in zip(outs, runs[0]):
            assert torch.equal(got.view(torch.int32), first.view(torch.int32))
