"""Pins the CPU oracle (oracle/tsfm_oracle.c) before it is trusted as the GPU checker.

Each oracle function is checked against at least one of: the reference's golden vectors
(tests/golden/*.json), the reference's own known-answer test restated (every mask, with and
without bias, against a float64 naive reference: src/core/attn.zig:156-189), an independent
float64 numpy formulation (tests/_ref.py), or a closed form / invariant chosen so that a plausible
slip (dropped scale, j < i instead of j <= i, bias after mask, transposed operand, wrong RoPE pair)
fails.
"""
import json
import pathlib

import numpy as np
import pytest

import _ref
from _oracle import ORC_CAUSAL, ORC_CAUSAL_KEYS, ORC_FULL, ORC_FULL_KEYS, ORC_KEYS_ADDITIVE

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
MASKS = [ORC_FULL, ORC_KEYS_ADDITIVE, ORC_CAUSAL, ORC_CAUSAL_KEYS, ORC_FULL_KEYS]


# ---- golden vectors ----------------------------------------------------------------------------


def test_relative_bucket_golden(orc):
    g = json.loads((GOLDEN / "t5_buckets_32_128.json").read_text())
    got = [orc.relative_bucket(g["rel_first"] + i, g["num_buckets"], g["max_distance"]) for i in range(len(g["buckets"]))]
    assert got == g["buckets"]


def test_mask_pick_truth_table(orc):
    g = json.loads((GOLDEN / "mask_pick.json").read_text())
    names = {"full": ORC_FULL, "keys_additive": ORC_KEYS_ADDITIVE, "causal": ORC_CAUSAL,
             "causal_keys": ORC_CAUSAL_KEYS, "full_keys": ORC_FULL_KEYS}
    for c in g["cases"]:
        assert orc.mask_pick(c["causal"], c["all_keys_valid"], c["additive"]) == names[c["mask"]]


# ---- the reference's known-answer test (src/core/attn.zig:156-189) ------------------------------


def _kat_inputs():
    n, hd = 11, 8
    ld = 3 * hd + 2  # fused-qkv-like stride with padding
    rng = np.random.default_rng(0x7A11)
    qkv = (rng.random(n * ld, dtype=np.float32) * 2 - 1).astype(np.float32)
    key_valid = np.array([i % 3 != 1 for i in range(n)], np.uint8)
    bias = (rng.random(n * n, dtype=np.float32) * 4 - 2).astype(np.float32)
    return n, hd, ld, qkv, key_valid, bias


@pytest.mark.parametrize("mask", MASKS)
@pytest.mark.parametrize("with_bias", [False, True])
def test_self_attend_matches_f64_reference(orc, mask, with_bias):
    n, hd, ld, qkv, key_valid, bias = _kat_inputs()
    st = (ld, ld, ld, hd)
    q, k, v = qkv[0:], qkv[hd:], qkv[2 * hd:]
    got = np.zeros(n * hd, np.float32)
    orc.self_attend(mask, q, k, v, got, st, n, hd, 0.35, key_valid, bias if with_bias else None)
    want = orc.reference_attend_f64(mask, q, k, v, st, n, hd, 0.35, key_valid, bias if with_bias else None)
    np.testing.assert_allclose(got.reshape(n, hd), want, atol=1e-4, rtol=0)
    # And the float64 reference itself against the independent numpy formulation.
    Q = np.stack([qkv[i * ld: i * ld + hd] for i in range(n)])
    K = np.stack([qkv[i * ld + hd: i * ld + 2 * hd] for i in range(n)])
    V = np.stack([qkv[i * ld + 2 * hd: i * ld + 3 * hd] for i in range(n)])
    np_ref = _ref.naive_attend(Q, K, V, _ref.allowed_matrix(mask, n, n, key_valid), 0.35,
                               bias.reshape(n, n) if with_bias else None)
    np.testing.assert_allclose(want, np_ref, atol=1e-12, rtol=0)


@pytest.mark.parametrize("mask", MASKS)
def test_self_attend_head_sized(orc, mask):
    """Head-sized case (n = 129, hd = 64, the Chronos-Bolt shape) at the f32 tolerance."""
    rng = np.random.default_rng(1)
    n, hd, ld = 129, 64, 3 * 64
    qkv = rng.standard_normal(n * ld).astype(np.float32)
    kv = (rng.random(n) > 0.3).astype(np.uint8)
    kv[-1] = 1
    bias = (rng.standard_normal(n * n) * 0.5).astype(np.float32)
    got = np.zeros(n * hd, np.float32)
    orc.self_attend(mask, qkv[0:], qkv[hd:], qkv[2 * hd:], got, (ld, ld, ld, hd), n, hd, 0.125, kv, bias)
    Q = qkv.reshape(n, ld)[:, :hd]
    K = qkv.reshape(n, ld)[:, hd:2 * hd]
    V = qkv.reshape(n, ld)[:, 2 * hd:]
    want = _ref.naive_attend(Q, K, V, _ref.allowed_matrix(mask, n, n, kv), 0.125, bias.reshape(n, n))
    assert _ref.scaled_err(got.reshape(n, hd), want) < 2e-6


# ---- closed forms and invariants ---------------------------------------------------------------


def _qkv(rng, n, hd):
    return [rng.standard_normal(n * hd).astype(np.float32) for _ in range(3)]


@pytest.mark.parametrize("mask", MASKS)
def test_single_key_returns_v(orc, mask):
    """Softmax over one key is exactly 1, so o == v bit for bit (src/chronos2/model.zig:264-269)."""
    rng = np.random.default_rng(2)
    q, k, v = _qkv(rng, 1, 64)
    o = np.zeros(64, np.float32)
    orc.self_attend(mask, q, k, v, o, (64, 64, 64, 64), 1, 64, 0.7, np.ones(1, np.uint8), None)
    assert np.array_equal(o, v)


def test_zero_query_gives_mean_of_allowed_values(orc):
    rng = np.random.default_rng(3)
    n, hd = 37, 64
    _, k, v = _qkv(rng, n, hd)
    q = np.zeros(n * hd, np.float32)
    kv = (rng.random(n) > 0.5).astype(np.uint8)
    kv[0] = 1
    for mask in (ORC_FULL, ORC_FULL_KEYS):
        o = np.zeros(n * hd, np.float32)
        orc.self_attend(mask, q, k, v, o, (hd,) * 4, n, hd, 1.0, kv, None)
        V = v.reshape(n, hd)
        for i in (0, 5, n - 1):
            sel = np.ones(n, bool) if mask == ORC_FULL else (kv.astype(bool) | (np.arange(n) == i))
            np.testing.assert_allclose(o.reshape(n, hd)[i], V[sel].mean(axis=0), atol=2e-6)


def test_constant_values_pass_through(orc):
    rng = np.random.default_rng(4)
    n, hd = 50, 64
    q, k, _ = _qkv(rng, n, hd)
    row = rng.standard_normal(hd).astype(np.float32)
    v = np.tile(row, n)
    for mask in MASKS:
        o = np.zeros(n * hd, np.float32)
        orc.self_attend(mask, q, k, v, o, (hd,) * 4, n, hd, 0.125, np.ones(n, np.uint8), None)
        np.testing.assert_allclose(o.reshape(n, hd), np.tile(row, (n, 1)), rtol=2e-6, atol=2e-6)


def test_causal_first_row_is_v0(orc):
    rng = np.random.default_rng(5)
    n, hd = 20, 64
    q, k, v = _qkv(rng, n, hd)
    o = np.zeros(n * hd, np.float32)
    orc.self_attend(ORC_CAUSAL, q, k, v, o, (hd,) * 4, n, hd, 0.3, None, None)
    assert np.array_equal(o[:hd], v[:hd])


@pytest.mark.parametrize("mask", [ORC_CAUSAL_KEYS, ORC_FULL_KEYS, ORC_KEYS_ADDITIVE])
def test_masked_keys_carry_no_weight(orc, mask):
    """-inf keys get exactly zero weight, -FLT_MAX keys ~1e-38: perturbing their k and v leaves o
    unchanged bit for bit."""
    rng = np.random.default_rng(6)
    n, hd = 33, 64
    q, k, v = _qkv(rng, n, hd)
    kv = (rng.random(n) > 0.4).astype(np.uint8)
    kv[-1] = 1
    o1 = np.zeros(n * hd, np.float32)
    orc.self_attend(mask, q, k, v, o1, (hd,) * 4, n, hd, 0.125, kv, None)
    k2, v2 = k.copy().reshape(n, hd), v.copy().reshape(n, hd)
    bad = np.where(kv == 0)[0]
    k2[bad] += 3.0
    v2[bad] *= -7.0
    o2 = np.zeros(n * hd, np.float32)
    orc.self_attend(mask, q, k2.ravel(), v2.ravel(), o2, (hd,) * 4, n, hd, 0.125, kv, None)
    rows = [i for i in range(n) if mask == ORC_KEYS_ADDITIVE or kv[i]]  # diagonal rows read themselves
    assert np.array_equal(o1.reshape(n, hd)[rows], o2.reshape(n, hd)[rows])


def test_keys_additive_all_invalid_is_uniform(orc):
    """With every key invalid each score becomes -FLT_MAX and softmax is uniform over all keys."""
    rng = np.random.default_rng(7)
    n, hd = 9, 64
    q, k, v = _qkv(rng, n, hd)
    o = np.zeros(n * hd, np.float32)
    orc.self_attend(ORC_KEYS_ADDITIVE, q, k, v, o, (hd,) * 4, n, hd, 1.0, np.zeros(n, np.uint8), None)
    np.testing.assert_allclose(o.reshape(n, hd), np.tile(v.reshape(n, hd).mean(axis=0), (n, 1)), atol=2e-6)


def test_key_permutation_invariance(orc):
    rng = np.random.default_rng(8)
    n, hd = 40, 64
    q, k, v = _qkv(rng, n, hd)
    perm = rng.permutation(n)
    o1 = np.zeros(n * hd, np.float32)
    o2 = np.zeros(n * hd, np.float32)
    orc.self_attend(ORC_FULL, q, k, v, o1, (hd,) * 4, n, hd, 0.125, None, None)
    orc.self_attend(ORC_FULL, q, k.reshape(n, hd)[perm].ravel(), v.reshape(n, hd)[perm].ravel(), o2, (hd,) * 4, n,
                    hd, 0.125, None, None)
    np.testing.assert_allclose(o1, o2, atol=2e-6)


def test_bias_shifts_scores_before_softmax(orc):
    """A bias that is constant along each row leaves softmax unchanged; a bias of +50 on one key
    makes that key dominate (a bias applied after the softmax would fail both)."""
    rng = np.random.default_rng(9)
    n, hd = 16, 64
    q, k, v = _qkv(rng, n, hd)
    base = np.zeros(n * hd, np.float32)
    orc.self_attend(ORC_FULL, q, k, v, base, (hd,) * 4, n, hd, 0.125, None, None)
    rowconst = np.repeat(rng.standard_normal(n).astype(np.float32), n)
    o = np.zeros(n * hd, np.float32)
    orc.self_attend(ORC_FULL, q, k, v, o, (hd,) * 4, n, hd, 0.125, None, rowconst)
    np.testing.assert_allclose(o, base, atol=2e-6)
    spike = np.zeros((n, n), np.float32)
    spike[:, 3] = 50.0
    orc.self_attend(ORC_FULL, q, k, v, o, (hd,) * 4, n, hd, 0.125, None, spike.ravel())
    np.testing.assert_allclose(o.reshape(n, hd), np.tile(v.reshape(n, hd)[3], (n, 1)), atol=1e-5)


# ---- nn.zig primitives -------------------------------------------------------------------------


def test_exp_vec_accuracy_and_clamp(orc):
    xs = np.concatenate([np.linspace(-87.0, 0.0, 4001), np.linspace(0, 80, 801)]).astype(np.float32)
    got = np.array([orc.exp_vec(x) for x in xs], np.float64)
    want = np.exp(xs.astype(np.float64))
    assert np.max(np.abs(got - want) / want) < 3e-7  # about 2 ulp
    assert orc.exp_vec(0.0) == np.float32(1.0)
    assert orc.exp_vec(-1e9) == orc.exp_vec(-87.33654)  # clamped to the smallest normal range
    assert 1.0e-38 < float(orc.exp_vec(-1e9)) < 1.3e-38


@pytest.mark.parametrize("n", [1, 7, 8, 16, 17, 129, 577])
def test_softmax(orc, n):
    rng = np.random.default_rng(10 + n)
    row = (rng.standard_normal(n) * 4).astype(np.float32)
    if n > 3:
        row[[1, n - 2]] = -np.inf
    x = row.copy()
    orc.softmax(x)
    r64 = row.astype(np.float64)
    e = np.where(np.isinf(r64), 0.0, np.exp(r64 - r64.max()))
    np.testing.assert_allclose(x, e / e.sum(), atol=1e-7, rtol=3e-6)
    assert np.all(x[np.isinf(row)] == 0.0)


def test_gemm_nt_and_tiling_independence(orc):
    rng = np.random.default_rng(11)
    m, n, k, lda, ldb, ldc = 37, 29, 71, 75, 80, 33
    a = rng.standard_normal(m * lda).astype(np.float32)
    b = rng.standard_normal(n * ldb).astype(np.float32)
    c = np.full(m * ldc, -12345.0, np.float32)
    orc.gemm_nt(c, ldc, a, lda, b, ldb, m, n, k, 0.7)
    A = a.reshape(m, lda)[:, :k].astype(np.float64)
    B = b.reshape(n, ldb)[:, :k].astype(np.float64)
    np.testing.assert_allclose(c.reshape(m, ldc)[:, :n], 0.7 * A @ B.T, atol=1e-4, rtol=1e-5)
    assert np.all(c.reshape(m, ldc)[:, n:] == -12345.0)  # padding untouched (gpu_test.zig:30-34)
    # Each output depends only on its own row and column: row-by-row calls are bit-identical.
    c1 = np.zeros(ldc, np.float32)
    for i in (0, 1, m - 1):
        orc.gemm_nt(c1, ldc, a[i * lda:], lda, b, ldb, 1, n, k, 0.7)
        assert np.array_equal(c1[:n], c.reshape(m, ldc)[i, :n])


def test_gemm_nn_skips_zero_probabilities(orc):
    rng = np.random.default_rng(12)
    m, n, k = 13, 64, 41
    a = rng.random((m, k)).astype(np.float32)
    a[:, ::3] = 0.0
    b = rng.standard_normal((k, n)).astype(np.float32)
    c = np.zeros((m, n), np.float32)
    orc.gemm_nn(c, n, a, k, b, n, m, n, k)
    np.testing.assert_allclose(c, a.astype(np.float64) @ b.astype(np.float64), atol=1e-5, rtol=1e-5)
    b2 = b.copy()
    b2[::3] = np.nan  # rows of B with an all-zero A column are never read
    c2 = np.zeros((m, n), np.float32)
    orc.gemm_nn(c2, n, a, k, b2, n, m, n, k)
    assert np.array_equal(c, c2)


def test_dot_matches_f64(orc):
    rng = np.random.default_rng(13)
    a = rng.standard_normal(67).astype(np.float32)
    b = rng.standard_normal(67).astype(np.float32)
    assert abs(float(orc.dot(a, b)) - float(a.astype(np.float64) @ b.astype(np.float64))) < 1e-5


def test_rope_invariants(orc):
    """RoPE preserves each pair's norm and makes q.k depend only on the position difference."""
    hd, seq = 64, 40
    cos_t, sin_t = orc.chronos2_rope_tables(seq, hd, 10000.0)
    np.testing.assert_allclose(cos_t.astype(np.float64) ** 2 + sin_t.astype(np.float64) ** 2, 1.0, atol=1e-6)
    inv = 1.0 / 10000.0 ** (np.arange(0, hd, 2, dtype=np.float64) / hd)
    np.testing.assert_allclose(cos_t.reshape(seq, hd // 2), np.cos(np.outer(np.arange(seq), inv)), atol=3e-6)
    rng = np.random.default_rng(14)
    q0 = rng.standard_normal(hd).astype(np.float32)
    k0 = rng.standard_normal(hd).astype(np.float32)

    def rot(x, pos):
        y = x.copy()
        orc.rope_half(y, cos_t[pos * 32:], sin_t[pos * 32:], 32)
        return y

    for p in (0, 3, 17):
        y = rot(q0, p)
        np.testing.assert_allclose(y[:32] ** 2 + y[32:] ** 2, q0[:32] ** 2 + q0[32:] ** 2, rtol=1e-5, atol=1e-6)
    d1 = float(rot(q0, 10) @ rot(k0, 4))
    d2 = float(rot(q0, 20) @ rot(k0, 14))
    d3 = float(rot(q0, 6) @ rot(k0, 0))
    assert abs(d1 - d2) < 1e-4 and abs(d1 - d3) < 1e-4
    assert abs(d1 - float(q0 @ k0)) > 1e-3  # rotation is not the identity


def test_position_bias_layout(orc):
    rng = np.random.default_rng(15)
    table = _ref.t5_bias_table(rng, 32, 12)
    seq = 21
    bias = orc.position_bias(table, seq, 12, 32, 128).reshape(12, seq, seq)
    for h in (0, 7):
        for i, j in ((0, 0), (3, 15), (20, 1)):
            assert bias[h, i, j] == table[orc.relative_bucket(j - i, 32, 128), h]


# ---- family jobs -------------------------------------------------------------------------------


def test_bolt_cross_attention(orc):
    rng = np.random.default_rng(16)
    nb, seq, nh, hd = 3, 33, 8, 64
    inner = nh * hd
    q = rng.standard_normal(nb * inner).astype(np.float32)
    k = rng.standard_normal(nb * seq * inner).astype(np.float32)
    v = rng.standard_normal(nb * seq * inner).astype(np.float32)
    kv = _ref.left_pad_valid(rng, nb, seq, 10, tail_valid=1)
    o = np.zeros(nb * inner, np.float32)
    orc.bolt_cross_attention(2, q, k, v, o, kv.ravel(), nb, seq, inner, nh, hd)
    for r in range(nb):
        for h in range(nh):
            Q = q.reshape(nb, nh, hd)[r, h][None]
            K = k.reshape(nb, seq, nh, hd)[r, :, h]
            V = v.reshape(nb, seq, nh, hd)[r, :, h]
            want = _ref.naive_attend(Q, K, V, kv[r][None].astype(bool), 1.0)
            assert _ref.scaled_err(o.reshape(nb, nh, hd)[r, h], want[0]) < 2e-6


def test_bolt_self_attention(orc):
    rng = np.random.default_rng(17)
    nb, seq, nh, hd = 2, 33, 4, 64
    inner = nh * hd
    q, k, v = (rng.standard_normal(nb * seq * inner).astype(np.float32) for _ in range(3))
    table = _ref.t5_bias_table(rng, 32, nh)
    bias = orc.position_bias(table, seq, nh, 32, 128)
    kv = _ref.left_pad_valid(rng, nb, seq, 8, tail_valid=1)
    o = np.zeros(nb * seq * inner, np.float32)
    orc.bolt_self_attention(2, q, k, v, o, bias, kv.ravel(), False, nb, seq, inner, nh, hd)
    B3 = bias.reshape(nh, seq, seq)
    for r in range(nb):
        for h in range(nh):
            sl = lambda x: x.reshape(nb, seq, nh, hd)[r, :, h]  # noqa: E731
            want = _ref.naive_attend(sl(q), sl(k), sl(v), _ref.allowed_matrix(1, seq, seq, kv[r]), 1.0, B3[h])
            # Unscaled T5 scores reach |s| ~ 30: f32 rounding of s alone gives ~2e-6 here.
            assert _ref.scaled_err(sl(o), want) < 5e-6


def test_chronos2_time_attention_and_threads(orc):
    rng = np.random.default_rng(18)
    b, seq, nh, hd = 2, 45, 3, 64
    d = nh * hd
    q, k, v = (rng.standard_normal(b * seq * d).astype(np.float32) for _ in range(3))
    kv = _ref.left_pad_valid(rng, b, seq, 10, tail_valid=5)
    cos_t, sin_t = orc.chronos2_rope_tables(seq, hd)
    qr, kr = q.copy(), k.copy()
    orc.chronos2_rope(qr, kr, cos_t, sin_t, b * seq, seq, d, nh, hd)
    o1 = np.zeros_like(q)
    o4 = np.zeros_like(q)
    orc.chronos2_time_attention(1, qr, kr, v, o1, kv.ravel(), False, b, seq, d, nh, hd, 0.125)
    orc.chronos2_time_attention(4, qr, kr, v, o4, kv.ravel(), False, b, seq, d, nh, hd, 0.125)
    assert np.array_equal(o1, o4)  # thread count is bit-identical (README.md:282)
    # RoPE applied with numpy from the same tables, then the float64 reference.
    C = cos_t.reshape(seq, hd // 2).astype(np.float64)
    S = sin_t.reshape(seq, hd // 2).astype(np.float64)

    def rope64(x):
        lo, hi = x[:, :32], x[:, 32:]
        return np.concatenate([lo * C - hi * S, hi * C + lo * S], axis=1)

    for r in range(b):
        for h in range(nh):
            sl = lambda x: x.reshape(b, seq, nh, hd)[r, :, h].astype(np.float64)  # noqa: E731
            want = _ref.naive_attend(rope64(sl(q)), rope64(sl(k)), sl(v), _ref.allowed_matrix(1, seq, seq, kv[r]), 0.125)
            assert _ref.scaled_err(sl(o1), want) < 2e-6


@pytest.mark.parametrize("all_valid", [True, False])
def test_timestral_time_attention(orc, all_valid):
    rng = np.random.default_rng(19 + all_valid)
    rows, vall, ne, l, h, nh, hd = 4, 2, 24, 24, 6, 2, 64
    d = nh * hd
    sl = ne + h
    qkv = rng.standard_normal(rows * sl * 3 * d).astype(np.float32)
    kv = np.ones((rows, ne), np.uint8) if all_valid else _ref.left_pad_valid(rng, rows, ne, 6)
    bidir = np.array([0, 1, 0, 0], np.uint8)
    o = np.zeros(rows * sl * d, np.float32)
    orc.timestral_time_attention(2, qkv, o, kv.ravel(), all_valid, bidir, rows, ne, l, h, d, nh, hd)
    X = qkv.reshape(rows, sl, 3, nh, hd).astype(np.float64)
    O = o.reshape(rows, sl, nh, hd)
    for r in range(rows):
        for hh in range(nh):
            Q, K, V = X[r, :, 0, hh], X[r, :, 1, hh], X[r, :, 2, hh]
            enc_mask = (4 if bidir[r] else 3) if not all_valid else (0 if bidir[r] else 2)
            want = _ref.naive_attend(Q[:ne], K[:ne], V[:ne], _ref.allowed_matrix(enc_mask, ne, ne, kv[r]), 0.125)
            assert _ref.scaled_err(O[r, :ne, hh], want) < 2e-6
            dec = _ref.allowed_matrix(5, h, sl, np.concatenate([kv[r], np.ones(h, np.uint8)]), q_pos0=ne, ctx_keys=l,
                                      chain_start=ne)
            want = _ref.naive_attend(Q[ne:], K, V, dec, 0.125)
            assert _ref.scaled_err(O[r, ne:, hh], want) < 2e-6


def test_lane_counts_agree(orc, orc16):
    assert (orc.lanes, orc16.lanes) == (8, 16)
    rng = np.random.default_rng(21)
    n, hd = 70, 64
    q, k, v = _qkv(rng, n, hd)
    kv = (rng.random(n) > 0.2).astype(np.uint8)
    for mask in MASKS:
        o8 = np.zeros(n * hd, np.float32)
        o16 = np.zeros(n * hd, np.float32)
        orc.self_attend(mask, q, k, v, o8, (hd,) * 4, n, hd, 0.125, kv, None)
        orc16.self_attend(mask, q, k, v, o16, (hd,) * 4, n, hd, 0.125, kv, None)
        assert _ref.scaled_err(o16, o8) < 1e-6


@pytest.mark.parametrize("mask", MASKS)
@pytest.mark.parametrize("with_bias", [False, True])
def test_batched_self_attend_matches_f64_per_item(orc, mask, with_bias):
    """orc_batched_self_attend, the oracle of every generic-mask GPU test, on its own: each
    (series, head) item against float64 attention over that item's own slices. Odd token and batch
    strides that differ per tensor, a bias that differs per head, key validity that differs per
    series (one series all invalid), threads over the items; a wrong batch or head offset, a shared
    bias slice or one series' validity applied to another fails. Padding between views stays
    untouched."""
    rng = np.random.default_rng(40 + mask + 10 * with_bias)
    nb, nh, n, hd, scale = 3, 2, 23, 64, 0.21
    q_tok, k_tok, v_tok, o_tok = nh * hd + 3, nh * hd + 5, 2 * nh * hd + 1, nh * hd + 7
    q_b, k_b, v_b, o_b = n * q_tok + 11, n * k_tok + 2, n * v_tok + 9, n * o_tok + 13
    q = rng.standard_normal(nb * q_b).astype(np.float32)
    k = rng.standard_normal(nb * k_b).astype(np.float32)
    v = rng.standard_normal(nb * v_b).astype(np.float32)
    kv_b = n + 4
    kv = (rng.random(nb * kv_b) > 0.35).astype(np.uint8)
    kv[kv_b: kv_b + n] = 0  # series 1: no valid key
    bias = (rng.standard_normal(nh * n * n) * 0.7).astype(np.float32) if with_bias else None
    sentinel = np.float32(-777.25)
    o = np.full(nb * o_b, sentinel, np.float32)
    orc.batched_self_attend(3, mask, q, q_tok, q_b, k, k_tok, k_b, v, v_tok, v_b, o, o_tok, o_b, kv, kv_b, bias, nb, nh,
                            n, hd, scale)
    written = np.zeros(o.size, bool)
    for b in range(nb):
        for h in range(nh):
            rows = lambda x, tok, bat: np.stack([x[b * bat + t * tok + h * hd:][:hd] for t in range(n)])
            Q, K, V = rows(q, q_tok, q_b), rows(k, k_tok, k_b), rows(v, v_tok, v_b)
            allowed = _ref.allowed_matrix(mask, n, n, kv[b * kv_b: b * kv_b + n])
            want = _ref.naive_attend(Q, K, V, allowed, scale, None if bias is None else bias[h * n * n:][:n * n].reshape(n, n))
            got = rows(o, o_tok, o_b)
            assert _ref.scaled_err(got, want) < 2e-6, (b, h)
            for t in range(n):
                written[b * o_b + t * o_tok + h * hd:][:hd] = True
    assert (o[~written] == sentinel).all()


# ---- Timestral variate attention (VariateJob.run, src/timestral/model.zig:648-709) -------------


def _variate_inputs(seed, groups, vall, ne, h, d, p_valid=0.7):
    rng = np.random.default_rng(seed)
    sl = ne + h
    qkv = rng.standard_normal((groups * vall, sl, 3 * d)).astype(np.float32)
    kv = (rng.random((groups * vall, ne)) < p_valid).astype(np.uint8)
    return qkv, kv


@pytest.mark.parametrize("vall,cov", [(1, False), (3, False), (5, True), (8, True), (24, True), (33, False)])
def test_variate_attention_matches_f64(orc, vall, cov):
    groups, ne, h, nh, hd = 3, 9, 4, 2, 16
    d = nh * hd
    qkv, kv = _variate_inputs(vall, groups, vall, ne, h, d)
    roles = np.array(([_ref.ROLE_TARGET, _ref.ROLE_PAST, _ref.ROLE_KNOWN] * 11)[:vall], np.uint8)
    o = np.zeros((groups * vall, ne + h, d), np.float32)
    orc.timestral_variate_attention(4, qkv, o, kv, roles, cov, groups, vall, ne, h, d, nh, hd)
    want = _ref.variate_attend_f64(qkv, kv, roles, cov, groups, vall, ne, h, d, nh, hd)
    assert _ref.scaled_err(o, want) <= 1e-5


def test_variate_singleton_is_v(orc):
    """vall = 1: every row reads only itself, so o = v exactly (a singleton series pins the gather without any softmax arithmetic)."""
    groups, ne, h, nh, hd = 4, 7, 3, 2, 16
    d = nh * hd
    qkv, kv = _variate_inputs(1, groups, 1, ne, h, d, p_valid=0.0)
    o = np.zeros((groups, ne + h, d), np.float32)
    orc.timestral_variate_attention(2, qkv, o, kv, np.zeros(1, np.uint8), False, groups, 1, ne, h, d, nh, hd)
    assert np.array_equal(o, qkv[:, :, 2 * d:])


def test_variate_firewalls_and_validity(orc):
    """What a row may not read does not move its output: with covariates, past/known rows ignore
    the target row; known rows ignore past rows; on encoder slots an invalid key row is ignored,
    on decoder slots (tok >= ne) it is read."""
    groups, vall, ne, h, nh, hd = 1, 4, 6, 3, 2, 16
    d = nh * hd
    roles = np.array([_ref.ROLE_TARGET, _ref.ROLE_PAST, _ref.ROLE_KNOWN, _ref.ROLE_KNOWN], np.uint8)
    qkv, kv = _variate_inputs(11, groups, vall, ne, h, d, p_valid=1.0)
    kv[3, 2] = 0  # row 3 is not a valid key at slot 2

    def run(x):
        o = np.zeros((vall, ne + h, d), np.float32)
        orc.timestral_variate_attention(1, x, o, kv, roles, True, groups, vall, ne, h, d, nh, hd)
        return o

    base = run(qkv)
    bumped = qkv.copy()
    bumped[0, :, d:] += 3.0  # the target row's k and v
    o = run(bumped)
    assert np.array_equal(o[1:], base[1:]) and not np.array_equal(o[0], base[0])
    bumped = qkv.copy()
    bumped[1, :, d:] += 3.0  # the past row's k and v: the target reads it, known rows do not
    o = run(bumped)
    assert np.array_equal(o[2:], base[2:]) and not np.array_equal(o[0], base[0])
    bumped = qkv.copy()
    bumped[3, 2, d:] += 3.0  # invalid key at encoder slot 2: only row 3 itself sees it
    o = run(bumped)
    assert np.array_equal(o[:3, 2], base[:3, 2]) and not np.array_equal(o[3, 2], base[3, 2])
    kv2 = kv.copy()
    kv2[:] = 0  # decoder slots read every row whatever key_valid says
    o2 = np.zeros((vall, ne + h, d), np.float32)
    orc.timestral_variate_attention(1, qkv, o2, kv2, roles, True, groups, vall, ne, h, d, nh, hd)
    assert np.array_equal(o2[:, ne:], base[:, ne:])


def test_mul_sigmoid_closed_form(orc):
    rng = np.random.default_rng(5)
    n = 37  # whole vectors and a tail
    x = rng.standard_normal(n).astype(np.float32)
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    out = np.zeros(n, np.float32)
    orc.mul_sigmoid(out, x, g)
    want = x.astype(np.float64) / (1.0 + np.exp(-g.astype(np.float64)))
    assert np.max(np.abs(out - want)) <= 1e-6 * max(1.0, np.abs(want).max())
    zero = np.zeros(n, np.float32)
    orc.mul_sigmoid(out, x, zero)
    assert np.array_equal(out, x * np.float32(0.5))  # sigmoid(0) = 1/2 exactly


def test_linear_matches_f64_and_thread_count(orc):
    """nn.linear: y = x w^T + bias, with the column blocks split over threads above 2^20 products."""
    rng = np.random.default_rng(21)
    rows, inp, out = 40, 160, 200  # 1.28e6 products: the threaded column-block path
    x = rng.standard_normal((rows, inp)).astype(np.float32)
    w = (rng.standard_normal((out, inp)) / np.sqrt(inp)).astype(np.float32)
    bias = rng.standard_normal(out).astype(np.float32)
    y1 = np.zeros((rows, out), np.float32)
    orc.linear(1, y1, x, rows, w, out, inp, bias)
    want = x.astype(np.float64) @ w.astype(np.float64).T + bias
    assert np.max(np.abs(y1 - want) / np.maximum(np.abs(want), 1.0)) < 5e-6
    for threads in (3, 8):  # blocks of 16 columns: the result does not depend on the split
        y = np.zeros_like(y1)
        orc.linear(threads, y, x, rows, w, out, inp, bias)
        assert np.array_equal(y, y1)
    small = np.zeros((3, 24), np.float32)  # below the threshold: one linearCols call
    orc.linear(4, small, x[:3], 3, w[:24], 24, inp)
    want_small = x[:3].astype(np.float64) @ w[:24].astype(np.float64).T
    assert np.max(np.abs(small - want_small)) < 5e-6


def test_linear_permutation_weight_is_exact(orc):
    """A permutation weight picks columns of x exactly: y[:, j] = x[:, perm[j]] (a transposed
    operand would apply the inverse permutation)."""
    rng = np.random.default_rng(22)
    rows, n = 9, 48
    x = rng.standard_normal((rows, n)).astype(np.float32)
    perm = rng.permutation(n)
    w = np.zeros((n, n), np.float32)
    w[np.arange(n), perm] = 1.0
    y = np.zeros((rows, n), np.float32)
    orc.linear(2, y, x, rows, w, n, n)
    assert np.array_equal(y, x[:, perm])
    assert not np.array_equal(y, x[:, np.argsort(perm)])


def test_rms_norm_matches_definition(orc):
    rng = np.random.default_rng(31)
    rows, dim = 70, 100  # whole lane groups and a tail
    x = (rng.standard_normal((rows, dim)) * 3).astype(np.float32)
    scale = (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
    out = np.zeros_like(x)
    orc.rms_norm(4, out, x, rows, dim, scale, 1e-6)
    assert _ref.scaled_err(out, _ref.rms_norm_f64(x, scale, 1e-6)) < 2e-6
    y = x.copy()
    orc.rms_norm(1, y, y, rows, dim, scale, 1e-6)  # in place, one thread: the same bits
    assert np.array_equal(y, out)
    z = np.zeros((2, dim), np.float32)  # a zero row: eps keeps it finite and it stays zero
    orc.rms_norm(1, z, z, 2, dim, scale, 1e-6)
    assert np.array_equal(z, np.zeros_like(z))


def test_relu_closed_form(orc):
    x = np.array([-2.0, -0.0, 0.0, 1e-30, 3.5, -1e30], np.float32)
    y = x.copy()
    orc.relu(y)
    assert np.array_equal(y, np.maximum(x, 0))


@pytest.mark.parametrize("scale", [0.125, 1.0])
def test_chronos2_encode_matches_f64(orc, scale):
    """Model.encode's layer loop against the same stack written from its definition in float64."""
    rng = np.random.default_rng(33)
    b, seq, nh, d_ff, n_layers, eps = 2, 21, 2, 256, 2, 1e-6
    d = nh * 64
    x = rng.standard_normal((b * seq, d)).astype(np.float32)
    kv = _ref.left_pad_valid(rng, b, seq, 6, tail_valid=3)
    kv[0, :] = 1
    layers = _ref.chronos2_layers(rng, n_layers, d, d_ff)
    fn = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    cos_t, sin_t = orc.chronos2_rope_tables(seq, 64, 10000.0)
    got = x.copy()
    orc.chronos2_encode(4, got, kv.ravel().copy(), b, seq, d, nh, 64, d_ff, layers, fn, eps, cos_t, sin_t, scale)
    want = _ref.chronos2_encode_f64(x, kv, b, seq, nh, layers, fn, eps, cos_t, sin_t, scale)
    assert _ref.scaled_err(got, want) < 2e-5
    # no layers: the final norm alone
    y = x.copy()
    orc.chronos2_encode(1, y, kv.ravel().copy(), b, seq, d, nh, 64, d_ff, [], fn, eps, cos_t, sin_t, scale)
    z = np.zeros_like(x)
    orc.rms_norm(1, z, x, b * seq, d, fn, eps)
    assert np.array_equal(y, z)


def test_resblock_matches_definition(orc):
    rng = np.random.default_rng(41)
    rows, d_in, hid, d_out = 37, 48, 64, 40
    rb = _ref.resblock(rng, d_in, hid, d_out)
    x = rng.standard_normal((rows, d_in)).astype(np.float32)
    y = np.zeros((rows, d_out), np.float32)
    orc.resblock_relu(4, y, x, rows, rb)
    assert _ref.scaled_err(y, _ref.resblock_f64(rb, x)) < 5e-6


def test_chronos2_model_forward_matches_f64(orc):
    """The model part of runChunk: embed, [context; REG; future], encode, future rows, head."""
    rng = np.random.default_rng(43)
    b, n_ctx, n_out, nh, d_ff, ps, q = 2, 12, 3, 2, 256, 16, 3
    d, seq = nh * 64, n_ctx + 1 + n_out
    feats = rng.standard_normal((b * n_ctx, 3 * ps)).astype(np.float32)
    fut = rng.standard_normal((b * n_out, 3 * ps)).astype(np.float32)
    cv = (rng.random((b, n_ctx)) < 0.8).astype(np.uint8)
    reg = rng.standard_normal(d).astype(np.float32)
    layers = _ref.chronos2_layers(rng, 2, d, d_ff)
    fn = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    ie, oe = _ref.resblock(rng, 3 * ps, d_ff, d), _ref.resblock(rng, d, d_ff, q * ps)
    cos_t, sin_t = orc.chronos2_rope_tables(seq, 64, 10000.0)
    raw = np.zeros((b * n_out, q * ps), np.float32)
    orc.chronos2_model_forward(4, raw, feats, fut, cv, reg, b, n_ctx, n_out, d, nh, 64, d_ff, layers, fn, 1e-6, cos_t,
                               sin_t, 1.0, ie, oe)
    want = _ref.chronos2_model_forward_f64(feats, fut, cv, reg, b, n_ctx, n_out, nh, layers, fn, 1e-6, cos_t, sin_t,
                                           1.0, ie, oe)
    assert _ref.scaled_err(raw, want) < 3e-5


def test_bolt_model_forward_matches_f64(orc):
    """The model part of the Chronos-Bolt chunk: embed, [patches; REG], T5 encoder with the relative
    bias, one-token decoder with cross-attention, output head; against float64 from the definition."""
    rng = np.random.default_rng(47)
    b, n_patch, nh, d_ff, ps, out = 3, 10, 2, 256, 16, 36
    d = inner = nh * 64
    seq = n_patch + 1
    feats = rng.standard_normal((b * n_patch, 2 * ps)).astype(np.float32)
    pv = (rng.random((b, n_patch)) < 0.8).astype(np.uint8)
    reg, start = (rng.standard_normal(d).astype(np.float32) for _ in range(2))
    table = _ref.t5_bias_table(rng, 32, nh)
    enc, dec = _ref.bolt_layers(rng, 2, 2, d, inner, d_ff)
    ef, df = ((1 + 0.1 * rng.standard_normal(d)).astype(np.float32) for _ in range(2))
    ie, oe = _ref.resblock(rng, 2 * ps, d_ff, d), _ref.resblock(rng, d, d_ff, out)
    raw = np.zeros((b, out), np.float32)
    orc.bolt_model_forward(4, raw, feats, pv, reg, start, table, 32, 128, b, n_patch, d, nh, 64, d_ff, enc, ef, dec,
                           df, 1e-6, ie, oe)
    bias = orc.position_bias(table, seq, nh, 32, 128)
    want = _ref.bolt_model_forward_f64(feats, pv, reg, start, bias, b, n_patch, nh, enc, ef, dec, df, 1e-6, ie, oe)
    assert _ref.scaled_err(raw, want) < 3e-5


def test_bolt_forecast_instance_norm_and_patching(orc):
    """The forecaster's preparation and inverse norm around the model (src/chronos_bolt/
    forecaster.zig:150-219), pinned by numpy's nanmean / nanstd (population) for loc and scale, a
    left pad of (16 - len % 16) % 16 missing steps, [values, mask] features with missing steps 0,
    and out = raw * scale + loc; plus the special cases: a constant series gets scale norm_eps, an
    all-missing one loc 0 and scale 1. Strided rows at an offset in a wider buffer."""
    rng = np.random.default_rng(48)
    n, length, stride, offset, nh, d_ff, ps, out, norm_eps = 4, 37, 45, 3, 1, 64, 16, 20, 1e-5
    d = inner = nh * 64
    buf = (2.0 + 3.0 * rng.standard_normal(n * stride + offset)).astype(np.float32)
    rows = [buf[i * stride + offset:][:length] for i in range(n)]
    rows[0][rng.random(length) < 0.3] = np.nan
    rows[1][:] = -1.5
    rows[2][:] = np.nan
    reg, start = (rng.standard_normal(d).astype(np.float32) for _ in range(2))
    table = _ref.t5_bias_table(rng, 32, nh)
    enc, dec = _ref.bolt_layers(rng, 1, 1, d, inner, d_ff)
    ef, df = ((1 + 0.1 * rng.standard_normal(d)).astype(np.float32) for _ in range(2))
    ie, oe = _ref.resblock(rng, 2 * ps, d_ff, d), _ref.resblock(rng, d, d_ff, out)
    got = np.zeros((n, out), np.float32)
    orc.bolt_forecast(2, got, buf, stride, offset, length, n, ps, norm_eps, reg, start, table, 32, 128, d, nh, 64, d_ff,
                      enc, ef, dec, df, 1e-6, ie, oe)

    pad = (ps - length % ps) % ps
    n_patch = (length + pad) // ps
    assert (pad, n_patch) == (11, 3)
    loc, scale = np.zeros(n, np.float32), np.ones(n, np.float32)
    feats = np.zeros((n, n_patch, 2 * ps), np.float32)
    pv = np.zeros((n, n_patch), np.uint8)
    for i, r in enumerate(rows):
        obs = ~np.isnan(r)
        if obs.any():
            loc[i] = np.float32(np.nanmean(r.astype(np.float64)))
            scale[i] = np.float32(np.sqrt(np.mean((r[obs] - loc[i]).astype(np.float64) ** 2)))
            if scale[i] == 0:
                scale[i] = norm_eps
        padded = np.concatenate([np.full(pad, np.nan, np.float32), r]).reshape(n_patch, ps)
        m = ~np.isnan(padded)
        feats[i, :, :ps] = np.where(m, (np.nan_to_num(padded) - loc[i]) / scale[i], 0)
        feats[i, :, ps:] = m
        pv[i] = m.any(axis=1)
    assert (loc[1], scale[1]) == (np.float32(-1.5), np.float32(norm_eps))
    assert (loc[2], scale[2]) == (0, 1) and not pv[2].any() and not feats[2].any()
    assert pv[3].all() and feats[3, 0, ps:ps + pad].sum() == 0  # 11 padded steps, then 5 observed values
    raw = np.zeros((n, out), np.float32)
    orc.bolt_model_forward(2, raw, feats.reshape(n * n_patch, 2 * ps), pv, reg, start, table, 32, 128, n, n_patch, d,
                           nh, 64, d_ff, enc, ef, dec, df, 1e-6, ie, oe)
    want = raw * scale[:, None] + loc[:, None]
    assert np.allclose(got, want, rtol=1e-6, atol=1e-6 * np.abs(want).max())


@pytest.mark.parametrize("arcsinh", [False, True])
def test_chronos2_forecast_preparation_and_inverse_scaling(orc, arcsinh):
    """runChunk around the model (src/chronos2/forecaster.zig:93-201), pinned by numpy: loc and
    scale are nanmean and the population nanstd (zero spread -> 1e-5, nothing observed -> 0 and 1),
    the context is left-padded by (16 - len % 16) % 16 missing steps, the time encodings are
    (j - n_ctx * 16) / time_scale and j / time_scale, values optionally go through arcsinh, and the
    (n * n_out, q * 16) raw head output is transposed to (n, horizon, q), through sinh, and
    scaled back. Strided rows at a start offset; horizon not a multiple of the patch."""
    rng = np.random.default_rng(49)
    n, length, stride, start, nh, d_ff, ps, q, horizon, tsc = 4, 41, 50, 6, 1, 64, 16, 3, 21, 512.0
    d = nh * 64
    buf = (2.0 + 3.0 * rng.standard_normal(n * stride + start)).astype(np.float32)
    rows = [buf[i * stride + start:][:length] for i in range(n)]
    rows[0][rng.random(length) < 0.3] = np.nan
    rows[1][:] = 7.0
    rows[2][:] = np.nan
    reg = rng.standard_normal(d).astype(np.float32)
    layers = _ref.chronos2_layers(rng, 1, d, d_ff)
    fn = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    ie, oe = _ref.resblock(rng, 3 * ps, d_ff, d), _ref.resblock(rng, d, d_ff, q * ps)
    pad = (ps - length % ps) % ps
    n_ctx, n_out = (length + pad) // ps, (horizon + ps - 1) // ps
    assert (pad, n_ctx, n_out) == (7, 3, 2)
    cos_t, sin_t = orc.chronos2_rope_tables(n_ctx + 1 + n_out, 64, 10000.0)
    got = np.zeros((n, horizon, q), np.float32)
    orc.chronos2_forecast(2, got, buf, stride, start, length, n, ps, horizon, tsc, arcsinh, reg, d, nh, 64, d_ff,
                          layers, fn, 1e-6, cos_t, sin_t, 1.0, ie, oe)

    loc, scale = np.zeros(n, np.float32), np.ones(n, np.float32)
    feats = np.zeros((n, n_ctx, 3 * ps), np.float32)
    fut = np.zeros((n, n_out, 3 * ps), np.float32)
    cv = np.zeros((n, n_ctx), np.uint8)
    j = np.arange(n_ctx * ps, dtype=np.float32).reshape(n_ctx, ps)
    for i, r in enumerate(rows):
        obs = ~np.isnan(r)
        if obs.any():
            loc[i] = np.float32(np.nanmean(r.astype(np.float64)))
            scale[i] = np.float32(np.sqrt(np.mean((r[obs] - loc[i]).astype(np.float64) ** 2)))
            if scale[i] == 0:
                scale[i] = 1e-5
        padded = np.concatenate([np.full(pad, np.nan, np.float32), r]).reshape(n_ctx, ps)
        m = ~np.isnan(padded)
        val = np.where(m, (np.nan_to_num(padded) - loc[i]) / scale[i], 0).astype(np.float32)
        feats[i, :, :ps] = (j - np.float32(n_ctx * ps)) / np.float32(tsc)
        feats[i, :, ps:2 * ps] = np.arcsinh(val) if arcsinh else val
        feats[i, :, 2 * ps:] = m
        cv[i] = m.any(axis=1)
        fut[i, :, :ps] = np.arange(n_out * ps, dtype=np.float32).reshape(n_out, ps) / np.float32(tsc)
    assert (loc[1], scale[1]) == (7, np.float32(1e-5)) and (loc[2], scale[2]) == (0, 1) and not cv[2].any()
    raw = np.zeros((n * n_out, q * ps), np.float32)
    orc.chronos2_model_forward(2, raw, feats.reshape(-1, 3 * ps), fut.reshape(-1, 3 * ps), cv, reg, n, n_ctx, n_out,
                               d, nh, 64, d_ff, layers, fn, 1e-6, cos_t, sin_t, 1.0, ie, oe)
    r = raw.reshape(n, n_out, q, ps).transpose(0, 1, 3, 2).reshape(n, n_out * ps, q)[:, :horizon]
    if arcsinh:
        r = np.sinh(r.astype(np.float64))
    want = r * scale[:, None, None] + loc[:, None, None]
    # arcsinh / sinh: libm's single-precision functions against numpy's double ones (an ulp or two).
    tol = 2e-6 if arcsinh else 1e-6
    assert np.allclose(got, want, rtol=tol, atol=tol * np.abs(want).max())


# ---- Timestral validity, first observation and partial RoPE (src/timestral/model.zig) -----------


@pytest.mark.parametrize("attend_missing", [True, False])
def test_timestral_key_valid_matches_definition(orc, attend_missing):
    """model.zig:343-362 against the numpy definition, on random observation masks with leading
    gaps, inner gaps and an all-missing row and group."""
    rng = np.random.default_rng(31)
    rows, vall, ne, ps = 12, 3, 9, 4
    obs = rng.random((rows, ne * ps)) < 0.15
    obs[0:3] = False                       # group 0 has no observation at all
    obs[4, :] = False                      # one all-missing row in an observed group
    obs[6, : 5 * ps] = False               # leading gap
    got_kv, got_first, got_all = orc.timestral_key_valid(obs, rows, vall, ne, ps, attend_missing)
    kv, first, all_valid = _ref.timestral_key_valid(obs, rows, vall, ne, ps, attend_missing)
    assert np.array_equal(got_kv, kv)
    assert np.array_equal(got_first, first)
    assert got_all == all_valid


def test_timestral_key_valid_hand_case(orc):
    """A case written out by hand: ps = 2, two groups of two rows.
    Row 0: patches (0,0) (1,0) (0,0) -> observed F T F; row 1: (0,0) (0,0) (0,1) -> F F T;
    group 0's first observed patch is 1. Group 1 (rows 2, 3) has no observation: first_obs 0."""
    obs = np.array([[0, 0, 1, 0, 0, 0],
                    [0, 0, 0, 0, 0, 1],
                    [0, 0, 0, 0, 0, 0],
                    [0, 0, 0, 0, 0, 0]], np.uint8)
    kv, first, all_valid = orc.timestral_key_valid(obs, 4, 2, 3, 2, True)
    assert kv.tolist() == [[0, 1, 1], [0, 0, 1], [0, 0, 0], [0, 0, 0]]
    assert first.tolist() == [1, 0] and not all_valid
    kv, first, _ = orc.timestral_key_valid(obs, 4, 2, 3, 2, False)
    assert kv.tolist() == [[0, 1, 0], [0, 0, 1], [0, 0, 0], [0, 0, 0]]
    assert first.tolist() == [1, 0]
    kv, first, all_valid = orc.timestral_key_valid(np.ones((2, 6), np.uint8), 2, 1, 3, 2, False)
    assert kv.all() and all_valid and first.tolist() == [0, 0]


@pytest.mark.parametrize("ne,l,h", [(20, 20, 6), (26, 20, 6)])
def test_timestral_rope_tables_match_definition(orc, ne, l, h):
    """model.zig:180-188, 447-463 against float64 tables from the definition. ne > l is the covariate
    window (decoder token j at time l + j, not ne + j). first_obs differs per group and exceeds some
    positions (negative times). Past rope_dim / 2 the tables are exactly cos 1, sin 0."""
    groups, hd, rope_dim, theta = 3, 64, 32, 10000.0
    first_obs = [0, 7, 25]
    c, s = orc.timestral_rope_tables(groups, ne, l, h, hd, rope_dim, theta, first_obs)
    c64, s64, ang = _ref.timestral_rope_tables_f64(groups, ne, l, h, hd, rope_dim, theta, first_obs)
    c = c.reshape(c64.shape)
    s = s.reshape(s64.shape)
    # f32 frequencies and products: relative error of the angle a few 1e-7
    tol = 1e-6 * (1.0 + np.abs(ang))
    assert np.all(np.abs(c - c64) <= tol) and np.all(np.abs(s - s64) <= tol)
    assert np.all(c[:, :, rope_dim // 2:] == 1.0) and np.all(s[:, :, rope_dim // 2:] == 0.0)
    # the decoder's time base is visible at i = 0 (frequency 1): a table built with ne + j instead
    # of l + j, or with +first_obs, would miss these by O(1)
    for g in range(groups):
        for j in range(h):
            assert abs(float(c[g, ne + j, 0]) - np.cos(l + j - first_obs[g])) <= 1e-5


def test_timestral_rope_application(orc):
    """TimeJob.rope (model.zig:558-577) against a float64 rotation with each row's group table
    (g = r // vall): q and k of every head rotated, v untouched, and the dims past rope_dim / 2 (and
    their partners) bit-identical."""
    rng = np.random.default_rng(32)
    rows, vall, ne, l, h, nh, hd, rope_dim = 6, 2, 12, 12, 4, 3, 64, 32
    d, sl = nh * hd, ne + h
    first_obs = [0, 5, 9]
    c, s = orc.timestral_rope_tables(rows // vall, ne, l, h, hd, rope_dim, 10000.0, first_obs)
    qkv = rng.standard_normal(rows * sl * 3 * d).astype(np.float32)
    got = qkv.copy()
    orc.timestral_rope(4, got, c, s, rows, sl, vall, d, nh, hd)
    want = _ref.timestral_rope_f64(qkv, c, s, rows, sl, vall, d, nh, hd)
    assert np.max(np.abs(got - want)) <= 2e-6 * max(1.0, np.max(np.abs(want)))
    g5 = got.reshape(rows, sl, 3, nh, hd)
    x5 = qkv.reshape(rows, sl, 3, nh, hd)
    assert np.array_equal(g5[:, :, 2], x5[:, :, 2])
    keep = np.r_[rope_dim // 2: hd // 2, hd // 2 + rope_dim // 2: hd]
    assert np.array_equal(g5[..., keep], x5[..., keep])
    # rotating with another group's table (a wrong g) would differ: rows 0 and 2 share tokens
    # but not tables
    assert not np.allclose(g5[0, :, 0], _ref.timestral_rope_f64(qkv, np.roll(c.reshape(3, -1), 1, 0).ravel(),
                                                                 np.roll(s.reshape(3, -1), 1, 0).ravel(), rows, sl,
                                                                 vall, d, nh, hd).reshape(rows, sl, 3, nh, hd)[0, :, 0])


# ---- Timestral model and forecaster (oracle/tsfm_oracle_timestral.c) ---------------------------


def test_silu_mul_silu_softplus_closed_forms(orc):
    x = np.linspace(-30, 30, 1001).astype(np.float32)
    y = x.copy()
    orc.silu_in_place(y)
    exact = x.astype(np.float64) / (1 + np.exp(-x.astype(np.float64)))
    assert np.max(np.abs(y - exact) / np.maximum(np.abs(exact), 1)) < 1e-6
    g = np.random.default_rng(1).standard_normal(1001).astype(np.float32)
    z = np.zeros_like(x)
    orc.mul_silu(z, g, x)  # gate * silu(up): a transposed operand order would fail
    assert np.max(np.abs(z - g * exact) / np.maximum(np.abs(g * exact), 1)) < 1e-6
    for v in (-30.0, -1.0, 0.0, 3.0, 19.9, 20.0, 20.5, 80.0):
        want = v if v > 20 else np.log1p(np.exp(v))
        assert abs(orc.softplus(v) - want) <= 1e-6 * max(1.0, abs(want))


def test_clamp_nonfinite_cases(orc):
    a = np.array([1.0, np.inf, -2.0, -np.inf, np.nan], np.float32)
    orc.clamp_nonfinite(a)
    assert a[0] == 1 and a[1] == 1 and a[2] == -2 and a[3] == -2 and np.isnan(a[4])
    b = np.array([np.inf, -np.inf], np.float32)
    orc.clamp_nonfinite(b)
    assert (b == 0).all()
    c = np.array([3.0, np.nan], np.float32)
    orc.clamp_nonfinite(c)  # no infinity: untouched
    assert c[0] == 3 and np.isnan(c[1])


def test_resblock_silu_matches_definition(orc):
    rng = np.random.default_rng(2)
    rb = _ref.resblock(rng, 32, 64, 48)
    x = rng.standard_normal((10, 32)).astype(np.float32)
    y = np.zeros((10, 48), np.float32)
    orc.resblock_silu(3, y, x, 10, rb)
    assert _ref.scaled_err(y, _ref.resblock_silu_f64(rb, x)) < 2e-6
    for k in ("hidden_b", "output_b", "residual_b"):
        rb[k] = None  # bias = false
    orc.resblock_silu(3, y, x, 10, rb)
    assert _ref.scaled_err(y, _ref.resblock_silu_f64(rb, x)) < 2e-6


def test_timestral_patch_stats_match_the_definition(orc):
    """StatsJob (model.zig:712-750) against two-pass numpy statistics of the observed prefix: the
    running mean, the sample std (ddof 1), min_scale below two values, loc 0 before any."""
    rng = np.random.default_rng(3)
    rows, ps, n = 5, 8, 12
    t = ps * n
    x = (3 + 2 * rng.standard_normal((rows, t))).astype(np.float32)
    obs = rng.random((rows, t)) < 0.7
    obs[1, :30] = False   # leading gap
    obs[2] = False        # never observed
    obs[3, :] = False
    obs[3, 17] = True     # exactly one observation
    loc, scale = orc.timestral_patch_stats(2, x, obs, rows, t, ps, 1e-6)
    wl, ws = _ref.patch_stats_f64(x, obs, ps, 1e-6)
    assert np.allclose(loc, wl, rtol=2e-7, atol=1e-7) and np.allclose(scale, ws, rtol=2e-7, atol=1e-7)
    assert (loc[2] == 0).all() and (scale[2] == np.float32(1e-6)).all()


@pytest.mark.parametrize("attend_missing", [True, False])
def test_timestral_predict_block_matches_f64(orc, attend_missing):
    """Model.predictBlock (model.zig:220-432) without covariates against a float64 model written
    from the definitions (tests/_ref.py): causal per-patch normalisation with asinh, the patch
    embedding, time attention (causal encoder rows with key validity, block-causal decoder rows,
    partial RoPE relative to each group's first observation, sigmoid gate), variate attention, the
    SiLU MLP, the head, and the monotone quantile transform back to data units. Two groups of two
    variates, leading gaps (one group starts late), scattered missing values."""
    rng = np.random.default_rng(4 + attend_missing)
    m = _ref.timestral_model(rng, d=128, nh=2, hid=128, attend_missing=attend_missing)
    groups, vall, t, h = 2, 2, 16 * 10, 4
    rows = groups * vall
    ctx = (5 + 3 * rng.standard_normal((rows, t))).astype(np.float32)
    obs = rng.random((rows, t)) < 0.9
    obs[2:4, :40] = False  # group 1's first observed patch is patch 2
    ctx[~obs] = 0
    got = orc.timestral_predict_block(3, m, ctx, obs, t, groups, vall, h)
    want = _ref.timestral_predict_block_f64(m, ctx, obs, t, groups, vall, h)
    assert got.shape == want.shape
    assert _ref.scaled_err(got, want) < 5e-5  # measured 5.5e-6


def test_timestral_refine_block_matches_definition(orc):
    rng = np.random.default_rng(6)
    m = _ref.timestral_model(rng, d=64, nh=1, hid=64)
    rows, ps, t, h, q = 3, 16, 16 * 8, 4, m["q"]
    ctx = (10 + 4 * rng.standard_normal((rows, t))).astype(np.float32)
    obs = rng.random((rows, t)) < 0.85
    obs[2, :70] = False
    ctx[~obs] = 0
    med = (10 + 4 * rng.standard_normal((rows, h * ps))).astype(np.float32)
    qs = np.sort(med[:, :, None] + rng.standard_normal((rows, h * ps, q)).astype(np.float32), axis=2)
    qs[:, :, m["median"]] = med
    got = qs.copy()
    orc.timestral_refine_block(got, m, ctx, obs, rows, t, h)
    want = _ref.timestral_refine_f64(qs, ctx, obs, ps, m["median"], m["minimum_scale"])
    assert _ref.scaled_err(got, want) < 1e-5
    assert not np.allclose(got[:, ps:], qs[:, ps:])  # later patches do move


def _ts_case(seed, b=2, v=2, t0=150, nan_frac=0.1, start_missing=0):
    rng = np.random.default_rng(seed)
    m = _ref.timestral_model(rng, d=64, nh=1, hid=64, schedule=("time_variate",))
    x = (20 + 5 * np.sin(np.arange(t0) / 4.0) + rng.standard_normal((b * v, t0))).astype(np.float32)
    obs = rng.random((b * v, t0)) >= nan_frac
    obs[:, :start_missing] = False
    x[~obs] = 0
    return m, x, obs


def _ts_decode_composed(orc, m, x, obs, b, v, horizon, per_shot, max_context):
    """blockDecode restated in Python over the oracle's predict_block and refine_block: each block's
    medians (0 if not finite or huge) become observed context, oldest steps dropped past
    max_context."""
    ps, q = m["ps"], m["q"]
    ctx, mask = _ref.timestral_context(x, obs, max_context, ps)
    out = np.zeros((b * v, horizon, q), np.float32)
    remaining, done = -(-horizon // ps), 0
    while remaining:
        block = min(per_shot, remaining)
        blen = block * ps
        t = ctx.shape[1]
        qs = orc.timestral_predict_block(3, m, ctx, mask, t, b, v, block)
        if block > 1:
            orc.timestral_refine_block(qs, m, ctx, mask, b * v, t, block)
        take = min(blen, horizon - done)
        out[:, done:done + take] = qs[:, :take]
        remaining -= block
        done += blen
        if not remaining:
            break
        medv = qs[:, :, m["median"]].copy()
        medv[~np.isfinite(medv) | (np.abs(medv) >= 1e30)] = 0
        ctx = np.concatenate([ctx, medv], axis=1)
        mask = np.concatenate([mask, np.ones_like(medv, bool)], axis=1)
        if ctx.shape[1] > max_context:
            keep = max(ps, max_context // ps * ps)
            ctx, mask = ctx[:, -keep:], mask[:, -keep:]
    return out


@pytest.mark.parametrize("horizon,per_shot,max_context", [(40, 4, 2048), (100, 2, 2048), (100, 2, 160)])
def test_timestral_forecast_block_decode_composition(orc, horizon, per_shot, max_context):
    """forecast (no averaging, no clip, no cap) = forecastRaw's forward-fill and padding, then
    blockDecode: one block refined (40 steps), several blocks with median feedback (100 steps in
    blocks of 2 patches), and a context cap that drops the oldest steps as it grows."""
    b, v = 2, 2
    m, x, obs = _ts_case(7, b, v, start_missing=20)
    rc, got = orc.timestral_forecast(3, m, x, obs, b, v, x.shape[1], horizon, max_context, per_shot, cap_k=0.0,
                                     symmetric=False, clip_nonnegative=False)
    assert rc == 0
    want = _ts_decode_composed(orc, m, x, obs, b, v, horizon, per_shot, max_context)
    assert np.array_equal(got.reshape(b * v, horizon, -1), want)


def test_timestral_forecast_symmetric_clip_and_cap(orc):
    """Symmetric averaging: 0.5 (f(x) - reverse(f(-x))) over the quantile levels; the clip to zero
    of series whose observed values are all non-negative; the quantile cap at the context's range
    widened by cap_k times its last patch scale."""
    b, v, horizon = 2, 2, 40
    m, x, obs = _ts_case(8, b, v)
    t0 = x.shape[1]
    kw = dict(cap_k=0.0, per_shot=32)
    _, f = orc.timestral_forecast(3, m, x, obs, b, v, t0, horizon, symmetric=False, clip_nonnegative=False, **kw)
    _, g = orc.timestral_forecast(3, m, -x, obs, b, v, t0, horizon, symmetric=False, clip_nonnegative=False, **kw)
    rc, s = orc.timestral_forecast(3, m, x, obs, b, v, t0, horizon, symmetric=True, clip_nonnegative=False, **kw)
    assert rc == 0
    assert np.allclose(s, 0.5 * (f - g[..., ::-1]), rtol=0, atol=1e-5 * np.abs(f).max())
    _, c = orc.timestral_forecast(3, m, x, obs, b, v, t0, horizon, symmetric=True, clip_nonnegative=True, **kw)
    assert np.array_equal(c, np.maximum(s, 0))  # every series here is positive
    cap = 0.05
    _, capped = orc.timestral_forecast(3, m, x, obs, b, v, t0, horizon, symmetric=False, clip_nonnegative=False,
                                       cap_k=cap, per_shot=32)
    ctx, mask = _ref.timestral_context(x, obs, 2048, m["ps"])
    _, sc = _ref.patch_stats_f64(ctx, mask, m["ps"], m["minimum_scale"])
    for r in range(b * v):
        vals = ctx[r][mask[r]]
        a = np.float32(sc[r, -1]) * np.float32(cap)
        lo, hi = vals.min() - a, vals.max() + a
        assert capped.reshape(b * v, -1)[r].min() >= lo - 1e-4 and capped.reshape(b * v, -1)[r].max() <= hi + 1e-4
    assert not np.array_equal(capped, f)


@pytest.mark.parametrize("asinh", [False, True])
@pytest.mark.parametrize("horizon,per_shot,max_context,cap_k,symmetric", [
    (40, 32, 2048, 0.0, False), (100, 2, 2048, 1e4, True), (100, 2, 176, 1e4, True), (64, 4, 2048, 0.05, True)])
def test_timestral_forecast_f64_composition_matches_oracle(orc, asinh, horizon, per_shot, max_context, cap_k,
                                                           symmetric):
    """_ref.timestral_forecast_f64 (the float64 forecast the GPU tests measure distances from, composed
    from the float64 predict_block and refine_block definitions with the feedback, window, cap,
    mirrored average and clip) against the oracle's forecast: one refined block, several blocks with
    feedback, a context window that drops steps, a cap that binds (cap_k 0.05), a negative series
    (the clip leaves it alone) and a series without observation. Within f32 distance in linear space
    (1e-5) and in asinh space (2e-4, where the sinh expansion amplifies the head's f32 error); a
    wrong mirror, cap or clip moves the forecast by orders of magnitude more."""
    b, v = 3, 1
    rng = np.random.default_rng(50 + int(asinh))
    m = _ref.timestral_model(rng, d=64, nh=1, hid=64, schedule=("time_variate", "time"), use_asinh=asinh)
    t0 = 150
    x = (20 + 5 * np.sin(np.arange(t0) / 4.0) + rng.standard_normal((b * v, t0))).astype(np.float32)
    x[1] = -x[1]
    obs = rng.random((b * v, t0)) >= 0.1
    obs[2] = False
    x[~obs] = 0
    rc, got = orc.timestral_forecast(3, m, x, obs, b, v, t0, horizon, max_context, per_shot, cap_k=cap_k,
                                     symmetric=symmetric, clip_nonnegative=True)
    assert rc == 0
    want = _ref.timestral_forecast_f64(m, x, obs, b, v, horizon, per_shot=per_shot, max_context=max_context,
                                       cap_k=cap_k, symmetric=symmetric, clip_nonnegative=True)
    assert _ref.scaled_err(got, want) < (2e-4 if asinh else 1e-5)
    assert (got[1] < 0).any() and (got[0] >= 0).all()  # the clip applies to the positive series only


# ---- Chronos-Bolt long horizons (src/chronos_bolt/forecaster.zig:22-92) ----------------------------


def test_quantile_linear_reference_cases(orc):
    """The reference's own test of quantileLinear (forecaster.zig:222-228)."""
    v = np.array([1, 2, 4, 8, 16], np.float32)
    assert orc.quantile_linear(v, 0.0) == 1
    assert orc.quantile_linear(v, 0.5) == 4
    assert orc.quantile_linear(v, 1.0) == 16
    assert abs(orc.quantile_linear(v, 0.375) - 3) <= 1e-6


@pytest.mark.parametrize("n", [2, 7, 81])
def test_quantile_linear_is_torch_quantile(orc, n):
    """torch.quantile (linear interpolation) over sorted random samples, levels on and between the
    sample ranks, both halves of the lerp: within one f32 rounding of torch's own result."""
    import torch

    rng = np.random.default_rng(n)
    for _ in range(20):
        v = np.sort(rng.standard_normal(n).astype(np.float32) * 10)
        for lv in (0.0, 0.1, 0.2, 0.25, 0.3, 0.5, 0.6, 0.7, 0.8, 0.9, 0.95, 1.0):
            want = torch.quantile(torch.from_numpy(v), torch.tensor(lv, dtype=torch.float32)).item()
            got = float(orc.quantile_linear(v, lv))
            assert abs(got - want) <= 2.4e-7 * max(1.0, abs(want)), (n, lv, got, want)


def _bolt_small(seed=0, P=16, q=9):
    from tsfm_attn import workloads

    w = workloads.bolt_forward(B=2, n_patch=2, H=2, d_ff=256, n_layers=1, quantiles=q, horizon=P, seed=seed)
    a, m = w.arrays, w.meta
    return dict(reg=a["reg"], dec_start=a["dec_start"], rel_table=a["rel_table"], enc=m["enc"], dec=m["dec"],
                enc_final_norm=a["enc_final_norm"], dec_final_norm=a["dec_final_norm"], ie=m["ie"], oe=m["oe"],
                d_model=m["d_model"], heads=w.H, d_ff=m["d_ff"], eps=m["eps"], buckets=m["buckets"],
                max_distance=m["max_distance"])


def _bolt_block(orc, w, ctx, P, q):
    ctx = np.ascontiguousarray(ctx, np.float32)
    n, length = ctx.shape
    out = np.zeros((n, q * P), np.float32)
    orc.bolt_forecast(1, out, ctx, length, 0, length, n, 16, 1e-5, w["reg"], w["dec_start"], w["rel_table"],
                      w["buckets"], w["max_distance"], w["d_model"], w["heads"], 64, w["d_ff"], w["enc"],
                      w["enc_final_norm"], w["dec"], w["dec_final_norm"], w["eps"], w["ie"], w["oe"])
    return out.reshape(n, q, P)


@pytest.mark.parametrize("t_in,max_ctx,horizon", [(70, 96, 50), (40, 2048, 16), (40, 2048, 7), (130, 64, 33)])
def test_bolt_forecast_horizon_composition(orc, t_in, max_ctx, horizon):
    """forecaster.forecast as a composition of the chunk forecast: block 0 from the last max_ctx
    steps; then each series' q quantile paths appended to its window (the oldest steps dropped past
    max_ctx), forecast as q rows each, sorted per step over the q * q outputs and reduced with
    quantileLinear. Written here with whole-array operations (repeat, concatenate, trailing slice,
    sort); the oracle's loop must give the same bits."""
    P, q = 16, 9
    w = _bolt_small(P=P, q=q)
    levels = np.linspace(0.1, 0.9, q).astype(np.float32)
    rng = np.random.default_rng(t_in)
    b = 2
    t = np.arange(t_in)
    x = (10 * np.sin(2 * np.pi * t / 24) + 0.05 * t + rng.standard_normal((b, t_in))).astype(np.float32)
    x[rng.random(x.shape) < 0.05] = np.nan
    got = orc.bolt_forecast_horizon(1, x, horizon, w, P, max_ctx, levels)

    ctx = x[:, -max_ctx:]
    pred = _bolt_block(orc, w, ctx, P, q)
    steps = [pred.transpose(0, 2, 1)]
    paths = np.repeat(ctx, q, axis=0)
    while sum(s.shape[1] for s in steps) < horizon:
        paths = np.concatenate([paths, pred.reshape(b * q, P)], axis=1)[:, -max_ctx:]
        srt = np.sort(_bolt_block(orc, w, paths, P, q).reshape(b, q * q, P), axis=1)
        pred = np.array([[[orc.quantile_linear(srt[s, :, p], lv) for p in range(P)] for lv in levels]
                         for s in range(b)], np.float32)
        steps.append(pred.transpose(0, 2, 1))
    want = np.concatenate(steps, axis=1)[:, :horizon]
    assert got.shape == (b, horizon, q)
    assert np.array_equal(got, want)


# ---- Timestral covariates (past-only and known-future rows) ------------------------------------

def _ts_cov_case(seed, b=2, v=1, n_past=1, n_known=2, t0=150, horizon=40):
    """Targets plus covariates of both kinds: a past-only row with a gap, a known-future row with
    missing steps in its future, and (with n_known > 1) a 0/1 indicator row."""
    rng = np.random.default_rng(seed)
    m, x, obs = _ts_case(seed, b, v, t0)
    past = (3 + rng.standard_normal((b, n_past, t0))).astype(np.float32)
    past[:, :, 40:55] = np.nan
    steps = np.arange(t0 + horizon)
    known = np.empty((b, n_known, t0 + horizon), np.float32)
    for k in range(n_known):
        known[:, k] = (np.cos(steps / 5.0 + k) * 4 + 10).astype(np.float32)
        if k == 1:
            known[:, k] = (steps % 7 < 2).astype(np.float32)
    known[:, 0, t0 + 3:t0 + 9] = np.nan
    return m, x, obs, past, known


@pytest.mark.parametrize("attend_missing", [True, False])
def test_timestral_predict_block_covariates_match_f64(orc, attend_missing):
    """predictBlock (model.zig:220-432) with covariate rows against the float64 model: the window
    spans context and horizon (blanks for past-only rows, real futures for known rows), known rows
    normalised by their whole-window mean and population std (0/1 rows neither shifted nor
    asinh'd), known rows bidirectional in time attention, the variate firewalls, and the head
    on the target rows only."""
    rng = np.random.default_rng(11 + attend_missing)
    m = _ref.timestral_model(rng, d=128, nh=2, hid=128, attend_missing=attend_missing)
    groups, t, h, ps = 2, 16 * 8, 3, 16
    roles = np.array([0, 0, 1, 2, 2], np.uint8)
    vall = len(roles)
    rows = groups * vall
    ctx = (5 + 3 * rng.standard_normal((rows, t))).astype(np.float32)
    obs = rng.random((rows, t)) < 0.9
    obs[vall:vall + 2, :35] = False  # group 1's targets start late
    kf = (2 + rng.standard_normal((rows, h * ps))).astype(np.float32)
    kfm = rng.random((rows, h * ps)) < 0.85
    for g in range(groups):  # the last row of each series is a 0/1 indicator
        r = g * vall + 4
        ctx[r] = (np.arange(t) % 5 == 0)
        kf[r] = (np.arange(h * ps) % 5 == 0)
    ctx[~obs] = 0
    kf[~kfm] = 0
    got = orc.timestral_predict_block_cov(3, m, ctx, obs, t, groups, vall, h, roles, kf, kfm)
    want = _ref.timestral_predict_block_f64(m, ctx, obs, t, groups, vall, h, roles, kf, kfm)
    assert got.shape == want.shape == (groups * 2, h * ps, m["q"])
    assert _ref.scaled_err(got, want) < 5e-5
    # The covariates reach the targets: blanking the known futures moves the forecast.
    blank = orc.timestral_predict_block_cov(3, m, ctx, obs, t, groups, vall, h, roles, None, None)
    assert _ref.scaled_err(blank, _ref.timestral_predict_block_f64(m, ctx, obs, t, groups, vall, h, roles)) < 5e-5
    assert not np.allclose(blank, got, rtol=1e-4, atol=1e-4)


def _ts_cov_decode_composed(orc, m, x, obs, past, known, b, v, horizon, per_shot, max_context):
    """forecastRaw + blockDecode with covariates restated over the oracle's predict_block_cov and
    refine_block: targets forward-filled, covariates NaN-masked; after each block targets carry
    their medians, known rows their real future, past-only rows a blank."""
    ps, q = m["ps"], m["q"]
    n_past, n_known = past.shape[1], known.shape[1]
    vall, t0 = v + n_past + n_known, x.shape[1]
    roles = np.array([0] * v + [1] * n_past + [2] * n_known, np.uint8)
    tctx, tmask = _ref.timestral_context(x, obs, max_context, ps)
    t = tctx.shape[1]
    keep = min(t0, max_context)
    rows = np.zeros((b, vall, t), np.float32)
    mask = np.zeros((b, vall, t), bool)
    rows[:, :v], mask[:, :v] = tctx.reshape(b, v, t), tmask.reshape(b, v, t)
    for k, src in ((v, past), (v + n_past, known[:, :, :t0])):
        win = src[:, :, t0 - keep:]
        rows[:, k:k + src.shape[1], t - keep:] = np.nan_to_num(win, nan=0.0)
        mask[:, k:k + src.shape[1], t - keep:] = ~np.isnan(win)
    fut = known[:, :, t0:]
    hpad = -(-horizon // ps) * ps
    kf = np.zeros((b, vall, hpad), np.float32)
    kfm = np.zeros((b, vall, hpad), bool)
    kf[:, v + n_past:, :horizon] = np.nan_to_num(fut, nan=0.0)
    kfm[:, v + n_past:, :horizon] = ~np.isnan(fut)
    ctx, cm = rows.reshape(b * vall, t), mask.reshape(b * vall, t)
    kf, kfm = kf.reshape(b * vall, hpad), kfm.reshape(b * vall, hpad)
    out = np.zeros((b * v, horizon, q), np.float32)
    tgt = [g * vall + i for g in range(b) for i in range(v)]
    remaining, done = -(-horizon // ps), 0
    while remaining:
        block = min(per_shot, remaining)
        blen = block * ps
        t = ctx.shape[1]
        qs = orc.timestral_predict_block_cov(3, m, ctx, cm, t, b, vall, block, roles, kf[:, done:done + blen],
                                             kfm[:, done:done + blen])
        if block > 1:
            for oi, r in enumerate(tgt):
                sub = qs[oi:oi + 1].copy()
                orc.timestral_refine_block(sub, m, ctx[r:r + 1], cm[r:r + 1], 1, t, block)
                qs[oi] = sub[0]
        take = min(blen, horizon - done)
        out[:, done:done + take] = qs[:, :take]
        remaining -= block
        if not remaining:
            break
        new = np.zeros((b * vall, blen), np.float32)
        newm = np.zeros((b * vall, blen), bool)
        medv = qs[:, :, m["median"]].copy()
        medv[~np.isfinite(medv) | (np.abs(medv) >= 1e30)] = 0
        new[tgt], newm[tgt] = medv, True
        kn = [g * vall + i for g in range(b) for i in range(v + n_past, vall)]
        new[kn], newm[kn] = kf[kn, done:done + blen], kfm[kn, done:done + blen]
        done += blen
        ctx, cm = np.concatenate([ctx, new], 1), np.concatenate([cm, newm], 1)
        if ctx.shape[1] > max_context:
            kt = max(ps, max_context // ps * ps)
            ctx, cm = ctx[:, -kt:], cm[:, -kt:]
    return out


@pytest.mark.parametrize("horizon,per_shot,max_context", [(40, 4, 2048), (100, 2, 2048), (100, 2, 160)])
def test_timestral_forecast_covariates_block_decode_composition(orc, horizon, per_shot, max_context):
    b, v = 2, 2
    m, x, obs, past, known = _ts_cov_case(21, b, v, horizon=horizon)
    rc, got = orc.timestral_forecast_cov(3, m, x, obs, b, v, x.shape[1], horizon, past, known, max_context, per_shot,
                                         cap_k=0.0, symmetric=False, clip_nonnegative=False)
    assert rc == 0
    want = _ts_cov_decode_composed(orc, m, x, obs, past, known, b, v, horizon, per_shot, max_context)
    assert np.array_equal(got.reshape(b * v, horizon, -1), want)


def test_timestral_forecast_covariates_mirror_and_causality(orc):
    """Symmetric averaging negates every covariate row in the mirrored pass: the forecast of
    (-x, -covariates) is exactly the reversed negation of that of (x, covariates) (a mirror that
    kept the covariates' sign breaks this). Known futures past the first block do not move the
    first block; the covariates do move the forecast."""
    b, v, horizon = 2, 1, 64
    m, x, obs, past, known = _ts_cov_case(22, b, v, horizon=horizon)
    t0 = x.shape[1]
    kw = dict(per_shot=2, cap_k=1e4, clip_nonnegative=False)
    _, f = orc.timestral_forecast_cov(3, m, x, obs, b, v, t0, horizon, past, known, **kw)
    _, g = orc.timestral_forecast_cov(3, m, -x, obs, b, v, t0, horizon, -past, -known, **kw)
    assert np.array_equal(g, -f[..., ::-1])
    _, g2 = orc.timestral_forecast_cov(3, m, -x, obs, b, v, t0, horizon, past, known, **kw)
    assert not np.array_equal(g2, -f[..., ::-1])
    k2 = known.copy()
    k2[:, :, t0 + 32:] += 50
    _, f2 = orc.timestral_forecast_cov(3, m, x, obs, b, v, t0, horizon, past, k2, **kw)
    assert np.array_equal(f2[:, :, :32], f[:, :, :32]) and not np.allclose(f2[:, :, 32:], f[:, :, 32:])
    _, f0 = orc.timestral_forecast_cov(3, m, x, obs, b, v, t0, horizon, **kw)
    _, f1 = orc.timestral_forecast(3, m, x, obs, b, v, t0, horizon, **kw)
    assert np.array_equal(f0, f1) and not np.allclose(f0, f, rtol=1e-3)


# ---- categorical covariates (forecaster.zig:201-301) ---------------------------------------------


def _cat_inputs(t, obs=None, values=None):
    x = np.zeros((1, 1, t), np.float32) if values is None else np.asarray(values, np.float32).reshape(1, 1, t)
    ob = np.ones((1, 1, t), np.uint8) if obs is None else np.asarray(obs, np.uint8).reshape(1, 1, t)
    return x, ob


def test_categorical_encoding_hand_case(orc):
    """Smoothed mean-target encoding worked by hand: target 1..6, codes (0, 1, 0, 1, NaN, 0): mean
    3.5; category 0 holds targets 1, 3, 6 -> (3.5 + 10) / 4; category 1 holds 2, 4 -> (3.5 + 6) / 3;
    the missing category holds 5 -> (3.5 + 5) / 2. Future codes: 1, NaN, an unseen 7 and +inf (both
    unseen: the mean)."""
    x, ob = _cat_inputs(6, values=[1, 2, 3, 4, 5, 6])
    codes = np.array([[[0, 1, 0, 1, np.nan, 0, 1, np.nan, 7, np.inf]]])
    got = orc.timestral_encode_categorical(codes, x, ob, 512)[0, 0]
    c0, c1, cm = np.float32(13.5 / 4), np.float32(9.5 / 3), np.float32(8.5 / 2)
    want = np.array([c0, c1, c0, c1, cm, c0, c1, cm, 3.5, 3.5], np.float32)
    assert np.array_equal(got, want)


def test_categorical_encoding_window_and_padding(orc):
    """The encoding target is forward-filled from the first observation and kept only over the
    last max_context steps: steps before it (or outside the window) carry no target, a missing code
    there stays NaN (padding), and any other code there still gets its category's value."""
    t = 8
    x, ob = _cat_inputs(t, obs=[0, 0, 1, 0, 1, 1, 0, 1], values=[0, 0, 2, 9, 4, 6, 9, 8])
    codes = np.array([[[np.nan, 5, 5, 5, np.nan, 3, 3, 5]]])
    # Target over the whole context: (NaN, NaN, 2, 2, 4, 6, 6, 8); mean 28 / 6.
    got = orc.timestral_encode_categorical(codes, x, ob, 100)[0, 0]
    mean = 28.0 / 6
    c5 = np.float32((mean + 2 + 2 + 8) / 4)
    c3 = np.float32((mean + 6 + 6) / 3)
    cm = np.float32((mean + 4) / 2)
    assert np.isnan(got[0]) and np.array_equal(got[1:], [c5, c5, c5, cm, c3, c3, c5])
    # Window of 4 steps: target (NaN x4, 4, 6, 6, 8); mean 6; step 3's code 5 keeps a value, step 0's
    # NaN is padding.
    got = orc.timestral_encode_categorical(codes, x, ob, 4)[0, 0]
    c5 = np.float32((6 + 8) / 2)
    c3 = np.float32((6 + 6 + 6) / 3)
    cm = np.float32((6 + 4) / 2)
    assert np.isnan(got[0]) and np.array_equal(got[1:], [c5, c5, c5, cm, c3, c3, c5])


def test_categorical_encoding_invariants(orc):
    """A constant target encodes every code to that constant (mean c, (c + n c) / (1 + n) = c); with
    more than one target variate the codes pass through as float32; a series with no observation
    encodes to 0 (mean 0, no counts) except its missing codes, which are padding."""
    rng = np.random.default_rng(3)
    t, n = 40, 55
    codes = rng.integers(0, 5, (2, 3, n)).astype(np.float64)
    codes[rng.random(codes.shape) < 0.2] = np.nan
    x = np.full((2, 1, t), 2.5, np.float32)
    ob = (rng.random((2, 1, t)) < 0.7).astype(np.uint8)
    ob[:, :, 0] = 1
    assert np.array_equal(orc.timestral_encode_categorical(codes, x, ob, 512), np.full((2, 3, n), 2.5, np.float32))
    x2 = rng.standard_normal((2, 2, t)).astype(np.float32)
    got = orc.timestral_encode_categorical(codes, x2, np.ones((2, 2, t), np.uint8), 512)
    assert np.array_equal(got, codes.astype(np.float32), equal_nan=True)
    got = orc.timestral_encode_categorical(codes, x, np.zeros((2, 1, t), np.uint8), 512)
    past = codes[:, :, :t]
    assert np.array_equal(np.isnan(got[:, :, :t]), np.isnan(past))
    assert (got[:, :, :t][~np.isnan(past)] == 0).all() and (got[:, :, t:] == 0).all()


def test_categorical_encoding_matches_a_dictionary_count(orc):
    """Random codes (NaN, infinities, unseen future codes), gaps and windows against a count by
    dictionary in float64, rounded once."""
    rng = np.random.default_rng(11)
    for trial in range(20):
        t, h = int(rng.integers(1, 60)), int(rng.integers(0, 30))
        b, c = 2, 2
        x = (rng.standard_normal((b, 1, t)) * 3).astype(np.float32)
        ob = (rng.random((b, 1, t)) < 0.6).astype(np.uint8)
        codes = rng.integers(-2, 6, (b, c, t + h)).astype(np.float64)
        codes[rng.random(codes.shape) < 0.15] = np.nan
        codes[rng.random(codes.shape) < 0.05] = np.inf
        window = int(rng.integers(1, 80))
        got = orc.timestral_encode_categorical(codes, x, ob, window)
        for s in range(b):
            tg = np.full(t, np.nan)
            last, started = 0.0, False
            for i in range(t):
                if ob[s, 0, i]:
                    started, last = True, float(x[s, 0, i])
                if started and (t <= window or i >= t - window):
                    tg[i] = last
            fin = np.isfinite(tg)
            mean = tg[fin].sum() / fin.sum() if fin.any() else 0.0
            for j in range(c):
                row = codes[s, j]
                seen = {float(v) for v in row[:t] if np.isfinite(v)}
                key = lambda v: float(v) if (np.isfinite(v) and float(v) in seen) else "missing"
                sums, counts = {}, {}
                for i in range(t):
                    if fin[i]:
                        k = key(row[i])
                        sums[k] = sums.get(k, 0.0) + tg[i]
                        counts[k] = counts.get(k, 0) + 1
                val = lambda k: (mean + sums.get(k, 0.0)) / (1.0 + counts.get(k, 0))
                want = np.empty(t + h, np.float32)
                for i in range(t):
                    want[i] = np.nan if (np.isnan(tg[i]) and np.isnan(row[i])) else val(key(row[i]))
                for i in range(t, t + h):
                    v = row[i]
                    want[i] = val("missing") if np.isnan(v) else (val(float(v)) if (np.isfinite(v) and float(v) in seen)
                                                                    else mean)
                np.testing.assert_allclose(got[s, j], want, rtol=2e-7, atol=0, equal_nan=True, err_msg=str(trial))
