"""GPU parity of the bf16/f16 attention path (f32 accumulation) and the KV-cached block decode,
through the C ABI.

Bar: max |gpu - oracle| / max(|oracle|, 1) <= 1e-2, with the oracle (the reference's f32 CPU
attention) run on the same inputs rounded to bf16/f16. The outputs are rounded to the input type,
so part of the error is that final rounding (2^-9 relative for bf16, 2^-12 for f16).
"""
import numpy as np
import pytest

import _ref

pytestmark = pytest.mark.gpu

TOL_HALF = 1e-2
THREADS = 16
DTYPES = ["bf16", "f16"]


def _torch():
    import torch

    return torch


def _tdtype(name):
    torch = _torch()
    return torch.bfloat16 if name == "bf16" else torch.float16


def _dev(x, name):
    """numpy f32 -> device half tensor, and the f32 values it holds (the oracle's input)."""
    torch = _torch()
    t = torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(_tdtype(name)).cuda()
    return t, t.float().cpu().numpy()


def _inputs(seed, B, H, n_q, n_k):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, n_q, H * 64), dtype=np.float32)
    k = rng.standard_normal((B, n_k, H * 64), dtype=np.float32)
    v = rng.standard_normal((B, n_k, H * 64), dtype=np.float32)
    kv = (rng.random((B, n_k)) > 0.3).astype(np.uint8)
    kv[:, -1] = 1
    return q, k, v, kv


def _run_half(ta, name, mask, q, k, v, kv, B, H, n_q, n_k, scale, **extra):
    """Device half attention; returns (output as f32 numpy, rounded q, k, v as f32 numpy)."""
    torch = _torch()
    row = H * 64
    qd, qr = _dev(q, name)
    kd, kr = _dev(k, name)
    vd, vr = _dev(v, name)
    od = torch.full((B, n_q, row), -7.0, dtype=_tdtype(name), device="cuda")
    kvd = torch.from_numpy(np.ascontiguousarray(kv)).cuda() if kv is not None else None
    ta.fwd_checked(ta.make_args(q=qd, k=kd, v=vd, o=od, mask=mask, batch=B, heads=H, n_q=n_q, n_k=n_k,
                                q_tok=row, q_batch=n_q * row, k_tok=row, k_batch=n_k * row, v_tok=row,
                                v_batch=n_k * row, o_tok=row, o_batch=n_q * row, scale=scale, key_valid=kvd,
                                kv_batch=kv.shape[1] if kv is not None else 0, **extra))
    torch.cuda.synchronize()
    return od.float().cpu().numpy(), qr, kr, vr


def _oracle(orc, mask, q, k, v, kv, B, H, n, scale):
    row = H * 64
    o = np.zeros((B, n, row), np.float32)
    orc.batched_self_attend(THREADS, mask, np.ascontiguousarray(q), row, n * row, np.ascontiguousarray(k), row,
                            n * row, np.ascontiguousarray(v), row, n * row, o, row, n * row,
                            None if kv is None else np.ascontiguousarray(kv), n if kv is not None else 0, None, B, H,
                            n, 64, scale)
    return o


@pytest.mark.parametrize("name", DTYPES)
@pytest.mark.parametrize("mask", [0, 1, 2, 3, 4])
@pytest.mark.parametrize("n", [1, 17, 64, 65, 130, 300])
def test_half_masks_match_oracle(ta, orc, gpu_ready, name, mask, n):
    B, H = 2, 3
    q, k, v, kv = _inputs(300 + n + 11 * mask, B, H, n, n)
    got, qr, kr, vr = _run_half(ta, name, mask, q, k, v, kv, B, H, n, n, 0.125)
    want = _oracle(orc, mask, qr, kr, vr, kv, B, H, n, 0.125)
    assert _ref.scaled_err(got, want) <= TOL_HALF


@pytest.mark.parametrize("name", DTYPES)
@pytest.mark.parametrize("mask", [3, 4])
def test_half_long_left_padding(ta, orc, gpu_ready, name, mask):
    """Rows whose first 200 of 300 keys are invalid: whole 64-key tiles with no valid key are
    skipped, except where a query's own (always open) diagonal falls in them."""
    B, H, n = 3, 2, 300
    q, k, v, _ = _inputs(41 + mask, B, H, n, n)
    kv = np.ones((B, n), np.uint8)
    kv[0, :200] = 0
    kv[1, :64] = 0
    kv[2, 100:164] = 0
    got, qr, kr, vr = _run_half(ta, name, mask, q, k, v, kv, B, H, n, n, 0.125)
    want = _oracle(orc, mask, qr, kr, vr, kv, B, H, n, 0.125)
    assert _ref.scaled_err(got, want) <= TOL_HALF


@pytest.mark.parametrize("name", DTYPES)
@pytest.mark.parametrize("mask", [0, 2, 3])
@pytest.mark.parametrize("growth", [1 / 64, 1 / 8])
def test_half_growing_scores(ta, orc, gpu_ready, name, mask, growth):
    """Keys scaled by 1 + growth * key: each row's maximum score keeps rising along the keys, by
    several exp2 units per 64-key tile, so mask-free tiles taken against the running max as it
    stands overflow the weights' range and are redone with the max pass, over and over."""
    B, H, n = 2, 2, 600
    q, k, v, kv = _inputs(500 + mask, B, H, n, n)
    k *= (1.0 + growth * np.arange(n, dtype=np.float32))[None, :, None]
    got, qr, kr, vr = _run_half(ta, name, mask, q, k, v, kv, B, H, n, n, 0.125)
    want = _oracle(orc, mask, qr, kr, vr, kv, B, H, n, 0.125)
    assert _ref.scaled_err(got, want) <= TOL_HALF


@pytest.mark.parametrize("name", DTYPES)
@pytest.mark.parametrize("mask", [0, 2, 3])
def test_half_scale_one(ta, orc, gpu_ready, name, mask):
    """Unscaled logits (scale 1.0, standard deviation 8 on these inputs): q is not pre-multiplied
    by scale * log2(e) (> 1), and the weights are far from uniform."""
    B, H, n = 2, 2, 400
    q, k, v, kv = _inputs(600 + mask, B, H, n, n)
    got, qr, kr, vr = _run_half(ta, name, mask, q, k, v, kv, B, H, n, n, 1.0)
    want = _oracle(orc, mask, qr, kr, vr, kv, B, H, n, 1.0)
    assert _ref.scaled_err(got, want) <= TOL_HALF


@pytest.mark.parametrize("name", DTYPES)
def test_half_decoder_mask_matches_float64(ta, gpu_ready, name):
    B, H, ne, h, l = 3, 2, 80, 9, 70
    sl = ne + h
    q, k, v, _ = _inputs(31, B, H, h, sl)
    rng = np.random.default_rng(32)
    kv = (rng.random((B, ne)) > 0.25).astype(np.uint8)
    got, qr, kr, vr = _run_half(ta, name, 5, q, k, v, kv, B, H, h, sl, 0.125, q_pos0=ne, ctx_keys=l, chain_start=ne)
    for b in range(B):
        allowed = _ref.allowed_matrix(5, h, sl, kv[b], q_pos0=ne, ctx_keys=l, chain_start=ne)
        for hh in range(H):
            sel = slice(hh * 64, hh * 64 + 64)
            want = _ref.naive_attend(qr[b, :, sel], kr[b, :, sel], vr[b, :, sel], allowed, 0.125)
            assert _ref.scaled_err(got[b, :, sel], want) <= TOL_HALF


@pytest.mark.parametrize("name", DTYPES)
def test_half_timestral_layout_with_rope(ta, orc, gpu_ready, name):
    """Timestral TimeJob in the fused (token, qkv, head, hd) layout with per-group partial RoPE,
    at half precision: the kernel rotates in f32 and rounds the rotated q/k to the input type."""
    torch = _torch()
    rng = np.random.default_rng(33)
    rows, vall, ne, l, h, nh = 6, 3, 96, 80, 32, 2
    d, sl, hd = nh * 64, ne + h, 64
    qkv32 = rng.standard_normal(rows * sl * 3 * d).astype(np.float32)
    kv = _ref.left_pad_valid(rng, rows, ne, 20)
    bidir = np.array([0, 1, 0, 0, 1, 0], np.uint8)
    cos_t, sin_t = _ref.timestral_rope_tables(rows // vall, ne, l, h, hd, hd // 2, 10000.0, [0, 7])
    qkv_d, qkv_r = _dev(qkv32, name)
    o_d = torch.zeros(rows * sl * d, dtype=_tdtype(name), device="cuda")
    tab = {n: torch.from_numpy(x).cuda() for n, x in (("c", cos_t), ("s", sin_t))}
    kv_d = torch.from_numpy(kv).cuda()
    rc = ta.timestral_time_attention(qkv_d, o_d, tab["c"], tab["s"], kv_d, False, bidir, rows, vall, ne, l, h, d, nh,
                                     hd)
    assert rc == ta.OK, ta.last_error()
    torch.cuda.synchronize()
    roped = qkv_r.copy()
    orc.timestral_rope(THREADS, roped, cos_t, sin_t, rows, sl, vall, d, nh, hd)
    want = np.zeros(rows * sl * d, np.float32)
    orc.timestral_time_attention(THREADS, roped, want, kv.ravel(), False, bidir, rows, ne, l, h, d, nh, hd)
    assert _ref.scaled_err(o_d.float().cpu().numpy(), want) <= TOL_HALF


def test_half_prefill_full_shape_f16(ta, orc, gpu_ready):
    """Timestral-shaped causal prefill, f16: B=32 rows, H=16, L=2048, 10 % of rows with their
    oldest 512 patches invalid (one CAUSAL_KEYS call for the chunk, as Mask.pick decides per
    chunk, src/timestral/model.zig:361-362, 609)."""
    from tsfm_attn import workloads

    w = workloads.timestral_prefill()
    a = w.arrays
    assert a["padded_rows"].any()
    got, qr, kr, vr = _run_half(ta, "f16", 3, a["q"], a["k"], a["v"], a["key_valid"], w.B, w.H, w.n_q, w.n_k,
                                w.scale)
    want = _oracle(orc, 3, qr, kr, vr, a["key_valid"], w.B, w.H, w.n_q, w.scale)
    assert _ref.scaled_err(got, want) <= TOL_HALF


def test_half_prefill_back_to_back_launches_agree(ta, gpu_ready):
    """The config-5 prefill launched six times back to back on one stream (no synchronisation in
    between, as a timed loop runs it) gives the same bits every time: the kernel is deterministic,
    so a copy into LDS that a wave read before it landed shows up as a difference."""
    torch = _torch()
    from tsfm_attn import workloads

    w = workloads.timestral_prefill()
    a = w.arrays
    row = w.H * 64
    qd, _ = _dev(a["q"], "f16")
    kd, _ = _dev(a["k"], "f16")
    vd, _ = _dev(a["v"], "f16")
    kvd = torch.from_numpy(np.ascontiguousarray(a["key_valid"])).cuda()
    outs = [torch.full((w.B, w.n_q, row), -7.0, dtype=torch.float16, device="cuda") for _ in range(6)]
    for od in outs:
        ta.fwd_checked(ta.make_args(q=qd, k=kd, v=vd, o=od, mask=3, batch=w.B, heads=w.H, n_q=w.n_q, n_k=w.n_k,
                                    q_tok=row, q_batch=w.n_q * row, k_tok=row, k_batch=w.n_k * row, v_tok=row,
                                    v_batch=w.n_k * row, o_tok=row, o_batch=w.n_q * row, scale=w.scale,
                                    key_valid=kvd, kv_batch=a["key_valid"].shape[1]))
    torch.cuda.synchronize()
    first = outs[0].view(torch.int16)
    for od in outs[1:]:
        assert torch.equal(od.view(torch.int16), first)


def _decode(ta, w, name, blocks=None, fused=False):
    """Prefix append, then per block: append 32 K/V, attend its 32 queries (fused: both in one
    tsfm_kv_append_attend call, the benchmark's decode step). Returns the decoded outputs
    (B, blocks*32, H*D) as f32 and the rounded inputs."""
    torch = _torch()
    a = w.arrays
    P, nb, blk = w.meta["prefix"], w.meta["blocks"], w.meta["block"]
    nb = nb if blocks is None else blocks
    row = w.H * 64
    T = P + nb * blk
    qd, qr = _dev(a["q"][:, :T], name)
    kd, kr = _dev(a["k"][:, :T], name)
    vd, vr = _dev(a["v"][:, :T], name)
    out = torch.zeros((w.B, nb * blk, row), dtype=_tdtype(name), device="cuda")
    dt = ta.DTYPE_BF16 if name == "bf16" else ta.DTYPE_F16
    with ta.KvCache(dt, w.B, w.H, T) as cache:
        cache.append(kd, vd, P, row, T * row, row, T * row)
        for i in range(nb):
            p0 = P + i * blk
            if fused:
                cache.append_attend(kd[:, p0:], vd[:, p0:], qd[:, p0:], out[:, i * blk:], blk, w.scale, row, T * row,
                                    row, T * row, row, T * row, row, nb * blk * row)
            else:
                cache.append(kd[:, p0:], vd[:, p0:], blk, row, T * row, row, T * row)
                cache.attend(qd[:, p0:], out[:, i * blk:], blk, p0, w.scale, row, T * row, row, nb * blk * row)
            assert len(cache) == p0 + blk
        torch.cuda.synchronize()
    return out.float().cpu().numpy(), qr, kr, vr


@pytest.mark.parametrize("name", DTYPES)
def test_kv_decode_matches_causal_rows(ta, orc, gpu_ready, name):
    """Block decode over the cache equals rows [P, P+32i+32) of causal attention over the
    concatenated sequence (the equivalence with the reference's re-encoding)."""
    from tsfm_attn import workloads

    w = workloads.timestral_decode(B=4, H=3, prefix=70, blocks=5, block=32, dtype=name)
    got, qr, kr, vr = _decode(ta, w, name)
    T = 70 + 5 * 32
    want = _oracle(orc, 2, qr, kr, vr, None, w.B, w.H, T, w.scale)
    assert _ref.scaled_err(got, want[:, 70:]) <= TOL_HALF


def test_kv_decode_full_shape_bf16(ta, orc, gpu_ready):
    """Timestral-shaped decode, bf16: B=128, H=16, prefix 256, 8 blocks of 32 queries, through the
    two calls per block and through the one-launch decode block the benchmark times
    (tsfm_kv_append_attend); both against the causal rows of the oracle, and with the same bits."""
    from tsfm_attn import workloads

    w = workloads.timestral_decode()
    got, qr, kr, vr = _decode(ta, w, "bf16")
    fused = _decode(ta, w, "bf16", fused=True)[0]
    T = 256 + 8 * 32
    want = _oracle(orc, 2, qr, kr, vr, None, w.B, w.H, T, w.scale)
    assert _ref.scaled_err(got, want[:, 256:]) <= TOL_HALF
    assert _ref.scaled_err(fused, want[:, 256:]) <= TOL_HALF
    assert np.array_equal(fused, got)


@pytest.mark.parametrize("name", DTYPES)
@pytest.mark.parametrize("prefix,blk,nb", [(256, 32, 4), (70, 32, 3), (64, 17, 4), (40, 48, 2)])
def test_kv_append_attend_equals_the_two_calls(ta, orc, gpu_ready, name, prefix, blk, nb):
    """One decode block per call (tsfm_kv_append_attend) gives the bits of tsfm_kv_append then
    tsfm_kv_attend: one launch for blocks of up to 32 tokens (prefixes that leave the new tokens in
    a partly filled 32-key chunk and 64-key tile), the two calls for 48; and the causal rows of the
    oracle. Host pointers run through the same entry point too."""
    from tsfm_attn import workloads

    torch = _torch()
    w = workloads.timestral_decode(B=3, H=2, prefix=prefix, blocks=nb, block=blk, dtype=name)
    a = w.arrays
    row, T = w.H * 64, prefix + nb * blk
    qd, qr = _dev(a["q"][:, :T], name)
    kd, kr = _dev(a["k"][:, :T], name)
    vd, vr = _dev(a["v"][:, :T], name)
    dt = ta.DTYPE_BF16 if name == "bf16" else ta.DTYPE_F16
    outs = []
    for fused in (False, True):
        out = torch.zeros((w.B, nb * blk, row), dtype=_tdtype(name), device="cuda")
        with ta.KvCache(dt, w.B, w.H, T) as cache:
            cache.append(kd, vd, prefix, row, T * row, row, T * row)
            for i in range(nb):
                p0 = prefix + i * blk
                if fused:
                    cache.append_attend(kd[:, p0:], vd[:, p0:], qd[:, p0:], out[:, i * blk:], blk, w.scale, row,
                                        T * row, row, T * row, row, T * row, row, nb * blk * row)
                else:
                    cache.append(kd[:, p0:], vd[:, p0:], blk, row, T * row, row, T * row)
                    cache.attend(qd[:, p0:], out[:, i * blk:], blk, p0, w.scale, row, T * row, row, nb * blk * row)
                assert len(cache) == p0 + blk
            torch.cuda.synchronize()
        outs.append(out.cpu())
    assert torch.equal(outs[0], outs[1])
    want = _oracle(orc, 2, qr, kr, vr, None, w.B, w.H, T, w.scale)
    assert _ref.scaled_err(outs[1].float().numpy(), want[:, prefix:]) <= TOL_HALF
    # host pointers: the same entry point stages and synchronises
    kh, vh, qh = (x.view(torch.int16).cpu().numpy() for x in (kd, vd, qd))  # the raw halves
    oh = np.zeros((w.B, blk, row), np.int16)
    with ta.KvCache(dt, w.B, w.H, T) as cache:
        cache.append(kh, vh, prefix, row, T * row, row, T * row)
        at = prefix * row * 2  # byte offset of token `prefix` in each (B, T, row) array
        cache.append_attend(kh.ctypes.data + at, vh.ctypes.data + at, qh.ctypes.data + at, oh, blk, w.scale, row,
                            T * row, row, T * row, row, T * row, row, blk * row)
    assert np.array_equal(oh, outs[0][:, :blk].view(torch.int16).numpy())


def test_kv_truncate_replays_identically(ta, gpu_ready):
    from tsfm_attn import workloads

    w = workloads.timestral_decode(B=2, H=2, prefix=64, blocks=2, block=32)
    torch = _torch()
    a = w.arrays
    row, T = w.H * 64, 128
    qd, _ = _dev(a["q"][:, :T], "bf16")
    kd, _ = _dev(a["k"][:, :T], "bf16")
    vd, _ = _dev(a["v"][:, :T], "bf16")
    outs = []
    with ta.KvCache(ta.DTYPE_BF16, w.B, w.H, T) as cache:
        cache.append(kd, vd, 64, row, T * row, row, T * row)
        for _ in range(2):
            cache.truncate(64)
            o = torch.zeros((w.B, 64, row), dtype=torch.bfloat16, device="cuda")
            for i in range(2):
                p0 = 64 + 32 * i
                cache.append(kd[:, p0:], vd[:, p0:], 32, row, T * row, row, T * row)
                cache.attend(qd[:, p0:], o[:, 32 * i:], 32, p0, 0.125, row, T * row, row, 64 * row)
            torch.cuda.synchronize()
            outs.append(o.cpu())
        with pytest.raises(ta.TsfmError):
            cache.append(kd, vd, 64, row, T * row, row, T * row)  # past the capacity
        with pytest.raises(ta.TsfmError):
            cache.attend(qd, o, 32, 120, 0.125, row, T * row, row, 64 * row)  # queries past the length
    assert torch.equal(outs[0], outs[1])
