"""Independent float64 attention in numpy, the parity metric, and seeded input builders.

`naive_attend` is written from the mathematics (softmax over an explicit allowed-key matrix),
not from the reference code, so it can pin the oracle: a dropped scale, a wrong mask index or a
transposed operand in the oracle shows up as a disagreement with it.
"""
import numpy as np

FLT_MAX = np.finfo(np.float32).max


def scaled_err(got, ref):
    """max |got - ref| / max(|ref|, 1): tests/compare.py:15 of the reference."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(got - ref) / np.maximum(np.abs(ref), 1.0))) if ref.size else 0.0


def allowed_matrix(mask, n_q, n_k, key_valid=None, q_pos0=0, ctx_keys=0, chain_start=0):
    """Boolean (n_q, n_k): which keys each query reads under a mask (attn.Mask semantics; for
    KEYS_ADDITIVE the invalid keys, whose weight is ~1e-38 in the reference)."""
    i = np.arange(n_q)[:, None] + q_pos0
    j = np.arange(n_k)[None, :]
    kv = np.ones(n_k, bool) if key_valid is None else np.asarray(key_valid[:n_k], bool)
    if mask == 0:
        return np.ones((n_q, n_k), bool)
    if mask == 1:
        return np.broadcast_to(kv[None, :], (n_q, n_k)).copy()
    if mask == 2:
        return j <= i
    if mask == 3:
        return (j == i) | (kv[None, :] & (j <= i))
    if mask == 4:
        return (j == i) | kv[None, :]
    if mask == 5:
        kvc = np.zeros(n_k, bool)
        kvc[: min(ctx_keys, n_k)] = kv[: min(ctx_keys, n_k)] if key_valid is not None else True
        return (kvc[None, :] & (j < ctx_keys)) | ((j >= chain_start) & (j <= i))
    raise ValueError(mask)


def naive_attend(q, k, v, allowed, scale, bias=None):
    """float64 o = softmax over allowed keys of (scale q.k + bias), times v. Rows with no allowed
    key are uniform over every key (what the additive -FLT_MAX mask gives in that case)."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    s = scale * (q @ k.T)
    if bias is not None:
        s = s + np.asarray(bias, np.float64)
    allowed = np.asarray(allowed, bool).copy()
    empty = ~allowed.any(axis=1)
    allowed[empty, :] = True
    s[empty, :] = 0.0  # equal scores: uniform weights
    s = np.where(allowed, s, -np.inf)
    s = s - s.max(axis=1, keepdims=True)
    p = np.where(allowed, np.exp(s), 0.0)
    p /= p.sum(axis=1, keepdims=True)
    return p @ v


def bf16_round(x):
    """Round float32 to bfloat16 (nearest-even), returned as float32 values."""
    x = np.ascontiguousarray(x, np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def f16_round(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def t5_bias_table(rng, buckets, heads):
    return (rng.standard_normal((buckets, heads)) * 0.1).astype(np.float32)


def left_pad_valid(rng, batch, n, max_pad, tail_valid=0):
    """Per-row key validity: the first pad_b ~ U{0..max_pad} of the first n - tail_valid keys are
    invalid (left-truncated / missing patches); the last tail_valid keys (REG, future) are valid."""
    kv = np.ones((batch, n), np.uint8)
    pads = rng.integers(0, max_pad + 1, size=batch)
    for b, p in enumerate(pads):
        kv[b, : min(p, n - tail_valid)] = 0
    return kv


def f64_errors(outs, q, k, v, key_valid, n_series, heads, n, scale, bias=None, mask=1, threads=16):
    """Max scaled error of each array in `outs` (all (B, n, heads*64)) against float64 attention
    over the first n_series series: how far each f32 evaluation is from exact arithmetic."""
    from concurrent.futures import ThreadPoolExecutor

    def one(b):
        allowed = allowed_matrix(mask, n, n, None if key_valid is None else key_valid[b])
        errs = [0.0] * len(outs)
        for h in range(heads):
            sel = slice(h * 64, h * 64 + 64)
            ref = naive_attend(q[b, :, sel], k[b, :, sel], v[b, :, sel], allowed, scale,
                               None if bias is None else bias[h])
            for i, o in enumerate(outs):
                errs[i] = max(errs[i], scaled_err(o[b, :, sel], ref))
        return errs

    with ThreadPoolExecutor(threads) as ex:
        per = list(ex.map(one, range(n_series)))
    return [max(e[i] for e in per) for i in range(len(outs))]


ROLE_TARGET, ROLE_PAST, ROLE_KNOWN = 0, 1, 2


def variate_allowed(vall, tok, ne, key_valid_rows, roles, cov):
    """(vall, vall) bool: row iq may read row ik at token slot tok (diagonal always; else the key is
    valid on an encoder slot, and with covariates no non-target -> target and no known -> non-known
    edge)."""
    a = np.zeros((vall, vall), bool)
    for iq in range(vall):
        for ik in range(vall):
            if iq == ik:
                a[iq, ik] = True
                continue
            valid = tok >= ne or bool(key_valid_rows[ik, tok])
            bad = cov and ((roles[iq] != ROLE_TARGET and roles[ik] == ROLE_TARGET) or
                           (roles[iq] == ROLE_KNOWN and roles[ik] != ROLE_KNOWN))
            a[iq, ik] = valid and not bad
    return a


def variate_attend_f64(qkv, key_valid, roles, cov, groups, vall, ne, h, d, nh, hd):
    """Variate attention in float64 from its definition: per (group, token slot, head), softmax over
    the allowed rows of q.k / sqrt(hd), then the weighted sum of v. qkv (groups*vall, sl, 3d)."""
    sl = ne + h
    x = qkv.reshape(groups * vall, sl, 3 * d).astype(np.float64)
    kv = key_valid.reshape(groups * vall, ne)
    o = np.zeros((groups * vall, sl, d))
    for g in range(groups):
        rows = slice(g * vall, (g + 1) * vall)
        for tok in range(sl):
            allowed = variate_allowed(vall, tok, ne, kv[rows], roles, cov)
            for hh in range(nh):
                c = slice(hh * hd, (hh + 1) * hd)
                q = x[rows, tok, c]
                k = x[rows, tok, d + hh * hd:d + (hh + 1) * hd]
                v = x[rows, tok, 2 * d + hh * hd:2 * d + (hh + 1) * hd]
                s = np.where(allowed, q @ k.T / np.sqrt(hd), -np.inf)
                w = np.exp(s - s.max(axis=1, keepdims=True))
                w /= w.sum(axis=1, keepdims=True)
                o[rows, tok, c] = w @ v
    return o


def rms_norm_f64(x, scale, eps):
    """nn.rmsNorm from its definition: x / sqrt(mean(x^2) + eps) * scale, per row, in float64."""
    x = np.asarray(x, np.float64)
    return x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps) * np.asarray(scale, np.float64)


def rope_f64(x, cos_t, sin_t, seq, nh, hd=64):
    """Rotate-half RoPE of every head of x (rows = b * seq tokens, token t uses row t % seq)."""
    x = np.asarray(x, np.float64).copy()
    half = hd // 2
    rows = x.shape[0]
    c = np.asarray(cos_t, np.float64).reshape(-1, half)[np.arange(rows) % seq]
    s = np.asarray(sin_t, np.float64).reshape(-1, half)[np.arange(rows) % seq]
    for h in range(nh):
        lo = x[:, h * hd:h * hd + half].copy()
        hi = x[:, h * hd + half:(h + 1) * hd].copy()
        x[:, h * hd:h * hd + half] = lo * c - hi * s
        x[:, h * hd + half:(h + 1) * hd] = hi * c + lo * s
    return x


def chronos2_encode_f64(x, key_valid, b, seq, nh, layers, final_norm, eps, cos_t, sin_t, scale, hd=64):
    """Chronos-2 Model.encode (src/chronos2/model.zig:144-206) written from its definition in
    float64: per layer x += o(attn(rope(q), rope(k), v)) over n1(x), x += o_g(v_g(n2(x))),
    x += wo(relu(wi(n3(x)))), then the final rmsNorm."""
    x = np.asarray(x, np.float64).copy()
    d = x.shape[1]
    kv = np.asarray(key_valid, bool).reshape(b, seq)
    W = lambda a: np.asarray(a, np.float64)
    for ly in layers:
        xn = rms_norm_f64(x, ly["time_norm"], eps)
        q = rope_f64(xn @ W(ly["time_q"]).T, cos_t, sin_t, seq, nh, hd)
        k = rope_f64(xn @ W(ly["time_k"]).T, cos_t, sin_t, seq, nh, hd)
        v = xn @ W(ly["time_v"]).T
        ab = np.zeros_like(x)
        for r in range(b):
            sl = slice(r * seq, (r + 1) * seq)
            allowed = allowed_matrix(1, seq, seq, kv[r])
            for h in range(nh):
                hs = slice(h * hd, (h + 1) * hd)
                ab[sl, hs] = naive_attend(q[sl, hs], k[sl, hs], v[sl, hs], allowed, scale)
        x = x + ab @ W(ly["time_o"]).T
        xn = rms_norm_f64(x, ly["group_norm"], eps)
        x = x + (xn @ W(ly["group_v"]).T) @ W(ly["group_o"]).T
        xn = rms_norm_f64(x, ly["mlp_norm"], eps)
        x = x + np.maximum(xn @ W(ly["mlp_wi"]).T, 0.0) @ W(ly["mlp_wo"]).T
    return rms_norm_f64(x, final_norm, eps)


def chronos2_layers(rng, n_layers, d, d_ff):
    """Random-init Chronos-2 layer weights (the (out, in) nn.Weight layout), scaled so activations
    stay O(1): linear weights ~ N(0, 1/in), norm scales ~ 1 + N(0, 0.1)."""
    def lin(o, i):
        return (rng.standard_normal((o, i)) / np.sqrt(i)).astype(np.float32)

    def norm():
        return (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32)

    return [dict(time_norm=norm(), time_q=lin(d, d), time_k=lin(d, d), time_v=lin(d, d), time_o=lin(d, d),
                 group_norm=norm(), group_v=lin(d, d), group_o=lin(d, d), mlp_norm=norm(), mlp_wi=lin(d_ff, d),
                 mlp_wo=lin(d, d_ff)) for _ in range(n_layers)]


def resblock(rng, d_in, hid, d_out):
    """Random-init ResBlock weights with biases ((out, in) layout)."""
    def lin(o, i):
        return (rng.standard_normal((o, i)) / np.sqrt(i)).astype(np.float32)

    def bias(o):
        return (0.1 * rng.standard_normal(o)).astype(np.float32)

    return dict(hidden_w=lin(hid, d_in), hidden_b=bias(hid), output_w=lin(d_out, hid), output_b=bias(d_out),
                residual_w=lin(d_out, d_in), residual_b=bias(d_out))


def resblock_f64(rb, x):
    """ResBlock(.relu) from its definition: output(relu(hidden(x))) + residual(x), with biases."""
    W = lambda k: np.asarray(rb[k], np.float64)
    x = np.asarray(x, np.float64)
    h = np.maximum(x @ W("hidden_w").T + W("hidden_b"), 0.0)
    return h @ W("output_w").T + W("output_b") + x @ W("residual_w").T + W("residual_b")


def chronos2_model_forward_f64(feats, fut_feats, ctx_valid, reg, b, n_ctx, n_out, nh, layers, final_norm, eps, cos_t,
                               sin_t, scale, input_embed, output_embed):
    """The model part of the Chronos-2 forecaster (src/chronos2/forecaster.zig:155-183) in float64:
    embed, [context; REG; future] with key validity, encode, the future rows, the output head."""
    emb = resblock_f64(input_embed, feats).reshape(b, n_ctx, -1)
    fut = resblock_f64(input_embed, fut_feats).reshape(b, n_out, -1)
    d = emb.shape[2]
    seq = n_ctx + 1 + n_out
    x = np.concatenate([emb, np.broadcast_to(np.asarray(reg, np.float64), (b, 1, d)), fut], axis=1).reshape(b * seq, d)
    kv = np.concatenate([np.asarray(ctx_valid, bool).reshape(b, n_ctx), np.ones((b, 1 + n_out), bool)], axis=1)
    x = chronos2_encode_f64(x, kv, b, seq, nh, layers, final_norm, eps, cos_t, sin_t, scale).reshape(b, seq, d)
    return resblock_f64(output_embed, x[:, n_ctx + 1:].reshape(b * n_out, d))


def bolt_layers(rng, n_enc, n_dec, d, inner, d_ff):
    """Random-init Chronos-Bolt encoder and decoder layer weights ((out, in) layout)."""
    def lin(o, i):
        return (rng.standard_normal((o, i)) / np.sqrt(i)).astype(np.float32)

    def norm():
        return (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32)

    enc = [dict(attn_norm=norm(), q=lin(inner, d), k=lin(inner, d), v=lin(inner, d), o=lin(d, inner), ffn_norm=norm(),
                wi=lin(d_ff, d), wo=lin(d, d_ff)) for _ in range(n_enc)]
    dec = [dict(self_norm=norm(), self_v=lin(inner, d), self_o=lin(d, inner), cross_norm=norm(), cross_q=lin(inner, d),
                cross_k=lin(inner, d), cross_v=lin(inner, d), cross_o=lin(d, inner), ffn_norm=norm(), wi=lin(d_ff, d),
                wo=lin(d, d_ff)) for _ in range(n_dec)]
    return enc, dec


def bolt_model_forward_f64(feats, patch_valid, reg, dec_start, bias, b, n_patch, nh, enc, enc_final_norm, dec,
                           dec_final_norm, eps, input_embed, output_embed, hd=64):
    """The model part of the Chronos-Bolt forecaster (src/chronos_bolt/forecaster.zig:199-213) in
    float64 from its definition: bias is the (H, seq, seq) T5 position bias."""
    W = lambda a: np.asarray(a, np.float64)
    emb = resblock_f64(input_embed, feats).reshape(b, n_patch, -1)
    d = emb.shape[2]
    seq = n_patch + 1
    x = np.concatenate([emb, np.broadcast_to(W(reg), (b, 1, d))], axis=1).reshape(b * seq, d)
    kv = np.concatenate([np.asarray(patch_valid, bool).reshape(b, n_patch), np.ones((b, 1), bool)], axis=1)
    bias = W(bias).reshape(nh, seq, seq)
    for ly in enc:
        xn = rms_norm_f64(x, ly["attn_norm"], eps)
        q, k, v = xn @ W(ly["q"]).T, xn @ W(ly["k"]).T, xn @ W(ly["v"]).T
        ab = np.zeros_like(q)
        for r in range(b):
            sl = slice(r * seq, (r + 1) * seq)
            allowed = allowed_matrix(1, seq, seq, kv[r])
            for h in range(nh):
                hs = slice(h * hd, (h + 1) * hd)
                ab[sl, hs] = naive_attend(q[sl, hs], k[sl, hs], v[sl, hs], allowed, 1.0, bias[h])
        x = x + ab @ W(ly["o"]).T
        xn = rms_norm_f64(x, ly["ffn_norm"], eps)
        x = x + np.maximum(xn @ W(ly["wi"]).T, 0.0) @ W(ly["wo"]).T
    x = rms_norm_f64(x, enc_final_norm, eps)
    y = np.broadcast_to(W(dec_start), (b, d)).copy()
    for ly in dec:
        y = y + (rms_norm_f64(y, ly["self_norm"], eps) @ W(ly["self_v"]).T) @ W(ly["self_o"]).T
        qd = rms_norm_f64(y, ly["cross_norm"], eps) @ W(ly["cross_q"]).T
        k, v = x @ W(ly["cross_k"]).T, x @ W(ly["cross_v"]).T
        ad = np.zeros_like(qd)
        for r in range(b):
            sl = slice(r * seq, (r + 1) * seq)
            for h in range(nh):
                hs = slice(h * hd, (h + 1) * hd)
                ad[r:r + 1, hs] = naive_attend(qd[r:r + 1, hs], k[sl, hs], v[sl, hs], kv[r][None, :], 1.0)
        y = y + ad @ W(ly["cross_o"]).T
        y = y + np.maximum(rms_norm_f64(y, ly["ffn_norm"], eps) @ W(ly["wi"]).T, 0.0) @ W(ly["wo"]).T
    return resblock_f64(output_embed, rms_norm_f64(y, dec_final_norm, eps))


# ---- Timestral (src/timestral/model.zig) written from the definitions --------------------------


def timestral_positions(ne, l, h, first_obs_g):
    """Time of every token of a group relative to its first observed patch: encoder token p sits at
    p, decoder token j (index ne + j) at l + j."""
    tok = np.arange(ne + h)
    time = np.where(tok < ne, tok, l + (tok - ne))
    return time - int(first_obs_g)


def timestral_rope_tables_f64(groups, ne, l, h, hd, rope_dim, theta, first_obs):
    """float64 (groups, ne + h, hd/2) cos and sin: frequency theta^(-2i/rope_dim) for i < rope_dim/2,
    zero beyond (those dims are not rotated)."""
    half = hd // 2
    i = np.arange(half, dtype=np.float64)
    inv = np.where(i < rope_dim // 2, theta ** (-2.0 * i / rope_dim), 0.0)
    ang = np.stack([timestral_positions(ne, l, h, first_obs[g]).astype(np.float64)[:, None] * inv[None, :]
                    for g in range(groups)])
    return np.cos(ang), np.sin(ang), ang


def timestral_rope_tables(groups, ne, l, h, hd, rope_dim, theta, first_obs):
    """The float64 tables rounded once to float32, flattened as the kernels take them: an input
    builder for the GPU tests that does not go through the oracle."""
    c, s, _ = timestral_rope_tables_f64(groups, ne, l, h, hd, rope_dim, theta, first_obs)
    return c.astype(np.float32).ravel(), s.astype(np.float32).ravel()


def timestral_rope_f64(qkv, cos_t, sin_t, rows, sl, vall, d, nh, hd):
    """Rotate-half RoPE of every head of q and k (parts 0 and 1 of the (token, qkv, head, hd)
    layout) in float64; row r uses its group's table, g = r // vall."""
    half = hd // 2
    x = np.asarray(qkv, np.float64).reshape(rows, sl, 3, nh, hd).copy()
    c = np.asarray(cos_t, np.float64).reshape(-1, sl, half)
    s = np.asarray(sin_t, np.float64).reshape(-1, sl, half)
    for r in range(rows):
        cg, sg = c[r // vall][:, None, :], s[r // vall][:, None, :]
        for part in (0, 1):
            lo, hi = x[r, :, part, :, :half].copy(), x[r, :, part, :, half:].copy()
            x[r, :, part, :, :half] = lo * cg - hi * sg
            x[r, :, part, :, half:] = hi * cg + lo * sg
    return x.ravel()


def timestral_key_valid(obs, rows, vall, ne, ps, attend_missing=True):
    """(key_valid (rows, ne), first_obs (groups,), keys_all_valid): a patch is observed when any of
    its steps is; with attend_missing, every patch from a row's first observed patch on is valid.
    first_obs is the earliest observed patch over the rows of a group, 0 if it has none."""
    patch = np.asarray(obs, bool).reshape(rows, ne, ps).any(axis=2)
    kv = np.logical_or.accumulate(patch, axis=1) if attend_missing else patch
    groups = rows // vall
    gp = patch.reshape(groups, vall, ne).any(axis=1)
    first = np.where(gp.any(axis=1), gp.argmax(axis=1), 0)
    return kv.astype(np.uint8), first.astype(np.int64), bool(kv.all())


# ---- the f32 parity bar, derived from the reference itself ---------------------------------------


def reference_bar(lane8, lane16, exact=None):
    """The f32 bar for a GPU result compared with the 16-lane oracle, and its two ingredients.

    The reference computes in f32 with nn.lanes partial sums (src/core/nn.zig:296): 8 on an AVX2
    host, 16 on an AVX-512 host, so its own output moves with the host by s = |lane8 - lane16|.
    With a float64 evaluation `exact`, m = the larger distance of the two builds from it. An f32
    evaluation as accurate as the reference on its worse host is within m of exact, hence within
    2m of the 16-lane build (triangle inequality). Without `exact`, s stands in for m (s <= 2m;
    for independent rounding s ~ 1.4 m). Bar = max(1e-5, 2 max(s, m)): never tighter than the
    1e-5 parity target, never looser than the reference's own cross-host floor needs."""
    s = scaled_err(lane8, lane16)
    m = 0.0 if exact is None else max(scaled_err(lane8, exact), scaled_err(lane16, exact))
    return max(1e-5, 2.0 * max(s, m)), s, m


def assert_within_reference_bar(got, lane8, lane16, exact=None):
    bar, s, m = reference_bar(lane8, lane16, exact)
    err = scaled_err(got, lane16)
    assert err <= bar, f"GPU vs 16-lane oracle {err:.3e} > bar {bar:.3e} (cross-host spread {s:.3e}, f64 {m:.3e})"
    return err, bar


def assert_no_further_from_exact(got, lane8, lane16, exact):
    """The GPU result is at most as far from the float64 evaluation as the reference's worse host
    build (8 or 16 nn.lanes): its own rounding is no worse than the reference's."""
    g = scaled_err(got, exact)
    m = max(scaled_err(lane8, exact), scaled_err(lane16, exact))
    print(f"distance from f64: GPU {g:.3e}, reference builds {scaled_err(lane8, exact):.3e} / "
          f"{scaled_err(lane16, exact):.3e}")
    assert g <= m, f"GPU {g:.3e} from f64 > the reference's {m:.3e}"
    return g, m


# ---- the Timestral model in float64, written from its definitions ---------------------------------


def timestral_model(rng, ps=16, d=128, nh=2, hid=256, schedule=("time_variate", "time"), knots=None, block_size=32,
                    context_length=2048, rope_factor=0.5, use_asinh=True, attend_missing=True, gated=True):
    """Random-init Timestral weights and config (src/timestral/model.zig:126-200, config.zig:6-45) as a
    dict: the fused qkv weights already in the permuted (qkv, head, head_dim) row order."""
    if knots is None:
        knots = np.array([0.1, 0.2, 0.3, 0.4, 0.5, 0.6, 0.7, 0.8, 0.9])
    knots = np.ascontiguousarray(knots, np.float64)
    q = len(knots)

    def lin(o, i):
        return (rng.standard_normal((o, i)) / np.sqrt(i)).astype(np.float32)

    def norm():
        return (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32)

    axes = {"time": [True], "variate": [False], "time_variate": [True, False], "variate_time": [False, True]}
    layers = []
    for kind in schedule:
        attns = [dict(is_time=t, norm=norm(), qkv=lin(3 * d, d), out=lin(d, d), gate=lin(d, d) if gated else None)
                 for t in axes[kind]]
        layers.append(dict(attns=attns, mlp_norm=norm(), w12=lin(2 * hid, d), w3=lin(d, hid)))
    pp = resblock(rng, 2 * ps, 4 * d, d)
    hb = resblock(rng, d, 4 * d, ps * q)
    for k in ("hidden_b", "output_b", "residual_b"):
        hb[k] = None  # the head has no biases (model.zig:145)
    return dict(ps=ps, d=d, nh=nh, hid=hid, q=q, median=int(np.where(knots == 0.5)[0][0]), block_size=block_size,
                context_length=context_length, rope_dim=int(64 * rope_factor), rope_theta=10000.0, norm_eps=1e-6,
                minimum_scale=1e-6, use_asinh=use_asinh, attend_missing=attend_missing, width_factor=2.0, knots=knots,
                patch_proj=pp, head=hb, forecast_query=rng.standard_normal(d).astype(np.float32), out_norm=norm(),
                layers=layers)


def silu_f64(x):
    return x / (1.0 + np.exp(-x))


def resblock_silu_f64(rb, x):
    """ResBlock(.silu): output(silu(hidden(x))) + residual(x), biases where present."""
    W = lambda k: np.asarray(rb[k], np.float64)
    B = lambda k: 0.0 if rb.get(k) is None else np.asarray(rb[k], np.float64)
    x = np.asarray(x, np.float64)
    h = silu_f64(x @ W("hidden_w").T + B("hidden_b"))
    return h @ W("output_w").T + B("output_b") + x @ W("residual_w").T + B("residual_b")


def patch_stats_f64(x, obs, ps, min_scale):
    """Causal per-patch (mean, std) of each row: over the observed values up to the patch's last step,
    the mean (0 without any) and the sample standard deviation (ddof 1; 0 below two values), at least
    min_scale. Two-pass numpy statistics, not a running recurrence."""
    x = np.asarray(x, np.float64)
    obs = np.asarray(obs, bool)
    rows, t = x.shape
    n = t // ps
    loc = np.zeros((rows, n))
    scale = np.zeros((rows, n))
    for r in range(rows):
        for p in range(n):
            v = x[r, :(p + 1) * ps][obs[r, :(p + 1) * ps]]
            loc[r, p] = v.mean() if v.size else 0.0
            sd = v.std(ddof=1) if v.size >= 2 else 0.0
            scale[r, p] = max(sd, min_scale)
    return loc, scale


def softplus_f64(x):
    return np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))


def timestral_predict_block_f64(m, ctx, obs, t, groups, vall, h, roles=None, kf=None, kfm=None):
    """Model.predictBlock in float64: (groups * n_targets, h * ps, q) quantiles in data units. roles
    (vall) in model.Role order (ROLE_TARGET, ROLE_PAST, ROLE_KNOWN; None = all targets); kf/kfm
    (rows, h * ps) known-future values and observations. With covariates the window spans the
    context and the horizon, known rows use whole-window mean/std (none for 0/1 rows, which also
    skip the asinh) and read every valid key, and the variate firewalls apply."""
    ps, d, nh, hid, q = m["ps"], m["d"], m["nh"], m["hid"], m["q"]
    hd, rows = 64, groups * vall
    roles = [ROLE_TARGET] * vall if roles is None else list(roles)
    cov = any(r != ROLE_TARGET for r in roles)
    hl = h * ps
    w = t + hl if cov else t
    l, n = t // ps, w // ps
    ne = n
    sl = ne + h
    ctx = np.asarray(ctx, np.float64).reshape(rows, t)
    obs = np.asarray(obs, bool).reshape(rows, t)
    if cov:
        fut = np.zeros((rows, hl)) if kf is None else np.asarray(kf, np.float64).reshape(rows, hl)
        fob = np.zeros((rows, hl), bool) if kf is None else np.asarray(kfm, bool).reshape(rows, hl)
        ctx, obs = np.concatenate([ctx, fut], 1), np.concatenate([obs, fob], 1)
    loc, scale = patch_stats_f64(ctx, obs, ps, m["minimum_scale"])
    lo_t, sc_t = np.repeat(loc, ps, axis=1), np.repeat(scale, ps, axis=1)
    asinh_row = np.ones(rows, bool)
    for r in range(rows):
        if cov and roles[r % vall] == ROLE_KNOWN:
            vals = ctx[r][obs[r]]
            mu = vals.mean() if vals.size else 0.0
            sd = max(np.sqrt(((vals - mu) ** 2).mean()) if vals.size else 0.0, m["minimum_scale"])
            if vals.size and np.all((vals == 0) | (vals == 1)):
                mu, sd, asinh_row[r] = 0.0, 1.0, False
            lo_t[r], sc_t[r] = mu, sd
    sc = np.maximum(sc_t, float(np.finfo(np.float32).eps))
    v = np.where(obs, (ctx - lo_t) / sc, 0.0)
    if m["use_asinh"]:
        v = np.where(asinh_row[:, None], np.arcsinh(v), v)
    feats = np.concatenate([v.reshape(rows, n, ps), (~obs).reshape(rows, n, ps).astype(np.float64)], axis=2)
    x = np.zeros((rows, sl, d))
    x[:, :ne] = resblock_silu_f64(m["patch_proj"], feats.reshape(rows * n, 2 * ps)).reshape(rows, n, d)
    x[:, ne:] = np.asarray(m["forecast_query"], np.float64)
    kv, first, _ = timestral_key_valid(obs.astype(np.uint8), rows, vall, ne, ps, m["attend_missing"])
    c64, s64, _ = timestral_rope_tables_f64(groups, ne, l, h, hd, m["rope_dim"], m["rope_theta"], first)
    W = lambda a: np.asarray(a, np.float64)
    half = hd // 2

    def rope(y, g):  # y (sl, nh, hd)
        cg, sg = c64[g][:, None, :], s64[g][:, None, :]
        lo, hi = y[..., :half].copy(), y[..., half:].copy()
        return np.concatenate([lo * cg - hi * sg, hi * cg + lo * sg], axis=-1)

    enc_allowed = [allowed_matrix(4 if cov and roles[r % vall] == ROLE_KNOWN else 3, ne, ne, kv[r])
                   for r in range(rows)]
    dec_allowed = [allowed_matrix(5, h, sl, kv[r], q_pos0=ne, ctx_keys=l, chain_start=ne) for r in range(rows)]
    for ly in m["layers"]:
        for a in ly["attns"]:
            xn = rms_norm_f64(x, a["norm"], m["norm_eps"])
            qkv = (xn @ W(a["qkv"]).T).reshape(rows, sl, 3, nh, hd)
            if a["is_time"]:
                o = np.zeros((rows, sl, nh, hd))
                for r in range(rows):
                    qr, kr, vr = rope(qkv[r, :, 0], r // vall), rope(qkv[r, :, 1], r // vall), qkv[r, :, 2]
                    for hh in range(nh):
                        o[r, :ne, hh] = naive_attend(qr[:ne, hh], kr[:ne, hh], vr[:ne, hh], enc_allowed[r], hd ** -0.5)
                        o[r, ne:, hh] = naive_attend(qr[ne:, hh], kr[:, hh], vr[:, hh], dec_allowed[r], hd ** -0.5)
                o = o.reshape(rows, sl, d)
            else:
                o = variate_attend_f64(qkv.reshape(rows * sl, 3 * d), kv, roles, cov, groups, vall,
                                       ne, h, d, nh, hd).reshape(rows, sl, d)
            if a.get("gate") is not None:
                o = o / (1.0 + np.exp(-(xn @ W(a["gate"]).T)))
            x = x + o @ W(a["out"]).T
        xn = rms_norm_f64(x, ly["mlp_norm"], m["norm_eps"])
        hh_ = xn @ W(ly["w12"]).T
        x = x + (hh_[..., :hid] * silu_f64(hh_[..., hid:])) @ W(ly["w3"]).T
    tgt = [r for r in range(rows) if roles[r % vall] == ROLE_TARGET]
    dec = rms_norm_f64(x[tgt, ne:], m["out_norm"], m["norm_eps"])
    raw = resblock_silu_f64(m["head"], dec.reshape(len(tgt) * h, d)).reshape(len(tgt), h * ps, q)
    knots, med = np.asarray(m["knots"]), m["median"]
    widths = np.zeros(q)
    widths[med + 1:] = knots[med + 1:] - knots[med:-1]
    widths[:med] = knots[1:med + 1] - knots[:med]
    inc = m["width_factor"] * widths * softplus_f64(raw)
    out = np.empty_like(raw)
    out[..., med] = raw[..., med]
    out[..., med + 1:] = raw[..., med:med + 1] + np.cumsum(inc[..., med + 1:], axis=-1)
    out[..., :med] = raw[..., med:med + 1] - np.cumsum(inc[..., :med][..., ::-1], axis=-1)[..., ::-1]
    if m["use_asinh"]:
        out = np.sinh(out)
    return out * scale[tgt, l - 1, None, None] + loc[tgt, l - 1, None, None]


def timestral_refine_f64(qs, ctx, obs, ps, med, min_scale, exact=False):
    """refineBlock (src/timestral/forecaster.zig:582-662) from its definition, with two-pass numpy
    statistics: horizon patch j is re-framed with the mean and std (ddof 1) of the observed context
    plus the medians of patches 0..j-1 mapped into their own frames (clipped around the context
    mean), patch 0 keeping the context's last-patch frame. The frames are kept in f32 as the
    reference stores them; exact=True keeps every value in float64 instead."""
    f = np.float64 if exact else np.float32
    qs = np.asarray(qs, f)
    rows, hps, q = qs.shape
    h = hps // ps
    t = ctx.shape[1]
    l = t // ps
    loc, scale = patch_stats_f64(ctx, obs, ps, min_scale)
    clip = np.sqrt(np.float64(np.finfo(np.float32).max)) / 1e3
    out = np.empty_like(qs)
    for r in range(rows):
        loc0, scale0 = f(loc[r, l - 1]), f(scale[r, l - 1])
        vals = np.asarray(ctx[r], np.float64)[np.asarray(obs[r], bool)]
        sinh_med = (qs[r, :, med].astype(np.float64) - np.float64(loc0)) / np.float64(scale0)
        offset = vals.mean() if vals.size else 0.0
        lj, sj = [], []
        for j in range(h):
            mean = vals.mean() if vals.size else 0.0
            m2 = ((vals - mean) ** 2).sum()
            sc = max(np.sqrt(max(m2 / max(vals.size - 1.0, 1.0), 0.0)), min_scale)
            lj.append(f(mean))
            sj.append(f(sc))
            folded = np.clip(sinh_med[j * ps:(j + 1) * ps] * sc + mean - offset, -clip, clip) + offset
            vals = np.concatenate([vals, folded])
        lj[0], sj[0] = loc0, scale0
        for s in range(hps):
            a = (qs[r, s] - loc0) / scale0
            out[r, s] = a * sj[s // ps] + lj[s // ps]
    return out


def timestral_forecast_f64(m, x, obs, b, v, horizon, per_shot=32, max_context=0, cap_k=1e4, extreme=1e30,
                           symmetric=True, clip_nonnegative=True):
    """forecaster.forecast (src/timestral/forecaster.zig:57-180) for target rows in float64, composed
    from the definitions above: forecastRaw's context (forward fill, window, left padding), then
    blockDecode (predict_block, refine_block when a block has more than one patch, medians fed back
    as observed context, 0 when not finite or at least `extreme`, the oldest steps dropped past
    max_context), the quantile cap at the context's observed range widened by cap_k times its last
    patch scale, the symmetric average 0.5 (f(x) - reverse(f(-x))) over the levels, and the clip to
    zero of series whose observed values are all non-negative. (b, v, horizon, q)."""
    ps, q, med = m["ps"], m["q"], m["median"]
    max_context = max_context or m["context_length"]
    per_shot = min(per_shot, m["block_size"])
    x = np.asarray(x, np.float32).reshape(b * v, -1)
    obs = np.asarray(obs, bool).reshape(b * v, -1)

    def raw(xs):
        ctx, mask = timestral_context(xs, obs, max_context, ps)
        ctx = ctx.astype(np.float64)
        ctx0, mask0 = ctx.copy(), mask.copy()
        out = np.zeros((b * v, horizon, q))
        remaining, done = -(-horizon // ps), 0
        while remaining:
            block = min(per_shot, remaining)
            blen = block * ps
            qs = timestral_predict_block_f64(m, ctx, mask, ctx.shape[1], b, v, block)
            if block > 1:
                qs = timestral_refine_f64(qs, ctx, mask, ps, med, m["minimum_scale"], exact=True)
            take = min(blen, horizon - done)
            out[:, done:done + take] = qs[:, :take]
            remaining -= block
            done += blen
            if not remaining:
                break
            fed = qs[:, :, med].copy()
            fed[~np.isfinite(fed) | (np.abs(fed) >= extreme)] = 0.0
            ctx = np.concatenate([ctx, fed], axis=1)
            mask = np.concatenate([mask, np.ones_like(fed, bool)], axis=1)
            if ctx.shape[1] > max_context:
                keep = max(ps, max_context // ps * ps)
                ctx, mask = ctx[:, -keep:], mask[:, -keep:]
        if cap_k > 0:
            _, sc = patch_stats_f64(ctx0, mask0, ps, m["minimum_scale"])
            for r in range(b * v):
                vals = ctx0[r][mask0[r]]
                hi, lo = (vals.max(), vals.min()) if vals.size else (0.0, 0.0)
                a = sc[r, -1] * cap_k
                out[r] = np.clip(out[r], lo - a, hi + a)
        return out

    out = raw(x)
    if symmetric:
        out = 0.5 * (out - raw(-x)[..., ::-1])
    if clip_nonnegative:
        for r in range(b * v):
            seen = obs[r] & np.isfinite(x[r])
            if seen.any() and (x[r][seen] >= 0).all():
                out[r] = np.maximum(out[r], 0.0)
    return out.reshape(b, v, horizon, q)


def timestral_context(inputs, observed, max_context, ps):
    """forecastRaw's preparation (src/timestral/forecaster.zig:327-379) for target rows: forward-fill
    (leading gaps 0), keep the last max_context steps, left-pad to whole patches. (rows, t) values
    and mask."""
    x = np.asarray(inputs, np.float32)
    o = np.asarray(observed, bool)
    rows, t0 = x.shape
    keep = min(t0, max_context)
    t = (keep + ps - 1) // ps * ps
    vals = np.zeros((rows, t), np.float32)
    mask = np.zeros((rows, t), bool)
    for r in range(rows):
        last, seen = 0.0, False
        filled = np.zeros(t0, np.float32)
        for j in range(t0):
            if o[r, j]:
                last, seen = x[r, j], True
            filled[j] = last if seen else 0.0
        vals[r, t - keep:] = filled[t0 - keep:]
        mask[r, t - keep:] = o[r, t0 - keep:]
    return vals, mask
