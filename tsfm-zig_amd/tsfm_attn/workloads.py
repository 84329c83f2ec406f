"""Synthetic attention workloads at the shapes of tsfm-zig's model families, with their
algorithmic FLOP and byte counts. Used by the benchmark and the parity tests; numpy only.

Counting rules (per call):
  FLOPs = 4 * D * (scored query-key pairs): non-causal pairs are n_q * n_k per (b, h) with padding
          not subtracted; causal pairs are n(n+1)/2; decode pairs are each query's visible prefix.
  bytes = q + k + v + o read/written once at the element size (plus, for decode, the cache re-read
          of every block).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict

import numpy as np

MI355X_PEAK = {  # dense, per GPU
    "f32_mfma_tflops": 157.3,
    "f16_mfma_tflops": 2516.6,
    "bf16_mfma_tflops": 2516.6,
    "hbm_gbps": 8000.0,
}


def left_pad_valid(rng: np.random.Generator, batch: int, n: int, max_pad: int, lead: int) -> np.ndarray:
    """(batch, n) uint8 key validity: the first pad_b ~ U{0..max_pad} of the first `lead` keys are
    invalid (left-padded / missing leading patches); everything else is valid."""
    kv = np.ones((batch, n), np.uint8)
    pads = rng.integers(0, max_pad + 1, size=batch)
    for b, p in enumerate(pads):
        kv[b, : min(int(p), lead)] = 0
    return kv


@dataclass
class Workload:
    name: str
    dtype: str
    B: int
    H: int
    n_q: int
    n_k: int
    D: int = 64
    scale: float = 1.0
    arrays: Dict[str, np.ndarray] = field(default_factory=dict)
    meta: Dict[str, object] = field(default_factory=dict)

    @property
    def pairs(self) -> int:
        return int(self.meta.get("pairs", self.B * self.H * self.n_q * self.n_k))

    @property
    def flops(self) -> float:
        if "flops" in self.meta:  # not an attention count (the projection workload)
            return float(self.meta["flops"])
        return 4.0 * self.D * self.pairs

    @property
    def bytes(self) -> float:
        return float(self.meta["bytes"])


def chronos2(B: int = 64, H: int = 12, n_ctx: int = 512, n_fut: int = 64, seed: int = 0, scale: float = 0.125,
             theta: float = 10000.0) -> Workload:
    """Chronos-2 encoder time attention: sequence [512 context patches; REG; 64 future patches]
    (src/chronos2/forecaster.zig:162-174), RoPE on q and k, additive key mask with 0-25% of the
    context patches of each series left-padded invalid. Inputs (B, L, H*D) f32 ~ N(0, 1)."""
    L = n_ctx + 1 + n_fut
    D = 64
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, L, H * D), dtype=np.float32)
    k = rng.standard_normal((B, L, H * D), dtype=np.float32)
    v = rng.standard_normal((B, L, H * D), dtype=np.float32)
    kv = left_pad_valid(rng, B, L, n_ctx // 4, n_ctx)
    half = D // 2
    inv = (1.0 / np.power(np.float32(theta), np.arange(0, D, 2, dtype=np.float32) / np.float32(D))).astype(np.float32)
    ang = (np.arange(L, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float32)
    cos_t = np.cos(ang).astype(np.float32).reshape(L * half)
    sin_t = np.sin(ang).astype(np.float32).reshape(L * half)
    w = Workload("chronos2_time_attention", "f32", B, H, L, L, D, scale,
                 dict(q=q, k=k, v=v, key_valid=kv, rope_cos=cos_t, rope_sin=sin_t),
                 dict(n_ctx=n_ctx, n_fut=n_fut, theta=theta, seed=seed, num_layers=12))
    w.meta["bytes"] = 4.0 * 4 * B * L * H * D
    return w


def bolt(B: int = 256, H: int = 12, n_patch: int = 128, seed: int = 0, buckets: int = 32, max_distance: int = 128
         ) -> Workload:
    """Chronos-Bolt-base encoder self-attention: [128 patches; REG], no score scale, T5 relative
    bias from a (buckets, H) table ~ N(0, 0.1), additive mask over left-truncated NaN patches."""
    L = n_patch + 1
    D = 64
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, L, H * D), dtype=np.float32)
    k = rng.standard_normal((B, L, H * D), dtype=np.float32)
    v = rng.standard_normal((B, L, H * D), dtype=np.float32)
    kv = left_pad_valid(rng, B, L, n_patch // 4, n_patch)
    table = (rng.standard_normal((buckets, H)) * 0.1).astype(np.float32)
    w = Workload("bolt_self_attention", "f32", B, H, L, L, D, 1.0, dict(q=q, k=k, v=v, key_valid=kv, rel_table=table),
                 dict(buckets=buckets, max_distance=max_distance, seed=seed, num_layers=12))
    w.meta["bytes"] = 4.0 * 4 * B * L * H * D
    return w


def timestral_prefill(B: int = 32, H: int = 16, L: int = 2048, seed: int = 0, dtype: str = "f16",
                      pad_rows: float = 0.1, pad_keys: int = 512) -> Workload:
    """Timestral-shaped causal prefill over L patches: rows (series x variates) folded into B; a
    fraction of the rows get causal_keys with their oldest `pad_keys` patches invalid."""
    D = 64
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, L, H * D), dtype=np.float32)
    k = rng.standard_normal((B, L, H * D), dtype=np.float32)
    v = rng.standard_normal((B, L, H * D), dtype=np.float32)
    padded = rng.random(B) < pad_rows
    kv = np.ones((B, L), np.uint8)
    kv[padded, :pad_keys] = 0
    w = Workload("timestral_causal_prefill", dtype, B, H, L, L, D, 1.0 / np.sqrt(D),
                 dict(q=q, k=k, v=v, key_valid=kv, padded_rows=padded.astype(np.uint8)),
                 dict(seed=seed, pairs=B * H * L * (L + 1) // 2))
    w.meta["bytes"] = 2.0 * 4 * B * L * H * D
    return w


def timestral_decode(B: int = 128, H: int = 16, prefix: int = 256, blocks: int = 8, block: int = 32, seed: int = 0,
                     dtype: str = "bf16") -> Workload:
    """Block-autoregressive decode against a KV cache: a prefix of `prefix` tokens, then `blocks`
    blocks of `block` queries; each block is causal over the cache and earlier rows of the block,
    and appends its K/V before the next block."""
    D = 64
    rng = np.random.default_rng(seed)
    T = prefix + blocks * block
    q = rng.standard_normal((B, T, H * D), dtype=np.float32)
    k = rng.standard_normal((B, T, H * D), dtype=np.float32)
    v = rng.standard_normal((B, T, H * D), dtype=np.float32)
    pairs = 0
    reread = 0
    for i in range(blocks):
        p0 = prefix + i * block
        pairs += sum(p0 + t + 1 for t in range(block))
        reread += (p0 + block) * D * 2 * 2  # K and V of the whole cache, per (b, h)
    w = Workload("timestral_kv_decode", dtype, B, H, blocks * block, T, D, 1.0 / np.sqrt(D),
                 dict(q=q, k=k, v=v), dict(prefix=prefix, blocks=blocks, block=block, seed=seed, pairs=B * H * pairs))
    # q + o of the decoded blocks, the new K/V written once, and every block's cache read.
    w.meta["bytes"] = float(B * H * (2 * blocks * block * D * 2 + 2 * blocks * block * D * 2) + B * H * reread)
    return w


def timestral_variate(groups: int = 8, vall: int = 4, H: int = 16, L: int = 2048, seed: int = 0,
                      pad_rows: float = 0.1, pad_keys: int = 512) -> Workload:
    """Timestral variate attention at the prefill shape: `groups` series of `vall` rows (target,
    past covariate, two known-future covariates) over L token slots; at every slot the rows of a
    series attend each other, per head, with the covariate firewalls and key validity; the result
    is gated by sigmoid(gate). f32 (the reference arithmetic). FLOPs count the vall x vall pairs of
    every (series, slot, head); bytes are the fused qkv, the gate and o, once."""
    D = 64
    d = H * D
    rows = groups * vall
    rng = np.random.default_rng(seed)
    qkv = rng.standard_normal((rows, L, 3 * d), dtype=np.float32)
    gate = rng.standard_normal((rows, L, d), dtype=np.float32)
    padded = rng.random(rows) < pad_rows
    kv = np.ones((rows, L), np.uint8)
    kv[padded, :pad_keys] = 0
    roles = np.array(([0, 1, 2, 2] * 4)[:vall], np.uint8)
    w = Workload("timestral_variate_attention", "f32", groups, H, vall, vall, D, 1.0 / np.sqrt(D),
                 dict(qkv=qkv, gate=gate, key_valid=kv, roles=roles),
                 dict(seed=seed, groups=groups, vall=vall, L=L, pairs=groups * L * H * vall * vall))
    w.meta["bytes"] = 4.0 * rows * L * (3 * d + d + d)
    return w


def chronos2_projection(B: int = 64, H: int = 12, n_ctx: int = 512, n_fut: int = 64, seed: int = 0,
                        theta: float = 10000.0) -> Workload:
    """Chronos-2 time-attention projections at the attention's shape (src/chronos2/model.zig:232-245):
    x (B * L, d) ~ N(0, 1) standing for the rmsNorm output, W_q, W_k, W_v (d, d) ~ N(0, 1/d), RoPE
    tables (L, 32) as the attention workload's. FLOPs = 2 * tokens * d * 3d; bytes = x and the three
    weights read once, q, k, v written once, plus the tables."""
    L, D = n_ctx + 1 + n_fut, 64
    d = H * D
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((B * L, d), dtype=np.float32)
    ws = [(rng.standard_normal((d, d), dtype=np.float32) / np.float32(np.sqrt(d))).astype(np.float32)
          for _ in range(3)]
    half = D // 2
    inv = (1.0 / np.power(np.float32(theta), np.arange(0, D, 2, dtype=np.float32) / np.float32(D))).astype(np.float32)
    ang = (np.arange(L, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float32)
    cos_t = np.cos(ang).astype(np.float32).reshape(L * half)
    sin_t = np.sin(ang).astype(np.float32).reshape(L * half)
    tokens = B * L
    flops = 2.0 * tokens * d * 3 * d
    nbytes = 4.0 * (tokens * d + 3 * d * d + 3 * tokens * d + 2 * L * half)
    return Workload("chronos2_qkv_projection", "f32", B, H, L, L, D, 1.0,
                    dict(x=x, wq=ws[0], wk=ws[1], wv=ws[2], rope_cos=cos_t, rope_sin=sin_t),
                    dict(d_model=d, tokens=tokens, flops=flops, bytes=nbytes, seed=seed, num_layers=12))


def chronos2_encoder(B: int = 64, H: int = 12, n_ctx: int = 512, n_fut: int = 64, d_ff: int = 3072,
                     n_layers: int = 12, seed: int = 0, eps: float = 1e-6, theta: float = 10000.0) -> Workload:
    """The Chronos-2 encoder stack (src/chronos2/model.zig:144-206) at the Chronos-2-base size:
    d_model 768, 12 heads, d_ff 3072, 12 layers, over the attention workload's 64 series x 577
    tokens with the same left padding. Random-init weights (linear ~ N(0, 1/in), norm scales
    ~ 1 + N(0, 0.1)); x ~ N(0, 1) stands for the embedded patches. FLOPs per call: per layer
    2 * tokens * (6 d^2 + 2 d d_ff) for the seven linear layers plus the time attention's
    4 * 64 * H * B * L^2, times the layers. Bytes: x in and out once, the weights once, and per layer
    the activations each launch streams (norm in/out, q/k/v, attention in/out, the MLP hidden)."""
    L, D = n_ctx + 1 + n_fut, 64
    d = H * D
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((B * L, d), dtype=np.float32)
    kv = left_pad_valid(rng, B, L, n_ctx // 4, n_ctx)

    def lin(o, i):
        return (rng.standard_normal((o, i), dtype=np.float32) / np.float32(np.sqrt(i))).astype(np.float32)

    def norm():
        return (1.0 + 0.1 * rng.standard_normal(d, dtype=np.float32)).astype(np.float32)

    layers = [dict(time_norm=norm(), time_q=lin(d, d), time_k=lin(d, d), time_v=lin(d, d), time_o=lin(d, d),
                   group_norm=norm(), group_v=lin(d, d), group_o=lin(d, d), mlp_norm=norm(), mlp_wi=lin(d_ff, d),
                   mlp_wo=lin(d, d_ff)) for _ in range(n_layers)]
    half = D // 2
    inv = (1.0 / np.power(np.float32(theta), np.arange(0, D, 2, dtype=np.float32) / np.float32(D))).astype(np.float32)
    ang = (np.arange(L, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float32)
    tokens = B * L
    flops = n_layers * (2.0 * tokens * (6 * d * d + 2 * d * d_ff) + 4.0 * D * H * B * L * L)
    w_bytes = 4.0 * n_layers * (6 * d * d + 2 * d * d_ff + 3 * d)
    act = 4.0 * tokens * (2 * d + 3 * d + 4 * d + 2 * d + 2 * d + 2 * d + 2 * d_ff + 2 * d_ff + 2 * d)
    nbytes = 4.0 * tokens * d * 2 + w_bytes + n_layers * act
    return Workload("chronos2_encoder", "f32", B, H, L, L, D, 1.0,
                    dict(x=x, key_valid=kv, rope_cos=np.cos(ang).astype(np.float32).reshape(L * half),
                         rope_sin=np.sin(ang).astype(np.float32).reshape(L * half),
                         final_norm=norm()),
                    dict(layers=layers, d_model=d, d_ff=d_ff, n_layers=n_layers, eps=eps, tokens=tokens, flops=flops,
                         bytes=nbytes, seed=seed, num_layers=n_layers))


def chronos2_forecast(B: int = 64, context: int = 8192, horizon: int = 1024, quantiles: int = 21, patch: int = 16,
                      seed: int = 0) -> Workload:
    """The whole Chronos-2-base forecast at the attention workload's shape: 64 series of 8192 raw
    steps (512 context patches) and a 1024-step horizon (64 future patches), so the sequence is the
    attention's 577 tokens, through the 12-layer encoder of chronos2_encoder (same weights), the
    input and output ResBlocks (hidden d_ff, 21 quantiles) and the forecaster's instance norm,
    asinh space and inverse scaling (time_encoding_scale 8192). Each series is a period-24
    sinusoid of amplitude 10 plus a trend plus N(0, 1) noise, with its oldest 0-25 % of steps
    missing (whole patches, as the attention workload's left padding) and 2 % of the rest.
    FLOPs: the encoder's plus both ResBlocks' products."""
    w = chronos2_encoder(B=B, n_ctx=context // patch, n_fut=(horizon + patch - 1) // patch, seed=seed)
    a, m = w.arrays, w.meta
    d, F = m["d_model"], m["d_ff"]
    n_ctx, n_out = context // patch, (horizon + patch - 1) // patch
    rng = np.random.default_rng(seed + 1)

    def block(i, h, o):
        return dict(hidden_w=(rng.standard_normal((h, i)) / np.sqrt(i)).astype(np.float32),
                    hidden_b=(0.1 * rng.standard_normal(h)).astype(np.float32),
                    output_w=(rng.standard_normal((o, h)) / np.sqrt(h)).astype(np.float32),
                    output_b=(0.1 * rng.standard_normal(o)).astype(np.float32),
                    residual_w=(rng.standard_normal((o, i)) / np.sqrt(i)).astype(np.float32),
                    residual_b=(0.1 * rng.standard_normal(o)).astype(np.float32))

    ie, oe = block(3 * patch, F, d), block(d, F, quantiles * patch)
    t = np.arange(context, dtype=np.float64)
    slope = rng.uniform(-0.01, 0.01, (B, 1))
    ctx = 10.0 * np.sin(2 * np.pi * t / 24.0) + slope * t + rng.standard_normal((B, context))
    ctx[rng.random(ctx.shape) < 0.02] = np.nan
    pad = rng.integers(0, n_ctx // 4 + 1, B)
    for b in range(B):
        ctx[b, : pad[b] * patch] = np.nan
    rows_in, rows_out = B * (n_ctx + n_out), B * n_out
    f_res = 2.0 * rows_in * (3 * patch * F + F * d + 3 * patch * d) + \
        2.0 * rows_out * (d * F + F * quantiles * patch + d * quantiles * patch)
    return Workload("chronos2_forecast", "f32", B, w.H, w.n_q, w.n_k, 64, 1.0,
                    dict(ctx=ctx.astype(np.float32), rope_cos=a["rope_cos"], rope_sin=a["rope_sin"],
                         final_norm=a["final_norm"], reg=(rng.standard_normal(d)).astype(np.float32)),
                    dict(m, ie=ie, oe=oe, context=context, horizon=horizon, quantiles=quantiles, patch=patch,
                         time_scale=float(context), flops=m["flops"] + f_res))


def bolt_forward(B: int = 16, n_patch: int = 32, H: int = 8, d_ff: int = 2048, n_layers: int = 6, quantiles: int = 9,
                 horizon: int = 64, patch: int = 16, buckets: int = 32, max_distance: int = 128, seed: int = 0,
                 eps: float = 1e-6) -> Workload:
    """The Chronos-Bolt-small model forward at the end-to-end configuration: 16 series x 512 context
    steps = 32 patches of 16 + [REG], d_model 512, 8 heads of 64, d_ff 2048, 6 encoder + 6 decoder
    layers, 9 quantiles x 64 steps. Random-init weights (linear ~ N(0, 1/in), biases ~ N(0, 0.01),
    norm scales ~ 1 + N(0, 0.1)); patch features [values ~ N(0, 1), mask] with 2 % of the steps
    missing. FLOPs: every linear layer (2 rows out in) and the attention products."""
    rng = np.random.default_rng(seed)
    d = inner = H * 64
    seq = n_patch + 1
    out = quantiles * horizon
    vals = rng.standard_normal((B * n_patch, patch)).astype(np.float32)
    mask = (rng.random((B * n_patch, patch)) >= 0.02).astype(np.float32)
    feats = np.concatenate([vals * mask, mask], axis=1).astype(np.float32)
    pv = (mask.reshape(B, n_patch, patch).max(axis=2) > 0).astype(np.uint8)

    def lin(o, i):
        return (rng.standard_normal((o, i), dtype=np.float32) / np.float32(np.sqrt(i))).astype(np.float32)

    def norm():
        return (1.0 + 0.1 * rng.standard_normal(d, dtype=np.float32)).astype(np.float32)

    def block(i, h, o):
        return dict(hidden_w=lin(h, i), hidden_b=(0.1 * rng.standard_normal(h)).astype(np.float32),
                    output_w=lin(o, h), output_b=(0.1 * rng.standard_normal(o)).astype(np.float32),
                    residual_w=lin(o, i), residual_b=(0.1 * rng.standard_normal(o)).astype(np.float32))

    enc = [dict(attn_norm=norm(), q=lin(inner, d), k=lin(inner, d), v=lin(inner, d), o=lin(d, inner), ffn_norm=norm(),
                wi=lin(d_ff, d), wo=lin(d, d_ff)) for _ in range(n_layers)]
    dec = [dict(self_norm=norm(), self_v=lin(inner, d), self_o=lin(d, inner), cross_norm=norm(), cross_q=lin(inner, d),
                cross_k=lin(inner, d), cross_v=lin(inner, d), cross_o=lin(d, inner), ffn_norm=norm(), wi=lin(d_ff, d),
                wo=lin(d, d_ff)) for _ in range(n_layers)]
    ie, oe = block(2 * patch, d_ff, d), block(d, d_ff, out)
    rows = B * seq
    f_enc = n_layers * (2.0 * rows * (4 * d * inner + 2 * d * d_ff) + 4.0 * 64 * H * B * seq * seq)
    f_dec = n_layers * (2.0 * B * (4 * d * inner + 2 * d * d_ff) + 2.0 * rows * 2 * d * inner + 4.0 * 64 * H * B * seq)
    f_emb = 2.0 * B * n_patch * (2 * patch * d_ff + d_ff * d + 2 * patch * d) + 2.0 * B * (d * d_ff + d_ff * out + d * out)
    w_bytes = 4.0 * (sum(a.size for ly in enc + dec for a in ly.values()) + sum(a.size for a in ie.values()) +
                     sum(a.size for a in oe.values()))
    # The raw context of the end-to-end run: each series a period-24 sinusoid of amplitude 10 plus
    # a linear trend plus N(0, 1) noise (its own generator from the seed), 2 % of the steps NaN.
    crng = np.random.default_rng(seed)
    t = np.arange(n_patch * patch, dtype=np.float64)
    slope = crng.uniform(-0.05, 0.05, (B, 1))
    ctx = 10.0 * np.sin(2 * np.pi * t / 24.0) + slope * t + crng.standard_normal((B, t.size))
    ctx[crng.random(ctx.shape) < 0.02] = np.nan
    return Workload("bolt_small_forward", "f32", B, H, seq, seq, 64, 1.0,
                    dict(feats=feats, patch_valid=pv, ctx=ctx.astype(np.float32), reg=norm(), dec_start=norm(),
                         rel_table=(0.1 * rng.standard_normal((buckets, H))).astype(np.float32),
                         enc_final_norm=norm(), dec_final_norm=norm()),
                    dict(enc=enc, dec=dec, ie=ie, oe=oe, d_model=d, d_ff=d_ff, n_patch=n_patch, out=out, eps=eps,
                         buckets=buckets, max_distance=max_distance, flops=f_enc + f_dec + f_emb,
                         bytes=w_bytes + 4.0 * (feats.size + B * out), seed=seed, num_layers=2 * n_layers))


def timestral_forecast(B: int = 128, context_patches: int = 256, blocks: int = 8, per_shot: int = 32, d: int = 1024,
                       H: int = 16, hid: int = 2816, patch: int = 16, seed: int = 0,
                       schedule=("time_variate", "time", "time_variate", "time")) -> Workload:
    """The Timestral forecast at the decode configuration's shape: 128 univariate series of
    context_patches x 16 steps (4096), a horizon of 8 decode blocks of 32 patches (4096 steps), a
    Timestral-shaped model of d_model 1024, 16 heads of 64, four layers (time+variate, time,
    time+variate, time; sigmoid gates), SwiGLU width 2816 (2/3 of 4 d, rounded to 256), 9 quantile
    knots, asinh space, random-init f32 weights (linear ~ N(0, 1/in), norm scales ~ 1 + N(0, 0.1)).
    The model dict has the keys of the forecast binding (tsfm_attn.timestral_forecast_args). Each
    series is a period-24 sinusoid of amplitude 10 plus a trend plus N(0, 1) noise, its oldest
    0-25 % of steps missing and 2 % of the rest. Symmetric averaging doubles the rows (the mirrored
    pass). meta carries the FLOP counts of the cached decode (each block runs its new patches and
    decoder tokens) and of the reference's re-encoding decode (each block re-encodes the grown
    context)."""
    rng = np.random.default_rng(seed)
    knots = np.array([0.1, 0.2, 0.3, 0.4, 0.5, 0.6, 0.7, 0.8, 0.9])
    q = len(knots)

    def lin(o, i):
        return (rng.standard_normal((o, i)) / np.sqrt(i)).astype(np.float32)

    def norm():
        return (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32)

    def resblock(i, h, o, biases=True):
        rb = dict(hidden_w=lin(h, i), output_w=lin(o, h), residual_w=lin(o, i))
        for k, n in (("hidden_b", h), ("output_b", o), ("residual_b", o)):
            rb[k] = (0.1 * rng.standard_normal(n)).astype(np.float32) if biases else None
        return rb

    axes = {"time": [True], "variate": [False], "time_variate": [True, False], "variate_time": [False, True]}
    layers = []
    for kind in schedule:
        attns = [dict(is_time=t, norm=norm(), qkv=lin(3 * d, d), out=lin(d, d), gate=lin(d, d)) for t in axes[kind]]
        layers.append(dict(attns=attns, mlp_norm=norm(), w12=lin(2 * hid, d), w3=lin(d, hid)))
    model = dict(ps=patch, d=d, nh=H, hid=hid, q=q, median=4, block_size=per_shot, context_length=8192, rope_dim=32,
                 rope_theta=10000.0, norm_eps=1e-6, minimum_scale=1e-6, use_asinh=True, attend_missing=True,
                 width_factor=2.0, knots=knots, patch_proj=resblock(2 * patch, 4 * d, d),
                 head=resblock(d, 4 * d, patch * q, biases=False), forecast_query=rng.standard_normal(d).astype(np.float32),
                 out_norm=norm(), layers=layers)
    t = context_patches * patch
    horizon = blocks * per_shot * patch
    steps = np.arange(t, dtype=np.float64)
    slope = rng.uniform(-0.01, 0.01, (B, 1))
    x = 10.0 * np.sin(2 * np.pi * steps / 24.0) + slope * steps + rng.standard_normal((B, t))
    obs = rng.random((B, t)) >= 0.02
    lead = rng.integers(0, context_patches // 4 + 1, B) * patch
    for b in range(B):
        obs[b, : lead[b]] = False
    x[~obs] = 0.0
    rows = 2 * B  # the mirrored pass of the symmetric average runs in the same batch
    n_time = sum(1 for ly in layers for a in ly["attns"] if a["is_time"])
    n_var = sum(1 for ly in layers for a in ly["attns"] if not a["is_time"])

    def flops(cached: bool) -> float:
        f = 0.0
        for i in range(blocks):
            l = context_patches + i * per_shot  # encoder tokens (context patches) of block i
            p0 = l - per_shot if (cached and i > 0) else 0  # first encoder token this block runs
            m, h = l - p0, per_shot
            n = m + h
            f += 2.0 * m * (2 * patch * 4 * d + 4 * d * d + 2 * patch * d)       # patch embedding
            f += len(layers) * 2.0 * n * 3 * hid * d                                # SwiGLU MLPs
            f += (n_time + n_var) * 2.0 * n * 5 * d * d                             # q/k/v, gate, out
            enc_pairs = sum(p0 + j + 1 for j in range(m))                           # causal encoder rows
            dec_pairs = h * l + h * (h + 1) // 2                                    # context + own chain
            f += n_time * 4.0 * 64 * H * (enc_pairs + dec_pairs)
            f += n_var * 4.0 * 64 * H * n                                           # one row per series
            f += 2.0 * h * (d * 4 * d + 4 * d * patch * q + d * patch * q)         # quantile head
        return rows * f

    w = Workload("timestral_forecast", "f32", B, H, blocks * per_shot, context_patches + blocks * per_shot, 64,
                 0.125, dict(inputs=x.astype(np.float32), observed=obs.astype(np.uint8)),
                 dict(model=model, context=t, horizon=horizon, per_shot=per_shot, blocks=blocks, d_model=d, hid=hid,
                      n_layers=len(layers), schedule=list(schedule), flops=flops(True),
                      reencode_flops=flops(False), bytes=0.0, seed=seed, num_layers=len(layers)))
    return w
