"""Independent float64 numpy restatement of the t0 forward (tests only).

Written from crates/t0-core/src/{model.rs:177-300, 448-531, ops.rs, mask.rs,
scaler.rs, data.rs} with whole-array numpy ops (einsum, broadcasting, cumulative
sums) instead of the oracle's C loops, so that an indexing or ordering slip in
either shows up as a disagreement.

A fully blocked softmax row (every key masked) is uniform in the reference's
f32 arithmetic, where -1e9 + score rounds to -1e9 for every key; float64 keeps
the scores, so `mhsa` takes the uniform row explicitly.

The forecast wrapper (`forecast_window` and its callers) restates the window,
causal scaler, rescale and slice of model.rs:448-531 / scaler.rs:44-148 with
the closed-form running mean and variance instead of the Welford recurrence."""
import numpy as np

BLOCK = -1.0e9


def rms(x, scale, eps=1e-8):
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * scale


def linear(x, w, b):
    return x @ w.T + b


def residual_block(x, T, prefix):
    h = np.maximum(linear(x, T[f"{prefix}.mlp.hidden_layer.weight"], T[f"{prefix}.mlp.hidden_layer.bias"]), 0.0)
    o = linear(h, T[f"{prefix}.mlp.output_layer.weight"], T[f"{prefix}.mlp.output_layer.bias"])
    return o + linear(x, T[f"{prefix}.residual_layer.weight"], T[f"{prefix}.residual_layer.bias"])


def rope_tables(p, hd):
    half = hd // 2
    pos = np.arange(p, dtype=np.float64)[:, None]
    j = np.arange(half, dtype=np.float64)[None, :]
    ang = pos * (1.0 / 10000.0 ** (2 * j / hd))
    power = (pos - np.floor((p - 1) / 2.0)) / 512.0
    s = ((2 * j + 0.4 * hd) / (1.4 * hd)) ** power
    cos = np.repeat(np.cos(ang), 2, axis=1)   # interleaved f0,f0,f1,f1
    sin = np.repeat(np.sin(ang), 2, axis=1)
    scale = np.concatenate([s, s], axis=1)    # halves-concat
    return cos, sin, scale


def rotate_half(x):
    x2 = x.reshape(*x.shape[:-1], -1, 2)
    return np.stack([-x2[..., 1], x2[..., 0]], axis=-1).reshape(x.shape)


def mhsa(x, T, li, heads, mask, rope):
    o_, s_, E = x.shape
    hd = E // heads
    p = f"transformer.layers.{li}.attention_block.attention"
    qkv = linear(x, T[f"{p}.wQKV.weight"], T[f"{p}.wQKV.bias"]).reshape(o_, s_, 3, heads, hd)
    q = qkv[:, :, 0].transpose(0, 2, 1, 3)
    k = qkv[:, :, 1].transpose(0, 2, 1, 3)
    v = qkv[:, :, 2].transpose(0, 2, 1, 3)
    q = rms(q, T[f"{p}.q_norm.scale"])
    k = rms(k, T[f"{p}.k_norm.scale"])
    if rope is not None:
        cos, sin, sc = rope
        q = q * cos * sc + rotate_half(q) * sin * sc
        k = k * cos / sc + rotate_half(k) * sin / sc
    s = np.einsum("ohid,ohjd->ohij", q, k) / np.sqrt(hd) + np.where(mask[:, None], 0.0, BLOCK)
    s = s - s.max(-1, keepdims=True)
    a = np.exp(s)
    a = a / a.sum(-1, keepdims=True)
    blocked = ~mask.any(-1)[:, None, :, None]  # [o, 1, i, 1]
    a = np.where(blocked, 1.0 / mask.shape[-1], a)
    out = np.einsum("ohij,ohjd->ohid", a, v).transpose(0, 2, 1, 3).reshape(o_, s_, E)
    return linear(out, T[f"{p}.wO.weight"], T[f"{p}.wO.bias"])


def reduce_meta(meta, mask, ps):
    v, t = mask.shape
    m = meta.reshape(v, t // ps, ps)
    k = mask.reshape(v, t // ps, ps)
    nonpad = k != 1
    first = np.argmax(nonpad, axis=-1)
    val = np.take_along_axis(m, first[..., None], -1)[..., 0]
    return np.where(nonpad.any(-1), val, -1), nonpad.any(-1)


def forward(T, cfg, variates, mask, group_ids, variate_type):
    ps, E, heads, H, nq = cfg["patch_size"], cfg["embed_dim"], cfg["num_heads"], cfg["mlp_hidden_dim"], cfg["n_q"]
    v, t = variates.shape
    p = t // ps
    vals = variates.reshape(v, p, ps).astype(np.float64)
    kk = np.broadcast_to(np.arange(ps) / ps, (v, p, ps))
    valid = (mask.reshape(v, p, ps) == 0).astype(np.float64)
    concat = np.concatenate([vals, kk, valid], axis=-1)
    x = residual_block(concat, T, "patch_encoder.projection")
    pvt, att = reduce_meta(variate_type, mask, ps)
    pg, _ = reduce_meta(group_ids, mask, ps)
    x = x + T["patch_encoder.type_embeddings.weight"][np.maximum(pvt, 0)]
    future = (pvt[:, 0] == 2)[:, None, None]
    ii, jj = np.meshgrid(np.arange(p), np.arange(p), indexing="ij")
    same = (pg[:, :, None] >= 0) & (pg[:, :, None] == pg[:, None, :])
    tmask = same & (future | (jj <= ii)[None]) & att[:, None, :]
    gsame = (pg.T[:, :, None] >= 0) & (pg.T[:, :, None] == pg.T[:, None, :])
    rope = rope_tables(p, E // heads)
    n = cfg["group_every_n"]
    layers = cfg["num_layers"] if n <= 0 else (cfg["num_layers"] // n) * n  # config.rs:45-56 truncates
    for li in range(layers):
        is_group = n > 0 and li % n == n - 1
        normed = rms(x, T[f"transformer.layers.{li}.attention_block.norm.scale"])
        if is_group:
            a = mhsa(normed.transpose(1, 0, 2), T, li, heads, gsame, None).transpose(1, 0, 2)
        else:
            a = mhsa(normed, T, li, heads, tmask, rope)
        x = x + a
        h = linear(rms(x, T[f"transformer.layers.{li}.norm.scale"]), T[f"transformer.layers.{li}.mlp.0.weight"],
                   T[f"transformer.layers.{li}.mlp.0.bias"])
        g, u = h[..., :H], h[..., H:]
        x = x + linear(g / (1 + np.exp(-g)) * u, T[f"transformer.layers.{li}.mlp.2.weight"],
                       T[f"transformer.layers.{li}.mlp.2.bias"])
    x = rms(x, T["transformer.out_norm.scale"])
    d = residual_block(x, T, "decoder").reshape(v, p, ps, nq)
    inc = np.log1p(np.exp(d[..., 1:]))
    return np.concatenate([d[..., :1], d[..., :1] + np.cumsum(inc, axis=-1)], axis=-1)


# ---- forecast wrapper: model.rs:448-531, scaler.rs:44-148, data.rs:52-155 ------------------------
VALID, PAD, MISSING, WITHHELD = 0, 1, 2, 4


def from_context(ctx, t_ctx, horizon, row_group=None):
    """data.rs:52-86: NaN -> MISSING (value 0); `horizon` WITHHELD steps appended; group 0 per row
    (or `row_group[r]`, the explicit per-row ids of the grouped batch)."""
    v = ctx.shape[0]
    t = t_ctx + horizon
    x = np.zeros((v, t))
    mask = np.full((v, t), WITHHELD, np.int8)
    nan = np.isnan(ctx)
    x[:, :t_ctx] = np.where(nan, 0.0, ctx)
    mask[:, :t_ctx] = np.where(nan, MISSING, VALID)
    g = np.zeros((v, t), np.int64) if row_group is None else np.repeat(np.asarray(row_group, np.int64)[:, None], t, 1)
    return x, mask, g, np.zeros((v, t), np.int64)


def pad(series, ps, context_end, pad_right=False):
    """data.rs:110-155 TimeSeries::pad: PAD columns on the left up to a patch boundary (group and
    type -1), then the horizon rounded up to whole patches with the row's last group/type, WITHHELD
    for targets.  `pad_right` puts the context's PAD columns after the context instead (a planted
    mistake for negative controls)."""
    x, mask, g, vt = series
    if pad_right:
        n = (ps - context_end % ps) % ps
        ins = lambda a, fill: np.concatenate([a[:, :context_end], np.full((a.shape[0], n), fill, a.dtype),
                                              a[:, context_end:]], axis=1)
        x, mask, g, vt = ins(x, 0.0), ins(mask, PAD), ins(g, -1), ins(vt, -1)
        context_end += n
    v, t = x.shape
    horizon = t - context_end
    pl = (ps - context_end % ps) % ps
    pr = -(-horizon // ps) * ps - horizon
    nt = pl + t + pr
    X = np.zeros((v, nt))
    M = np.full((v, nt), PAD, np.int8)
    G = np.full((v, nt), -1, np.int64)
    VT = np.full((v, nt), -1, np.int64)
    X[:, pl:pl + t], M[:, pl:pl + t], G[:, pl:pl + t], VT[:, pl:pl + t] = x, mask, g, vt
    G[:, pl + t:] = g[:, -1:]
    VT[:, pl + t:] = vt[:, -1:]
    M[:, pl + t:] = np.where(vt[:, -1:] == 0, WITHHELD, PAD)
    return X, M, G, VT


def causal_stats(x, mask, group, eps, variance_offset):
    """scaler.rs:44-118 in closed form: at step c the mean and sample variance of the VALID values
    in [0, c] (mean 0 and variance 0 before two of them), scale = sqrt(var + eps) or max(sqrt(var),
    eps); loc 0 / scale 1 where the group id is negative."""
    valid = (mask == VALID).astype(np.float64)
    n = np.cumsum(valid, axis=1)
    shift = np.where(valid.sum(1, keepdims=True) > 0,
                     (x * valid).sum(1, keepdims=True) / np.maximum(valid.sum(1, keepdims=True), 1), 0.0)
    d = (x - shift) * valid  # variance is shift-invariant; shifting keeps the sums well conditioned
    s1 = np.cumsum(d, axis=1)
    s2 = np.cumsum(d * d, axis=1)
    mean_d = np.where(n > 0, s1 / np.maximum(n, 1), 0.0)
    loc = np.where(n > 0, mean_d + shift, 0.0)
    var = np.where(n > 1, np.maximum(s2 - n * mean_d * mean_d, 0.0) / np.maximum(n - 1, 1), 0.0)
    scale = np.sqrt(var + eps) if variance_offset else np.maximum(np.sqrt(var), eps)
    neg = group < 0
    return np.where(neg, 0.0, loc), np.where(neg, 1.0, scale)


def forecast_window(T, cfg, raw, t_ctx, horizon, slice_shift=0, rescale_step=None, pad_right=False):
    """model.rs:448-531 (forecast_series_prepare + forecast_series_finish) on one raw window.

    The keyword arguments plant mistakes for negative controls: `slice_shift` moves the first
    output patch off context_patches - 1, `rescale_step` rescales with another step of each patch
    than its last, `pad_right` pads the context on the wrong side."""
    ps, nq = cfg["patch_size"], cfg["n_q"]
    pl = (ps - t_ctx % ps) % ps
    padded_h = -(-horizon // ps) * ps
    ctx_p = (t_ctx + pl) // ps
    x, mask, g, vt = pad(raw, ps, t_ctx, pad_right)
    v, t = x.shape
    loc, scale = causal_stats(x, mask, g, cfg.get("scaler_eps", 0.1), cfg.get("variance_offset", True))
    z = (x - loc) / scale
    scaled = np.arcsinh(z) if cfg.get("use_arcsinh", True) else z
    pred = forward(T, cfg, scaled, mask, g, vt)  # [v, p, ps, nq]
    p = t // ps
    step = ps - 1 if rescale_step is None else rescale_step
    l = loc.reshape(v, p, ps)[:, :, step][:, :, None, None]
    s = scale.reshape(v, p, ps)[:, :, step][:, :, None, None]
    u = np.sinh(pred) if cfg.get("use_arcsinh", True) else pred
    pred = u * s + l
    first = ctx_p - 1 + slice_shift
    out = pred[:, first:first + padded_h // ps].reshape(v, padded_h, nq)
    return out[:, :horizon]


def forecast(T, cfg, ctx, t_ctx, horizon, **plant):
    """model.rs:322-333 forecast: the v rows of `ctx` form one joint series (group 0)."""
    return forecast_window(T, cfg, from_context(np.asarray(ctx, np.float64), t_ctx, horizon), t_ctx, horizon, **plant)


def forecast_grouped(T, cfg, ctx, row_group, t_ctx, horizon, **plant):
    """One window, an explicit group id per row (the grouped batch)."""
    raw = from_context(np.asarray(ctx, np.float64), t_ctx, horizon, row_group)
    return forecast_window(T, cfg, raw, t_ctx, horizon, **plant)


def forecast_rows(T, cfg, rows, horizon, **plant):
    """crates/t0-fast/src/lib.rs:175-242: ragged rows, each left-padded with PAD to the longest
    patch-aligned length, group id = row index, one window."""
    ps = cfg["patch_size"]
    common = max(-(-len(r) // ps) * ps for r in rows)
    n, t = len(rows), common + horizon
    x = np.zeros((n, t))
    mask = np.full((n, t), PAD, np.int8)
    g = np.full((n, t), -1, np.int64)
    vt = np.full((n, t), -1, np.int64)
    for i, r in enumerate(rows):
        r = np.asarray(r, np.float64)
        lead = common - len(r)
        nan = np.isnan(r)
        x[i, lead:common] = np.where(nan, 0.0, r)
        mask[i, lead:common] = np.where(nan, MISSING, VALID)
        g[i, lead:] = i
        vt[i, lead:] = 0
        mask[i, common:] = WITHHELD
    return forecast_window(T, cfg, (x, mask, g, vt), common, horizon, **plant)
