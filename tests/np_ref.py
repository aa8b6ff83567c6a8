"""Independent float64 numpy restatement of the t0 forward (tests only).

Written from crates/t0-core/src/{model.rs:177-300, ops.rs, mask.rs} with
whole-array numpy ops (einsum, broadcasting) instead of the oracle's C loops,
so that an indexing or ordering slip in either shows up as a disagreement.
Valid for inputs without whole-PAD patches (a fully blocked softmax row is
uniform in the reference's f32 arithmetic but not in float64)."""
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
