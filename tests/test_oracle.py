"""Pins the oracle (the CPU restatement of t0-core) before it is trusted as the
GPU checker (CPU only).

  * the reference's own known-answer tests: crates/t0-core/tests/ops_tests.rs:11-72
    (RMSNorm, RoPE tables) and crates/t0-core/src/quantile.rs:82-97;
  * closed forms in float64 numpy: linear, RoPE/xPos tables, quantile head,
    causal Welford scaler, the two attention masks, weighted quantiles;
  * an independent float64 numpy forward (tests/np_ref.py) on small models;
  * the reference's integration-test invariants (batch isolation, chunking,
    ragged rows, rollout's saturating_sub) run on the oracle itself."""
import numpy as np
import pytest

import np_ref
from util import TINY, sine_mix


# ---- ops_tests.rs -------------------------------------------------------------
def test_rmsnorm_hand_computation(oracle):  # ops_tests.rs:11-24
    got = oracle.rmsnorm(np.array([[3.0, 4.0]], np.float32), np.ones(2, np.float32))
    d = np.sqrt(12.5)
    assert np.allclose(got, [[3 / d, 4 / d]], atol=1e-5)


def test_rmsnorm_applies_scale(oracle):  # ops_tests.rs:26-35
    s = np.array([2.0, 0.5, -1.0, 3.0], np.float32)
    assert (oracle.rmsnorm(np.ones((1, 4), np.float32), s)[0] == s).all()


def test_rope_zero_position_identity(oracle):  # ops_tests.rs:37-52
    c, s, x = oracle.rope_tables(1, 4)
    assert (c == 1).all() and (s == 0).all() and np.allclose(x, 1, atol=1e-6)


def test_rope_scale_halves_concat(oracle):  # ops_tests.rs:54-72
    _, _, x = oracle.rope_tables(3, 4)
    row = x[2]
    assert abs(row[0] - row[2]) < 1e-9 and abs(row[1] - row[3]) < 1e-9
    assert row[0] != row[1]


def test_rope_tables_closed_form(oracle):
    for p in (1, 2, 19, 66, 130):
        c, s, x = oracle.rope_tables(p, 64)
        wc, ws, wx = np_ref.rope_tables(p, 64)
        assert np.array_equal(c, wc.astype(np.float32))
        assert np.array_equal(s, ws.astype(np.float32))
        assert np.max(np.abs(x - wx.astype(np.float32)) / wx) < 2e-7


# ---- linear / quantile head / quantile.rs ------------------------------------------
def test_linear_matches_float64(oracle, rng):
    for m, k, n in ((1, 96, 5), (37, 768, 130), (200, 64, 300)):
        x = rng.standard_normal((m, k)).astype(np.float32)
        w = rng.standard_normal((n, k)).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        want = x.astype(np.float64) @ w.T.astype(np.float64) + b
        got = oracle.linear(x, w, b)
        assert np.max(np.abs(got - want)) <= 1e-5 * np.sqrt(k) * np.max(np.abs(want))
        assert (oracle.linear(x, w, b, relu=True) == np.maximum(got, 0)).all()


def test_quantile_head_closed_form(oracle, rng):
    x = rng.standard_normal((50, 9)).astype(np.float32)
    want = np.concatenate([x[:, :1], x[:, :1] + np.cumsum(np.log1p(np.exp(x[:, 1:].astype(np.float64))), 1)], 1)
    got = oracle.quantile_head(x)
    assert np.max(np.abs(got - want)) < 1e-5
    assert (np.diff(got, axis=1) > 0).all()
    one = rng.standard_normal((4, 1)).astype(np.float32)
    assert (oracle.quantile_head(one) == one).all()  # n_q == 1 is the identity


def test_interpolate_identity_at_trained_levels(oracle):  # quantile.rs:85-92
    lv = np.array([0.1, 0.25, 0.5, 0.75, 0.9], np.float32)
    vals = np.array([1, 2, 3, 4, 5], np.float32)
    assert np.allclose(oracle.interpolate_quantiles(lv, lv, vals), vals, atol=1e-6)


def test_prob_mass_sums_to_one(oracle):  # quantile.rs:94-97
    m = oracle.prob_mass(np.array([0.1, 0.25, 0.5, 0.75, 0.9], np.float32))
    assert abs(m.sum() - 1) < 1e-6
    assert np.allclose(m, np.array([0.25, 0.4, 0.5, 0.4, 0.25]) / 1.8, atol=1e-6)


def test_interpolation_and_weighted_quantile_brute_force(oracle, rng):
    lv = np.array([0.1, 0.25, 0.5, 0.75, 0.9], np.float32)
    vals = np.sort(rng.standard_normal(5)).astype(np.float32)
    q = np.array([0.0, 0.05, 0.1, 0.3, 0.5, 0.77, 0.95, 1.0], np.float32)
    want = np.interp(q, np.concatenate([[0], lv, [1]]), np.concatenate([[vals[0]], vals, [vals[-1]]]))
    assert np.allclose(oracle.interpolate_quantiles(q, lv, vals), want, atol=1e-6)
    s = rng.standard_normal(15).astype(np.float32)
    w = rng.uniform(0.1, 1, 15).astype(np.float32)
    order = np.argsort(s, kind="stable")
    cw = np.clip(np.cumsum(w[order] / w.sum()), 0, 1)
    want = np.interp(q, np.concatenate([[0], cw, [1]]) if cw[-1] < 1 else np.concatenate([[0], cw]),
                     np.concatenate([[s[order][0]], s[order], [s[order][-1]]]) if cw[-1] < 1
                     else np.concatenate([[s[order][0]], s[order]]))
    assert np.allclose(oracle.weighted_quantile(q, w, s), want, atol=1e-5)


# ---- scaler.rs / mask.rs ------------------------------------------------------------
def welford_closed_form(x, mask, group, eps, offset):
    v, t = x.shape
    loc, scale = np.zeros((v, t)), np.ones((v, t))
    for r in range(v):
        for c in range(t):
            sel = x[r, :c + 1][mask[r, :c + 1] == 0].astype(np.float64)
            n = sel.size
            mean = sel.mean() if n else 0.0
            var = sel.var(ddof=1) if n > 1 else 0.0
            loc[r, c] = mean
            scale[r, c] = np.sqrt(var + eps) if offset else max(np.sqrt(var), eps)
            if group[r, c] < 0:
                loc[r, c], scale[r, c] = 0.0, 1.0
    return loc, scale


@pytest.mark.parametrize("offset,eps", [(True, 0.1), (False, 0.01)])
def test_causal_scaler_closed_form(oracle, rng, offset, eps):
    v, t = 3, 300
    x = (5 + 3 * rng.standard_normal((v, t))).astype(np.float32)
    mask = np.zeros((v, t), np.int8)
    mask[0, 40:90] = 2                  # missing
    mask[1, :32] = 1                    # pad
    mask[:, 270:] = 4                   # withheld
    group = np.zeros((v, t), np.int64)
    group[1, :32] = -1
    x[mask != 0] = 0.0
    sc, loc, scale = oracle.scale_input(x, mask, group, np.zeros((v, t), np.int64), True, eps, offset)
    wl, ws = welford_closed_form(x, mask, group, eps, offset)
    assert np.max(np.abs(loc - wl)) < 1e-5 * 8
    assert np.max(np.abs(scale - ws) / ws) < 1e-5
    assert np.max(np.abs(sc - np.arcsinh((x - loc.astype(np.float32)) / scale.astype(np.float32)))) < 2e-6
    with pytest.raises(oracle.OracleError) as e:  # scaler.rs:52-54
        oracle.scale_input(x, mask, group, np.full((v, t), 2, np.int64))
    assert e.value.code == -10


def test_masks_brute_force(oracle, rng):
    v, p = 4, 7
    pg = rng.integers(-1, 2, (v, p)).astype(np.int64)
    pvt = np.zeros((v, p), np.int64)
    pvt[2, 0] = 2  # a FUTURE row attends bidirectionally
    att = rng.integers(0, 2, (v, p)).astype(np.uint8)
    import ctypes as C
    L = oracle.lib()
    tm = np.zeros((v, p, p), np.float32)
    gm = np.zeros((p, v, v), np.float32)
    L.t0r_build_time_mask(pg.ctypes.data_as(C.c_void_p), pvt.ctypes.data_as(C.c_void_p),
                          att.ctypes.data_as(C.c_void_p), v, p, tm.ctypes.data_as(C.c_void_p))
    L.t0r_build_group_mask(pg.ctypes.data_as(C.c_void_p), v, p, gm.ctypes.data_as(C.c_void_p))
    for r in range(v):
        for i in range(p):
            for j in range(p):
                ok = pg[r, i] >= 0 and pg[r, i] == pg[r, j] and (pvt[r, 0] == 2 or j <= i) and att[r, j]
                assert tm[r, i, j] == (0.0 if ok else -1e9)
    for pi in range(p):
        for a in range(v):
            for b in range(v):
                ok = pg[a, pi] >= 0 and pg[a, pi] == pg[b, pi]
                assert gm[pi, a, b] == (0.0 if ok else -1e9)


# ---- the whole forward against an independent float64 restatement -----------------------
def model_tensors(om, names):
    return {n: om.tensor(n).astype(np.float64) for n in names}


@pytest.mark.parametrize("gen,levels", [(3, (0.1, 0.25, 0.5, 0.75, 0.9)), (2, (0.5,)), (0, (0.1, 0.9))])
def test_forward_matches_float64_numpy(oracle, t0hip, rng, gen, levels):
    cfg = dict(TINY, group_every_n=gen, quantile_levels=levels)
    g = t0hip.synth_model_gguf(t0hip.make_config(**cfg), quant=0, seed=21)
    om = oracle.Model(g)
    import struct
    # every tensor name from the GGUF header
    n_t, n_m = struct.unpack_from("<QQ", g, 8)
    T = {}
    for name in [l for l in _tensor_names(g)]:
        T[name] = om.tensor(name).astype(np.float64)
    v, t = 4, 320
    x = sine_mix(rng, v, t)
    mask = np.zeros((v, t), np.int8)
    mask[1, 50:90] = 2
    mask[:, 256:] = 4
    x[mask != 0] = 0
    grp = np.repeat(np.array([[0], [0], [1], [1]]), t, 1).astype(np.int64)
    vt = np.zeros((v, t), np.int64)
    vt[3] = 1
    got = om.forward(x, mask, grp, vt)
    c = dict(cfg, n_q=len(levels))
    want = np_ref.forward(T, c, x.astype(np.float64), mask, grp, vt)
    assert np.max(np.abs(got - want)) < 1e-4 * max(1.0, np.max(np.abs(want)))


def _tensor_names(g):
    import struct
    n_t, n_m = struct.unpack_from("<QQ", g, 8)
    pos = 24

    def rstr(p):
        n = struct.unpack_from("<Q", g, p)[0]
        return g[p + 8:p + 8 + n].decode(), p + 8 + n

    for _ in range(n_m):
        _, pos = rstr(pos)
        ty = struct.unpack_from("<I", g, pos)[0]
        pos += 4
        pos += {4: 4, 6: 4, 7: 1}.get(ty, 0)
        if ty == 8:
            _, pos = rstr(pos)
        elif ty == 9:
            n = struct.unpack_from("<Q", g, pos + 4)[0]
            pos += 12 + 4 * n
    names = []
    for _ in range(n_t):
        name, pos = rstr(pos)
        nd = struct.unpack_from("<I", g, pos)[0]
        pos += 4 + 8 * nd + 12
        names.append(name)
    return names


# ---- reference integration-test invariants, on the oracle --------------------------------
@pytest.fixture(scope="module")
def tiny_oracle(oracle, t0hip):
    return oracle.Model(t0hip.synth_model_gguf(t0hip.make_config(**TINY), quant=8, seed=4))


def test_batch_equals_singles(tiny_oracle):
    """crates/t0-core/tests/batch.rs:36-66: batched signals equal single forecasts (<= 1e-5)."""
    rng = np.random.default_rng(5)
    ctx = sine_mix(rng, 6, 200)
    ctx[2, 20:60] = np.nan
    b = tiny_oracle.forecast_batch_chunked(ctx, 6, 200, 40, 0)
    for i in range(6):
        s = tiny_oracle.forecast(ctx[i:i + 1], 1, 200, 40)
        assert np.max(np.abs(b[i] - s[0])) <= 1e-5


def test_chunking_is_transparent(tiny_oracle):
    rng = np.random.default_rng(6)
    ctx = sine_mix(rng, 7, 128)
    outs = [tiny_oracle.forecast_batch_chunked(ctx, 7, 128, 32, c) for c in (1, 3, 16)]
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[1], outs[2])


def test_ragged_rows_match_standalone(tiny_oracle):
    """crates/t0-fast/tests/batch_rows.rs:30-65 gate (1e-4): rows of lengths 512/511/480/500."""
    rng = np.random.default_rng(7)
    lengths = [512, 511, 480, 500]
    rows = [sine_mix(rng, 1, L)[0] for L in lengths]
    b = tiny_oracle.forecast_batch_rows_chunked(np.concatenate(rows), lengths, 32, 0)
    for i, r in enumerate(rows):
        s = tiny_oracle.forecast(r[None], 1, len(r), 32)
        assert np.max(np.abs(b[i] - s[0])) <= 1e-4


def test_rollout_short_is_interpolated_forecast(tiny_oracle, oracle):
    rng = np.random.default_rng(8)
    ctx = sine_mix(rng, 1, 256)[0]
    q = np.array([0.1, 0.3, 0.5, 0.9], np.float32)
    r = tiny_oracle.forecast_rollout(ctx, 256, 40, q)
    f = tiny_oracle.forecast(ctx[None], 1, 256, 64)[0]
    want = np.stack([oracle.interpolate_quantiles(q, tiny_oracle.levels, f[h]) for h in range(40)])
    assert np.array_equal(r, want)


def test_rollout_saturating_tail(tiny_oracle):
    """model.rs:653-660: 1200 = 1024 + 176 steps; the last block (192) overshoots and must stop."""
    rng = np.random.default_rng(9)
    ctx = sine_mix(rng, 1, 256)[0]
    out = tiny_oracle.forecast_rollout(ctx, 256, 1200, np.array([0.2, 0.5, 0.8], np.float32))
    assert out.shape == (1200, 3) and np.isfinite(out).all()
    assert (np.diff(out, axis=1) >= -1e-6).all()  # query quantiles stay ordered


def test_horizon_limit(tiny_oracle, oracle):
    with pytest.raises(oracle.OracleError) as e:
        tiny_oracle.forecast(np.zeros((1, 64), np.float32), 1, 64, 1025)
    assert e.value.code == -9


def test_grouped_is_per_group_forecast(tiny_oracle):
    """Grouped batch (one group id per row) equals t0_core::forecast on each group's rows alone:
    groups never see each other (mask.rs:49-82) and share one window (lib.rs:50-97)."""
    rng = np.random.default_rng(10)
    ctx = sine_mix(rng, 5, 160)
    ctx[3, 40:90] = np.nan
    groups = np.array([7, 7, 2, 2, 2], np.int64)
    g = tiny_oracle.forecast_grouped(ctx, groups, 160, 48)
    for rows in ([0, 1], [2, 3, 4]):
        s = tiny_oracle.forecast(ctx[rows], len(rows), 160, 48)
        assert np.max(np.abs(g[rows] - s)) <= 1e-5


def test_grouped_ar_is_repeated_forecast(tiny_oracle):
    """Each AR step appends the median-level forecast (the level closest to 0.5) to every row and
    forecasts again from the trailing t_ctx values, as forecast_rollout does (model.rs:582-665)."""
    rng = np.random.default_rng(11)
    t_ctx, h = 128, 32
    ctx = sine_mix(rng, 4, t_ctx)
    groups = np.array([0, 0, 1, 1], np.int64)
    ar = tiny_oracle.forecast_grouped_ar(ctx, groups, t_ctx, h, 3)
    qi = int(np.argmin(np.abs(np.asarray(tiny_oracle.levels) - 0.5)))
    cur = ctx.copy()
    for step in range(3):
        f = tiny_oracle.forecast_grouped(cur, groups, t_ctx, h)
        assert np.array_equal(ar[:, step * h:(step + 1) * h], f)
        cur = np.concatenate([cur, f[:, :, qi]], axis=1)[:, -t_ctx:]
