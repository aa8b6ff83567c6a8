"""End-to-end parity on the GPU: forward pass and every forecast entry point
against the oracle (the CPU restatement of t0-core) on the same GGUF bytes.

Gate: quantiles within 5e-3 max-abs of the oracle, measured in units of each
series' own scale (the causal scaler's std at the forecast origin) so that
series multiplied by a large lognormal factor are held to the same relative
standard; the raw max-abs is asserted too for unit-scale inputs."""
import os

import numpy as np
import pytest

from util import BASELINE, SMALL, TINY, nan_gaps, sine_mix

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = 5e-3


@pytest.fixture(scope="module")
def models(t0hip, oracle, engine):
    out = {}
    for name, cfg in (("tiny", TINY), ("small", SMALL)):
        for q in (t0hip.Q8_0, t0hip.Q4_0, t0hip.F16):
            g = t0hip.synth_model_gguf(t0hip.make_config(**cfg), quant=q, seed=11)
            out[(name, q)] = (t0hip.load_model_from_gguf(engine, g), oracle.Model(g))
    return out


def reference_contexts():
    """The reference's own fixture inputs (fixtures/*_context.f32): case0 sine, case1 trivariate, case2 NaN gap."""
    ctx = {}
    for name, v in (("case0_univariate_sine", 1), ("case1_trivariate_freqs", 3), ("case2_masked_gap", 1)):
        a = np.fromfile(os.path.join(GOLDEN, f"{name}_context.f32"), dtype="<f4")
        ctx[name] = (a.reshape(v, -1), v)
    return ctx


def row_scale(ctx):
    """Each row's std over its valid values (the scale the causal scaler divides by)."""
    s = np.array([np.nanstd(r) if np.isfinite(r).any() else 1.0 for r in ctx], np.float64)
    return np.maximum(s, 1e-3)


def assert_close(got, want, scale=None, tol=TOL):
    assert got.shape == want.shape
    assert np.isfinite(got).all()
    d = np.abs(got.astype(np.float64) - want)
    if scale is not None:
        d = d / scale.reshape(-1, *([1] * (d.ndim - 1)))
    assert d.max() <= tol, float(d.max())


def prepared_series(oracle, ctx, ps=32):
    """A padded + scaled series the way forecast_series_prepare builds one (model.rs:448-482)."""
    v, t_ctx = ctx.shape
    t = t_ctx + 64
    var = np.zeros((v, t), np.float32)
    var[:, :t_ctx] = np.nan_to_num(ctx)
    mask = np.full((v, t), 4, np.int8)
    mask[:, :t_ctx] = np.where(np.isnan(ctx), 2, 0)
    grp = np.zeros((v, t), np.int64)
    vt = np.zeros((v, t), np.int64)
    sc, _, _ = oracle.scale_input(var, mask, grp, vt)
    return sc, mask, grp, vt


@pytest.mark.parametrize("q", [8, 2, 1])
@pytest.mark.parametrize("name", ["tiny", "small"])
def test_forward_with_traces(models, t0hip, oracle, rng, name, q):
    gm, om = models[(name, q)]
    ctx = sine_mix(rng, 3, 512)
    ctx[1, 100:160] = np.nan
    sc, mask, grp, vt = prepared_series(oracle, ctx)
    out, pe, l0 = t0hip.forward(gm, sc, mask, grp, vt, trace=True)
    want, wpe, wl0 = om.forward(sc, mask, grp, vt, trace=True)
    assert_close(pe, wpe, tol=2e-3)
    assert_close(l0, wl0, tol=5e-3)
    assert_close(out, want)


@pytest.mark.parametrize("q", [8, 2])
def test_forecast_reference_fixture_inputs(models, t0hip, oracle, engine, q):
    """t0-cli parity --backend fast pattern (main.rs:583-664): same GGUF, same fixture contexts,
    GPU forecast vs the CPU path, context 512 / horizon 96."""
    gm, om = models[("small", q)]
    for name, (ctx, v) in reference_contexts().items():
        got = t0hip.forecast(engine, gm, ctx, v, ctx.shape[1], 96)
        want = om.forecast(ctx, v, ctx.shape[1], 96)
        assert_close(got, want, scale=row_scale(ctx))


def test_forecast_unaligned_and_short(models, t0hip, oracle, engine, rng):
    """Context and horizon not patch-aligned (left pad + right WITHHELD pad, data.rs:110-155)."""
    gm, om = models[("tiny", 8)]
    for t_ctx, h in ((500, 30), (33, 1), (64, 96), (1000, 8)):
        ctx = sine_mix(rng, 2, t_ctx)
        got = t0hip.forecast(engine, gm, ctx, 2, t_ctx, h)
        want = om.forecast(ctx, 2, t_ctx, h)
        assert_close(got, want, scale=row_scale(ctx))


def test_batch_chunked_and_isolation(models, t0hip, oracle, engine, rng):
    """forecast_batch_chunked vs the oracle, and batch isolation (t0-core tests/batch.rs:36-66):
    each signal in a batch equals its standalone forecast."""
    gm, om = models[("small", 8)]
    n, t_ctx, h = 20, 512, 64
    ctx = nan_gaps(rng, sine_mix(rng, n, t_ctx) * np.exp(rng.standard_normal((n, 1))).astype(np.float32))
    got = t0hip.forecast_batch_chunked(engine, gm, ctx, n, t_ctx, h, 8)
    want = om.forecast_batch_chunked(ctx, n, t_ctx, h, 16)
    assert_close(got, want, scale=row_scale(ctx))
    one_chunk = t0hip.forecast_batch_chunked(engine, gm, ctx, n, t_ctx, h, 0)
    for i in (0, 7, 19):
        single = t0hip.forecast(engine, gm, ctx[i:i + 1], 1, t_ctx, h)
        assert_close(single, one_chunk[i:i + 1], scale=row_scale(ctx[i:i + 1]), tol=1e-3)


def test_batch_rows_ragged(models, t0hip, oracle, engine, rng):
    """Ragged rows (t0-fast tests/batch_rows.rs:30-65: lengths 512/511/480/500) vs the oracle and
    vs standalone forecasts of each row."""
    gm, om = models[("small", 2)]
    lengths = [512, 511, 480, 500, 77]
    rows = [sine_mix(rng, 1, L)[0] for L in lengths]
    flat = np.concatenate(rows)
    got = t0hip.forecast_batch_rows_chunked(engine, gm, flat, lengths, 40, 0)
    want = om.forecast_batch_rows_chunked(flat, lengths, 40, 0)
    sc = row_scale(np.array([np.pad(r, (0, 512 - len(r)), constant_values=np.nan) for r in rows]))
    assert_close(got, want, scale=sc)
    for i, r in enumerate(rows):
        alone = t0hip.forecast(engine, gm, r[None], 1, len(r), 40)
        assert_close(alone, got[i:i + 1], scale=sc[i:i + 1], tol=1e-3)


def test_grouped_multivariate(models, t0hip, oracle, engine, rng):
    """Multivariate batch (BASELINE config 4 shape, scaled down): series of 3 variates sharing a
    group id, lognormal per-series scale, 10% NaN gaps in runs of 16-128."""
    gm, om = models[("small", 2)]
    n_series, v, t_ctx, h = 6, 3, 1024, 64
    base = sine_mix(rng, n_series * v, t_ctx)
    scale = np.repeat(np.exp(rng.standard_normal(n_series)), v).astype(np.float32)[:, None]
    ctx = nan_gaps(rng, base * scale)
    groups = np.repeat(np.arange(n_series) * 7 + 3, v)
    got = t0hip.forecast_grouped(engine, gm, ctx, groups, t_ctx, h)
    want = om.forecast_grouped(ctx, groups, t_ctx, h)
    assert_close(got, want, scale=row_scale(ctx))


def test_grouped_ar(models, t0hip, oracle, engine, rng):
    """BASELINE config 5 shape (scaled down): AR steps append each row's median quantile."""
    gm, om = models[("tiny", 8)]
    n_rows, t_ctx, h, steps = 8, 256, 64, 3
    ctx = sine_mix(rng, n_rows, t_ctx)
    groups = np.repeat(np.arange(2), 4)
    got = t0hip.forecast_grouped_ar(engine, gm, ctx, groups, t_ctx, h, steps)
    want = om.forecast_grouped_ar(ctx, groups, t_ctx, h, steps)
    assert_close(got, want, scale=row_scale(ctx), tol=2e-2)
    assert_close(got[:, :h], want[:, :h], scale=row_scale(ctx))


def test_rollout(models, t0hip, oracle, engine, rng):
    """forecast_rollout past MAX_HORIZON (model.rs:582-665): 1024 + 176 steps (the saturating_sub case)."""
    gm, om = models[("tiny", 8)]
    ctx = sine_mix(rng, 1, 300)
    q = np.array([0.1, 0.5, 0.9], np.float32)
    got = t0hip.forecast_rollout(engine, gm, ctx[0], 300, 1200, q)
    want = om.forecast_rollout(ctx[0], 300, 1200, q)
    assert got.shape == (1200, 3)
    assert_close(got[:1024], want[:1024], scale=row_scale(ctx))
    assert_close(got, want, scale=row_scale(ctx), tol=5e-2)


def test_two_models_interleaved_bit_identical(t0hip, engine, rng):
    """t0-fast tests/pool_isolation.rs:43-84: two models on one engine, calls A,B,A,B are
    bit-identical to isolated runs (each model owns its workspace)."""
    ga = t0hip.synth_model_gguf(t0hip.make_config(**TINY), quant=8, seed=1)
    gb = t0hip.synth_model_gguf(t0hip.make_config(**TINY), quant=2, seed=2)
    ctx = sine_mix(rng, 2, 256)
    a = t0hip.load_model_from_gguf(engine, ga)
    ra = t0hip.forecast(engine, a, ctx, 2, 256, 32)
    b = t0hip.load_model_from_gguf(engine, gb)
    rb = t0hip.forecast(engine, b, ctx, 2, 256, 32)
    for _ in range(2):
        assert np.array_equal(t0hip.forecast(engine, a, ctx, 2, 256, 32), ra)
        assert np.array_equal(t0hip.forecast(engine, b, ctx, 2, 256, 32), rb)


def test_error_paths_on_device(models, t0hip, engine, rng):
    gm, _ = models[("tiny", 8)]
    ctx = sine_mix(rng, 1, 64)
    with pytest.raises(t0hip.T0HipError) as e:
        t0hip.forecast(engine, gm, ctx, 1, 64, 1025)
    assert e.value.status == "HORIZON"
    with pytest.raises(t0hip.T0HipError) as e:
        t0hip.forecast(engine, gm, sine_mix(rng, 1, 9000), 1, 9000, 32)
    assert e.value.status == "UNSUPPORTED"
    with pytest.raises(t0hip.T0HipError) as e:
        t0hip.forecast_grouped(engine, gm, ctx, np.array([-1]), 64, 32)
    assert e.value.status == "INVALID_ARG"


def test_profiler_all_kinds_and_one_kind(models, t0hip, engine, rng):
    """Event timing of every kernel kind, then of one kind only: the one-kind run times the
    same launches of that kind and nothing else, and neither changes the forecast."""
    gm, _ = models[("tiny", 8)]
    layers = TINY["num_layers"]
    ctx = sine_mix(rng, 3, 256)
    want = t0hip.forecast(engine, gm, ctx, 3, 256, 32)
    gm.profile(True)
    got = t0hip.forecast(engine, gm, ctx, 3, 256, 32)
    full = gm.profile_report()
    gm.profile(False)
    assert np.array_equal(got, want)
    n_sw, ms_sw = full["gemm_w0_swiglu"]
    assert n_sw > 0 and n_sw % layers == 0 and ms_sw > 0
    assert sum(1 for n, _ in full.values() if n) >= 5
    gm.profile_kind("gemm_w0_swiglu")
    got = t0hip.forecast(engine, gm, ctx, 3, 256, 32)
    one = gm.profile_report()
    gm.profile(False)
    assert np.array_equal(got, want)
    assert one["gemm_w0_swiglu"][0] == n_sw and one["gemm_w0_swiglu"][1] > 0
    assert all(n == 0 for k, (n, _) in one.items() if k != "gemm_w0_swiglu")
    # stopped: a further forward records nothing
    t0hip.forecast(engine, gm, ctx, 3, 256, 32)
    assert all(n == 0 for n, _ in gm.profile_report().values())
    with pytest.raises(t0hip.T0HipError) as e:
        gm.profile_kind("")
    assert e.value.status == "INVALID_ARG"


def test_baseline_model_forecast(t0hip, oracle, engine, rng):
    """The BASELINE synthetic model (12 layers, embed 768, Q8_0), config 3 input: one series,
    sum of 3 sines + N(0, 0.1), context 2048, horizon 64."""
    g = t0hip.synth_model_gguf(t0hip.make_config(**BASELINE), quant=8, seed=0)
    gm = t0hip.load_model_from_gguf(engine, g)
    om = oracle.Model(g)
    ctx = sine_mix(rng, 1, 2048)
    got = t0hip.forecast(engine, gm, ctx, 1, 2048, 64)
    want = om.forecast(ctx, 1, 2048, 64)
    assert_close(got, want, scale=row_scale(ctx))
    assert_close(got, want)


def test_config5_windows_small_model(t0hip, oracle, engine, rng):
    """BASELINE config 5's window (ctx 4096: 130 patches, the long time-attention path) on a small
    model, 2 series x 8 variates, 3 autoregressive steps of 64 against the oracle."""
    from util import trend_season_t
    g = t0hip.synth_model_gguf(t0hip.make_config(**SMALL), quant=8, seed=12)
    gm = t0hip.load_model_from_gguf(engine, g)
    om = oracle.Model(g)
    n_series, v, t_ctx, h, steps = 2, 8, 4096, 64, 3
    ctx = trend_season_t(rng, n_series * v, t_ctx)
    groups = np.repeat(np.arange(n_series), v).astype(np.int64)
    got = t0hip.forecast_grouped_ar(engine, gm, ctx, groups, t_ctx, h, steps)
    want = om.forecast_grouped_ar(ctx, groups, t_ctx, h, steps)
    scale = row_scale(ctx)
    assert_close(got[:, :h], want[:, :h], scale=scale)
    assert_close(got, want, scale=scale, tol=2e-2)


def test_config5_full_size(t0hip, oracle, engine, rng):
    """BASELINE config 5 at full size: 64 series x 8 variates, ctx 4096, 8 autoregressive steps of 64,
    Q8_0 BASELINE model with weights resident across steps.  Checked by batch isolation (series 0
    alone gives the same steps; not bit for bit, since its 16 decoder rows take the exact-f32
    small-M GEMM while the full batch takes the f16-operand MFMA one) and, for series 0's first
    step, against the oracle."""
    from util import trend_season_t
    g = t0hip.synth_model_gguf(t0hip.make_config(**BASELINE), quant=8, seed=0)
    gm = t0hip.load_model_from_gguf(engine, g)
    n_series, v, t_ctx, h, steps = 64, 8, 4096, 64, 8
    ctx = trend_season_t(rng, n_series * v, t_ctx)
    groups = np.repeat(np.arange(n_series), v).astype(np.int64)
    full = t0hip.forecast_grouped_ar(engine, gm, ctx, groups, t_ctx, h, steps)
    assert full.shape == (n_series * v, steps * h, 9) and np.isfinite(full).all()
    alone = t0hip.forecast_grouped_ar(engine, gm, ctx[:v], groups[:v], t_ctx, h, steps)
    scale = row_scale(ctx[:v])
    assert_close(full[:v, :h], alone[:, :h], scale=scale, tol=1e-3)
    assert_close(full[:v], alone, scale=scale, tol=2e-2)
    om = oracle.Model(g)
    want = om.forecast_grouped(ctx[:v], groups[:v], t_ctx, h)
    assert_close(full[:v, :h], want, scale=scale)


def test_config4_full_size(t0hip, oracle, engine, rng):
    """BASELINE config 4 at full size, as bench.py times it: 256 series x 3 variates (one group id
    per series), ctx 2048, horizon 64, sine mixture x lognormal scale with 10% NaN gaps in runs of
    16-128, Q4_0 BASELINE model; 50,688 patch rows, so every layer GEMM runs the register-operand
    MFMA kernel.  Two series of the full batch against the oracle (5e-3 of each row's scale), and
    batch isolation: series 0 alone (its 198 rows take the medium-M kernel) gives the same forecast
    up to 1e-2, the sum of the two paths' allowed distances from the oracle (each is checked
    against it at 5e-3; rows leaking across series would differ by order 1)."""
    n_series, v, t_ctx, h = 256, 3, 2048, 64
    g = t0hip.synth_model_gguf(t0hip.make_config(**BASELINE), quant=2, seed=0)
    gm = t0hip.load_model_from_gguf(engine, g)
    x = sine_mix(rng, n_series * v, t_ctx) * np.repeat(np.exp(rng.standard_normal(n_series)), v)[:, None].astype(np.float32)
    x = nan_gaps(rng, x)
    groups = np.repeat(np.arange(n_series), v).astype(np.int64)
    full = t0hip.forecast_grouped(engine, gm, x, groups, t_ctx, h)
    assert full.shape == (n_series * v, h, 9) and np.isfinite(full).all()
    om = oracle.Model(g)
    for s in (0, 137):
        rows = slice(s * v, (s + 1) * v)
        want = om.forecast_grouped(x[rows], groups[rows], t_ctx, h)
        assert_close(full[rows], want, scale=row_scale(x[rows]))
    alone = t0hip.forecast_grouped(engine, gm, x[:v], groups[:v], t_ctx, h)
    assert_close(alone, om.forecast_grouped(x[:v], groups[:v], t_ctx, h), scale=row_scale(x[:v]))
    assert_close(full[:v], alone, scale=row_scale(x[:v]), tol=2 * TOL)
