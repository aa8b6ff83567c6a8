"""End-to-end parity on the GPU: forward pass and every forecast entry point
against the oracle (the CPU restatement of t0-core) on the same GGUF bytes.

Gate: quantiles within 5e-3 max-abs of the oracle, measured in units of each
series' own scale, the causal scaler's scale at the forecast origin
(sqrt(sample variance of the valid values + eps), scaler.rs:91-118, the unit
the model's inputs and outputs are measured in), so that series multiplied by a
large lognormal factor are held to the same relative standard; the raw max-abs
is asserted too for unit-scale inputs and printed beside the normalized figure
for scaled ones.  Autoregressive and rollout steps are held to the same bar by
feeding both paths the oracle's own windows at every step (teacher forcing);
the GPU loops themselves are checked bit for bit against the GPU's single-step
calls on the windows they build."""
import os

import numpy as np
import pytest

from util import BASELINE, SMALL, TINY, ar_windows, median_index, nan_gaps, rollout_blocks, sine_mix

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


def row_scale(ctx, eps=0.1):
    """Each row's causal-scaler scale at the forecast origin, sqrt(var + eps) over its valid
    values (scaler.rs:91-118, variance_offset mode, the tests' models' eps): the factor the
    model's outputs are multiplied by on their way back to the series' units."""
    out = []
    for r in np.atleast_2d(ctx):
        x = r[np.isfinite(r)].astype(np.float64)
        var = x.var(ddof=1) if x.size > 1 else 0.0
        out.append(np.sqrt(var + eps))
    return np.array(out)


def assert_close(got, want, scale=None, tol=TOL):
    assert got.shape == want.shape
    assert np.isfinite(got).all()
    d = np.abs(got.astype(np.float64) - want)
    if scale is not None:
        d = d / scale.reshape(-1, *([1] * (d.ndim - 1)))
    assert d.max() <= tol, float(d.max())


def report(tag, got, want, scale):
    """Raw and normalized max-abs error, printed (pytest -s shows them) and returned."""
    d = np.abs(got.astype(np.float64) - want)
    raw = float(d.max())
    norm = float((d / scale.reshape(-1, *([1] * (d.ndim - 1)))).max())
    print(f"{tag}: raw max-abs {raw:.3e}, normalized {norm:.3e} (row scales {scale.min():.3g}..{scale.max():.3g})",
          flush=True)
    return raw, norm


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


def mixed_series(rng, t=320, inconsistent=False):
    """A padded + scaled series exercising every mask branch (mask.rs:12-82): a TARGET row, a
    FUTURE row (bidirectional time attention) and a HISTORICAL row led by two whole-PAD patches
    sharing group 5; rows of groups 7 and 8; a row whose group id is negative throughout (every
    key blocked: uniform attention); MISSING and WITHHELD steps.  With `inconsistent`, one row
    switches group from 7 to 8 half-way, so group attention cannot use per-row segments."""
    ps, v = 32, 7
    x = rng.standard_normal((v, t)).astype(np.float32)
    mask = np.zeros((v, t), np.int8)
    grp = np.zeros((v, t), np.int64)
    vt = np.zeros((v, t), np.int64)
    grp[0:3] = 5
    vt[1] = 2
    vt[2] = 1
    mask[2, :2 * ps] = 1
    grp[2, :2 * ps] = -1
    vt[2, :2 * ps] = -1
    grp[3] = 7
    if inconsistent:
        grp[3, t // 2:] = 8
    grp[4] = 7
    grp[5] = 8
    grp[6] = -1
    mask[0, 40:75] = 2
    mask[4, 100:110] = 2
    mask[[0, 3, 4, 5], t - 48:] = 4
    x[mask != 0] = 0.0
    return x, mask, grp, vt


@pytest.mark.parametrize("inconsistent", [False, True])
@pytest.mark.parametrize("q", [8, 2])
def test_forward_future_pad_and_groups(models, t0hip, oracle, rng, q, inconsistent):
    """t0h_forward against the oracle on FUTURE, whole-PAD, negative-group and per-patch
    inconsistent-group rows (the branches a forecast window never produces): both traces and
    the output at the usual bars."""
    gm, om = models[("small", q)]
    sc, mask, grp, vt = mixed_series(rng, inconsistent=inconsistent)
    out, pe, l0 = t0hip.forward(gm, sc, mask, grp, vt, trace=True)
    want, wpe, wl0 = om.forward(sc, mask, grp, vt, trace=True)
    assert_close(pe, wpe, tol=2e-3)
    assert_close(l0, wl0, tol=5e-3)
    assert_close(out, want)


@pytest.mark.parametrize("q", [8, 2])
def test_forward_long_window(models, t0hip, oracle, rng, q):
    """A window longer than the LDS-resident time attention holds (300 patches > 256): the keys
    stream through workspace with an online softmax, on the same mask branches as above (FUTURE,
    whole-PAD, negative-group and inconsistent-group rows)."""
    gm, om = models[("small", q)]
    sc, mask, grp, vt = mixed_series(rng, t=300 * 32, inconsistent=True)
    out, pe, l0 = t0hip.forward(gm, sc, mask, grp, vt, trace=True)
    want, wpe, wl0 = om.forward(sc, mask, grp, vt, trace=True)
    assert_close(pe, wpe, tol=2e-3)
    assert_close(l0, wl0, tol=5e-3)
    assert_close(out, want)


@pytest.mark.parametrize("t_ctx,h", [(9000, 64), (20000, 40)])
def test_forecast_long_context(models, t0hip, oracle, engine, rng, t_ctx, h):
    """Contexts past 256 patches (t0-core takes any length): 9000 steps (284 patches, the streamed
    time attention) and 20000 steps (628 patches, where the window prep's per-row arrays no longer
    fit the LDS and live in device memory), two series with NaN gaps."""
    gm, om = models[("small", 8)]
    ctx = nan_gaps(rng, sine_mix(rng, 2, t_ctx), frac=0.1, lo=16, hi=128)
    got = t0hip.forecast(engine, gm, ctx, 2, t_ctx, h)
    want = om.forecast(ctx, 2, t_ctx, h)
    scale = row_scale(ctx)
    report(f"long context {t_ctx}", got, want, scale)
    assert_close(got, want, scale=scale)


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


@pytest.mark.parametrize("sizes", [(1, 3, 5, 8, 2), (4, 1, 4, 3), (2, 2, 1)])
def test_grouped_ragged_segments(models, t0hip, oracle, engine, rng, sizes):
    """Groups of different sizes in one batch, their rows interleaved in the input order: the group
    attention's segments (largest 8, 4 and 2 rows) hold fewer members than the kernel instance, and
    a segment's rows are not adjacent rows of the batch."""
    gm, om = models[("small", 2)]
    t_ctx, h = 512, 32
    groups = np.concatenate([np.full(n, 11 * g + 5, np.int64) for g, n in enumerate(sizes)])
    groups = groups[rng.permutation(len(groups))]
    v = len(groups)
    ctx = nan_gaps(rng, sine_mix(rng, v, t_ctx) * np.exp(rng.standard_normal(v)).astype(np.float32)[:, None])
    got = t0hip.forecast_grouped(engine, gm, ctx, groups, t_ctx, h)
    want = om.forecast_grouped(ctx, groups, t_ctx, h)
    assert_close(got, want, scale=row_scale(ctx))


def test_grouped_ar(models, t0hip, oracle, engine, rng):
    """BASELINE config 5 shape (scaled down): AR steps append each row's median quantile.
    (1) The GPU loop equals the GPU's single-step forecasts on the windows it builds (the device
    shift and store, k_ar_shift / k_ar_store), bit for bit.  (2) Every step, teacher-forced: the
    GPU forecasts the oracle's own window of that step within 5e-3, raw and normalized.  (3) The
    free-running loops, which feed back their own medians, are reported as drift."""
    gm, om = models[("tiny", 8)]
    n_rows, t_ctx, h, steps = 8, 256, 64, 3
    ctx = sine_mix(rng, n_rows, t_ctx)
    groups = np.repeat(np.arange(2), 4)
    qi = median_index(om.levels)
    got = t0hip.forecast_grouped_ar(engine, gm, ctx, groups, t_ctx, h, steps)
    mine, _ = ar_windows(lambda w: t0hip.forecast_grouped(engine, gm, w, groups, t_ctx, h), ctx, t_ctx, h, steps, qi)
    assert np.array_equal(got, mine)
    want = om.forecast_grouped_ar(ctx, groups, t_ctx, h, steps)
    _, wins = ar_windows(lambda w: om.forecast_grouped(w, groups, t_ctx, h), ctx, t_ctx, h, steps, qi)
    for st, w in enumerate(wins):
        step = t0hip.forecast_grouped(engine, gm, w, groups, t_ctx, h)
        assert_close(step, want[:, st * h:(st + 1) * h])
        assert_close(step, want[:, st * h:(st + 1) * h], scale=row_scale(w))
    report("grouped AR free-running drift", got, want, row_scale(ctx))


def test_rollout(models, t0hip, oracle, engine):
    """forecast_rollout (model.rs:582-665, lib.rs:259-341) on the reference's long-rollout fixture
    context (ctx 4096, horizon 1200: a 1024-step block, then 5 paths over a saturating 192-step
    block of 134 patches).  (1) The C++ driver equals the Python driver (tests/util.py, pinned
    against the oracle's rollout on the CPU) run over the GPU's own forecasts, within f32 rounding
    of the host reducer.  (2) Each block teacher-forced: the GPU forecasts the oracle's windows
    within 5e-3.  (3) Free-running drift reported."""
    gm, om = models[("tiny", 8)]
    ctx = np.fromfile(os.path.join(GOLDEN, "case_long_rollout_context.f32"), "<f4")
    q = np.array([0.1, 0.25, 0.5, 0.75, 0.9], np.float32)
    n = ctx.size
    got = t0hip.forecast_rollout(engine, gm, ctx, n, 1200, q)
    assert got.shape == (1200, 5)
    mine, _ = rollout_blocks(lambda x, h: t0hip.forecast(engine, gm, x[None], 1, x.size, h),
                             lambda w, h: t0hip.forecast_batch_chunked(engine, gm, w, w.shape[0], w.shape[1], h, 0),
                             oracle, om.levels, ctx, n, 1200, q)
    assert np.max(np.abs(got - mine)) <= 1e-6 * max(1.0, float(np.max(np.abs(mine))))
    want, wins = rollout_blocks(lambda x, h: om.forecast(x[None], 1, x.size, h),
                                lambda w, h: om.forecast_batch_chunked(w, w.shape[0], w.shape[1], h, 0),
                                oracle, om.levels, ctx, n, 1200, q)
    sc = row_scale(ctx[None])
    assert_close(got[:1024], want[:1024])
    for w in wins:
        g_ = t0hip.forecast_batch_chunked(engine, gm, w, w.shape[0], w.shape[1], 192, 0)
        o_ = om.forecast_batch_chunked(w, w.shape[0], w.shape[1], 192, 0)
        assert_close(g_, o_)
        assert_close(g_, o_, scale=row_scale(w))
    report("rollout free-running drift", got, want, sc)


@pytest.mark.parametrize("q", [8, 2])
def test_load_model_from_safetensors(t0hip, oracle, engine, rng, q):
    """t0_fast::load_model(engine, weights, config, quant) (lib.rs:34-36): an F32 model.safetensors
    (written by the safetensors package) and its config.json straight onto the device; forecasts
    equal those of the GGUF the same export writes (loaded through t0h_model_load_gguf), and match
    the oracle on that GGUF."""
    import json
    import safetensors.numpy
    from test_oracle import _tensor_names
    g32 = t0hip.synth_model_gguf(t0hip.make_config(**SMALL), quant=0, seed=23)
    om32 = oracle.Model(g32)
    st = safetensors.numpy.save({n: np.ascontiguousarray(om32.tensor(n)) for n in _tensor_names(g32)})
    cj = json.dumps({k: SMALL[k] for k in ("embed_dim", "num_layers", "num_heads", "mlp_hidden_dim", "patch_size",
                                           "group_every_n")} |
                    {"dropout": 0.0, "quantile_levels": [float(np.float32(x)) for x in SMALL["quantile_levels"]]})
    gm = t0hip.load_model(engine, st, cj, q)
    gguf = t0hip.export_gguf_from_safetensors(st, cj, q)
    ref = t0hip.load_model_from_gguf(engine, gguf)
    ctx = nan_gaps(rng, sine_mix(rng, 3, 700))
    got = t0hip.forecast(engine, gm, ctx, 3, 700, 64)
    assert np.array_equal(got, t0hip.forecast(engine, ref, ctx, 3, 700, 64))
    assert_close(got, oracle.Model(gguf).forecast(ctx, 3, 700, 64), scale=row_scale(ctx))


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


def test_graph_replay_matches_eager(t0hip, engine, torch_cuda, rng):
    """The window forward captured as a HIP graph and replayed: every replay equals the eager
    result bit for bit, with other eager work (another model, another window shape) and
    synchronizations between replays; a new output pointer, and the autoregressive loop's two
    alternating context buffers, are captured on their own."""
    g = t0hip.synth_model_gguf(t0hip.make_config(**TINY), quant=8, seed=3)
    gm = t0hip.load_model_from_gguf(engine, g)
    other = t0hip.load_model_from_gguf(engine, t0hip.synth_model_gguf(t0hip.make_config(**TINY), quant=2, seed=4))
    ctx = sine_mix(rng, 3, 500)
    ctx[1, 50:90] = np.nan
    gm.graph_replay(False)
    eager = t0hip.forecast(engine, gm, ctx, 3, 500, 40)
    eager_short = t0hip.forecast(engine, gm, ctx[:, :300], 3, 300, 40)
    gm.graph_replay(True)
    for i in range(5):
        assert np.array_equal(t0hip.forecast(engine, gm, ctx, 3, 500, 40), eager), i
        t0hip.forecast(engine, other, ctx, 3, 500, 40)
        assert np.array_equal(t0hip.forecast(engine, gm, ctx[:, :300], 3, 300, 40), eager_short), i
        torch_cuda.cuda.synchronize()
    # device entry point: the output pointer is part of what a graph bakes in
    n_rows, t_ctx, h = 6, 256, 32
    x = sine_mix(rng, n_rows, t_ctx)
    groups = np.repeat(np.arange(3), 2).astype(np.int64)
    d_x = torch_cuda.from_numpy(x).cuda()
    outs = [torch_cuda.empty((n_rows, h, 5), dtype=torch_cuda.float32, device="cuda") for _ in range(2)]
    gm.graph_replay(False)
    want = t0hip.forecast_grouped(engine, gm, x, groups, t_ctx, h)
    gm.graph_replay(True)
    for i in range(6):
        o = outs[i % 2]
        o.zero_()
        torch_cuda.cuda.synchronize()
        t0hip.forecast_grouped_dev(gm, d_x.data_ptr(), groups, t_ctx, h, o.data_ptr())
        torch_cuda.cuda.synchronize()  # device-wide: includes the model's stream
        assert np.array_equal(o.cpu().numpy(), want), i
    gm.graph_replay(False)
    ar_eager = t0hip.forecast_grouped_ar(engine, gm, x, groups, t_ctx, h, 4)
    gm.graph_replay(True)
    for i in range(3):
        assert np.array_equal(t0hip.forecast_grouped_ar(engine, gm, x, groups, t_ctx, h, 4), ar_eager), i


def test_error_paths_on_device(models, t0hip, engine, rng):
    gm, _ = models[("tiny", 8)]
    ctx = sine_mix(rng, 1, 64)
    with pytest.raises(t0hip.T0HipError) as e:
        t0hip.forecast(engine, gm, ctx, 1, 64, 1025)
    assert e.value.status == "HORIZON"
    with pytest.raises(t0hip.T0HipError) as e:
        t0hip.forecast_grouped(engine, gm, ctx, np.array([-1]), 64, 32)
    assert e.value.status == "INVALID_ARG"


def test_numeric_guard_on_f16_overflow(t0hip, oracle, engine, torch_cuda, rng):
    """An f16 activation beyond 65504 (the SwiGLU hidden of layer 0, its gate/up weights scaled by
    2000) becomes inf on the GPU where the reference's f32 path stays finite: the host-output entry
    points return NUMERIC, a device-output call leaves the report to check_numerics, which clears
    it; a model without the overflow is unaffected."""
    import json

    import safetensors.numpy
    from test_oracle import _tensor_names
    g = t0hip.synth_model_gguf(t0hip.make_config(**TINY), quant=0, seed=17)
    om = oracle.Model(g)
    tensors = {n: np.ascontiguousarray(om.tensor(n), np.float32) for n in _tensor_names(g)}
    tensors["transformer.layers.0.mlp.0.weight"] *= np.float32(2000.0)
    config = {k: TINY[k] for k in ("embed_dim", "num_layers", "num_heads", "mlp_hidden_dim", "patch_size",
                                   "group_every_n")}
    config.update(dropout=0.0, quantile_levels=[float(np.float32(q)) for q in TINY["quantile_levels"]])
    big = t0hip.export_gguf_from_safetensors(safetensors.numpy.save(tensors), json.dumps(config), 0)
    gm = t0hip.load_model_from_gguf(engine, big)
    ctx = sine_mix(rng, 2, 256)
    want = oracle.Model(big).forecast(ctx, 2, 256, 32)
    assert np.isfinite(want).all()
    for call in (lambda: t0hip.forecast(engine, gm, ctx, 2, 256, 32),
                 lambda: t0hip.forecast_grouped(engine, gm, ctx, np.array([0, 1]), 256, 32),
                 lambda: t0hip.forecast_grouped_ar(engine, gm, ctx, np.array([0, 1]), 256, 32, 2)):
        with pytest.raises(t0hip.T0HipError) as e:
            call()
        assert e.value.status == "NUMERIC", e.value
    torch = torch_cuda
    d_x = torch.tensor(ctx, dtype=torch.float32, device="cuda")
    out = torch.empty((2, 32, 5), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    t0hip.forecast_grouped_dev(gm, d_x.data_ptr(), np.array([0, 1]), 256, 32, out.data_ptr())
    with pytest.raises(t0hip.T0HipError) as e:
        gm.check_numerics()
    assert e.value.status == "NUMERIC"
    gm.check_numerics()  # read and cleared
    ok = t0hip.load_model_from_gguf(engine, g)
    got = t0hip.forecast(engine, ok, ctx, 2, 256, 32)
    assert_close(got, om.forecast(ctx, 2, 256, 32), scale=row_scale(ctx))
    t0hip.forecast_grouped_dev(ok, d_x.data_ptr(), np.array([0, 1]), 256, 32, out.data_ptr())
    ok.check_numerics()


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


def test_baseline_model_long_context(t0hip, oracle, engine, rng):
    """The BASELINE model on one series of 12,000 steps (377 patches): the streamed time attention
    at full width (12 heads of 64).  Gated in the series' own scale (about 2 here); the raw figure
    is printed (5.4e-3 measured: about twice the normalized one, as the scale says)."""
    g = t0hip.synth_model_gguf(t0hip.make_config(**BASELINE), quant=8, seed=0)
    gm = t0hip.load_model_from_gguf(engine, g)
    om = oracle.Model(g)
    ctx = sine_mix(rng, 1, 12000)
    got = t0hip.forecast(engine, gm, ctx, 1, 12000, 64)
    want = om.forecast(ctx, 1, 12000, 64)
    report("baseline long context", got, want, row_scale(ctx))
    assert_close(got, want, scale=row_scale(ctx))


def test_config5_windows_small_model(t0hip, oracle, engine, rng):
    """BASELINE config 5's window (ctx 4096: 130 patches, the long time-attention path) on a small
    model, 2 series x 8 variates, 3 autoregressive steps of 64: every step teacher-forced against
    the oracle at 5e-3, and the GPU loop against its own single steps bit for bit."""
    from util import trend_season_t
    g = t0hip.synth_model_gguf(t0hip.make_config(**SMALL), quant=8, seed=12)
    gm = t0hip.load_model_from_gguf(engine, g)
    om = oracle.Model(g)
    n_series, v, t_ctx, h, steps = 2, 8, 4096, 64, 3
    ctx = trend_season_t(rng, n_series * v, t_ctx)
    groups = np.repeat(np.arange(n_series), v).astype(np.int64)
    qi = median_index(om.levels)
    got = t0hip.forecast_grouped_ar(engine, gm, ctx, groups, t_ctx, h, steps)
    mine, _ = ar_windows(lambda w: t0hip.forecast_grouped(engine, gm, w, groups, t_ctx, h), ctx, t_ctx, h, steps, qi)
    assert np.array_equal(got, mine)
    want, wins = ar_windows(lambda w: om.forecast_grouped(w, groups, t_ctx, h), ctx, t_ctx, h, steps, qi)
    for st, w in enumerate(wins):
        step = t0hip.forecast_grouped(engine, gm, w, groups, t_ctx, h)
        report(f"config-5 window step {st}", step, want[:, st * h:(st + 1) * h], row_scale(w))
        assert_close(step, want[:, st * h:(st + 1) * h], scale=row_scale(w))
    report("config-5 window free-running drift", got, want, row_scale(ctx))


def test_config5_full_size(t0hip, oracle, engine, rng):
    """BASELINE config 5 at full size: 64 series x 8 variates, ctx 4096, 8 autoregressive steps of 64,
    Q8_0 BASELINE model with weights resident across steps (66,560 patch rows per step).
    (1) The GPU loop equals the GPU's own single-step forecasts of the windows it builds, bit for
    bit, at every step.  (2) Every step teacher-forced for series 0: the full 512-row batch is
    forecast with series 0's rows replaced by the oracle's window of that step, and those rows are
    held to 5e-3 of the oracle (normalized; the raw figure is printed)."""
    from util import trend_season_t
    g = t0hip.synth_model_gguf(t0hip.make_config(**BASELINE), quant=8, seed=0)
    gm = t0hip.load_model_from_gguf(engine, g)
    om = oracle.Model(g)
    n_series, v, t_ctx, h, steps = 64, 8, 4096, 64, 8
    ctx = trend_season_t(rng, n_series * v, t_ctx)
    groups = np.repeat(np.arange(n_series), v).astype(np.int64)
    qi = median_index(om.levels)
    full = t0hip.forecast_grouped_ar(engine, gm, ctx, groups, t_ctx, h, steps)
    assert full.shape == (n_series * v, steps * h, 9) and np.isfinite(full).all()
    mine, gwins = ar_windows(lambda w: t0hip.forecast_grouped(engine, gm, w, groups, t_ctx, h), ctx, t_ctx, h,
                             steps, qi)
    assert np.array_equal(full, mine)
    want, owins = ar_windows(lambda w: om.forecast_grouped(w, groups[:v], t_ctx, h), ctx[:v], t_ctx, h, steps, qi)
    worst = 0.0
    for st in range(steps):
        batch = gwins[st].copy()
        batch[:v] = owins[st]
        step = t0hip.forecast_grouped(engine, gm, batch, groups, t_ctx, h)[:v]
        _, norm = report(f"config-5 step {st}", step, want[:, st * h:(st + 1) * h], row_scale(owins[st]))
        worst = max(worst, norm)
    assert worst <= TOL, worst
    report("config-5 series 0 free-running drift", full[:v], want, row_scale(ctx[:v]))


def test_config4_full_size(t0hip, oracle, engine, rng):
    """BASELINE config 4 at full size, as bench.py times it: 256 series x 3 variates (one group id
    per series), ctx 2048, horizon 64, sine mixture x lognormal scale with 10% NaN gaps in runs of
    16-128, Q4_0 BASELINE model; 50,688 patch rows, so every layer GEMM runs the register-operand
    MFMA kernel.  16 series of the full batch against the oracle, the largest- and the
    smallest-scale series among them: 5e-3 normalized by each row's scale on all of them, 5e-3
    raw on those whose scale is at most 1 (raw error grows with the series' scale: f16 MFMA
    operands round relative to the values), raw and normalized printed.  Batch isolation: series
    0 alone (its 198 rows take the medium-M kernel) gives the same forecast up to 1e-2 normalized,
    the sum of the two paths' allowed distances from the oracle."""
    n_series, v, t_ctx, h = 256, 3, 2048, 64
    g = t0hip.synth_model_gguf(t0hip.make_config(**BASELINE), quant=2, seed=0)
    gm = t0hip.load_model_from_gguf(engine, g)
    amp = np.exp(rng.standard_normal(n_series))
    x = sine_mix(rng, n_series * v, t_ctx) * np.repeat(amp, v)[:, None].astype(np.float32)
    x = nan_gaps(rng, x)
    groups = np.repeat(np.arange(n_series), v).astype(np.int64)
    full = t0hip.forecast_grouped(engine, gm, x, groups, t_ctx, h)
    assert full.shape == (n_series * v, h, 9) and np.isfinite(full).all()
    om = oracle.Model(g)
    pick = [int(np.argmax(amp)), int(np.argmin(amp)), 0, 137]
    pick += [int(s) for s in rng.choice([i for i in range(n_series) if i not in pick], 16 - len(pick), replace=False)]
    raw_unit, norm_all, raw_all = 0.0, 0.0, 0.0
    for s in pick:
        rows = slice(s * v, (s + 1) * v)
        want = om.forecast_grouped(x[rows], groups[rows], t_ctx, h)
        sc = row_scale(x[rows])
        raw, norm = report(f"config-4 series {s} (amplitude {amp[s]:.3g})", full[rows], want, sc)
        norm_all, raw_all = max(norm_all, norm), max(raw_all, raw)
        if sc.max() <= 1.0:
            raw_unit = max(raw_unit, raw)
    print(f"config-4 over {len(pick)} series: normalized {norm_all:.3e}, raw {raw_all:.3e}, "
          f"raw on unit-scale series {raw_unit:.3e}", flush=True)
    assert norm_all <= TOL, norm_all
    assert raw_unit <= TOL, raw_unit
    alone = t0hip.forecast_grouped(engine, gm, x[:v], groups[:v], t_ctx, h)
    assert_close(alone, om.forecast_grouped(x[:v], groups[:v], t_ctx, h), scale=row_scale(x[:v]))
    assert_close(full[:v], alone, scale=row_scale(x[:v]), tol=2 * TOL)
