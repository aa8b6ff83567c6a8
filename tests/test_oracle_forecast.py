"""Pins the oracle's forecast wrapper (CPU only): the window (left PAD to a patch boundary,
WITHHELD horizon), the causal scaler, the rescale at each patch's last step and the slice from
patch context_patches - 1 (crates/t0-core/src/model.rs:448-531, scaler.rs:44-148,
data.rs:52-155; crates/t0-fast/src/lib.rs:50-97, 175-242).

The oracle's C wrapper (oracle/t0ref.c forecast_window) is compared with tests/np_ref.py's
float64 restatement, which computes the scaler statistics in closed form (cumulative sums)
rather than by the Welford recurrence.  Each planted mistake (slice one patch early or late, rescale
with another step of each patch than its last, context padding on the wrong side) must fail the
same comparison, so the comparison is shown to see them."""
import numpy as np
import pytest

import np_ref
from test_oracle import _tensor_names
from util import TINY, nan_gaps, sine_mix

TOL = 1e-5  # float32 oracle against float64, relative to max(1, max |want|)


def _model(t0hip, oracle, **over):
    cfg = dict(TINY, **over)
    g = t0hip.synth_model_gguf(t0hip.make_config(**cfg), quant=0, seed=33)
    om = oracle.Model(g)
    T = {n: om.tensor(n).astype(np.float64) for n in _tensor_names(g)}
    c = dict(cfg, n_q=len(cfg["quantile_levels"]), scaler_eps=over.get("eps", 0.1),
             variance_offset=over.get("variance_offset", True), use_arcsinh=over.get("use_arcsinh", True))
    return om, T, c


@pytest.fixture(scope="module")
def tiny(t0hip, oracle):
    return _model(t0hip, oracle)


def _err(got, want):
    return float(np.max(np.abs(got - want)) / max(1.0, float(np.max(np.abs(want)))))


def _inputs(seed, v, t_ctx):
    rng = np.random.default_rng(seed)
    x = sine_mix(rng, v, t_ctx) * rng.lognormal(0.0, 1.0, (v, 1)).astype(np.float32) + 3.0
    if t_ctx >= 200:
        x = nan_gaps(rng, x, frac=0.1, lo=16, hi=min(128, t_ctx // 4))
    return x


@pytest.mark.parametrize("t_ctx,h,v", [(500, 30, 3), (33, 1, 2), (2048, 64, 2), (64, 32, 1), (95, 33, 3)])
def test_forecast_matches_float64(tiny, t_ctx, h, v):
    om, T, c = tiny
    x = _inputs(t_ctx + h, v, t_ctx)
    got = om.forecast(x, v, t_ctx, h)
    want = np_ref.forecast(T, c, x, t_ctx, h)
    assert got.shape == want.shape == (v, h, c["n_q"])
    assert _err(got, want) < TOL


def test_forecast_std_clamp_scaler(t0hip, oracle):
    """The beta scaler (eps 0.01, std_clamp) and no arcsinh go through the same wrapper."""
    for over in (dict(eps=0.01, variance_offset=False), dict(use_arcsinh=False)):
        om, T, c = _model(t0hip, oracle, **over)
        x = _inputs(7, 2, 300)
        assert _err(om.forecast(x, 2, 300, 40), np_ref.forecast(T, c, x, 300, 40)) < TOL


def test_grouped_and_ragged_match_float64(tiny):
    om, T, c = tiny
    x = _inputs(11, 5, 257)
    groups = np.array([4, 4, 9, 9, 9], np.int64)
    assert _err(om.forecast_grouped(x, groups, 257, 48), np_ref.forecast_grouped(T, c, x, groups, 257, 48)) < TOL
    rng = np.random.default_rng(12)
    lengths = [300, 299, 257, 33]
    rows = [sine_mix(rng, 1, L)[0] + 2.0 for L in lengths]
    rows[0][100:140] = np.nan
    got = om.forecast_batch_rows_chunked(np.concatenate(rows), lengths, 40, 0)
    assert _err(got, np_ref.forecast_rows(T, c, rows, 40)) < TOL


@pytest.mark.parametrize("t_ctx,plant", [(2048, dict(slice_shift=1)), (2048, dict(slice_shift=-1)),
                                         (2048, dict(rescale_step=0)), (500, dict(rescale_step=15)),
                                         (500, dict(pad_right=True)), (33, dict(pad_right=True))])
def test_planted_wrapper_mistakes_are_seen(tiny, t_ctx, plant):
    """Negative controls: each mistake, planted in the float64 restatement, fails the comparison
    by a wide margin.  (A whole extra PAD patch on the left would not: RoPE and xPos depend only
    on the distance between patches and PAD patches are never attended, which is what makes the
    reference's ragged-row batching exact, lib.rs:160-174.)"""
    om, T, c = tiny
    x = _inputs(t_ctx + 64, 2, t_ctx)
    got = om.forecast(x, 2, t_ctx, 64)
    assert _err(got, np_ref.forecast(T, c, x, t_ctx, 64)) < TOL
    assert _err(got, np_ref.forecast(T, c, x, t_ctx, 64, **plant)) > 100 * TOL


def test_causal_stats_closed_form_matches_oracle_scaler(oracle):
    """np_ref's cumulative-sum scaler against the oracle's Welford recurrence (scaler.rs:91-118) on
    a long row with NaN runs, a PAD lead and a WITHHELD tail."""
    rng = np.random.default_rng(3)
    v, t = 3, 2112
    x = (50.0 + 7.0 * rng.standard_normal((v, t))).astype(np.float32)
    mask = np.zeros((v, t), np.int8)
    mask[0, 100:230] = 2
    mask[1, :17] = 1
    mask[:, 2048:] = 4
    g = np.zeros((v, t), np.int64)
    g[1, :17] = -1
    x[mask != 0] = 0.0
    for offset, eps in ((True, 0.1), (False, 0.01)):
        _, loc, scale = oracle.scale_input(x, mask, g, np.zeros((v, t), np.int64), True, eps, offset)
        wl, ws = np_ref.causal_stats(x.astype(np.float64), mask, g, eps, offset)
        assert np.max(np.abs(loc - wl)) < 2e-4
        assert np.max(np.abs(scale - ws) / ws) < 1e-4


def test_rollout_driver_reproduces_oracle_rollout(tiny, oracle):
    """tests/util.py's rollout driver (lib.rs:259-341 in Python, reused by the GPU tests to feed
    both paths the same windows) reproduces the oracle's forecast_rollout bit for bit, on the
    reference's long-rollout fixture context (ctx 4096, horizon 1200: one 1024-step block, then the
    saturating 192-step block over 134 patches)."""
    import os
    from util import rollout_blocks
    om, T, c = tiny
    ctx = np.fromfile(os.path.join(os.path.dirname(__file__), "golden", "case_long_rollout_context.f32"), "<f4")
    q = np.array([0.1, 0.25, 0.5, 0.75, 0.9], np.float32)
    want = om.forecast_rollout(ctx, ctx.size, 1200, q)
    got, wins = rollout_blocks(lambda x, h: om.forecast(x[None], 1, x.size, h),
                               lambda w, h: om.forecast_batch_chunked(w, w.shape[0], w.shape[1], h, 0),
                               oracle, om.levels, ctx, ctx.size, 1200, q)
    assert len(wins) == 1 and wins[0].shape == (5, 4096)
    assert np.array_equal(got, want)
