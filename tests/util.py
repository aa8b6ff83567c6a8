"""Shared helpers for the test-suite (synthetic inputs, model configs, error metrics)."""
import numpy as np

TINY = dict(embed_dim=128, num_layers=3, num_heads=2, mlp_hidden_dim=256, patch_size=32, group_every_n=3,
            quantile_levels=(0.1, 0.25, 0.5, 0.75, 0.9))
SMALL = dict(embed_dim=256, num_layers=6, num_heads=4, mlp_hidden_dim=512, patch_size=32, group_every_n=3,
             quantile_levels=(0.1, 0.2, 0.3, 0.4, 0.5, 0.6, 0.7, 0.8, 0.9))
BASELINE = dict(embed_dim=768, num_layers=12, num_heads=12, mlp_hidden_dim=2048, patch_size=32, group_every_n=3,
                quantile_levels=(0.1, 0.2, 0.3, 0.4, 0.5, 0.6, 0.7, 0.8, 0.9))


def sine_mix(rng, n_rows, t, n_sines=3, noise=0.1):
    """Sum of sines with periods U[7,365] plus N(0, noise)."""
    tt = np.arange(t, dtype=np.float64)
    out = np.zeros((n_rows, t))
    for _ in range(n_sines):
        period = rng.uniform(7, 365, size=(n_rows, 1))
        phase = rng.uniform(0, 2 * np.pi, size=(n_rows, 1))
        amp = rng.uniform(0.5, 2.0, size=(n_rows, 1))
        out += amp * np.sin(2 * np.pi * tt / period + phase)
    out += noise * rng.standard_normal((n_rows, t))
    return out.astype(np.float32)


def nan_gaps(rng, x, frac=0.1, lo=16, hi=128):
    """Mask about `frac` of each row as NaN in contiguous runs of lo..hi steps."""
    x = x.copy()
    n_rows, t = x.shape
    for r in range(n_rows):
        target = int(frac * t)
        masked = 0
        while masked < target:
            L = int(rng.integers(lo, hi + 1))
            s = int(rng.integers(0, max(1, t - L)))
            x[r, s:s + L] = np.nan
            masked = int(np.isnan(x[r]).sum())
    return x


def rel_err(got, ref):
    """max |got-ref| / max |ref| (normwise relative error)."""
    return float(np.max(np.abs(got.astype(np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def trend_season_t(rng, n_rows, t, df=3):
    """BASELINE config 5 inputs: linear trend + two seasonal terms + Student-t(df) noise."""
    tt = np.arange(t, dtype=np.float64)
    slope = rng.normal(0.0, 0.01, size=(n_rows, 1))
    level = rng.normal(0.0, 5.0, size=(n_rows, 1))
    season = np.zeros((n_rows, t))
    for period in (24.0, 168.0):
        amp = rng.uniform(0.5, 3.0, size=(n_rows, 1))
        phase = rng.uniform(0, 2 * np.pi, size=(n_rows, 1))
        season += amp * np.sin(2 * np.pi * tt / period + phase)
    noise = rng.standard_t(df, size=(n_rows, t)) * 0.3
    return (level + slope * tt + season + noise).astype(np.float32)


def median_index(levels):
    """The trained level closest to 0.5 (the AR loop appends that quantile)."""
    return int(np.argmin(np.abs(np.asarray(levels, np.float32) - np.float32(0.5))))


def ar_windows(forecast_grouped, ctx, t_ctx, h, steps, qi):
    """The grouped autoregressive loop in Python over any one-step forecaster
    `forecast_grouped(window) -> [rows, h, n_q]`: every step appends each row's median-level
    quantile and keeps the trailing t_ctx values.  Returns (outputs [rows, steps*h, n_q], the window
    each step forecast from)."""
    cur = np.array(ctx, np.float32)
    outs, wins = [], []
    for _ in range(steps):
        wins.append(cur)
        f = forecast_grouped(cur)
        outs.append(f)
        cur = np.concatenate([cur, f[:, :, qi]], axis=1)[:, -t_ctx:]
    return np.concatenate(outs, axis=1), wins


def rollout_blocks(forecast, forecast_batch, oracle, levels, ctx, t_ctx, prediction_length, query, ps=32):
    """crates/t0-fast/src/lib.rs:259-341 forecast_rollout in Python over any forecaster:
    `forecast(ctx, horizon) -> [1, horizon, n_q]`, `forecast_batch(windows, horizon) ->
    [paths, horizon, n_q]`; the reducer is the oracle's (quantile.rs:16-76).  Returns the
    rollout [prediction_length, n_query] and, per batched block, the windows it forecast from."""
    MAX_H = 1024
    levels = np.asarray(levels, np.float32)
    query = np.asarray(query, np.float32)
    nq, nt = len(query), len(levels)
    ru = lambda x: -(-x // ps) * ps
    width = ru(t_ctx)
    h0 = min(ru(prediction_length), MAX_H)
    b0 = forecast(np.asarray(ctx, np.float32), h0)[0]
    first = np.stack([oracle.interpolate_quantiles(query, levels, b0[i]) for i in range(h0)])
    if prediction_length <= h0:
        return first[:prediction_length], []
    paths = [list(np.asarray(ctx, np.float32)) for _ in range(nq)]
    remaining, prev, chunks, windows = prediction_length - h0, first, [first], []
    tm, qm = oracle.prob_mass(levels), oracle.prob_mass(query)
    weights = (qm[:, None] * tm[None, :]).astype(np.float32).reshape(-1)
    while remaining > 0:
        for j in range(nq):
            paths[j].extend(prev[:, j])
        h = min(ru(remaining), MAX_H)
        win = np.zeros((nq, width), np.float32)
        for j in range(nq):
            w = np.asarray(paths[j][-width:], np.float32)
            win[j, width - len(w):] = w
        windows.append(win)
        blocks = forecast_batch(win, h)
        red = np.stack([oracle.weighted_quantile(query, weights, blocks[:, i, :].reshape(-1)) for i in range(h)])
        chunks.append(red)
        prev = red
        remaining = max(0, remaining - h)
    return np.concatenate(chunks)[:prediction_length], windows
