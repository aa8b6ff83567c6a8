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
