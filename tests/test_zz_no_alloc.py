"""The no-allocation entry point (t0h_forecast_grouped_dev_noalloc) against the entry point it
varies (t0h_forecast_grouped_dev) through the C ABI: two calls in a row, the second on a smaller
window, each bit-identical to the allocating path's result (the same kernels on the same inputs);
the model's workspace makes no allocation during them; a window beyond the scratch is rejected
before any work and leaves the output untouched."""
import numpy as np
import pytest

from util import BASELINE, nan_gaps, sine_mix

pytestmark = pytest.mark.gpu


def test_noalloc_matches_allocating_entry_point(t0hip, engine, torch_cuda, rng):
    torch = torch_cuda
    g = t0hip.synth_model_gguf(t0hip.make_config(**BASELINE), quant=8, seed=0)
    gm = t0hip.load_model_from_gguf(engine, g)
    cases = [(3, 3, 2048, 64), (1, 2, 1000, 40)]  # (series, variates, ctx, horizon); the second smaller
    inputs = []
    for n_series, v, t_ctx, h in cases:
        x = nan_gaps(rng, sine_mix(rng, n_series * v, t_ctx) * 3.0)
        groups = np.repeat(np.arange(n_series) * 5 + 1, v).astype(np.int64)
        inputs.append((torch.from_numpy(x).cuda(), groups, t_ctx, h))
    _, allocs0 = gm.workspace()
    got = []
    for d_x, groups, t_ctx, h in inputs:
        out = torch.full((groups.size, h, 9), float("nan"), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        t0hip.forecast_grouped_dev_noalloc(gm, d_x.data_ptr(), groups, t_ctx, h, out.data_ptr())
        torch.cuda.synchronize()
        got.append(out.cpu().numpy())
    assert gm.workspace()[1] == allocs0  # no workspace allocation on the no-allocation path
    for (d_x, groups, t_ctx, h), mine in zip(inputs, got):
        out = torch.empty((groups.size, h, 9), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        t0hip.forecast_grouped_dev(gm, d_x.data_ptr(), groups, t_ctx, h, out.data_ptr())
        torch.cuda.synchronize()
        want = out.cpu().numpy()
        assert np.isfinite(mine).all()
        assert np.array_equal(mine, want)
    # 256 series x 3 variates needs far more than the scratch
    n_rows, t_ctx, h = 768, 2048, 64
    d_big = torch.zeros((n_rows, t_ctx), dtype=torch.float32, device="cuda")
    out = torch.full((n_rows, h, 9), 7.0, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    with pytest.raises(t0hip.T0HipError) as e:
        t0hip.forecast_grouped_dev_noalloc(gm, d_big.data_ptr(), np.repeat(np.arange(256), 3), t_ctx, h,
                                           out.data_ptr())
    assert e.value.status == "UNSUPPORTED" and "scratch" in str(e.value)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
    # a window past the no-allocation limit (300 patches > NOALLOC_MAX_PATCHES) is rejected too
    d_long = torch.zeros((1, 300 * 32 - 64), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    with pytest.raises(t0hip.T0HipError) as e:
        t0hip.forecast_grouped_dev_noalloc(gm, d_long.data_ptr(), np.array([0]), 300 * 32 - 64, 64, out.data_ptr())
    assert e.value.status == "UNSUPPORTED" and "patches" in str(e.value)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
    # still usable after the rejection
    d_x, groups, t_ctx, h = inputs[1]
    again = torch.empty((groups.size, h, 9), dtype=torch.float32, device="cuda")
    t0hip.forecast_grouped_dev_noalloc(gm, d_x.data_ptr(), groups, t_ctx, h, again.data_ptr())
    torch.cuda.synchronize()
    assert np.array_equal(again.cpu().numpy(), got[1])
