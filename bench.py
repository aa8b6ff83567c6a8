#!/usr/bin/env python3
"""Throughput benchmark of the t0hip quantized-inference path on one MI355X.

Step = one batched forecast of BASELINE config 4: 256 series x 3 variates, each
with a 2048-step context (sine mixture x lognormal scale, 10% NaN gaps in runs
of 16-128), horizon 64, through the 12-layer / embed 768 synthetic t0 model
with Q4_0 weights (random init from a fixed seed).  Inputs are resident in HBM
(t0h_forecast_grouped_dev); `value` is series forecasts per second.

Also reported on the same JSON line:
  roofline      the dominant kernel of the step (by total time), timed with HIP
                events on the model's stream inside the real forward;
  cpu_baseline  the oracle (this repo's C restatement of t0-core's ndarray path,
                f32 dequant-at-load + OpenMP GEMM) on a bounded sample of the
                same workload on this host's cores;
  gemm_sweep    BASELINE configs 1-2: the kernel-level Q-GEMM (f32 in/out) at
                M in {1,16,64,512,8192} x (K,N) shapes, TFLOP/s and GB/s;
                small-M cases rotate through >256 MB of weight copies so the
                Infinity Cache cannot serve them;
  workloads     BASELINE config 3 (one series, latency) and config 5 (64 x 8
                autoregressive rollout, Q8_0) through the host-buffer entry
                points, with the oracle on a bounded sample beside each.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "t0-web_amd"))

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
METRIC = "Q-GEMM TFLOPS & HBM GB/s vs roofline; forecasts/sec at 256 series on 1 GPU"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def config4_inputs(n_series=256, n_var=3, t_ctx=2048, seed=0):
    """Sine mixture x lognormal scale per series, 10% NaN gaps in contiguous runs of 16..128."""
    rng = np.random.default_rng(seed)
    rows = n_series * n_var
    tt = np.arange(t_ctx, dtype=np.float64)
    x = np.zeros((rows, t_ctx))
    for _ in range(3):
        period = rng.uniform(7, 365, (rows, 1))
        phase = rng.uniform(0, 2 * np.pi, (rows, 1))
        x += rng.uniform(0.5, 2.0, (rows, 1)) * np.sin(2 * np.pi * tt / period + phase)
    x += 0.1 * rng.standard_normal((rows, t_ctx))
    x *= np.repeat(np.exp(rng.standard_normal(n_series)), n_var)[:, None]
    for r in range(rows):
        while np.isnan(x[r]).sum() < 0.1 * t_ctx:
            L = int(rng.integers(16, 129))
            s = int(rng.integers(0, t_ctx - L))
            x[r, s:s + L] = np.nan
    groups = np.repeat(np.arange(n_series), n_var).astype(np.int64)
    return x.astype(np.float32), groups


def config3_input(t_ctx=2048, seed=3):
    """One univariate series: sum of 3 sines (periods U[7,365]) + N(0, 0.1) noise."""
    rng = np.random.default_rng(seed)
    tt = np.arange(t_ctx, dtype=np.float64)
    x = sum(np.sin(2 * np.pi * tt / rng.uniform(7, 365) + rng.uniform(0, 2 * np.pi)) for _ in range(3))
    return (x + 0.1 * rng.standard_normal(t_ctx)).astype(np.float32)


def config5_inputs(n_series=64, n_var=8, t_ctx=4096, seed=5):
    """Linear trend + daily and weekly seasonal terms + Student-t(3) noise per row."""
    rng = np.random.default_rng(seed)
    rows = n_series * n_var
    tt = np.arange(t_ctx, dtype=np.float64)
    x = rng.normal(0.0, 5.0, (rows, 1)) + rng.normal(0.0, 0.01, (rows, 1)) * tt
    for period in (24.0, 168.0):
        x = x + rng.uniform(0.5, 3.0, (rows, 1)) * np.sin(2 * np.pi * tt / period + rng.uniform(0, 2 * np.pi, (rows, 1)))
    x += 0.3 * rng.standard_t(3, (rows, t_ctx))
    return x.astype(np.float32), np.repeat(np.arange(n_series), n_var).astype(np.int64)


def median_time(fn, reps):
    ts = []
    for _ in range(reps):
        t = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t)
    return float(np.median(ts))


def other_workloads(torch, t0hip, engine, cfg, with_cpu, reps=5):
    """BASELINE configs 3 and 5 through the host-buffer entry points (upload of the context and
    download of the result included, as the reference's own bench times them), median of `reps`
    after one warm-up, and config 3 also with device-resident input and output; the oracle beside
    each on a bounded sample when `with_cpu`."""
    res = {}
    gguf = t0hip.synth_model_gguf(cfg, quant=t0hip.Q8_0, seed=0)
    model = t0hip.load_model_from_gguf(engine, gguf)
    om = None
    if with_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import t0ref  # the CPU checker/baseline, test infrastructure
        om = t0ref.Model(gguf)

    x3 = config3_input()
    run3 = lambda: t0hip.forecast(engine, model, x3, 1, x3.size, 64)
    run3()
    ms3 = median_time(run3, 4 * reps) * 1e3
    res["config3"] = {"workload": "1 series, sum of 3 sines + N(0,0.1), ctx 2048, horizon 64, Q8_0",
                      "ms_per_forecast": round(ms3, 3), "gemm_rows": 66}
    if om is not None:
        om.forecast(x3, 1, x3.size, 64)
        res["config3"]["cpu_ms_per_forecast"] = round(median_time(lambda: om.forecast(x3, 1, x3.size, 64), 3) * 1e3, 1)
    # the same forecast with the context already in HBM and the output left there
    # (t0h_forecast_grouped_dev), ten back to back and one synchronization: device time
    d_x3 = torch.tensor(x3, device="cuda").reshape(1, -1)
    d_o3 = torch.empty((1, 64, cfg.n_quantiles), dtype=torch.float32, device="cuda")
    g3 = np.zeros(1, np.int64)
    torch.cuda.synchronize()

    def dev3():
        for _ in range(10):
            t0hip.forecast_grouped_dev(model, d_x3.data_ptr(), g3, x3.size, 64, d_o3.data_ptr())
        torch.cuda.synchronize()

    dev3()
    res["config3"]["device_ms_per_forecast"] = round(median_time(dev3, 2 * reps) * 1e2, 3)
    log(f"config 3: {ms3:.3f} ms per forecast ({res['config3']['device_ms_per_forecast']:.3f} device)")

    x5, g5 = config5_inputs()
    t_ctx, h, steps = x5.shape[1], 64, 8
    run5 = lambda: t0hip.forecast_grouped_ar(engine, model, x5, g5, t_ctx, h, steps)
    run5()
    s5 = median_time(run5, reps)
    p5 = (t_ctx + h + 31) // 32
    flops = 2.0 * x5.shape[0] * p5 * 7077888 * cfg.num_layers * steps
    res["config5"] = {"workload": "64 series x 8 variates, trend + seasonality + Student-t(3), ctx 4096, "
                                  "8 AR steps of horizon 64, Q8_0, weights resident across steps",
                      "ms_per_rollout": round(s5 * 1e3, 2), "series_rollouts_per_s": round(64 / s5, 2),
                      "gemm_rows_per_step": x5.shape[0] * p5,
                      "layer_gemm_tflops_effective": round(flops / s5 * 1e-12, 1)}
    if om is not None:
        # one series (8 variates), 2 of the 8 AR steps
        t = time.perf_counter()
        om.forecast_grouped_ar(x5[:8], g5[:8], t_ctx, h, 2)
        dt = time.perf_counter() - t
        res["config5"]["cpu_sample"] = {"series_rollouts_per_s": round(2 / steps / dt, 4),
                                        "sample": f"1 series x 8 variates, 2 of 8 AR steps, {dt:.1f} s"}
    log(f"config 5: {s5 * 1e3:.1f} ms per rollout")
    model.close()
    return res


def gemm_flops(name, M, cfg):
    E, H = cfg.embed_dim, cfg.mlp_hidden_dim
    return {"gemm_w0_swiglu": 2 * M * 2 * H * E, "gemm_qkv": 2 * M * 3 * E * E,
            "gemm_w2_resid": 2 * M * E * H, "gemm_wo_resid": 2 * M * E * E}.get(name)


def gemm_bytes(name, M, cfg, wbytes_per_val):
    """Algorithmic HBM bytes of one launch: weight blocks + f16 activations in + outputs."""
    E, H = cfg.embed_dim, cfg.mlp_hidden_dim
    if name == "gemm_w0_swiglu":
        return 2 * H * E * wbytes_per_val + M * E * 2 + M * H * 2 + 2 * H * 4
    if name == "gemm_qkv":
        return 3 * E * E * wbytes_per_val + M * E * 2 + M * 3 * E * 2 + 3 * E * 4
    if name == "gemm_w2_resid":
        return E * H * wbytes_per_val + M * H * 2 + 2 * M * E * 4 + E * 4
    if name == "gemm_wo_resid":
        return E * E * wbytes_per_val + M * E * 2 + 2 * M * E * 4 + E * 4
    return None


def stream_read_us(torch, buf, nbytes, n_copies, reps):
    """Event-timed average of t0p_stream_read over nbytes of each of the n_copies copies in buf
    (libt0probe.so, a measurement helper built beside libt0hip.so); None when it is not built."""
    import ctypes

    path = os.path.join(ROOT, "t0-web_amd", "libt0probe.so")
    if not os.path.exists(path):
        return None
    lib = ctypes.CDLL(path)
    lib.t0p_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p]
    lib.t0p_stream_read_out_words.argtypes = [ctypes.c_size_t]
    lib.t0p_stream_read_out_words.restype = ctypes.c_size_t
    out = torch.empty(int(lib.t0p_stream_read_out_words(nbytes)), dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream()

    def run(i):
        rc = lib.t0p_stream_read(buf.data_ptr() + (i % n_copies) * nbytes, nbytes, out.data_ptr(), stream.cuda_stream)
        if rc != 0:
            raise RuntimeError(f"t0p_stream_read: hip error {rc}")

    for i in range(3):
        run(i)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(reps):
        run(i)
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / reps


def gemm_sweep(torch, t0hip, iters=20):
    """BASELINE configs 1-2 through the kernel-level t0h_gemm_q (f32 x in, f32 y out)."""
    rng = np.random.default_rng(7)
    stream = torch.cuda.current_stream()
    out = []
    # BASELINE config 2 shapes at every M, plus one large weight (4096 x 16384) at the GEMV end,
    # where bandwidth rather than launch latency bounds a single call
    shapes = [(768, 2304), (768, 768), (768, 2048), (2048, 768), (768, 4096), (4096, 16384)]
    for qtype, qname, bpv in ((t0hip.Q8_0, "q8_0", 34 / 32), (t0hip.Q4_0, "q4_0", 18 / 32)):
        for K, N in shapes:
            W = (0.02 * rng.standard_normal((N, K))).astype(np.float32)
            blocks = t0hip.quantize(qtype, W)
            for M in ((1, 16) if N * K > 2**24 else (1, 16, 64, 512, 8192)):
                # rotate weight copies past the 256 MB Infinity Cache for the bandwidth-bound cases
                n_copies = max(1, int(np.ceil(320e6 / blocks.size))) if M <= 64 else 1
                # copies 256-byte aligned (the GEMM entry points take 16-byte aligned weights)
                src = np.concatenate([blocks, np.zeros((-blocks.size) % 256, np.uint8)])
                dW = torch.from_numpy(src).cuda().repeat(n_copies)
                x = torch.randn((M, K), dtype=torch.float32, device="cuda")
                y = torch.empty((M, N), dtype=torch.float32, device="cuda")
                stride = src.size

                def run(i):
                    t0hip.gemm_q_dev(qtype, dW.data_ptr() + (i % n_copies) * stride, x.data_ptr(), 0, y.data_ptr(),
                                     M, N, K, 0, stream.cuda_stream)

                for i in range(3):
                    run(i)
                reps = max(iters, n_copies)
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                for i in range(reps):
                    run(i)
                e1.record(stream)
                torch.cuda.synchronize()
                us = e0.elapsed_time(e1) * 1e3 / reps
                flops = 2.0 * M * N * K
                nbytes = N * K * bpv + M * K * 4 + M * N * 4
                tflops = flops / us * 1e-6
                gbs = nbytes / us * 1e-3
                ai = flops / nbytes
                bound = "mfma" if ai * HBM_PEAK_GBS * 1e9 > MFMA_F16_PEAK_TFLOPS * 1e12 else "hbm"
                frac = tflops / MFMA_F16_PEAK_TFLOPS if bound == "mfma" else gbs / HBM_PEAK_GBS
                rec = {"quant": qname, "M": M, "K": K, "N": N, "us": round(us, 2), "tflops": round(tflops, 2),
                       "gbs": round(gbs, 1), "bound": bound, "frac": round(frac, 3)}
                if M == 1 and N * K > 2**24:
                    # the same weight copies read once by a plain streaming-read kernel, timed the same way:
                    # what a launch that only reads these bytes costs on this box
                    rd_us = stream_read_us(torch, dW, stride, n_copies, reps)
                    if rd_us is not None:
                        rec["read_only_us"] = round(rd_us, 2)
                        rec["read_only_frac"] = round(stride / rd_us * 1e-3 / HBM_PEAK_GBS, 3)
                out.append(rec)
                del dW, x, y
    return out


def cpu_baseline(gguf, x, groups, t_ctx, horizon, budget_s=12.0):
    """Oracle forecast on a bounded sample of the same workload (whole series, 3 variates each)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import t0ref  # the CPU checker/baseline, test infrastructure

    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or (os.cpu_count() or 1)
    t0ref.set_threads(threads)
    om = t0ref.Model(gguf)
    n_var = 3
    n = 2
    t = time.perf_counter()
    om.forecast_grouped(x[: n * n_var], groups[: n * n_var], t_ctx, horizon)
    first = time.perf_counter() - t
    n = max(1, min(64, int(budget_s / max(first / 2, 1e-3))))
    t = time.perf_counter()
    om.forecast_grouped(x[: n * n_var], groups[: n * n_var], t_ctx, horizon)
    dt = time.perf_counter() - t
    return {"value": round(n / dt, 3), "unit": "forecasts/s", "cores": threads, "kind": "port",
            "sample": f"{n} series x {n_var} variates (of 256), ctx {t_ctx}, h {horizon}, one forecast_grouped call, "
                      f"{dt:.1f} s"}


# Device kernel behind each profiled GEMM kind of the forward at config 4
# (template args: weight type 2 = Q4_0 / 8 = Q8_0, epilogue 1 f16 store / 3 SwiGLU,
# waves, f32 activations).
KERNEL_OF = {("gemm_w0_swiglu", "q4_0"): "k_gemm_bf<2, 3, 4, false, 256>",
             ("gemm_w0_swiglu", "q8_0"): "k_gemm_bf<8, 3, 4, false, 256>",
             ("gemm_qkv", "q4_0"): "k_gemm_bf<2, 1, 4, false, 256>",
             ("gemm_qkv", "q8_0"): "k_gemm_bf<8, 1, 4, false, 256>"}
COPY_BYTES = 256 << 20  # the --calibrate-copy kernel reads and writes this many bytes
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_config4.json")


def _pmc_per_dispatch(d):
    """{dispatch_id: (kernel_name, grid, value)} from a rocprofv3 --pmc csv directory."""
    import csv
    import glob
    out = {}
    for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
        for r in csv.DictReader(open(f)):
            k = (f, r["Dispatch_Id"])
            name, grid, v = out.get(k, (r["Kernel_Name"], int(r["Grid_Size"]), 0.0))
            out[k] = (name, grid, v + float(r["Counter_Value"]))
    return out


def traffic_of(kind, quant):
    """HBM bytes per launch of `kind`'s kernel from the committed --pmc summary, or None."""
    try:
        rec = json.load(open(TRAFFIC_FILE))
    except (OSError, ValueError):
        return None
    same = (rec.get("kind"), rec.get("quant"), rec.get("kernel")) == (kind, quant, KERNEL_OF.get((kind, quant)))
    return rec.get("traffic") if same else None


def summarize(prof_dir, fetch_dir, write_dir, quant, kind):
    """Summaries of a --kernel-trace --stats run and two --pmc runs (FETCH_SIZE, WRITE_SIZE;
    KiB per dispatch) of this script: per-kernel time table and the HBM traffic of `kind`'s
    kernel, each counter scaled by what it reads for the 256 MiB calibration copy."""
    import csv
    import glob
    lines = []
    stats = glob.glob(os.path.join(prof_dir, "**", "*kernel_stats.csv"), recursive=True)
    if stats:
        rows = list(csv.DictReader(open(stats[0])))
        rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
        lines += ["| kernel | calls | total us | avg us | % |", "|---|---|---|---|---|"]
        for r in rows[:16]:
            lines.append(f"| `{r['Name'][:110]}` | {r['Calls']} | {float(r['TotalDurationNs']) / 1e3:.1f} | "
                         f"{float(r['AverageNs']) / 1e3:.2f} | {float(r['Percentage']):.2f} |")
    res = {"kind": kind, "quant": quant, "kernel": KERNEL_OF[(kind, quant)]}
    for ctr, d in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        disp = _pmc_per_dispatch(d)
        copies = [v for (n, g, v) in disp.values() if "copyBuffer" in n and v * 1024 > COPY_BYTES / 4]
        if not copies:
            raise SystemExit(f"{d}: no calibration copy dispatch (run with --calibrate-copy)")
        factor = COPY_BYTES / (max(copies) * 1024)
        vals = [v for (n, g, v) in disp.values() if KERNEL_OF[(kind, quant)] in n]
        if not vals:
            raise SystemExit(f"{d}: no dispatch of {KERNEL_OF[(kind, quant)]}")
        per = sum(vals) / len(vals) * 1024 * factor
        res[ctr.lower()] = {"kib_per_dispatch_raw": round(sum(vals) / len(vals), 1), "copy_factor": round(factor, 3),
                            "bytes_per_launch": int(per), "dispatches": len(vals)}
    res["traffic"] = res["fetch_size"]["bytes_per_launch"] + res["write_size"]["bytes_per_launch"]
    lines += ["", f"HBM traffic of `{KERNEL_OF[(kind, quant)]}` ({kind}, {quant}) per launch:",
              f"FETCH_SIZE {res['fetch_size']['kib_per_dispatch_raw']} KiB x {res['fetch_size']['copy_factor']} "
              f"+ WRITE_SIZE {res['write_size']['kib_per_dispatch_raw']} KiB x {res['write_size']['copy_factor']} "
              f"= {res['traffic'] / 1e6:.1f} MB"]
    return "\n".join(lines), res


def trace_table(trace_dir, min_calls=1):
    """Per (kernel, grid) median / mean duration from a rocprofv3 --kernel-trace csv directory,
    in first-dispatch order: consecutive launches of one shape (the GEMM sweep, a forecast's
    kernel sequence) each get a row."""
    import csv
    import glob
    import re
    files = glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True)
    if not files:
        raise SystemExit(f"{trace_dir}: no kernel_trace.csv")
    rows = list(csv.DictReader(open(files[0])))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    groups, order = {}, []
    for r in rows:
        name = re.sub(r"\(t0h::\w+(, t0h::\w+)?\)$|\(.*\)$", "", r["Kernel_Name"].replace("(anonymous namespace)::", ""))
        name = name.replace("void ", "").replace("t0h::", "")
        key = (name, int(r["Grid_Size_X"]), int(r["Workgroup_Size_X"]))
        if key not in groups:
            groups[key] = []
            order.append(key)
        groups[key].append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    lines = ["| kernel | workgroups x threads | calls | median us | mean us |", "|---|---|---|---|---|"]
    for key in order:
        d = groups[key]
        if len(d) < min_calls:
            continue
        d.sort()
        lines.append(f"| `{key[0][:100]}` | {key[1] // max(key[2], 1)} x {key[2]} | {len(d)} | {d[len(d) // 2] / 1e3:.2f} | "
                     f"{sum(d) / len(d) / 1e3:.2f} |")
    return "\n".join(lines)


def main():
    if len(sys.argv) > 1 and sys.argv[1] == "--trace-table":
        sp = argparse.ArgumentParser()
        sp.add_argument("--trace-table", metavar="TRACE_DIR", required=True)
        sp.add_argument("--min-calls", type=int, default=1)
        a = sp.parse_args()
        print(trace_table(a.trace_table, a.min_calls))
        return
    if len(sys.argv) > 1 and sys.argv[1] == "--summarize":
        sp = argparse.ArgumentParser()
        sp.add_argument("--summarize", nargs=3, metavar=("PROF_DIR", "FETCH_DIR", "WRITE_DIR"), required=True)
        sp.add_argument("--quant", default="q4_0", choices=["q4_0", "q8_0"])
        sp.add_argument("--kind", default="gemm_w0_swiglu")
        sp.add_argument("--traffic-out", default=None, help="write the traffic record (JSON) here")
        a = sp.parse_args()
        text, res = summarize(*a.summarize, a.quant, a.kind)
        print(text)
        if a.traffic_out:
            json.dump(res, open(a.traffic_out, "w"), indent=1)
        return
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--profile-steps", type=int, default=5)
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-workloads", action="store_true", help="skip BASELINE configs 3 and 5")
    ap.add_argument("--quant", default="q4_0", choices=["q4_0", "q8_0"])
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="first run one plain 256 MiB device-to-device copy (reference for PMC byte counters)")
    args = ap.parse_args()
    if args.steps < 1 or args.profile_steps < 1:
        ap.error("--steps and --profile-steps must be at least 1")
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build runs the whole forecast on a single MI355X "
              "(series would shard across GPUs with no collectives). Use --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    import t0hip

    if args.calibrate_copy:
        src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    qtype = t0hip.Q4_0 if args.quant == "q4_0" else t0hip.Q8_0
    bpv = 18 / 32 if args.quant == "q4_0" else 34 / 32
    cfg = t0hip.make_config()  # 12 layers, embed 768, 12 heads, hidden 2048, patch 32, 9 quantiles
    log("synthesizing model")
    gguf = t0hip.synth_model_gguf(cfg, quant=qtype, seed=0)
    engine = t0hip.Engine(0)
    model = t0hip.load_model_from_gguf(engine, gguf)
    n_series, n_var, t_ctx, horizon = 256, 3, 2048, 64
    x, groups = config4_inputs(n_series, n_var, t_ctx)
    d_x = torch.from_numpy(x).cuda()
    d_out = torch.empty((n_series * n_var, horizon, cfg.n_quantiles), dtype=torch.float32, device="cuda")

    def step():
        t0hip.forecast_grouped_dev(model, d_x.data_ptr(), groups, t_ctx, horizon, d_out.data_ptr())

    log(f"warmup {args.warmup}")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # per-kernel-kind event timing of every launch of the forward, in untimed steps of their own
    # (recording all of them costs the step about 5 %); it names the dominant GEMM kind
    M = n_series * n_var * ((t_ctx + horizon + 31) // 32)
    model.profile(True)
    for _ in range(args.profile_steps):
        step()
    torch.cuda.synchronize()
    prof = model.profile_report()
    model.profile(False)
    kernels = {k: {"launches": n, "avg_us": round(ms / max(n, 1) * 1e3, 2), "total_ms_per_step": round(ms / args.profile_steps, 3)}
               for k, (n, ms) in prof.items()}
    gemm_names = [k for k in prof if gemm_flops(k, M, cfg)]
    dom = max(gemm_names, key=lambda k: prof[k][1])
    total_gemm_flops = sum(gemm_flops(k, M, cfg) * prof[k][0] for k in gemm_names) / args.profile_steps
    total_gemm_ms = sum(prof[k][1] for k in gemm_names) / args.profile_steps

    # the timed steps; HIP events on the model's stream bracket each launch of the dominant kind
    # only (two event records per launch, 12 launches a step)
    log(f"timing {args.steps} steps")
    model.profile_kind(dom)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    n_l, ms_l = model.profile_report()[dom]
    model.profile(False)
    ms_per_step = elapsed / args.steps * 1e3
    value = n_series * args.steps / elapsed
    log(f"{ms_per_step:.3f} ms/step, {value:.1f} forecasts/s")

    avg_s = ms_l / n_l * 1e-3
    flops = gemm_flops(dom, M, cfg)
    achieved = flops / avg_s * 1e-12
    roofline = {"kernel": dom, "bound": "mfma", "achieved": round(achieved, 1), "peak": MFMA_F16_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / MFMA_F16_PEAK_TFLOPS, 4), "traffic": traffic_of(dom, args.quant),
                "flops_per_launch": flops, "algorithmic_bytes_per_launch": int(gemm_bytes(dom, M, cfg, bpv)),
                "avg_launch_us": round(avg_s * 1e6, 2), "timed_launches": n_l}
    log(f"dominant kernel {dom}: {roofline['avg_launch_us']} us over {n_l} timed launches, {achieved:.0f} TFLOP/s")

    # the same step with host buffers (t0h_forecast_grouped: context upload and result download
    # included); reported beside `value`, never as it
    host_steps = max(1, min(5, args.steps))
    t0hip.forecast_grouped(engine, model, x, groups, t_ctx, horizon)
    t0 = time.perf_counter()
    for _ in range(host_steps):
        t0hip.forecast_grouped(engine, model, x, groups, t_ctx, horizon)
    host_rate = n_series * host_steps / (time.perf_counter() - t0)
    log(f"host buffers: {host_rate:.1f} forecasts/s")

    sweep = None
    if not args.no_sweep:
        log("GEMM sweep (configs 1-2)")
        sweep = gemm_sweep(torch, t0hip)
    workloads = None
    if not args.no_workloads:
        log("BASELINE configs 3 and 5")
        workloads = other_workloads(torch, t0hip, engine, cfg, not args.no_cpu)
    cpu = None
    if not args.no_cpu:
        log("CPU baseline (oracle)")
        cpu = cpu_baseline(gguf, x, groups, t_ctx, horizon)
        log(f"cpu {cpu['value']} forecasts/s on {cpu['cores']} threads")

    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "forecasts/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f16", "data": "synthetic",
        "config": {"workload": "BASELINE config 4: 256 series x 3 variates, ctx 2048, horizon 64, "
                               f"{args.quant.upper()} synthetic t0 (12 layers, embed 768, 12 heads, SwiGLU 2048, "
                               "9 quantiles), sine mixture x lognormal scale, 10% NaN gaps",
                   "rows": n_series * n_var, "patches": M // (n_series * n_var), "gemm_rows": M},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "forward_gemm_tflops": round(total_gemm_flops / (total_gemm_ms * 1e-3) * 1e-12, 1),
        "host_buffers_forecasts_per_s": round(host_rate, 2),
        "kernels": kernels,
        "gemm_sweep": sweep,
        "workloads": workloads,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
