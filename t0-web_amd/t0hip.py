"""Python binding of libt0hip.so, mirroring t0-fast's public interface.

Reference surface (crates/t0-fast/src/lib.rs:22-341): `Engine`, `GpuModel`,
`load_model_from_gguf`, `forecast`, `forecast_batch_chunked`,
`forecast_batch_rows_chunked`, `forecast_rollout`, plus `model::forward_async`
(crates/t0-fast/src/model.rs:693-808).  Names, argument meaning and output
layouts follow the reference; errors surface as `T0HipError` carrying the C-ABI
status code and message (the reference's anyhow::Error / panics).

All compute goes through the C ABI declared in include/t0hip.h; this module
only marshals arrays.  There is no CPU fallback: without the built library or a
gfx950 device the calls raise.
"""
import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libt0hip.so")

F32, F16, Q4_0, Q8_0 = 0, 1, 2, 8
MAX_Q = 64
MAX_HORIZON = 1024
NOALLOC_MAX_PATCHES = 256
MASK_VALID, MASK_PAD, MASK_MISSING, MASK_CENSORED, MASK_WITHHELD = 0, 1, 2, 3, 4
VT_TARGET, VT_HISTORICAL, VT_FUTURE = 0, 1, 2

STATUS = {
    0: "OK", -1: "INVALID_ARG", -2: "GGUF_MAGIC", -3: "GGUF_VERSION", -4: "GGUF_TENSOR_TYPE",
    -5: "GGUF_META_TYPE", -6: "GGUF_BOUNDS", -7: "MISSING_TENSOR", -8: "METADATA", -9: "HORIZON",
    -10: "FUTURE_ROWS", -11: "NO_DEVICE", -12: "HIP", -13: "SHAPE", -14: "UNSUPPORTED", -15: "OOM",
    -16: "SAFETENSORS", -17: "CONFIG", -18: "NUMERIC",
}


class T0HipError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"{STATUS.get(code, code)} ({code}): {msg}")
        self.code = code
        self.status = STATUS.get(code, str(code))


class Config(C.Structure):
    """≡ T0Config (crates/t0-core/src/config.rs:6-22)."""
    _fields_ = [
        ("embed_dim", C.c_uint32), ("num_layers", C.c_uint32), ("num_heads", C.c_uint32),
        ("mlp_hidden_dim", C.c_uint32), ("patch_size", C.c_uint32), ("group_every_n", C.c_int64),
        ("dropout", C.c_float), ("n_quantiles", C.c_uint32), ("quantile_levels", C.c_float * MAX_Q),
        ("scaler_use_arcsinh", C.c_int32), ("scaler_eps", C.c_float), ("scaler_variance_offset", C.c_int32),
    ]

    @property
    def levels(self):
        return np.array(self.quantile_levels[: self.n_quantiles], np.float32)

    @property
    def head_dim(self):
        return self.embed_dim // self.num_heads


class Series(C.Structure):
    """≡ t0_core::data::TimeSeries (data.rs:24-33)."""
    _fields_ = [("v", C.c_size_t), ("t", C.c_size_t), ("variates", C.c_void_p), ("mask", C.c_void_p),
                ("group_ids", C.c_void_p), ("variate_type", C.c_void_p)]


class SynthSpec(C.Structure):
    _fields_ = [("config", Config), ("seed", C.c_uint64), ("weight_std", C.c_float), ("bias_std", C.c_float),
                ("norm_std", C.c_float), ("emb_std", C.c_float), ("increment_bias", C.c_float)]


_lib = None
SYMBOLS = [
    "t0h_last_error", "t0h_abi_version", "t0h_ctx_create", "t0h_ctx_destroy", "t0h_gguf_inspect",
    "t0h_model_load_gguf", "t0h_model_destroy", "t0h_model_config", "t0h_model_weight_bytes", "t0h_model_stream",
    "t0h_model_workspace", "t0h_model_profile", "t0h_model_profile_kind", "t0h_model_profile_entry", "t0h_model_graph_replay", "t0h_model_check_numerics", "t0h_forward", "t0h_forecast", "t0h_forecast_batch_chunked",
    "t0h_forecast_batch_rows_chunked", "t0h_forecast_grouped", "t0h_forecast_grouped_dev",
    "t0h_forecast_grouped_dev_noalloc",
    "t0h_forecast_grouped_ar", "t0h_forecast_rollout", "t0h_dequant", "t0h_gemm_q", "t0h_gemm_f16", "t0h_row_bytes",
    "t0h_quantize", "t0h_synth_model_gguf", "t0h_export_gguf", "t0h_export_gguf_from_safetensors",
    "t0h_model_load_safetensors",
]


def lib():
    """Load libt0hip.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `make -C t0-web_amd` or __graft_entry__.build()")
    L = C.CDLL(LIB_PATH)
    P, S, I = C.c_void_p, C.c_size_t, C.c_int
    L.t0h_last_error.restype = C.c_char_p
    L.t0h_last_error.argtypes = []
    L.t0h_abi_version.argtypes = []
    L.t0h_ctx_create.argtypes = [I, C.POINTER(P)]
    L.t0h_ctx_destroy.restype = None
    L.t0h_ctx_destroy.argtypes = [P]
    L.t0h_gguf_inspect.argtypes = [P, S, C.POINTER(Config), C.POINTER(S)]
    L.t0h_model_load_gguf.argtypes = [P, P, S, C.POINTER(P)]
    L.t0h_model_destroy.restype = None
    L.t0h_model_destroy.argtypes = [P]
    L.t0h_model_config.argtypes = [P, C.POINTER(Config)]
    L.t0h_model_weight_bytes.argtypes = [P, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]
    L.t0h_model_stream.restype = P
    L.t0h_model_stream.argtypes = [P]
    L.t0h_model_workspace.argtypes = [P, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]
    L.t0h_model_profile.argtypes = [P, I]
    L.t0h_model_profile_kind.argtypes = [P, C.c_char_p]
    L.t0h_model_profile_entry.argtypes = [P, S, C.c_char_p, S, C.POINTER(C.c_uint64), C.POINTER(C.c_double)]
    L.t0h_model_graph_replay.argtypes = [P, I]
    L.t0h_model_check_numerics.argtypes = [P]
    L.t0h_forward.argtypes = [P, C.POINTER(Series), P, S, P, P]
    L.t0h_forecast.argtypes = [P, P, S, S, S, P, S]
    L.t0h_forecast_batch_chunked.argtypes = [P, P, S, S, S, S, P, S]
    L.t0h_forecast_batch_rows_chunked.argtypes = [P, P, P, S, S, S, P, S]
    L.t0h_forecast_grouped.argtypes = [P, P, P, S, S, S, P, S]
    L.t0h_forecast_grouped_dev.argtypes = [P, P, P, S, S, S, P]
    L.t0h_forecast_grouped_dev_noalloc.argtypes = [P, P, P, S, S, S, P]
    L.t0h_forecast_grouped_ar.argtypes = [P, P, P, S, S, S, S, P, S]
    L.t0h_forecast_rollout.argtypes = [P, P, S, S, P, S, P, S]
    L.t0h_dequant.argtypes = [I, P, S, P, P]
    L.t0h_gemm_q.argtypes = [I, P, P, P, P, S, S, S, I, P]
    L.t0h_gemm_f16.argtypes = [I, P, P, P, P, S, S, S, I, I, P]
    L.t0h_row_bytes.restype = S
    L.t0h_row_bytes.argtypes = [I, S]
    L.t0h_quantize.argtypes = [I, P, S, P, S]
    L.t0h_synth_model_gguf.argtypes = [C.POINTER(SynthSpec), I, P, S, C.POINTER(S)]
    L.t0h_export_gguf.argtypes = [P, S, I, P, S, C.POINTER(S)]
    L.t0h_export_gguf_from_safetensors.argtypes = [P, S, C.c_char_p, I, P, S, C.POINTER(S)]
    L.t0h_model_load_safetensors.argtypes = [P, P, S, C.c_char_p, I, C.POINTER(P)]
    _lib = L
    return L


def _check(rc):
    if rc != 0:
        raise T0HipError(rc, lib().t0h_last_error().decode(errors="replace"))


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---------------------------------------------------------------------------
# codec / export / synthetic model (host side, no GPU needed)
# ---------------------------------------------------------------------------
def row_bytes(qtype, n):
    return lib().t0h_row_bytes(qtype, n)


def quantize(qtype, x):
    """≡ quantize_for (crates/t0-core/src/gguf.rs:192-211)."""
    x = _f32(x).ravel()
    out = np.zeros(row_bytes(qtype, x.size), np.uint8)
    _check(lib().t0h_quantize(qtype, _p(x), x.size, _p(out), out.size))
    return out


def inspect_gguf(gguf_bytes):
    b = np.frombuffer(bytes(gguf_bytes), np.uint8)
    cfg = Config()
    n = C.c_size_t()
    _check(lib().t0h_gguf_inspect(_p(b), b.size, C.byref(cfg), C.byref(n)))
    return cfg, n.value


def make_config(embed_dim=768, num_layers=12, num_heads=12, mlp_hidden_dim=2048, patch_size=32, group_every_n=3,
                quantile_levels=(0.1, 0.2, 0.3, 0.4, 0.5, 0.6, 0.7, 0.8, 0.9), use_arcsinh=True, eps=0.1,
                variance_offset=True):
    c = Config()
    c.embed_dim, c.num_layers, c.num_heads = embed_dim, num_layers, num_heads
    c.mlp_hidden_dim, c.patch_size, c.group_every_n = mlp_hidden_dim, patch_size, group_every_n
    c.dropout = 0.0
    c.n_quantiles = len(quantile_levels)
    for i, q in enumerate(quantile_levels):
        c.quantile_levels[i] = q
    c.scaler_use_arcsinh, c.scaler_eps, c.scaler_variance_offset = int(use_arcsinh), eps, int(variance_offset)
    return c


def synth_model_gguf(config=None, quant=Q8_0, seed=0, weight_std=0.02, bias_std=0.02, norm_std=0.1, emb_std=0.02,
                     increment_bias=-3.0):
    """Seeded random-init model written as GGUF with export_gguf's policy (weights.rs:187-227)."""
    spec = SynthSpec()
    spec.config = config if config is not None else make_config()
    spec.seed, spec.weight_std, spec.bias_std = seed, weight_std, bias_std
    spec.norm_std, spec.emb_std, spec.increment_bias = norm_std, emb_std, increment_bias
    n = C.c_size_t()
    _check(lib().t0h_synth_model_gguf(C.byref(spec), quant, None, 0, C.byref(n)))
    out = np.zeros(n.value, np.uint8)
    _check(lib().t0h_synth_model_gguf(C.byref(spec), quant, _p(out), out.size, C.byref(n)))
    return out.tobytes()


def export_gguf(gguf_bytes, quant):
    """Re-export every tensor of a GGUF with another quantization (≡ Weights::export_gguf)."""
    b = np.frombuffer(bytes(gguf_bytes), np.uint8)
    n = C.c_size_t()
    _check(lib().t0h_export_gguf(_p(b), b.size, quant, None, 0, C.byref(n)))
    out = np.zeros(n.value, np.uint8)
    _check(lib().t0h_export_gguf(_p(b), b.size, quant, _p(out), out.size, C.byref(n)))
    return out.tobytes()


def export_gguf_from_safetensors(st_bytes, config_json, quant):
    """≡ t0-cli export-gguf (crates/cli/src/main.rs:283-295): F32 model.safetensors bytes + the
    checkpoint's config.json text -> GGUF bytes with Weights::export_gguf's policy."""
    b = np.frombuffer(bytes(st_bytes), np.uint8)
    cj = config_json.encode() if isinstance(config_json, str) else bytes(config_json)
    n = C.c_size_t()
    _check(lib().t0h_export_gguf_from_safetensors(_p(b), b.size, cj, quant, None, 0, C.byref(n)))
    out = np.zeros(n.value, np.uint8)
    _check(lib().t0h_export_gguf_from_safetensors(_p(b), b.size, cj, quant, _p(out), out.size, C.byref(n)))
    return out.tobytes()


# ---------------------------------------------------------------------------
# Engine / GpuModel
# ---------------------------------------------------------------------------
class Engine:
    """≡ t0_fast::Engine (crates/t0-fast/src/engine.rs:18-44): one GPU, shareable by models."""

    def __init__(self, device=0):
        self._lib = lib()  # held so that close() still reaches it while the interpreter exits
        h = C.c_void_p()
        _check(self._lib.t0h_ctx_create(device, C.byref(h)))
        self.h = h

    def close(self):
        if getattr(self, "h", None):
            self._lib.t0h_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()


class GpuModel:
    """≡ t0_fast::GpuModel (crates/t0-fast/src/model.rs:170-187): resident weights + own workspace/stream.
    Calls on one model must be serialized by the caller."""

    def __init__(self, engine, gguf_bytes=None, _handle=None):
        self.engine = engine  # keep the context alive
        self._lib = lib()
        if _handle is None:
            self._bytes = np.frombuffer(bytes(gguf_bytes), np.uint8)
            h = C.c_void_p()
            _check(lib().t0h_model_load_gguf(engine.h, _p(self._bytes), self._bytes.size, C.byref(h)))
        else:
            h = _handle
        self.h = h
        cfg = Config()
        _check(lib().t0h_model_config(self.h, C.byref(cfg)))
        self.config = cfg

    def close(self):
        if getattr(self, "h", None):
            self._lib.t0h_model_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    @property
    def n_quantiles(self):
        return self.config.n_quantiles

    @property
    def stream(self):
        return lib().t0h_model_stream(self.h)

    def quantizable_gpu_bytes(self):
        q, t = C.c_uint64(), C.c_uint64()
        _check(lib().t0h_model_weight_bytes(self.h, C.byref(q), C.byref(t)))
        return q.value

    def total_weight_bytes(self):
        q, t = C.c_uint64(), C.c_uint64()
        _check(lib().t0h_model_weight_bytes(self.h, C.byref(q), C.byref(t)))
        return t.value

    def profile(self, enable=True):
        """Start (reset) or stop per-kernel-kind event timing of this model's forward."""
        _check(lib().t0h_model_profile(self.h, int(enable)))

    def profile_kind(self, kind):
        """Start (reset) event timing of the launches of one kernel kind only; stop with profile(False)."""
        _check(lib().t0h_model_profile_kind(self.h, kind.encode()))

    def profile_report(self):
        """{kernel kind: (launches, total_ms)} recorded since profile(True)."""
        out = {}
        i = 0
        name = C.create_string_buffer(128)
        while True:
            n, ms = C.c_uint64(), C.c_double()
            rc = lib().t0h_model_profile_entry(self.h, i, name, 128, C.byref(n), C.byref(ms))
            if rc != 0:
                break
            out[name.value.decode()] = (n.value, ms.value)
            i += 1
        return out

    def graph_replay(self, enable=True):
        """Capture and replay each window forward as a HIP graph (default) or run it eagerly."""
        _check(lib().t0h_model_graph_replay(self.h, int(enable)))

    def check_numerics(self):
        """Wait for the model's stream; raise T0HipError("NUMERIC") if a forecast since the last
        check (device-output calls included) produced non-finite model outputs."""
        _check(lib().t0h_model_check_numerics(self.h))

    def workspace(self):
        r, a = C.c_uint64(), C.c_uint64()
        _check(lib().t0h_model_workspace(self.h, C.byref(r), C.byref(a)))
        return r.value, a.value


def load_model_from_gguf(engine, gguf_bytes):
    """≡ t0_fast::load_model_from_gguf (lib.rs:42-44)."""
    return GpuModel(engine, gguf_bytes)


def load_model(engine, st_bytes, config_json, quant):
    """≡ t0_fast::load_model(engine, weights, config, quant) (lib.rs:34-36): an F32
    model.safetensors and its config.json, big matmuls quantized as `quant`."""
    b = np.frombuffer(bytes(st_bytes), np.uint8)
    cj = config_json.encode() if isinstance(config_json, str) else bytes(config_json)
    h = C.c_void_p()
    _check(lib().t0h_model_load_safetensors(engine.h, _p(b), b.size, cj, quant, C.byref(h)))
    return GpuModel(engine, _handle=h)


def forward(model, variates, mask, group_ids, variate_type, trace=False):
    """≡ model::forward_async (t0-fast model.rs:693-808): padded + scaled [v, t] series ->
    [v, p, patch_size, n_quantiles] (plus the patch-embedding and layer-0 taps when trace)."""
    x = _f32(variates)
    v, t = x.shape
    m = np.ascontiguousarray(mask, np.int8)
    g = np.ascontiguousarray(group_ids, np.int64)
    vt = np.ascontiguousarray(variate_type, np.int64)
    ps = model.config.patch_size
    p = t // ps if ps else 0
    out = np.zeros((v, p, ps, model.n_quantiles), np.float32)
    E = model.config.embed_dim
    pe = np.zeros((v, p, E), np.float32) if trace else None
    l0 = np.zeros((v, p, E), np.float32) if trace else None
    s = Series(v, t, x.ctypes.data, m.ctypes.data, g.ctypes.data, vt.ctypes.data)
    _check(lib().t0h_forward(model.h, C.byref(s), _p(out), out.size, _p(pe), _p(l0)))
    return (out, pe, l0) if trace else out


def forecast(engine, model, context, v, t_ctx, horizon):
    """≡ t0_fast::forecast (lib.rs:102-109) -> [v, horizon, n_quantiles]."""
    c = _f32(context)
    out = np.zeros((v, horizon, model.n_quantiles), np.float32)
    _check(lib().t0h_forecast(model.h, _p(c), v, t_ctx, horizon, _p(out), out.size))
    return out


def forecast_batch_chunked(engine, model, contexts, n_signals, t_ctx, horizon, chunk_size):
    """≡ t0_fast::forecast_batch_chunked (lib.rs:118-146) -> [n_signals, horizon, n_quantiles]."""
    c = _f32(contexts)
    out = np.zeros((n_signals, horizon, model.n_quantiles), np.float32)
    _check(lib().t0h_forecast_batch_chunked(model.h, _p(c), n_signals, t_ctx, horizon, chunk_size, _p(out), out.size))
    return out


def forecast_batch_rows_chunked(engine, model, contexts, lengths, horizon, chunk_size):
    """≡ t0_fast::forecast_batch_rows_chunked (lib.rs:175-248); contexts concatenated per lengths."""
    c = _f32(contexts)
    ln = np.ascontiguousarray(lengths, np.uint64)
    if c.size != int(ln.sum()):
        raise T0HipError(-1, "forecast_batch_rows: contexts.len() must equal sum(lengths)")
    out = np.zeros((ln.size, horizon, model.n_quantiles), np.float32)
    _check(lib().t0h_forecast_batch_rows_chunked(model.h, _p(c), _p(ln), ln.size, horizon, chunk_size, _p(out),
                                                 out.size))
    return out


def forecast_grouped(engine, model, contexts, row_group, t_ctx, horizon):
    """Multivariate batch with one group id per row -> [n_rows, horizon, n_quantiles]."""
    c = _f32(contexts)
    g = np.ascontiguousarray(row_group, np.int64)
    out = np.zeros((g.size, horizon, model.n_quantiles), np.float32)
    _check(lib().t0h_forecast_grouped(model.h, _p(c), _p(g), g.size, t_ctx, horizon, _p(out), out.size))
    return out


def forecast_grouped_dev_noalloc(model, d_contexts, row_group, t_ctx, horizon, d_out):
    """forecast_grouped_dev without any device or pinned allocation: the window's workspace is a
    slice of the library's static per-GPU scratch (T0H_NOALLOC_SCRATCH_BYTES)."""
    g = np.ascontiguousarray(row_group, np.int64)
    _check(lib().t0h_forecast_grouped_dev_noalloc(model.h, C.c_void_p(d_contexts), _p(g), g.size, t_ctx, horizon,
                                                  C.c_void_p(d_out)))


def forecast_grouped_dev(model, d_contexts, row_group, t_ctx, horizon, d_out):
    """Device-resident variant: d_contexts / d_out are device addresses (ints); enqueued on model.stream."""
    g = np.ascontiguousarray(row_group, np.int64)
    _check(lib().t0h_forecast_grouped_dev(model.h, C.c_void_p(d_contexts), _p(g), g.size, t_ctx, horizon,
                                          C.c_void_p(d_out)))


def forecast_grouped_ar(engine, model, contexts, row_group, t_ctx, horizon, steps):
    """AR loop over forecast_grouped, appending each row's median and re-windowing."""
    c = _f32(contexts)
    g = np.ascontiguousarray(row_group, np.int64)
    out = np.zeros((g.size, steps * horizon, model.n_quantiles), np.float32)
    _check(lib().t0h_forecast_grouped_ar(model.h, _p(c), _p(g), g.size, t_ctx, horizon, steps, _p(out), out.size))
    return out


def forecast_rollout(engine, model, context, t_ctx, prediction_length, query_quantile_levels):
    """≡ t0_fast::forecast_rollout (lib.rs:259-341) -> [prediction_length, n_query]."""
    c = _f32(context)
    q = _f32(query_quantile_levels)
    out = np.zeros((prediction_length, q.size), np.float32)
    _check(lib().t0h_forecast_rollout(model.h, _p(c), t_ctx, prediction_length, _p(q), q.size, _p(out), out.size))
    return out


# ---------------------------------------------------------------------------
# kernel-level entry points on device pointers (ints) + a hipStream_t
# ---------------------------------------------------------------------------
def dequant_dev(qtype, d_blocks, n, d_out, stream=None):
    _check(lib().t0h_dequant(qtype, C.c_void_p(d_blocks), n, C.c_void_p(d_out), C.c_void_p(stream)))


def gemm_q_dev(wtype, d_w, d_x, d_bias, d_y, m, n, k, act=0, stream=None):
    _check(lib().t0h_gemm_q(wtype, C.c_void_p(d_w), C.c_void_p(d_x), C.c_void_p(d_bias) if d_bias else None,
                            C.c_void_p(d_y), m, n, k, act, C.c_void_p(stream)))


EPI_STORE_F32, EPI_STORE_F16, EPI_RESID_F32, EPI_SWIGLU_F16 = 0, 1, 2, 3


def gemm_f16_dev(wtype, d_w, d_x, d_bias, d_y, m, n, k, epilogue, tile=0, stream=None):
    """The forward's GEMM kernels on device pointers: f16 x [m, k]; see t0hip.h t0h_gemm_f16."""
    _check(lib().t0h_gemm_f16(wtype, C.c_void_p(d_w), C.c_void_p(d_x), C.c_void_p(d_bias) if d_bias else None,
                              C.c_void_p(d_y), m, n, k, epilogue, tile, C.c_void_p(stream)))
