"""ctypes binding of oracle/libt0ref.so — TEST INFRASTRUCTURE ONLY.

The CPU restatement of t0-core used as the parity checker by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg.  The product
(t0-web_amd/) never imports this module.
"""
import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libt0ref.so")

F32, F16, Q4_0, Q8_0 = 0, 1, 2, 8
MAX_Q = 64


class Config(C.Structure):
    _fields_ = [
        ("embed_dim", C.c_uint32), ("num_layers", C.c_uint32), ("num_heads", C.c_uint32),
        ("mlp_hidden_dim", C.c_uint32), ("patch_size", C.c_uint32), ("group_every_n", C.c_int64),
        ("dropout", C.c_float), ("n_quantiles", C.c_uint32), ("quantile_levels", C.c_float * MAX_Q),
        ("scaler_use_arcsinh", C.c_int32), ("scaler_eps", C.c_float), ("scaler_variance_offset", C.c_int32),
    ]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle` (or __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        P, S = C.c_void_p, C.c_size_t
        L.t0r_f16_to_f32.restype = C.c_float
        L.t0r_f16_to_f32.argtypes = [C.c_uint16]
        L.t0r_f32_to_f16.restype = C.c_uint16
        L.t0r_f32_to_f16.argtypes = [C.c_float]
        L.t0r_row_bytes.restype = S
        L.t0r_row_bytes.argtypes = [C.c_int, S]
        for n in ("t0r_quantize_q8_0", "t0r_quantize_q4_0", "t0r_dequantize_q8_0", "t0r_dequantize_q4_0"):
            getattr(L, n).restype = None
            getattr(L, n).argtypes = [P, S, P]
        L.t0r_dequantize_for.argtypes = [C.c_int, P, S, P]
        L.t0r_quantize_for.argtypes = [C.c_int, P, S, P]
        L.t0r_model_load_gguf.argtypes = [P, S, C.POINTER(P)]
        L.t0r_model_free.restype = None
        L.t0r_model_free.argtypes = [P]
        L.t0r_model_config.argtypes = [P, C.POINTER(Config)]
        L.t0r_model_tensor.restype = S
        L.t0r_model_tensor.argtypes = [P, C.c_char_p, P, S, P, P]
        L.t0r_model_tensor_count.restype = S
        L.t0r_model_tensor_count.argtypes = [P]
        L.t0r_export_gguf.restype = S
        L.t0r_export_gguf.argtypes = [P, C.c_int, P, S]
        L.t0r_set_threads.restype = None
        L.t0r_set_threads.argtypes = [C.c_int]
        L.t0r_linear.restype = None
        L.t0r_linear.argtypes = [P, P, P, P, S, S, S, C.c_int]
        L.t0r_rmsnorm.restype = None
        L.t0r_rmsnorm.argtypes = [P, P, P, S, S, C.c_float]
        L.t0r_rope_tables.restype = None
        L.t0r_rope_tables.argtypes = [S, S, P, P, P]
        L.t0r_quantile_head.restype = None
        L.t0r_quantile_head.argtypes = [P, P, S, S]
        L.t0r_interpolate_quantiles.restype = None
        L.t0r_interpolate_quantiles.argtypes = [P, S, P, P, S, P]
        L.t0r_weighted_quantile.restype = None
        L.t0r_weighted_quantile.argtypes = [P, S, P, P, S, P]
        L.t0r_prob_mass.restype = None
        L.t0r_prob_mass.argtypes = [P, S, P]
        L.t0r_scale_input.argtypes = [P, P, P, P, S, S, C.c_int, C.c_float, C.c_int, P, P, P]
        L.t0r_build_time_mask.restype = None
        L.t0r_build_time_mask.argtypes = [P, P, P, S, S, P]
        L.t0r_build_group_mask.restype = None
        L.t0r_build_group_mask.argtypes = [P, S, S, P]
        L.t0r_forward.argtypes = [P, S, S, P, P, P, P, P, P, P]
        L.t0r_forecast.argtypes = [P, P, S, S, S, P]
        L.t0r_forecast_batch_chunked.argtypes = [P, P, S, S, S, S, P]
        L.t0r_forecast_batch_rows_chunked.argtypes = [P, P, P, S, S, S, P]
        L.t0r_forecast_grouped.argtypes = [P, P, P, S, S, S, P]
        L.t0r_forecast_grouped_ar.argtypes = [P, P, P, S, S, S, S, P]
        L.t0r_forecast_rollout.argtypes = [P, P, S, S, P, S, P]
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


class OracleError(RuntimeError):
    def __init__(self, code, what):
        super().__init__(f"{what} failed with oracle status {code}")
        self.code = code


def _check(rc, what):
    if rc != 0:
        raise OracleError(rc, what)


# ---- codec ----
def f32_to_f16_bits(x):
    L = lib()
    return np.array([L.t0r_f32_to_f16(float(v)) for v in np.asarray(x, np.float32).ravel()], np.uint16)


def f16_bits_to_f32(h):
    L = lib()
    return np.array([L.t0r_f16_to_f32(int(v)) for v in np.asarray(h, np.uint16).ravel()], np.float32)


def row_bytes(ty, n):
    return lib().t0r_row_bytes(ty, n)


def quantize(ty, x):
    x = np.ascontiguousarray(x, np.float32).ravel()
    out = np.zeros(row_bytes(ty, x.size), np.uint8)
    _check(lib().t0r_quantize_for(ty, _p(x), x.size, _p(out)), "quantize")
    return out


def dequantize(ty, b, n):
    b = np.ascontiguousarray(b, np.uint8)
    out = np.zeros(n, np.float32)
    _check(lib().t0r_dequantize_for(ty, _p(b), n, _p(out)), "dequantize")
    return out


# ---- ops ----
def linear(x, w, b=None, relu=False):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    m, k = x.shape
    n = w.shape[0]
    y = np.zeros((m, n), np.float32)
    bb = None if b is None else np.ascontiguousarray(b, np.float32)
    lib().t0r_linear(_p(x), _p(w), None if bb is None else _p(bb), _p(y), m, k, n, int(relu))
    return y


def rmsnorm(x, scale, eps=1e-8):
    x = np.ascontiguousarray(x, np.float32)
    s = np.ascontiguousarray(scale, np.float32)
    y = np.zeros_like(x)
    lib().t0r_rmsnorm(_p(x), _p(s), _p(y), x.shape[0], x.shape[1], eps)
    return y


def rope_tables(seq_len, head_dim):
    c = np.zeros((seq_len, head_dim), np.float32)
    s = np.zeros_like(c)
    x = np.zeros_like(c)
    lib().t0r_rope_tables(seq_len, head_dim, _p(c), _p(s), _p(x))
    return c, s, x


def quantile_head(x):
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros_like(x)
    lib().t0r_quantile_head(_p(x), _p(y), x.shape[0], x.shape[1])
    return y


def interpolate_quantiles(query, levels, values):
    q = np.ascontiguousarray(query, np.float32)
    l = np.ascontiguousarray(levels, np.float32)
    v = np.ascontiguousarray(values, np.float32)
    out = np.zeros(q.size, np.float32)
    lib().t0r_interpolate_quantiles(_p(q), q.size, _p(l), _p(v), l.size, _p(out))
    return out


def weighted_quantile(query, weights, samples):
    q = np.ascontiguousarray(query, np.float32)
    w = np.ascontiguousarray(weights, np.float32)
    s = np.ascontiguousarray(samples, np.float32)
    out = np.zeros(q.size, np.float32)
    lib().t0r_weighted_quantile(_p(q), q.size, _p(w), _p(s), s.size, _p(out))
    return out


def prob_mass(levels):
    l = np.ascontiguousarray(levels, np.float32)
    out = np.zeros(l.size, np.float32)
    lib().t0r_prob_mass(_p(l), l.size, _p(out))
    return out


def scale_input(variates, mask, group_ids, variate_type, use_arcsinh=True, eps=0.1, variance_offset=True):
    x = np.ascontiguousarray(variates, np.float32)
    v, t = x.shape
    m = np.ascontiguousarray(mask, np.int8)
    g = np.ascontiguousarray(group_ids, np.int64)
    vt = np.ascontiguousarray(variate_type, np.int64)
    sc, loc, scl = np.zeros_like(x), np.zeros_like(x), np.zeros_like(x)
    _check(lib().t0r_scale_input(_p(x), _p(m), _p(g), _p(vt), v, t, int(use_arcsinh), eps, int(variance_offset),
                                 _p(sc), _p(loc), _p(scl)), "scale_input")
    return sc, loc, scl


def set_threads(n):
    lib().t0r_set_threads(int(n))


# ---- model ----
class Model:
    """GGUF-loaded CPU model (every tensor dequantized to f32, weights.rs:151-163)."""

    def __init__(self, gguf_bytes):
        self._buf = np.frombuffer(bytes(gguf_bytes), np.uint8).copy()
        h = C.c_void_p()
        _check(lib().t0r_model_load_gguf(_p(self._buf), self._buf.size, C.byref(h)), "t0r_model_load_gguf")
        self.h = h
        cfg = Config()
        _check(lib().t0r_model_config(self.h, C.byref(cfg)), "config")
        self.cfg = cfg
        self.n_q = cfg.n_quantiles
        self.patch = cfg.patch_size
        self.levels = np.array(cfg.quantile_levels[: cfg.n_quantiles], np.float32)

    def __del__(self):
        if getattr(self, "h", None):
            lib().t0r_model_free(self.h)
            self.h = None

    def tensor(self, name):
        shape = (C.c_size_t * 4)()
        rank = C.c_int()
        n = lib().t0r_model_tensor(self.h, name.encode(), None, 0, shape, C.byref(rank))
        if n == 0:
            raise KeyError(name)
        out = np.zeros(n, np.float32)
        lib().t0r_model_tensor(self.h, name.encode(), _p(out), n, None, None)
        return out.reshape([shape[i] for i in range(rank.value)])

    def export_gguf(self, quant):
        n = lib().t0r_export_gguf(self.h, quant, None, 0)
        out = np.zeros(n, np.uint8)
        lib().t0r_export_gguf(self.h, quant, _p(out), n)
        return out.tobytes()

    def forward(self, variates, mask, group_ids, variate_type, trace=False):
        x = np.ascontiguousarray(variates, np.float32)
        v, t = x.shape
        p = t // self.patch
        E = self.cfg.embed_dim
        out = np.zeros((v, p, self.patch, self.n_q), np.float32)
        pe = np.zeros((v, p, E), np.float32) if trace else None
        l0 = np.zeros((v, p, E), np.float32) if trace else None
        m = np.ascontiguousarray(mask, np.int8)
        g = np.ascontiguousarray(group_ids, np.int64)
        vt = np.ascontiguousarray(variate_type, np.int64)
        _check(lib().t0r_forward(self.h, v, t, _p(x), _p(m), _p(g), _p(vt), _p(out),
                                 None if pe is None else _p(pe), None if l0 is None else _p(l0)), "t0r_forward")
        return (out, pe, l0) if trace else out

    def forecast(self, ctx, v, t_ctx, horizon):
        c = np.ascontiguousarray(ctx, np.float32)
        out = np.zeros((v, horizon, self.n_q), np.float32)
        _check(lib().t0r_forecast(self.h, _p(c), v, t_ctx, horizon, _p(out)), "t0r_forecast")
        return out

    def forecast_batch_chunked(self, ctx, n_signals, t_ctx, horizon, chunk=16):
        c = np.ascontiguousarray(ctx, np.float32)
        out = np.zeros((n_signals, horizon, self.n_q), np.float32)
        _check(lib().t0r_forecast_batch_chunked(self.h, _p(c), n_signals, t_ctx, horizon, chunk, _p(out)),
               "t0r_forecast_batch_chunked")
        return out

    def forecast_batch_rows_chunked(self, ctx, lengths, horizon, chunk=16):
        c = np.ascontiguousarray(ctx, np.float32)
        ln = np.ascontiguousarray(lengths, np.uint64)
        out = np.zeros((ln.size, horizon, self.n_q), np.float32)
        _check(lib().t0r_forecast_batch_rows_chunked(self.h, _p(c), _p(ln), ln.size, horizon, chunk, _p(out)),
               "t0r_forecast_batch_rows_chunked")
        return out

    def forecast_grouped(self, ctx, row_group, t_ctx, horizon):
        c = np.ascontiguousarray(ctx, np.float32)
        g = np.ascontiguousarray(row_group, np.int64)
        out = np.zeros((g.size, horizon, self.n_q), np.float32)
        _check(lib().t0r_forecast_grouped(self.h, _p(c), _p(g), g.size, t_ctx, horizon, _p(out)),
               "t0r_forecast_grouped")
        return out

    def forecast_grouped_ar(self, ctx, row_group, t_ctx, horizon, steps):
        c = np.ascontiguousarray(ctx, np.float32)
        g = np.ascontiguousarray(row_group, np.int64)
        out = np.zeros((g.size, steps * horizon, self.n_q), np.float32)
        _check(lib().t0r_forecast_grouped_ar(self.h, _p(c), _p(g), g.size, t_ctx, horizon, steps, _p(out)),
               "t0r_forecast_grouped_ar")
        return out

    def forecast_rollout(self, ctx, t_ctx, prediction_length, query):
        c = np.ascontiguousarray(ctx, np.float32)
        q = np.ascontiguousarray(query, np.float32)
        out = np.zeros((prediction_length, q.size), np.float32)
        _check(lib().t0r_forecast_rollout(self.h, _p(c), t_ctx, prediction_length, _p(q), q.size, _p(out)),
               "t0r_forecast_rollout")
        return out
