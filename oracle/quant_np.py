"""Independent numpy restatement of the GGUF Q8_0/Q4_0 block codec.

TEST INFRASTRUCTURE ONLY.  A second restatement of
crates/t0-core/src/gguf.rs:100-174 (quantize_q8_0, dequantize_q8_0,
quantize_q4_0, dequantize_q4_0), written with numpy vector ops instead of C
loops so that a transcription slip in either restatement shows up as a
bit-level disagreement between the two.

numpy details that matter for bit-exactness:
  * all arithmetic stays float32 (numpy would silently promote Python floats);
  * np.round is half-to-even, the reference's f32::round is half-away-from-zero,
    so rounding is done as trunc(x + copysign(0.5, x)) evaluated in float64
    (exact for float32 inputs) rather than np.round;
  * float32 -> float16 via astype(np.float16) is IEEE round-to-nearest-even,
    the same as `half::f16::from_f32`.
"""
import numpy as np

QK = 32


def _round_half_away(x32):
    """f32::round (ties away from zero), exact for float32 inputs."""
    x = x32.astype(np.float64)
    r = np.trunc(x + np.copysign(0.5, x))
    # x + 0.5 is exact in float64 for |x| < 2^52; ties resolve away from zero.
    return r.astype(np.float32)


def quantize_q8_0(x):
    """gguf.rs:100-114."""
    x = np.asarray(x, np.float32).reshape(-1, QK)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        amax = np.fmax.reduce(np.abs(x), axis=1, initial=np.float32(0.0)).astype(np.float32)
        d = (amax / np.float32(127.0)).astype(np.float32)
        id_ = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, np.float32(1.0)), np.float32(0.0)).astype(np.float32)
        prod = (x * id_[:, None]).astype(np.float32)
        r = _round_half_away(prod)
        r = np.where(np.isnan(r), np.float32(0.0), np.clip(r, -128.0, 127.0)).astype(np.float32)
    q = r.astype(np.int8)
    dh = d.astype(np.float16).view(np.uint16)
    out = np.zeros((x.shape[0], 2 + QK), np.uint8)
    out[:, 0] = (dh & 0xFF).astype(np.uint8)
    out[:, 1] = (dh >> 8).astype(np.uint8)
    out[:, 2:] = q.view(np.uint8)
    return out.ravel()


def dequantize_q8_0(b, n):
    """gguf.rs:116-126."""
    b = np.asarray(b, np.uint8).reshape(-1, 2 + QK)[: n // QK]
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(-1, 1)
    q = b[:, 2:].view(np.int8).astype(np.float32)
    return (d * q).astype(np.float32).ravel()


def quantize_q4_0(x):
    """gguf.rs:133-157: d = max/-8 with max the first value of largest |x|."""
    x = np.asarray(x, np.float32).reshape(-1, QK)
    ax = np.abs(x)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        # strict `>` scan keeps the FIRST index of the maximum (np.argmax does too);
        # NaN never wins a `>` comparison, so mask NaNs out first.
        axn = np.where(np.isnan(ax), np.float32(-1.0), ax)
        idx = np.argmax(axn, axis=1)
        mx = x[np.arange(x.shape[0]), idx]
        mx = np.where(axn[np.arange(x.shape[0]), idx] > 0, mx, np.float32(0.0)).astype(np.float32)
        d = (mx / np.float32(-8.0)).astype(np.float32)
        id_ = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, np.float32(1.0)), np.float32(0.0)).astype(np.float32)
        y = (x * id_[:, None]).astype(np.float32)
        f = np.floor((y + np.float32(8.5)).astype(np.float32))
        f = np.where(np.isnan(f), 0.0, f)
        qi = np.clip(f, 0, 15).astype(np.uint8)
    dh = d.astype(np.float16).view(np.uint16)
    out = np.zeros((x.shape[0], 2 + QK // 2), np.uint8)
    out[:, 0] = (dh & 0xFF).astype(np.uint8)
    out[:, 1] = (dh >> 8).astype(np.uint8)
    out[:, 2:] = qi[:, : QK // 2] | (qi[:, QK // 2:] << 4)
    return out.ravel()


def dequantize_q4_0(b, n):
    """gguf.rs:159-174."""
    b = np.asarray(b, np.uint8).reshape(-1, 2 + QK // 2)[: n // QK]
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(-1, 1)
    lo = (b[:, 2:] & 0x0F).astype(np.float32) - np.float32(8.0)
    hi = (b[:, 2:] >> 4).astype(np.float32) - np.float32(8.0)
    return np.concatenate([(d * lo).astype(np.float32), (d * hi).astype(np.float32)], axis=1).ravel()
