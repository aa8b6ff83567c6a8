"""Q8_0/Q4_0 block codec and f16 conversions (CPU).

Three restatements must agree bit for bit: the oracle (C), an independent
numpy restatement (oracle/quant_np.py) and the product's host codec
(t0h_quantize).  They are also pinned by the reference's own known-answer tests
(crates/t0-core/src/gguf.rs:411-433, crates/t0-fast/src/quant.rs:161-185) and by
closed-form special cases (ties, zero blocks, subnormal scales)."""
import numpy as np
import pytest

import quant_np

Q8, Q4 = 8, 2


def sample(n):  # gguf.rs:411-413
    return (np.sin(np.arange(n, dtype=np.float32) * np.float32(0.37)) * np.float32(3.0)).astype(np.float32)


def edge(rng, nblocks=2048):
    x = (rng.standard_normal(32 * nblocks) * rng.choice([0.02, 1.0, 1e-6, 3e-8, 500.0, 7e4], 32 * nblocks)).astype(np.float32)
    x[:32] = 0.0
    x[32:64] = 2.5
    x[64:96] = -np.arange(32, dtype=np.float32)
    x[96:128] = 3e-7
    x[128:160] = np.linspace(-1, 1, 32)
    x[160:192] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.5, 126.5, -127.0] * 4  # ties at d = 1
    x[192:224] = [-8.0, 4.0, -4.0, 0.5, 7.0, -7.5, 3.5, 1.0] * 4         # Q4_0 ties with d = 1
    return x


@pytest.mark.parametrize("qtype", [Q8, Q4])
def test_three_restatements_agree(oracle, t0hip, rng, qtype):
    for trial in range(4):
        x = edge(rng)
        a = oracle.quantize(qtype, x)
        b = (quant_np.quantize_q8_0 if qtype == Q8 else quant_np.quantize_q4_0)(x)
        c = t0hip.quantize(qtype, x)
        assert a.tobytes() == b.tobytes()
        assert a.tobytes() == c.tobytes()
        da = oracle.dequantize(qtype, a, x.size)
        db = (quant_np.dequantize_q8_0 if qtype == Q8 else quant_np.dequantize_q4_0)(a, x.size)
        assert da.view(np.uint32).tobytes() == db.view(np.uint32).tobytes()


def test_reference_round_trip_bounds(oracle, t0hip):
    """gguf.rs:415-433: sample(320) round trip error < 0.03 (Q8_0) and < 0.4 (Q4_0)."""
    x = sample(320)
    for quant in (oracle.quantize, t0hip.quantize):
        y8 = oracle.dequantize(Q8, quant(Q8, x), 320)
        y4 = oracle.dequantize(Q4, quant(Q4, x), 320)
        assert np.max(np.abs(x - y8)) < 0.03
        assert np.max(np.abs(x - y4)) < 0.4


def test_reference_repack_case_bit_exact(oracle):
    """quant.rs:161-185 input ((i-32)*0.37, n=64): the dequantized value of every
    element equals f32(d) * i8 with d read back from the block (bit-exact)."""
    n = 64
    x = ((np.arange(n, dtype=np.float32) - np.float32(32.0)) * np.float32(0.37)).astype(np.float32)
    b = oracle.quantize(Q8, x).reshape(2, 34)
    d = b[:, :2].copy().view(np.float16).astype(np.float32)
    q = b[:, 2:].view(np.int8).astype(np.float32)
    assert (oracle.dequantize(Q8, b.ravel(), n).reshape(2, 32) == d * q).all()


def test_closed_form_special_cases(oracle):
    z = np.zeros(32, np.float32)
    b8 = oracle.quantize(Q8, z)
    assert b8[:2].tobytes() == b"\x00\x00" and not b8[2:].any()
    b4 = oracle.quantize(Q4, z)
    assert b4[:2].view(np.uint16)[0] == 0x8000  # d = 0 / -8 = -0.0
    assert (b4[2:] == 0x88).all()               # q = floor(0 + 8.5) = 8
    y4 = oracle.dequantize(Q4, b4, 32)
    assert (y4.view(np.uint32) == 0x80000000).all()  # -0.0 * 0.0 = -0.0
    # Q8_0 ties round half away from zero (f32::round), not to even
    x = np.zeros(32, np.float32)
    x[:6] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.5]
    q = oracle.quantize(Q8, x)[2:8].view(np.int8)
    assert list(q) == [127, 3, -3, 1, -1, 2]
    # Q4_0: d = max/-8 with max the signed value of largest magnitude (first wins)
    x = np.zeros(32, np.float32)
    x[3], x[5] = -8.0, 8.0
    b = oracle.quantize(Q4, x)
    assert b[:2].view(np.float16)[0] == np.float16(1.0)
    y = oracle.dequantize(Q4, b, 32)
    assert y[3] == -8.0 and y[5] == 7.0  # +8 clamps to nibble 15 -> 7 * d


def test_subnormal_scale_survives(oracle):
    x = np.full(32, 3e-4, np.float32)  # d = amax/127 = 2.4e-6 is an f16 subnormal
    b = oracle.quantize(Q8, x)
    d = b[:2].view(np.float16)[0]
    assert 0 < float(d) < 6.1e-5  # f16 subnormal
    y = oracle.dequantize(Q8, b, 32)
    assert (y == np.float32(d) * np.float32(127)).all()


def test_f16_exhaustive_and_rne(oracle, t0hip, rng):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = oracle.f16_bits_to_f32(h)
    same = (ref.view(np.uint32) == got.view(np.uint32)) | (np.isnan(ref) & np.isnan(got))
    assert same.all()
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 20000),
                        np.array([65504, 65519.99, 65520, 6.1035156e-05, 5.96e-08, 2.98e-08, 2.99e-08, -0.0,
                                  np.inf, -np.inf], np.float32)]).astype(np.float32)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert (oracle.f32_to_f16_bits(x) == want).all()
    assert (t0hip.quantize(1, x).view(np.uint16) == want).all()


def test_row_bytes(oracle, t0hip):
    for ty, per in ((0, 4), (1, 2)):
        assert oracle.row_bytes(ty, 96) == 96 * per == t0hip.row_bytes(ty, 96)
    assert oracle.row_bytes(Q8, 768) == 24 * 34 == t0hip.row_bytes(Q8, 768)
    assert oracle.row_bytes(Q4, 2048) == 64 * 18 == t0hip.row_bytes(Q4, 2048)
    assert oracle.row_bytes(Q8, 33) == 0 == t0hip.row_bytes(Q8, 33)
    with pytest.raises(t0hip.T0HipError) as e:
        t0hip.quantize(Q8, np.zeros(33, np.float32))
    assert e.value.status == "SHAPE"
