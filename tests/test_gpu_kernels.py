"""Kernel-level parity on the GPU: dequantization (bit-exact) and the quantized GEMM.

Reference contracts: dequantize_for (crates/t0-core/src/gguf.rs:213-226) and
linear() (crates/t0-fast/src/model.rs:406-504 ≡ ops.rs:40-42).  The checker is
the oracle's dequantization (itself pinned bit-for-bit against an independent
numpy restatement) followed by a float64 matmul."""
import numpy as np
import pytest

from util import rel_err

pytestmark = pytest.mark.gpu


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def edge_values(rng, n):
    x = (rng.standard_normal(n) * rng.choice([0.02, 1.0, 1e-6, 500.0], n)).astype(np.float32)
    x[:32] = 0.0                      # all-zero block: Q4_0 stores d = -0.0
    x[32:64] = 2.5                    # ties
    x[64:96] = -np.arange(32)         # exact amax
    x[96:128] = 3e-7                  # subnormal f16 scale
    x[128:160] = np.linspace(-1, 1, 32)
    return x


@pytest.mark.parametrize("qtype", [8, 2, 1, 0])
def test_dequant_bit_exact(torch_cuda, t0hip, oracle, rng, qtype):
    n = 32 * 4099
    x = edge_values(rng, n)
    blocks = oracle.quantize(qtype, x)
    want = oracle.dequantize(qtype, blocks, n)
    d_b = dev(torch_cuda, blocks)
    d_o = torch_cuda.empty(n, dtype=torch_cuda.float32, device="cuda")
    t0hip.dequant_dev(qtype, d_b.data_ptr(), n, d_o.data_ptr(), torch_cuda.cuda.current_stream().cuda_stream)
    torch_cuda.cuda.synchronize()
    got = d_o.cpu().numpy()
    assert got.view(np.uint32).tobytes() == want.view(np.uint32).tobytes()


def run_gemm(torch, t0hip, wtype, W_bytes, x, bias, n, act=0):
    m, k = x.shape
    d_w = dev(torch, W_bytes)
    d_x = dev(torch, x)
    d_b = dev(torch, bias) if bias is not None else None
    d_y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    t0hip.gemm_q_dev(wtype, d_w.data_ptr(), d_x.data_ptr(), d_b.data_ptr() if d_b is not None else 0,
                     d_y.data_ptr(), m, n, k, act, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return d_y.cpu().numpy()


@pytest.mark.parametrize("qtype", [8, 2, 1])
@pytest.mark.parametrize("m", [1, 40])
def test_reference_kernel_case(torch_cuda, t0hip, oracle, qtype, m):
    """crates/t0-fast/src/model.rs:825-872 verbatim inputs: k=512, n=4, bias 0.
    The reference gates its f32 kernels at 1e-5 abs; the small-M path here is exact
    f32 and keeps that gate; the MFMA path (f16 operands, f32 accumulation) is held
    to 1e-2 relative, the GEMM tolerance of this engine."""
    k, n = 512, 4
    i = np.arange(n * k, dtype=np.int64)
    w = ((((i * 2654435761) % 1000).astype(np.float32) / 1000.0 - 0.5) * 0.6).astype(np.float32)
    j = np.arange(m * k, dtype=np.int64)
    x = ((((j * 40503) % 1000).astype(np.float32) / 1000.0 - 0.5) * 0.4).astype(np.float32).reshape(m, k)
    blocks = oracle.quantize(qtype, w)
    deq = oracle.dequantize(qtype, blocks, n * k).reshape(n, k)
    want = oracle.linear(x, deq, np.zeros(n, np.float32))
    got = run_gemm(torch_cuda, t0hip, qtype, blocks, x, np.zeros(n, np.float32), n)
    if m == 1:
        assert np.max(np.abs(got - want)) < 1e-5
    else:
        assert rel_err(got, want.astype(np.float64)) < 1e-2


SHAPES = [(768, 2304), (768, 768), (768, 2048), (2048, 768), (768, 4096)]


@pytest.mark.parametrize("qtype", [8, 2])
@pytest.mark.parametrize("k,n", SHAPES)
@pytest.mark.parametrize("m", [1, 16, 64, 512])
def test_gemm_sweep(torch_cuda, t0hip, oracle, rng, qtype, k, n, m):
    """BASELINE config 2 sweep (M up to 512 here; 8192 below): W ~ N(0, 0.02), x ~ N(0, 1)."""
    W = (0.02 * rng.standard_normal((n, k))).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    b = (0.02 * rng.standard_normal(n)).astype(np.float32)
    blocks = oracle.quantize(qtype, W)
    deq = oracle.dequantize(qtype, blocks, n * k).reshape(n, k).astype(np.float64)
    want = x.astype(np.float64) @ deq.T + b
    got = run_gemm(torch_cuda, t0hip, qtype, blocks, x, b, n)
    e = rel_err(got, want)
    assert e < 1e-2, e
    if m <= 16:  # exact-f32 small-M path: ulp-level
        assert e < 1e-5, e


@pytest.mark.parametrize("qtype", [8, 2])
def test_gemm_config1(torch_cuda, t0hip, oracle, rng, qtype):
    """M=512, K=768, N=2304, every row."""
    k, n, m = 768, 2304, 512
    W = (0.02 * rng.standard_normal((n, k))).astype(np.float32)
    blocks = oracle.quantize(qtype, W)
    deq = oracle.dequantize(qtype, blocks, n * k).reshape(n, k).astype(np.float64)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got = run_gemm(torch_cuda, t0hip, qtype, blocks, x, None, n)
    assert rel_err(got, x.astype(np.float64) @ deq.T) < 1e-2


@pytest.mark.parametrize("qtype", [8, 2])
@pytest.mark.parametrize("k,n", SHAPES)
def test_gemm_m8192(torch_cuda, t0hip, oracle, rng, qtype, k, n):
    """The M=8192 end of the config-2 sweep at every (K, N) the bench reports (the f32-activation
    256x256 register-operand kernel, K = 2048 included): 512 sampled rows plus the first and last
    256-row tile against float64, bias on."""
    m = 8192
    W = (0.02 * rng.standard_normal((n, k))).astype(np.float32)
    b = (0.02 * rng.standard_normal(n)).astype(np.float32)
    blocks = oracle.quantize(qtype, W)
    deq = oracle.dequantize(qtype, blocks, n * k).reshape(n, k).astype(np.float64)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got = run_gemm(torch_cuda, t0hip, qtype, blocks, x, b, n)
    rows = np.unique(np.concatenate([np.arange(256), np.arange(m - 256, m), rng.choice(m, 512, replace=False)]))
    want = x[rows].astype(np.float64) @ deq.T + b
    assert np.isfinite(got).all()
    assert rel_err(got[rows], want) < 1e-2


@pytest.mark.parametrize("m", [1, 3, 40, 200])
def test_gemm_ragged_and_relu(torch_cuda, t0hip, oracle, rng, m):
    """Edge shapes: M not a tile multiple, N not a tile multiple, K % 64 == 32, ReLU."""
    for qtype, k, n in [(8, 96, 200), (2, 160, 33), (1, 96, 130), (8, 64, 17)]:
        W = rng.standard_normal((n, k)).astype(np.float32)
        x = rng.standard_normal((m, k)).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        blocks = oracle.quantize(qtype, W)
        deq = oracle.dequantize(qtype, blocks, n * k).reshape(n, k).astype(np.float64)
        want = np.maximum(x.astype(np.float64) @ deq.T + b, 0.0)
        got = run_gemm(torch_cuda, t0hip, qtype, blocks, x, b, n, act=1)
        assert rel_err(got, want) < 1e-2, (qtype, k, n, m)


def test_gemm_linearity_and_zero_weights(torch_cuda, t0hip, oracle, rng):
    """Invariants: zero weights give the bias exactly; y(2x) = 2 y(x) exactly (power-of-two scale)."""
    k, n, m = 768, 256, 300
    z = oracle.quantize(8, np.zeros((n, k), np.float32))
    b = rng.standard_normal(n).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got = run_gemm(torch_cuda, t0hip, 8, z, x, b, n)
    assert np.array_equal(got, np.broadcast_to(b, (m, n)))
    W = oracle.quantize(2, (0.02 * rng.standard_normal((n, k))).astype(np.float32))
    y1 = run_gemm(torch_cuda, t0hip, 2, W, x, None, n)
    y2 = run_gemm(torch_cuda, t0hip, 2, W, 2 * x, None, n)
    assert np.array_equal(2 * y1, y2)


# The forward's GEMM paths (f16 activations, fused epilogues) at model shapes,
# M ragged against every tile height: (k, n) per epilogue as in the layer
# (wO store, QKV f16, w2 residual, w0 SwiGLU with n hidden units).
FWD_SHAPES = {0: (768, 768), 1: (768, 2304), 2: (2048, 768), 3: (768, 2048)}


def check_forward_gemm(torch, t0hip, oracle, rng, qtype, tile, epi, m, k, n, sample=True):
    """Run t0h_gemm_f16 on random data and compare with float64 over the
    oracle's dequantized weights: 1e-2 relative."""
    wrows = 2 * n if epi == 3 else n
    W = (0.02 * rng.standard_normal((wrows, k))).astype(np.float32)
    b = (0.02 * rng.standard_normal(wrows)).astype(np.float32)
    x16 = rng.standard_normal((m, k)).astype(np.float16)
    blocks = oracle.quantize(qtype, W)
    deq = oracle.dequantize(qtype, blocks, wrows * k).reshape(wrows, k).astype(np.float64)
    d_w, d_x, d_b = dev(torch, blocks), dev(torch, x16), dev(torch, b)
    out_dtype = torch.float16 if epi in (1, 3) else torch.float32
    y0 = rng.standard_normal((m, n)).astype(np.float32)
    d_y = dev(torch, y0) if epi == 2 else torch.empty((m, n), dtype=out_dtype, device="cuda")
    t0hip.gemm_f16_dev(qtype, d_w.data_ptr(), d_x.data_ptr(), d_b.data_ptr(), d_y.data_ptr(), m, n, k, epi, tile,
                       torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    got = d_y.float().cpu().numpy()
    if sample:
        rows = np.sort(np.concatenate([rng.choice(m - 200, 312, replace=False), np.arange(m - 200, m)]))
    else:
        rows = np.arange(m)
    h = x16[rows].astype(np.float64) @ deq.T + b
    if epi == 3:
        g, u = h[:, :n], h[:, n:]
        want = g / (1.0 + np.exp(-g)) * u
    elif epi == 2:
        want = y0[rows] + h
    else:
        want = h
    e = rel_err(got[rows], want)
    assert e < 1e-2, (tile, epi, m, k, n, e)


@pytest.mark.parametrize("qtype", [8, 2])
@pytest.mark.parametrize("tile", [1, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("epi", [0, 1, 2, 3])
def test_forward_gemm_paths(torch_cuda, t0hip, oracle, rng, qtype, tile, epi):
    """linear() (model.rs:406-504) as the forward runs it: f16 x, f32 accumulation,
    epilogues bias / f16 store / residual add / SwiGLU (ops.rs:49-62); 1e-2 relative
    on a 512-row sample of M = 4192 rows (ragged against every tile height)."""
    k, n = FWD_SHAPES[epi]
    check_forward_gemm(torch_cuda, t0hip, oracle, rng, qtype, tile, epi, 4192, k, n)


@pytest.mark.parametrize("qtype", [8, 2])
@pytest.mark.parametrize("tile", [5, 6, 7, 8])
@pytest.mark.parametrize("epi", [0, 1, 2, 3])
@pytest.mark.parametrize("m,k,n", [(300, 192, 328), (257, 64, 330), (40, 128, 72)])
def test_register_b_gemm_edges(torch_cuda, t0hip, oracle, rng, qtype, tile, epi, m, k, n):
    """The register-operand kernels (tiles 5-8: 256, 192 and 128 rows) on partial tiles: M and N
    ragged (weight rows past N clamp to row 0), an odd number of 64-wide K steps
    (the step after the paired loop), one step, and N % 4 != 0 (scalar stores;
    SwiGLU needs N % 8 == 0 and takes n rounded down to 8)."""
    if epi == 3:
        n -= n % 8
    check_forward_gemm(torch_cuda, t0hip, oracle, rng, qtype, tile, epi, m, k, n, sample=False)


@pytest.mark.parametrize("qtype", [8, 2])
@pytest.mark.parametrize("m,k,n", [(1, 2560, 200), (4, 4096, 72), (16, 768, 40), (7, 2048, 17), (16, 1088, 24)])
def test_small_m_kernel(torch_cuda, t0hip, oracle, rng, qtype, m, k, n):
    """The small-M kernels (M = 1: 16 lanes per weight row; 2..16: the f32 MFMA) through t0h_gemm_q:
    exact f32 dequantization and accumulation, so the 1e-5 gate of the
    reference's f32 kernels holds; a partial last K tile (K = 2560, 1088), N not
    a multiple of the 16 weight rows of a workgroup."""
    W = (0.02 * rng.standard_normal((n, k))).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    b = (0.02 * rng.standard_normal(n)).astype(np.float32)
    blocks = oracle.quantize(qtype, W)
    deq = oracle.dequantize(qtype, blocks, n * k).reshape(n, k).astype(np.float64)
    want = x.astype(np.float64) @ deq.T + b
    got = run_gemm(torch_cuda, t0hip, qtype, blocks, x, b, n)
    assert rel_err(got, want) < 1e-5, (m, k, n)
    got = run_gemm(torch_cuda, t0hip, qtype, blocks, x, b, n, act=1)
    assert rel_err(got, np.maximum(want, 0.0)) < 1e-5, (m, k, n)


@pytest.mark.parametrize("qtype", [8, 2])
@pytest.mark.parametrize("k,n", [(4096, 200), (4096, 4104), (8192, 72), (8192, 1031)])
def test_gemv_long_rows(torch_cuda, t0hip, oracle, rng, qtype, k, n):
    """M = 1 at K = 4096 and 8192 through t0h_gemm_q (the kernel that holds a lane's activation
    spans in registers across its weight rows): exact f32, so the 1e-5 gate of the reference's
    f32 kernels holds, with and without ReLU; N not a multiple of a workgroup's rows."""
    W = (0.02 * rng.standard_normal((n, k))).astype(np.float32)
    x = rng.standard_normal((1, k)).astype(np.float32)
    b = (0.02 * rng.standard_normal(n)).astype(np.float32)
    blocks = oracle.quantize(qtype, W)
    deq = oracle.dequantize(qtype, blocks, n * k).reshape(n, k).astype(np.float64)
    want = x.astype(np.float64) @ deq.T + b
    assert rel_err(run_gemm(torch_cuda, t0hip, qtype, blocks, x, b, n), want) < 1e-5, (k, n)
    assert rel_err(run_gemm(torch_cuda, t0hip, qtype, blocks, x, b, n, act=1), np.maximum(want, 0.0)) < 1e-5


@pytest.mark.parametrize("qtype", [8, 2, 1])
@pytest.mark.parametrize("m,k,n", [(2, 96, 40), (3, 160, 33), (5, 4096, 300), (16, 32, 17), (12, 1056, 24),
                                   (16, 4096, 2048)])
def test_small_m_f32_mfma_kernel(torch_cuda, t0hip, oracle, rng, qtype, m, k, n):
    """The 2..16-row kernel on the f32 MFMA through t0h_gemm_q: every weight type, K % 64 == 32, one
    block (K = 32: seven of the eight waves get none), K split over the waves with a partial last
    batch, ragged N; exact f32 products, so the reference's 1e-5 gate holds, with and without ReLU."""
    W = (0.02 * rng.standard_normal((n, k))).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    b = (0.02 * rng.standard_normal(n)).astype(np.float32)
    blocks = oracle.quantize(qtype, W)
    deq = oracle.dequantize(qtype, blocks, n * k).reshape(n, k).astype(np.float64)
    want = x.astype(np.float64) @ deq.T + b
    assert rel_err(run_gemm(torch_cuda, t0hip, qtype, blocks, x, b, n), want) < 1e-5, (m, k, n)
    assert rel_err(run_gemm(torch_cuda, t0hip, qtype, blocks, x, b, n, act=1), np.maximum(want, 0.0)) < 1e-5


@pytest.mark.parametrize("qtype", [8, 2, 1])
@pytest.mark.parametrize("m,k,n", [(16, 256, 16400), (5, 512, 8200), (2, 96, 16384)])
def test_small_m_wide_matrix(torch_cuda, t0hip, oracle, rng, qtype, m, k, n):
    """The f32-MFMA small-M kernel with two (N >= 8192) and four (N >= 16384) groups of 16 columns
    a workgroup: exact f32 products, the 1e-5 gate, with and without ReLU; N ragged against 64."""
    W = (0.02 * rng.standard_normal((n, k))).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    b = (0.02 * rng.standard_normal(n)).astype(np.float32)
    blocks = oracle.quantize(qtype, W)
    deq = oracle.dequantize(qtype, blocks, n * k).reshape(n, k).astype(np.float64)
    want = x.astype(np.float64) @ deq.T + b
    assert rel_err(run_gemm(torch_cuda, t0hip, qtype, blocks, x, b, n), want) < 1e-5, (m, k, n)
    assert rel_err(run_gemm(torch_cuda, t0hip, qtype, blocks, x, b, n, act=1), np.maximum(want, 0.0)) < 1e-5


@pytest.mark.parametrize("qtype", [8, 2, 1])
@pytest.mark.parametrize("epi", [0, 1, 2, 3])
@pytest.mark.parametrize("m,k,n", [(1, 768, 136), (1, 4096, 136), (1, 8192, 40), (9, 2048, 72), (16, 768, 40),
                                   (2, 96, 24), (7, 256, 8200), (16, 256, 16400)])
def test_small_m_forward_epilogues(torch_cuda, t0hip, oracle, rng, qtype, epi, m, k, n):
    """The forward's GEMMs at M <= 16 (a single series, the decoder's forecast rows): f16
    activations, epilogues bias / f16 store / residual add / SwiGLU on the small-M kernels
    (quantized and f16 weights)."""
    check_forward_gemm(torch_cuda, t0hip, oracle, rng, qtype, 0, epi, m, k, n, sample=False)


@pytest.mark.parametrize("qtype", [8, 2])
@pytest.mark.parametrize("epi", [0, 1, 2, 3])
@pytest.mark.parametrize("m,k,n", [(17, 768, 136), (66, 2048, 72), (300, 64, 40), (260, 2048, 200), (1000, 4096, 48)])
def test_medium_m_forward_epilogues(torch_cuda, t0hip, oracle, rng, qtype, epi, m, k, n):
    """The medium-M kernel (16 < M < 1024, K split over the waves of a workgroup):
    f16 activations and every forward epilogue; one 64-wide K step (fewer steps
    than 32-row slices), four and two 32-column groups per workgroup (M >= 256),
    the 8-wave limit at K = 4096, ragged M and N."""
    check_forward_gemm(torch_cuda, t0hip, oracle, rng, qtype, 0, epi, m, k, n, sample=False)


@pytest.mark.parametrize("epi", [0, 1, 2, 3])
@pytest.mark.parametrize("m,k,n", [(66, 96, 768), (17, 32, 40), (300, 160, 72), (66, 768, 768), (200, 2048, 40),
                                   (1000, 96, 520)])
def test_medium_m_f16_weights(torch_cuda, t0hip, oracle, rng, epi, m, k, n):
    """F16 weights on the medium-M kernel (the patch encoder and decoder at one series: K = 96 and
    768): K % 64 == 32 (the upper lane half of the last 64-wide step is past K and contributes
    zeros), a single 32-wide step, up to four steps per wave, ragged M and N."""
    check_forward_gemm(torch_cuda, t0hip, oracle, rng, 1, 0, epi, m, k, n, sample=False)


@pytest.mark.parametrize("qtype", [8, 2])
@pytest.mark.parametrize("epi", [0, 1, 2, 3])
@pytest.mark.parametrize("m,k,n", [(1023, 768, 96), (1024, 768, 96), (512, 768, 2304), (513, 768, 2304),
                                   (600, 2048, 2000)])
def test_forward_dispatch_boundaries(torch_cuda, t0hip, oracle, rng, qtype, epi, m, k, n):
    """The automatic kernel choice (tile 0) on both sides of each boundary with
    every forward epilogue: the medium-M kernel up to M = 1023 and up to 512 x 2304
    outputs, the register-operand kernel from M = 1024, the LDS-staged kernel for
    medium M past 512 x 2304 outputs (513 x 2304, 600 x 2000)."""
    check_forward_gemm(torch_cuda, t0hip, oracle, rng, qtype, 0, epi, m, k, n, sample=False)


@pytest.mark.parametrize("qtype", [8, 2])
@pytest.mark.parametrize("m,k,n", [(1100, 192, 200), (1024, 768, 256), (2049, 64, 37)])
def test_f32_activations_large_m(torch_cuda, t0hip, oracle, rng, qtype, m, k, n):
    """t0h_gemm_q at M >= 1024 (f32 activations rounded to f16 while the 256x256
    register-operand kernel stages them): ragged M and N, an odd number of K
    steps, one step, bias and ReLU; 1e-2 relative."""
    W = (0.02 * rng.standard_normal((n, k))).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    b = (0.02 * rng.standard_normal(n)).astype(np.float32)
    blocks = oracle.quantize(qtype, W)
    deq = oracle.dequantize(qtype, blocks, n * k).reshape(n, k).astype(np.float64)
    want = x.astype(np.float64) @ deq.T + b
    assert rel_err(run_gemm(torch_cuda, t0hip, qtype, blocks, x, b, n), want) < 1e-2
    assert rel_err(run_gemm(torch_cuda, t0hip, qtype, blocks, x, b, n, act=1), np.maximum(want, 0.0)) < 1e-2
