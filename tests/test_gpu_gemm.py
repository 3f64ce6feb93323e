"""GPU: the int4 GEMM for prompts (dip_int4_gemm) against the fp64 oracle
(exact q*s weights) at the fp32-accumulation bars the GEMV kernels meet, and
against the reference's route for prompts, dequantize + F.linear (bf16
weights, library GEMM), within the reference's max|err|/max|ref| < 1e-2.
Shapes cover token counts that are not multiples of 16, output counts that
are not multiples of 64, each of the kernel's token tilings (<= 16, <= 32,
more) and the Qwen3 widths."""
import numpy as np
import pytest
import torch

import dip_oracle as O
from gpu_util import assert_fp32_close, dev, dev_bf16, gemv_abs_terms, host_bf16, random_bf16, \
    random_int4, rel_err

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def K():
    import _dip_hip
    return _dip_hip


@pytest.mark.parametrize("m,n,k", [(2, 256, 128), (7, 1040, 5120), (16, 4096, 4096),
                                   (17, 2048, 2560), (33, 8192, 5120), (64, 5120, 8192),
                                   (100, 1088, 1024)])
def test_int4_gemm_matches_oracle(K, m, n, k):
    print(f"int4_gemm m={m} n={n} k={k}", flush=True)
    rng = np.random.default_rng(m * 31 + n)
    qw, sc = random_int4(rng, n, k)
    xs = [random_bf16(rng, k) for _ in range(m)]
    x = dev_bf16(np.stack(xs))
    out = K.int4_gemm(dev(qw), dev_bf16(sc), x)
    assert out.shape == (m, n)
    got = host_bf16(out)
    rows = [0, 1, m // 2, m - 1]
    for t in sorted(set(rows)):
        ref = O.gemv_f64(qw, sc, xs[t])
        assert rel_err(got[t], ref) < 1e-2
        assert_fp32_close(got[t], ref, gemv_abs_terms(qw, sc, xs[t]))


@pytest.mark.parametrize("m,n,k", [(5, 25600, 5120), (32, 25600, 5120), (300, 1024, 5120)])
def test_int4_gemm_matches_dequant_linear(K, m, n, k):
    """The reference's prompt route: bf16(q*s) weights and F.linear."""
    from qlinear import dequantize
    print(f"int4_gemm vs dequant+linear m={m} n={n} k={k}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(m + n)
    from quantize import quantize_tensor_int4_groupwise
    qw, sc = quantize_tensor_int4_groupwise(torch.randn(n, k, device="cuda", generator=g) * 0.02)
    x = torch.randn(m, k, device="cuda", generator=g).to(torch.bfloat16)
    got = K.int4_gemm(qw, sc, x).float()
    ref = torch.nn.functional.linear(x, dequantize(qw, sc)).float()
    assert float((got - ref).abs().max() / ref.abs().max()) < 1e-2


def test_int4_gemm_zero_tokens_and_errors(K):
    qw = torch.zeros(64, 64, dtype=torch.int8, device="cuda")
    sc = torch.ones(64, 1, dtype=torch.bfloat16, device="cuda")
    out = K.int4_gemm(qw, sc, torch.zeros(0, 128, dtype=torch.bfloat16, device="cuda"))
    assert out.shape == (0, 64)
    with pytest.raises(RuntimeError):
        K.int4_gemm(qw, sc, torch.zeros(3, 64, dtype=torch.bfloat16, device="cuda"))


def _dequant_f64(qw, sc):
    """bf16(q*s) of the reference's dequantize, as float64."""
    return O.bf16_to_f32(O.dequantize(qw, sc)).astype(np.float64)


@pytest.mark.parametrize("m,k,n", [(1, 512, 128), (2, 3072, 2560), (7, 25600, 5120),
                                   (32, 25600, 5120), (33, 1000, 256), (64, 12288, 4096)])
def test_int4_gemm_t_matches_oracle(K, m, k, n):
    """The transposed layout (W = down_t [K, N/2], scales along N): each
    weight enters as the reference's bf16(q*s); fp32 sums within the
    fp32-accumulation bound of an fp64 product of the same bf16 weights."""
    print(f"int4_gemm_t m={m} k={k} n={n}", flush=True)
    rng = np.random.default_rng(m * 7 + k)
    qw, sc = random_int4(rng, k, n)
    xs = np.stack([random_bf16(rng, k) for _ in range(m)])
    out = K.int4_gemm_t(dev(qw), dev_bf16(sc), dev_bf16(xs))
    assert out.shape == (m, n)
    got = O.bf16_to_f32(host_bf16(out)).astype(np.float64)
    w = _dequant_f64(qw, sc)
    xf = O.bf16_to_f32(xs).astype(np.float64)
    ref = xf @ w
    terms = np.abs(xf) @ np.abs(w)
    bound = 2.0 ** -8 * np.abs(ref) + 2.0 ** -17 * terms
    assert (np.abs(got - ref) <= bound).all()
    assert float(np.abs(got - ref).max() / np.abs(ref).max()) < 1e-2


@pytest.mark.parametrize("m", [5, 32, 64])
def test_int4_gemm_t_matches_dense_route(K, m):
    """The reference's prompt route for down: h @ dequantize(down_t)."""
    from qlinear import dequantize
    from quantize import quantize_tensor_int4_groupwise
    g = torch.Generator(device="cuda").manual_seed(m)
    qw, sc = quantize_tensor_int4_groupwise(torch.randn(25600, 5120, device="cuda", generator=g)
                                            * 0.02)
    h = torch.randn(m, 25600, device="cuda", generator=g).to(torch.bfloat16)
    got = K.int4_gemm_t(qw, sc, h).float()
    ref = (h @ dequantize(qw, sc)).float()
    assert float((got - ref).abs().max() / ref.abs().max()) < 1e-2


@pytest.mark.parametrize("m,k,n", [(7, 25600, 5120), (32, 25600, 5120), (64, 1000, 256),
                                   (20, 3072, 2560)])
def test_int4_gemm_t_weights_bit_exact(K, m, k, n):
    """Token t is one-hot at row r_t, so out[t] is row r_t of the staged
    weights (one nonzero product per sum): equal, bit for bit, to the
    reference's bf16(q*s) row.  Scales span 2^-100 .. 2^100 with both signs
    and random significands, so q*s needs rounding and every exponent path
    of the conversion runs; the rows cover both rows of a staged pair, step
    and K-split edges, and the last row."""
    print(f"int4_gemm_t one-hot m={m} k={k} n={n}", flush=True)
    rng = np.random.default_rng(k + m)
    q = rng.integers(-8, 8, size=(k, n)).astype(np.int8)
    mant = rng.random((k, n // 128), dtype=np.float32) + 1.0
    expo = rng.integers(-100, 101, size=(k, n // 128)).astype(np.float32)
    sign = np.where(rng.random((k, n // 128)) < 0.5, -1.0, 1.0).astype(np.float32)
    sc = O.f32_to_bf16((sign * np.ldexp(mant, expo.astype(np.int32))).astype(np.float32))
    qw = O.pack_int4(q)
    edges = [0, 1, 126, 127, 128, 129, k - 2, k - 1]
    rows = (edges + list(rng.integers(0, k, size=m)))[:m]
    x = np.zeros((m, k), dtype=np.uint16)
    x[np.arange(m), rows] = 0x3F80  # bf16 1.0
    out = host_bf16(K.int4_gemm_t(dev(qw), dev_bf16(sc), dev_bf16(x)))
    want = O.dequantize(qw, sc)[rows]
    got_f, want_f = O.bf16_to_f32(out), O.bf16_to_f32(want)
    # +0 and -0 both sum to +0 in fp32, so zeros are compared by value
    assert np.array_equal(got_f, want_f)
    nz = want_f != 0
    assert np.array_equal(out[nz], want[nz])
