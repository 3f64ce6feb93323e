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
