"""GPU parity of the contiguous GEMV on int8 MFMA (DIP_TUNE_GATE_MFMA = 1).

The kernel splits x into exact base-128 digits per 128-column group and sums
16*q*digit products in int32, so its outputs must meet the same bars as the
row-dot GEMV against the fp64 oracle: the reference's metric
max|err|/max|ref| < 1e-2 and the per-element fp32-accumulation bound with at
most 1 % of outputs one bf16 ulp off the correctly rounded value.  It runs for
widths 5120 and 4096 when there are at least 2 * CUs * 2 16-row tiles.
"""
import numpy as np
import pytest
import torch

import dip_oracle as O
from gpu_util import (assert_fp32_close, dev, dev_bf16, gemv_abs_terms, host_bf16, random_bf16,
                      random_int4, rel_err, ulp_diff)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def K():
    import _dip_hip
    return _dip_hip


@pytest.fixture()
def mfma(K):
    old = K.get_tuning("gate_mfma")
    K.set_tuning("gate_mfma", 1)
    yield
    K.set_tuning("gate_mfma", old)


def _gemv(K, qw, sc, x, act=0):
    return host_bf16(K.int4_gemv(dev(qw), dev_bf16(sc), dev_bf16(x), act=act))


@pytest.mark.parametrize("rows,cols", [(25600, 5120), (16389, 5120), (17000, 4096)])
def test_mfma_gemv_matches_oracle(K, mfma, rows, cols):
    print(f"mfma gemv rows={rows} cols={cols}", flush=True)
    rng = np.random.default_rng(rows + 3 * cols)
    qw, sc = random_int4(rng, rows, cols)
    x = random_bf16(rng, cols)
    out = _gemv(K, qw, sc, x)
    ref = O.gemv_f64(qw, sc, x)
    assert rel_err(out, ref) < 1e-2
    assert_fp32_close(out, ref, gemv_abs_terms(qw, sc, x))


def test_mfma_gemv_wide_dynamic_range(K, mfma):
    """x spanning 2^-40 .. 2^12 within every group, exact zeros, a group of
    only tiny values and one of only zeros."""
    rows, cols = 16400, 5120
    rng = np.random.default_rng(5)
    qw, sc = random_int4(rng, rows, cols)
    mag = 2.0 ** rng.uniform(-40, 12, cols)
    xf = (mag * rng.choice([-1.0, 1.0], cols)).astype(np.float32)
    xf[rng.random(cols) < 0.1] = 0.0
    xf[128:256] *= 2.0 ** -60      # a group of tiny values
    xf[256:384] = 0.0              # a group of zeros
    x = O.f32_to_bf16(xf)
    out = _gemv(K, qw, sc, x)
    ref = O.gemv_f64(qw, sc, x)
    assert rel_err(out, ref) < 1e-2
    assert_fp32_close(out, ref, gemv_abs_terms(qw, sc, x))


def test_mfma_gemv_nonfinite_x_poisons(K, mfma):
    rows, cols = 16384, 4096
    rng = np.random.default_rng(6)
    qw, sc = random_int4(rng, rows, cols)
    x = random_bf16(rng, cols)
    x[777] = 0x7FC0  # NaN
    out = _gemv(K, qw, sc, x)
    assert np.isnan(O.bf16_to_f32(out)).all()


def test_mfma_silu_and_topk(K, mfma):
    """The gate + SiLU + top-k entry point on the MFMA gate: g is silu of the
    raw GEMV within one ulp, and the indices are the oracle's top-k of g."""
    rows, cols, k = 25600, 5120, 15360
    rng = np.random.default_rng(7)
    qw, sc = random_int4(rng, rows, cols)
    x = random_bf16(rng, cols)
    pre = _gemv(K, qw, sc, x)
    g, idx = K.gate_silu_topk(dev(qw), dev_bf16(sc), dev_bf16(x), k)
    g_h = host_bf16(g)
    d = ulp_diff(g_h, O.silu_bf16(pre))
    assert d.max() <= 1 and (d > 0).mean() < 1e-3
    assert np.array_equal(idx.cpu().numpy(), O.topk_select(g_h, k))


def test_mfma_matches_rowdot_closely(K):
    """Both GEMV kernels on the same inputs: at most one bf16 ulp apart, and
    equal on almost every row."""
    rows, cols = 25600, 5120
    rng = np.random.default_rng(8)
    qw, sc = random_int4(rng, rows, cols)
    x = random_bf16(rng, cols)
    old = K.get_tuning("gate_mfma")
    try:
        K.set_tuning("gate_mfma", 0)
        a = _gemv(K, qw, sc, x)
        K.set_tuning("gate_mfma", 1)
        b = _gemv(K, qw, sc, x)
    finally:
        K.set_tuning("gate_mfma", old)
    d = ulp_diff(a, b)
    assert d.max() <= 1 and (d > 0).mean() < 0.02


def test_mfma_decode_step_spec_matches_stagewise(K, mfma):
    """The decode step with the MFMA gate: speculative and stage-by-stage
    steps stay bit-identical over several tokens."""
    from quantize import quantize_tensor_int4_groupwise
    H, I = 5120, 25600
    gen = torch.Generator(device="cuda").manual_seed(9)
    W = []
    for _ in range(3):
        W += list(quantize_tensor_int4_groupwise(torch.randn(I, H, device="cuda", generator=gen)
                                                 * 0.02))
    k = O.keep_count(I, 0.6)
    state = K.mlp_state("cuda")
    for t in range(3):
        x = torch.randn(H, device="cuda", generator=gen).to(torch.bfloat16)
        a = [v.clone() for v in K.mlp_decode(*W, x, k, state=state)]
        b = [v.clone() for v in K.mlp_decode(*W, x, k)]
        for u, v in zip(a, b):
            uu = u.view(torch.int16) if u.dtype == torch.bfloat16 else u
            vv = v.view(torch.int16) if v.dtype == torch.bfloat16 else v
            assert torch.equal(uu, vv), t
