"""Helpers shared by the GPU tests: numpy <-> device conversions and error
metrics.  (Imported by tests only.)"""
import numpy as np
import torch


def dev_bf16(bits: np.ndarray) -> torch.Tensor:
    a = np.ascontiguousarray(bits, dtype=np.uint16)
    return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).cuda()


def host_bf16(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16).copy()


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def rel_err(got_bits: np.ndarray, ref: np.ndarray) -> float:
    """max|err| / max|ref| — the reference's metric (kernels/*/test_*.py)."""
    import dip_oracle as O
    g = O.bf16_to_f32(got_bits).astype(np.float64)
    r = np.asarray(ref, dtype=np.float64)
    return float(np.abs(g - r).max() / (np.abs(r).max() + 1e-30))


def ulp_diff(a_bits: np.ndarray, b_bits: np.ndarray) -> np.ndarray:
    """Distance in bf16 ulps between finite values of the same sign pattern."""
    a = a_bits.astype(np.int32)
    b = b_bits.astype(np.int32)
    # map sign-magnitude to a monotone integer line
    a = np.where(a & 0x8000, -(a & 0x7FFF), a)
    b = np.where(b & 0x8000, -(b & 0x7FFF), b)
    return np.abs(a - b)


def random_int4(rng, rows, cols, scale_lo=0.001, scale_hi=0.011):
    """Random packed weights as the reference tests draw them:
    q ~ U{-8..7}, s ~ U[0.001, 0.011) (test_int4_gemv.py:34-37)."""
    import dip_oracle as O
    q = rng.integers(-8, 8, size=(rows, cols)).astype(np.int8)
    sc = O.f32_to_bf16((rng.random((rows, cols // 128), dtype=np.float32) *
                        (scale_hi - scale_lo) + scale_lo))
    return O.pack_int4(q), sc


def random_bf16(rng, n, std=1.0):
    import dip_oracle as O
    return O.f32_to_bf16((rng.standard_normal(n) * std).astype(np.float32))


def assert_fp32_close(got_bits, ref, abs_terms, frac_ulp=0.01):
    """Bar for a bf16 output of an fp32-accumulated dot product:
    |got - ref| <= 2^-8 |ref| (one bf16 ulp) + 2^-17 * sum|terms| (fp32
    accumulation over the terms, generous for any summation order), and at
    most `frac_ulp` of the outputs off the correctly rounded value."""
    import dip_oracle as O
    g = O.bf16_to_f32(got_bits).astype(np.float64)
    r = np.asarray(ref, np.float64)
    bound = np.abs(r) * 2.0 ** -8 + np.asarray(abs_terms, np.float64) * 2.0 ** -17
    bad = np.abs(g - r) > bound
    assert not bad.any(), (int(bad.sum()), float((np.abs(g - r) / bound).max()))
    off = got_bits != O.f32_to_bf16(r.astype(np.float32))
    assert off.mean() <= frac_ulp, float(off.mean())


def gemv_abs_terms(qw, sc, x, rows=None):
    import dip_oracle as O
    if rows is not None:
        qw, sc = np.asarray(qw)[rows], np.asarray(sc)[rows]
    return np.abs(O.dequant_f32(qw, sc)).astype(np.float64) @ np.abs(
        O.bf16_to_f32(x).astype(np.float64))


def down_abs_terms(qw, sc, h, rows=None):
    import dip_oracle as O
    if rows is not None:
        qw, sc = np.asarray(qw)[rows], np.asarray(sc)[rows]
    return np.abs(O.bf16_to_f32(h).astype(np.float64)) @ np.abs(
        O.dequant_f32(qw, sc)).astype(np.float64)
