"""Property tests of the oracle's threshold top-k (topk_select.cu:30-164) on
tie-heavy inputs with zeros, subnormals, infinities and NaN: the numpy
restatement and the C restatement agree bit for bit, the result is k
in-range indices in the reference's output order (tier A, then tier B, each
in index order, then zero fillers for slots no value reaches), and on finite
inputs that the bisection isolates the selected set is the top k by
(|g| desc, id asc)."""
import ctypes

import numpy as np
import pytest
from hypothesis import given, settings, HealthCheck

import dip_oracle as O
from topk_strategies import topk_inputs


@pytest.fixture(scope="module")
def c_topk_fn():
    """oracle/topk_literal.c, the sequential C restatement of the top-k."""
    from build_oracle import build
    fn = ctypes.CDLL(str(build())).oracle_topk_literal
    fn.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                   ctypes.c_void_p, ctypes.c_void_p]
    fn.restype = ctypes.c_int

    def run(s, k):
        s = np.ascontiguousarray(s, dtype=np.uint16)
        idx = np.zeros(max(k, 1), dtype=np.int32)
        lo, hi = ctypes.c_float(), ctypes.c_float()
        fn(s.ctypes.data, s.size, k, idx.ctypes.data, ctypes.byref(lo), ctypes.byref(hi))
        return idx[:k], np.float32(lo.value), np.float32(hi.value)
    return run

SETTINGS = settings(max_examples=150, derandomize=True, database=None, deadline=None,
                    suppress_health_check=[HealthCheck.too_slow])


@SETTINGS
@given(topk_inputs())
def test_topk_numpy_equals_c_literal(c_topk_fn, case):
    g, k = case
    idx = O.topk_select(g, k)
    c_idx, _, _ = c_topk_fn(g, k)
    assert np.array_equal(idx, c_idx)


@SETTINGS
@given(topk_inputs())
def test_topk_output_shape_and_order(case):
    g, k = case
    idx = O.topk_select(g, k)
    assert idx.shape == (k,)
    assert k == 0 or (idx.min() >= 0 and idx.max() < g.size)
    # distinct indices, then (when fewer than k values pass the lower cut:
    # zeros, NaN) the zero fillers of torch::zeros (topk_select.cu:160)
    seen, m = set(), k
    for j, v in enumerate(idx.tolist()):
        if v in seen:
            m = j
            break
        seen.add(v)
    assert not idx[m:].any()
    # tier A then tier B, each ascending: at most one descent in the filled part
    assert int((np.diff(idx[:m]) < 0).sum()) <= 1


@SETTINGS
@given(topk_inputs())
def test_topk_finite_isolated_is_key_order(case):
    g, k = case
    f = O.bf16_to_f32(g)
    if not np.isfinite(f).all():
        return
    mags = np.sort(np.abs(f))[::-1]
    # the bisection isolates the k-th value when it is not too small against
    # the largest (the reference's 25 steps): skip the rest
    if k == 0 or k == g.size or mags[k] < mags[0] * 2.0 ** -16:
        return
    assert np.array_equal(np.sort(O.topk_select(g, k)), np.sort(O.topk_key_order(g, k)))
