"""Pins the CPU oracle (oracle/dip_oracle.py) before anything is compared to it.

The reference stores no golden vectors for this path, so each oracle function
is pinned by known-answer bytes, closed forms, invariants, an independent
second implementation (the C restatement of the top-k, oracle/topk_literal.c)
or brute force on tiny inputs — chosen so that a plausible slip (swapped
nibbles, missing sign extension, round-half-away, a dropped bf16 rounding, a
wrong tie order) fails at least one test.
"""
import ctypes
import itertools
from fractions import Fraction

import numpy as np
import pytest
import torch

import dip_oracle as O

# ---------------------------------------------------------------------------
# bf16 conversions
# ---------------------------------------------------------------------------


def test_bf16_roundtrip_all_patterns():
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    f = O.bf16_to_f32(bits)
    back = O.f32_to_bf16(f)
    nan = np.isnan(f)
    assert np.array_equal(back[~nan], bits[~nan])
    assert np.all(back[nan] == 0x7FC0)


def test_f32_to_bf16_matches_torch():
    rng = np.random.default_rng(0)
    u = rng.integers(0, 1 << 32, size=200_000, dtype=np.uint64).astype(np.uint32)
    f = u.view(np.float32)
    ours = O.f32_to_bf16(f)
    ref = torch.from_numpy(f.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(f)
    assert np.array_equal(ours[~nan], ref[~nan])
    # ties go to even: 1 + 2^-8 is halfway between bf16 1.0 and 1.0078125
    assert O.f32_to_bf16(np.float32(1.0 + 2.0 ** -8)) == 0x3F80
    assert O.f32_to_bf16(np.float32(1.0 + 3 * 2.0 ** -8)) == 0x3F82


# ---------------------------------------------------------------------------
# int4 format
# ---------------------------------------------------------------------------


def test_unpack_known_answers():
    b = np.array([[0x8F, 0x7F, 0x08, 0x00, 0xF0, 0x21]], dtype=np.uint8).view(np.int8)
    q = O.unpack_int4(b)
    assert q.tolist() == [[-1, -8, -1, 7, -8, 0, 0, 0, 0, -1, 1, 2]]


def test_pack_unpack_all_bytes():
    b = np.arange(256, dtype=np.uint8).reshape(1, 256).view(np.int8)
    q = O.unpack_int4(b)
    assert q.min() == -8 and q.max() == 7
    assert np.array_equal(O.pack_int4(q), b)
    # low nibble is the even column
    assert np.array_equal(q[0, 0::2], ((np.arange(256) & 0xF) ^ 8) - 8)


def test_dequant_exact_vs_bf16_rounding():
    # s = 1.0078125 (bf16 0x3F81), q = 3: exact product 3.0234375 is a bf16
    # tie that rounds to even (3.03125).  Kernels multiply with the exact fp32
    # value; qlinear.dequantize rounds to bf16.
    qw = O.pack_int4(np.array([[3] + [0] * 127], dtype=np.int8))
    sc = np.array([[0x3F81]], dtype=np.uint16)
    assert O.dequant_f32(qw, sc)[0, 0] == np.float32(3.0234375)
    assert O.bf16_to_f32(O.dequantize(qw, sc))[0, 0] == np.float32(3.03125)


def test_dequant_f32_equals_exact_product():
    rng = np.random.default_rng(1)
    q = rng.integers(-8, 8, size=(7, 384)).astype(np.int8)
    sc = O.f32_to_bf16(rng.random((7, 3), dtype=np.float32) * 0.01 + 0.001)
    got = O.dequant_f32(O.pack_int4(q), sc).astype(np.float64)
    want = q.astype(np.float64) * np.repeat(O.bf16_to_f32(sc).astype(np.float64), 128, axis=1)
    assert np.array_equal(got, want)


def test_quantizer_closed_forms():
    # group max 7 -> s = 1 exactly; halves round to even; -3.5 -> -4.
    w = np.zeros((2, 128), dtype=np.float32)
    w[0, :6] = [7.0, 2.5, -3.5, 0.5, 1.5, -7.0]
    qw, sc = O.quantize_int4_groupwise(w)
    q = O.unpack_int4(qw)
    assert q[0, :6].tolist() == [7, 2, -4, 0, 2, -7]
    assert O.bf16_to_f32(sc)[0, 0] == 1.0
    # all-zero group: scale clamps to 1e-8 (as bf16) and q = 0
    assert np.all(q[1] == 0)
    assert sc[1, 0] == O.f32_to_bf16(np.float32(1e-8))


def test_quantizer_invariants_random():
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((64, 512)) * 0.02).astype(np.float32)
    qw, sc = O.quantize_int4_groupwise(w)
    q = O.unpack_int4(qw).reshape(64, 4, 128)
    assert np.abs(q).max() <= 7
    # the group maximum maps to +-7
    assert np.all(np.abs(q).max(axis=2) == 7)
    s32 = np.maximum(np.abs(w.reshape(64, 4, 128)).max(axis=2) / np.float32(7), np.float32(1e-8))
    assert np.array_equal(sc, O.f32_to_bf16(s32))
    # reconstruction error bounded by half a step of the fp32 scale
    err = np.abs(q * s32[..., None] - w.reshape(64, 4, 128))
    assert np.all(err <= s32[..., None] * 0.5 * (1 + 1e-6))


def test_quantizer_recovers_grid_values():
    rng = np.random.default_rng(3)
    q_true = rng.integers(-7, 8, size=(16, 256)).astype(np.int8)
    q_true[:, 0] = 7
    q_true[:, 128] = -7
    s = np.float32(2.0 ** -7)
    qw, sc = O.quantize_int4_groupwise(q_true.astype(np.float32) * s)
    assert np.array_equal(O.unpack_int4(qw), q_true)
    assert np.all(O.bf16_to_f32(sc) == s)


def test_transpose_down_exact_on_grid():
    # If every 128-run along `out` is already an int4 grid with max 7*2^-6,
    # dequantize -> transpose -> requantize is lossless.
    rng = np.random.default_rng(4)
    out_f, inter = 256, 384
    qt = rng.integers(-7, 8, size=(inter, out_f)).astype(np.int8)
    qt[:, 0] = 7
    qt[:, 128] = -7
    s = np.float32(2.0 ** -6)
    down = (qt.T.astype(np.float32) * s)           # [out, inter]
    dq, ds = O.quantize_int4_groupwise(down)
    dtq, dts = O.transpose_down_to_int4(dq, ds)
    np.testing.assert_array_equal(O.dequant_f32(dtq, dts), O.dequant_f32(dq, ds).T)


def test_transpose_down_error_bound():
    rng = np.random.default_rng(5)
    down = (rng.standard_normal((256, 512)) * 0.02).astype(np.float32)
    dq, ds = O.quantize_int4_groupwise(down)
    dtq, dts = O.transpose_down_to_int4(dq, ds)
    assert dtq.shape == (512, 128) and dts.shape == (512, 2)
    w = O.bf16_to_f32(O.dequantize(dq, ds)).T
    wt = O.dequant_f32(dtq, dts)
    st = np.repeat(O.bf16_to_f32(dts), 128, axis=1)
    assert np.all(np.abs(wt - w) <= st * 0.5 + 1e-9 + np.abs(w) * 2 ** -8)


# ---------------------------------------------------------------------------
# GEMV / SiLU / h
# ---------------------------------------------------------------------------


def test_gemv_matches_exact_rational_sum():
    rng = np.random.default_rng(6)
    q = rng.integers(-8, 8, size=(3, 256)).astype(np.int8)
    sc = O.f32_to_bf16(rng.random((3, 2), dtype=np.float32) * 0.01 + 0.001)
    x = O.f32_to_bf16(rng.standard_normal(256).astype(np.float32))
    qw = O.pack_int4(q)
    got = O.gemv_f64(qw, sc, x)
    sf = O.bf16_to_f32(sc)
    xf = O.bf16_to_f32(x)
    for r in range(3):
        exact = sum(Fraction(int(q[r, c])) * Fraction(float(sf[r, c // 128])) *
                    Fraction(float(xf[c])) for c in range(256))
        assert abs(got[r] - float(exact)) <= 1e-12 * max(1.0, abs(float(exact)))


def test_gemv_one_hot_is_exact_dequant():
    rng = np.random.default_rng(7)
    q = rng.integers(-8, 8, size=(5, 128)).astype(np.int8)
    sc = O.f32_to_bf16(rng.random((5, 1), dtype=np.float32))
    x = np.zeros(128, dtype=np.uint16)
    x[17] = 0x3F80  # 1.0
    pre = O.gemv_bf16(O.pack_int4(q), sc, x)
    assert np.array_equal(pre, O.f32_to_bf16(q[:, 17].astype(np.float32) * O.bf16_to_f32(sc)[:, 0]))


def test_silu_numpy_matches_torch_exhaustively():
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    a = O.silu_bf16(bits)
    b = O.silu_bf16_np(bits)
    fa, fb = O.bf16_to_f32(a), O.bf16_to_f32(b)
    same = (a == b) | (np.isnan(fa) & np.isnan(fb))
    # torch's CPU exp and numpy's exp may land on opposite sides of a bf16
    # rounding boundary on a handful of inputs; never by more than one ulp.
    assert (~same).sum() <= 64, int((~same).sum())
    ulp = np.abs(a.astype(np.int32) - b.astype(np.int32))
    assert np.all(ulp[~same] <= 1)
    # known values
    one = O.f32_to_bf16(np.float32(1.0))
    assert O.bf16_to_f32(O.silu_bf16(np.array([one])))[0] == np.float32(0.73046875)
    assert O.silu_bf16(np.array([0], np.uint16))[0] == 0
    assert O.silu_bf16(O.f32_to_bf16(np.float32(-200.0)).reshape(1))[0] == 0x8000  # -0.0


def test_h_product_is_exact_before_rounding():
    rng = np.random.default_rng(8)
    g = O.f32_to_bf16(rng.standard_normal(4096).astype(np.float32))
    u = O.f32_to_bf16(rng.standard_normal(4096).astype(np.float32))
    exact = O.bf16_to_f32(g).astype(np.float64) * O.bf16_to_f32(u).astype(np.float64)
    assert np.array_equal(O.h_bf16(g, u), O.f32_to_bf16(exact.astype(np.float32)))
    assert np.array_equal(exact.astype(np.float32).astype(np.float64), exact)


def test_down_one_hot_row():
    rng = np.random.default_rng(9)
    q = rng.integers(-8, 8, size=(6, 256)).astype(np.int8)
    sc = O.f32_to_bf16(rng.random((6, 2), dtype=np.float32) * 0.01)
    h = np.zeros(6, np.uint16)
    h[4] = O.f32_to_bf16(np.array([-2.0], np.float32))[0]
    y = O.down_f64(O.pack_int4(q), sc, h)
    np.testing.assert_array_equal(y, -2.0 * O.dequant_f32(O.pack_int4(q), sc)[4])


# ---------------------------------------------------------------------------
# top-k
# ---------------------------------------------------------------------------


@pytest.fixture(scope="module")
def c_topk():
    from build_oracle import build
    lib = ctypes.CDLL(str(build()))
    fn = lib.oracle_topk_literal
    fn.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                   ctypes.c_void_p, ctypes.c_void_p]
    fn.restype = ctypes.c_int

    def run(s, k):
        s = np.ascontiguousarray(s, dtype=np.uint16)
        idx = np.zeros(max(k, 1), dtype=np.int32)
        lo = ctypes.c_float()
        hi = ctypes.c_float()
        fn(s.ctypes.data, s.size, k, idx.ctypes.data, ctypes.byref(lo), ctypes.byref(hi))
        return idx[:k], np.float32(lo.value), np.float32(hi.value)
    return run


def _special_inputs():
    rng = np.random.default_rng(10)
    cases = []
    g = O.f32_to_bf16((rng.standard_normal(25600)).astype(np.float32))
    cases += [(g, 15360), (g, 7680), (g, 1), (g, 25599), (g, 25600), (g, 0)]
    # heavy ties: few distinct magnitudes
    t = O.f32_to_bf16(rng.integers(-3, 4, size=4000).astype(np.float32))
    cases += [(t, 1500), (t, 2999), (t, 10)]
    # zeros, NaN, inf, subnormals, -0
    z = np.zeros(300, np.uint16)
    cases += [(z, 10), (z, 300)]
    sp = O.f32_to_bf16(rng.standard_normal(1000).astype(np.float32))
    sp[::7] = 0x7FC0            # NaN
    sp[3] = 0x7F80              # +inf
    sp[5] = 0xFF80              # -inf
    sp[11::13] = 0x0001         # subnormal
    sp[12::17] = 0x8000         # -0
    cases += [(sp, 50), (sp, 900), (sp, 999)]
    # all values near the bf16 maximum: lo + hi overflows to inf
    big = np.full(64, 0x7F7F, np.uint16)
    big[::2] = 0x7F70
    cases += [(big, 20), (big, 40)]
    # tiny magnitudes: thresholds become fp32 subnormals
    tiny = np.full(64, 0x0090, np.uint16)
    tiny[::3] = 0x0100
    cases += [(tiny, 10), (tiny, 30)]
    return cases


def test_topk_numpy_equals_c_literal(c_topk):
    for s, k in _special_inputs():
        a = O.topk_select(s, k)
        b, lo, hi = c_topk(s, k)
        assert np.array_equal(a, b), (s.size, k)
        lo2, hi2 = O.topk_bisect(s, k)
        assert lo == lo2 and hi == hi2


def test_topk_literal_equals_key_order_on_ordinary_data():
    rng = np.random.default_rng(11)
    for trial in range(40):
        n = int(rng.integers(100, 30000))
        k = int(rng.integers(1, n))
        g = O.f32_to_bf16((rng.standard_normal(n) * rng.uniform(0.1, 10)).astype(np.float32))
        a = O.topk_select(g, k)
        b = O.topk_key_order(g, k)
        assert np.array_equal(a, b), (trial, n, k)


def test_topk_brute_force_tiny():
    """Every selection over small value sets.  With distinct magnitudes far
    apart (relative to max / 2^25) the bisection band holds only
    A = a_{k+1}, the (k+1)-th largest |s|, so the output must be
    ascending {|s| > A} followed by ascending {|s| == A} up to k (nothing from
    the band when A = 0 or does not exist), zero-padded."""
    vals = [0x0000, 0x3F80, 0xBF80, 0x4000, 0x3F00]   # 0, 1, -1, 2, 0.5
    for n in range(1, 6):
        for combo in itertools.product(vals, repeat=n):
            s = np.array(combo, np.uint16)
            mags = [abs(float(O.bf16_to_f32(np.array([v], np.uint16))[0])) for v in combo]
            ranked = sorted(mags, reverse=True)
            for k in range(0, n + 1):
                got = O.topk_select(s, k).tolist()
                A = ranked[k] if k < n else 0.0
                want = [i for i in range(n) if mags[i] > A]
                if A > 0:
                    want += [i for i in range(n) if mags[i] == A]
                want = want[:k] + [0] * max(0, k - len(want))
                assert got == want, (combo, k, got, want)


def test_topk_differs_from_torch_topk_on_ties():
    """torch.topk (the reference's fallback) is not a valid index oracle."""
    rng = np.random.default_rng(12)
    g = O.f32_to_bf16(rng.standard_normal(25600).astype(np.float32) * 0.5)
    k = 15360
    ours = set(O.topk_select(g, k).tolist())
    t = torch.from_numpy(g.view(np.int16)).view(torch.bfloat16)
    theirs = set(t.abs().topk(k).indices.tolist())
    assert len(ours) == k
    # same magnitudes either way, different tie members
    mag = np.abs(O.bf16_to_f32(g))
    assert sorted(mag[list(ours)]) == sorted(mag[list(theirs)])


def test_topk_band_edge_cases():
    # fewer than k nonzeros: zeros never selected, tail stays 0
    s = np.zeros(10, np.uint16)
    s[[2, 7]] = O.f32_to_bf16(np.array([1.0, -3.0], np.float32))
    assert O.topk_select(s, 4).tolist() == [2, 7, 0, 0]
    # NaN is never selected.  With +inf present the reference's bisection
    # degenerates: max = inf, t = 0.5f*(0 + inf) = inf forever, so hi = inf,
    # lo = 0, tier A is empty and the band (0, inf] is emitted by index.
    s = O.f32_to_bf16(np.array([1.0, np.nan, 2.0, np.inf, 0.5], np.float32))
    assert O.topk_select(s, 2).tolist() == [0, 2]
    lo, hi = O.topk_bisect(s, 2)
    assert lo == 0 and np.isinf(hi)
    # without inf, NaN is skipped and the two largest finite values win
    s = O.f32_to_bf16(np.array([1.0, np.nan, 2.0, 3.0, 0.5], np.float32))
    assert O.topk_select(s, 2).tolist() == [2, 3]
    # subnormal magnitudes behave as zero (fast-math fabsf)
    s = np.array([0x0001, 0x3F80, 0x0040], np.uint16)
    assert O.topk_select(s, 2).tolist() == [1, 0]


# ---------------------------------------------------------------------------
# module-level pieces
# ---------------------------------------------------------------------------


def test_keep_count_bankers_rounding():
    assert O.keep_count(25600, 0.6) == 15360
    assert O.keep_count(25600, 0.3) == 7680
    assert O.keep_count(12288, 0.6) == 7373
    assert O.keep_count(12288, 0.3) == 3686
    assert O.keep_count(10, 0.25) == 2     # round(2.5) -> 2
    assert O.keep_count(10, 0.01) == 1     # max(1, ...)


def test_ca_split_brute_force():
    rng = np.random.default_rng(13)
    inter = 200
    hot = np.sort(rng.choice(inter, 60, replace=False))
    id2slot = np.full(inter, -1, np.int64)
    id2slot[hot] = np.arange(60)
    idx = rng.choice(inter, 120, replace=False).astype(np.int32)
    comb, src, row, n_hit, miss = O.ca_split(idx, id2slot)
    hits = [c for c in idx if id2slot[c] >= 0]
    misses = [c for c in idx if id2slot[c] < 0]
    assert comb.tolist() == hits + misses
    assert src.tolist() == [0] * len(hits) + [1] * len(misses)
    assert row.tolist() == [int(id2slot[c]) for c in hits] + list(range(len(misses)))
    assert n_hit == len(hits) and miss.tolist() == misses


def test_hot_set_key_order():
    rng = np.random.default_rng(14)
    cnt = rng.integers(0, 5, size=300)
    hot, id2slot = O.hot_set(cnt, 90)
    order = sorted(range(300), key=lambda i: (-cnt[i], i))[:90]
    assert hot.tolist() == sorted(order)
    assert np.array_equal(id2slot[hot], np.arange(90))
    assert np.all(id2slot[np.setdiff1d(np.arange(300), hot)] == -1)


def test_dip_forward_tiny_against_loops():
    L = O.make_layer(256, 512, seed=3)
    x = O.make_x(256, seed=4)
    k = O.keep_count(512, 0.6)
    out = O.dip_forward(L["gate_qw"], L["gate_sc"], L["up_qw"], L["up_sc"], L["down_t_qw"],
                        L["down_t_sc"], x, k)
    wg = O.dequant_f32(L["gate_qw"], L["gate_sc"]).astype(np.float64)
    wu = O.dequant_f32(L["up_qw"], L["up_sc"]).astype(np.float64)
    wd = O.dequant_f32(L["down_t_qw"], L["down_t_sc"]).astype(np.float64)
    xf = O.bf16_to_f32(x).astype(np.float64)
    idx = out["idx"]
    assert len(set(idx.tolist())) == k
    y = np.zeros(256)
    for j, c in enumerate(idx):
        g = O.bf16_to_f32(out["g"][c])
        u = O.bf16_to_f32(O.f32_to_bf16(np.float32(wu[c] @ xf)))
        h = O.bf16_to_f32(O.f32_to_bf16(np.float32(g * u)))
        y += float(h.reshape(-1)[0]) * wd[c]
    np.testing.assert_allclose(out["y_f64"], y, rtol=1e-9, atol=1e-12)
    pre = O.f32_to_bf16((wg @ xf).astype(np.float32))
    assert np.array_equal(out["pre"], pre)


# ---------------------------------------------------------------------------
# The PyTorch restatement (cpu_baseline of bench.py) against the numpy one
# ---------------------------------------------------------------------------


def _t(a):
    """numpy int8 / uint16-bf16 bits -> torch CPU tensor (int8 / bfloat16)."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)
    return torch.from_numpy(a)


def _bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def test_torch_unpack_and_dequantize_bit_identical():
    """torch_unpack_int4 / torch_dequantize (qlinear.py:28-64 in torch ops)
    equal the numpy unpack_int4 / dequantize on all 256 bytes, under random
    scales and the tie scale 0x3F81 (q = 3 gives 3.0234375, a bf16 tie that
    rounds to even), and on the known-answer bytes."""
    b = np.tile(np.arange(256, dtype=np.uint8), 3).reshape(6, 128).view(np.int8)
    assert np.array_equal(O.torch_unpack_int4(_t(b)).numpy(), O.unpack_int4(b))
    rng = np.random.default_rng(7)
    sc = O.f32_to_bf16(rng.random((6, 2), dtype=np.float32) * 0.05 + 1e-4)
    sc[0, :] = 0x3F81
    sc[1, 0] = 0x0000
    got = _bits(O.torch_dequantize(_t(b), _t(sc)))
    assert np.array_equal(got, O.dequantize(b, sc))
    kb = np.array([[0x8F, 0x7F, 0x08] + [0] * 61], dtype=np.uint8).view(np.int8)
    assert O.torch_unpack_int4(_t(kb)).numpy()[0, :6].tolist() == [-1, -8, -1, 7, -8, 0]
    tie = O.pack_int4(np.array([[3] * 128], dtype=np.int8))
    t_out = O.bf16_to_f32(_bits(O.torch_dequantize(_t(tie), _t(np.array([[0x3F81]], np.uint16)))))
    assert np.all(t_out == np.float32(3.03125))


def test_torch_cpu_forward_matches_the_numpy_route():
    """torch_cpu_forward (the timed cpu_baseline) computes the reference's
    forward: its idx is topk_select of its own g, its g is bf16(silu(bf16 of
    the bf16(q*s) GEMV)) within one bf16 ulp of a float64 evaluation, and its
    y is within 1e-2 of dip_forward's on that idx."""
    H, I = 256, 768
    k = O.keep_count(I, 0.6)
    L = O.make_layer(H, I, seed=11)
    x = O.make_x(H, seed=12)
    out = O.torch_cpu_forward(_t(L["gate_qw"]), _t(L["gate_sc"]), _t(L["up_qw"]), _t(L["up_sc"]),
                              _t(L["down_t_qw"]), _t(L["down_t_sc"]), _t(x), k, return_all=True)
    g = _bits(out["g"])
    idx = out["idx"].numpy()
    assert np.array_equal(idx, O.topk_select(g, k))
    wg = O.bf16_to_f32(O.dequantize(L["gate_qw"], L["gate_sc"])).astype(np.float64)
    pre = O.f32_to_bf16((wg @ O.bf16_to_f32(x).astype(np.float64)).astype(np.float32))
    g_ref = O.silu_bf16(pre)
    d = np.abs(g.astype(np.int32) - g_ref.astype(np.int32))
    assert d.max() <= 1 and np.count_nonzero(d) <= I // 50
    ref = O.dip_forward(L["gate_qw"], L["gate_sc"], L["up_qw"], L["up_sc"], L["down_t_qw"],
                        L["down_t_sc"], x, k, idx=idx)
    y = O.bf16_to_f32(_bits(out["y"])).astype(np.float64)
    assert np.abs(y - ref["y_f64"]).max() / np.abs(ref["y_f64"]).max() < 1e-2
    # a planted slip (h without g) is caught by the same bar
    slip = O.down_f64(L["down_t_qw"], L["down_t_sc"], ref["u"], rows=idx)
    assert np.abs(y - slip).max() / np.abs(ref["y_f64"]).max() > 1e-2


# ---------------------------------------------------------------------------
# ca_forward and the two dense routes
# ---------------------------------------------------------------------------


def test_ca_forward_equals_dip_forward_per_channel():
    """ca_forward (dip_ca.py:127-188) reorders the selection into [hits,
    misses] but computes the same h per channel and the same y: h of every
    channel equals dip_forward's for that channel, the split covers idx
    exactly once, and y_f64 agrees to float64 rounding (a different sum
    order)."""
    H, I = 256, 512
    k = O.keep_count(I, 0.6)
    L = O.make_layer(H, I, seed=5)
    x = O.make_x(H, seed=6)
    rng = np.random.default_rng(8)
    hot = np.sort(rng.choice(I, size=150, replace=False))
    id2slot = np.full(I, -1, dtype=np.int64)
    id2slot[hot] = np.arange(hot.size)
    ca = O.ca_forward(L["gate_qw"], L["gate_sc"], L["up_qw"], L["up_sc"], L["down_t_qw"],
                      L["down_t_sc"], id2slot, x, k)
    dip = O.dip_forward(L["gate_qw"], L["gate_sc"], L["up_qw"], L["up_sc"], L["down_t_qw"],
                        L["down_t_sc"], x, k, idx=ca["idx"])
    assert sorted(ca["combined"].tolist()) == sorted(ca["idx"].tolist())
    assert 0 < ca["n_hit"] < k
    h_by_ch = dict(zip(dip["idx"].tolist(), dip["h"].tolist()))
    assert [h_by_ch[c] for c in ca["combined"].tolist()] == ca["h"].tolist()
    np.testing.assert_allclose(ca["y_f64"], dip["y_f64"], rtol=1e-12, atol=1e-15)
    assert np.array_equal(ca["g"], dip["g"])


def test_dense_literal_uses_bf16_weights():
    """dense_literal_forward (_dense, dip_stream_predispatch.py:206-215)
    multiplies by bf16(q*s): with the tie scale 0x3F81 and q = 3 on one
    weight of up and of down_t, a one-hot x and one channel, u and y take the
    rounded weight 3.03125 where the kernels' route takes 3.0234375."""
    H, I = 128, 1
    one_q = np.zeros((I, H), dtype=np.int8)
    one_q[0, 0] = 3
    w3 = O.pack_int4(one_q)
    sc = np.array([[0x3F81]], dtype=np.uint16)
    g_q = np.zeros((I, H), dtype=np.int8)
    g_q[0, 0] = 4                      # pre = 4 * 1.0 * x0
    gate_sc = np.array([[0x3F80]], dtype=np.uint16)
    x = np.zeros(H, dtype=np.uint16)
    x[0] = 0x3F80                      # x0 = 1
    lit = O.dense_literal_forward(O.pack_int4(g_q), gate_sc, w3, sc, w3, sc, x)
    dense = O.dense_forward(O.pack_int4(g_q), gate_sc, w3, sc, w3, sc, x)
    assert O.bf16_to_f32(lit["u"])[0] == np.float32(3.03125)
    assert O.bf16_to_f32(dense["u"])[0] == np.float32(3.03125)  # bf16(3.0234375) is the tie too
    h = O.bf16_to_f32(lit["h"])[0]
    assert lit["y_f64"][0] == float(h) * 3.03125
    assert dense["y_f64"][0] == float(O.bf16_to_f32(dense["h"])[0]) * 3.0234375
    assert np.all(lit["y_f64"][1:] == 0)


def test_dense_literal_equals_dense_on_exact_grids():
    """With power-of-two scales every q*s is a bf16 value, so bf16(q*s) =
    q*s and the literal route equals the all-channel DIP route bit for bit;
    with ordinary scales they differ (the rounding is real) but agree to
    well within 1e-2."""
    H, I = 256, 384
    rng = np.random.default_rng(9)
    mats = []
    for _ in range(3):
        q = rng.integers(-8, 8, size=(I, H)).astype(np.int8)
        e = rng.integers(-9, -5, size=(I, H // 128))
        sc = O.f32_to_bf16(np.ldexp(np.float32(1.0), e).astype(np.float32))
        mats.append((O.pack_int4(q), sc))
    x = O.make_x(H, seed=10)
    (gq, gs), (uq, us), (dq, ds) = mats
    lit = O.dense_literal_forward(gq, gs, uq, us, dq, ds, x)
    den = O.dense_forward(gq, gs, uq, us, dq, ds, x)
    assert np.array_equal(lit["u"], den["u"]) and np.array_equal(lit["h"], den["h"])
    assert np.array_equal(lit["y_f64"], den["y_f64"])
    L = O.make_layer(H, I, seed=13)
    lit = O.dense_literal_forward(L["gate_qw"], L["gate_sc"], L["up_qw"], L["up_sc"],
                                  L["down_t_qw"], L["down_t_sc"], x)
    den = O.dense_forward(L["gate_qw"], L["gate_sc"], L["up_qw"], L["up_sc"],
                          L["down_t_qw"], L["down_t_sc"], x)
    assert not np.array_equal(lit["y_f64"], den["y_f64"])
    assert np.abs(lit["y_f64"] - den["y_f64"]).max() / np.abs(lit["y_f64"]).max() < 1e-2


def test_dense_literal_matches_torch_dense_route():
    """The reference's own ops for _dense on the CPU (dequantize + F.linear
    in bf16, g * u, h @ dequantize(down_t)) agree with dense_literal_forward:
    u within one bf16 ulp, y within 1e-2."""
    import torch.nn.functional as F
    H, I = 256, 512
    L = O.make_layer(H, I, seed=14)
    x = O.make_x(H, seed=15)
    lit = O.dense_literal_forward(L["gate_qw"], L["gate_sc"], L["up_qw"], L["up_sc"],
                                  L["down_t_qw"], L["down_t_sc"], x)
    xb = _t(x).reshape(1, -1)
    g = _t(lit["g"]).reshape(1, -1)
    u = F.linear(xb, O.torch_dequantize(_t(L["up_qw"]), _t(L["up_sc"])))
    h = g * u
    y = h @ O.torch_dequantize(_t(L["down_t_qw"]), _t(L["down_t_sc"]))
    du = np.abs(_bits(u).reshape(-1).astype(np.int32) - lit["u"].astype(np.int32))
    assert du.max() <= 1
    yt = O.bf16_to_f32(_bits(y).reshape(-1)).astype(np.float64)
    assert np.abs(yt - lit["y_f64"]).max() / np.abs(lit["y_f64"]).max() < 1e-2
