"""GPU parity of each kernel against the CPU oracle (through the C ABI).

Bars: top-k indices, dequantized values, h and the CA tables bit-exact;
GEMV / down outputs within the reference's metric max|err|/max|ref| and at
most one bf16 ulp from the correctly rounded oracle value.
"""
import numpy as np
import pytest
import torch

import dip_oracle as O
from gpu_util import (assert_fp32_close, dev, dev_bf16, down_abs_terms, gemv_abs_terms, host_bf16,
                      random_bf16, random_int4, rel_err, ulp_diff)

pytestmark = pytest.mark.gpu

GEMV_SHAPES = [(4096, 5120), (512, 4096), (300, 2560), (100, 128), (257, 256), (64, 1024),
               (96, 2048), (128, 512), (40, 8192), (77, 1536), (50, 3072), (33, 6144),
               # 8192-wide rows (an o projection): 1, 2 and 7 rows per lane group
               (5120, 8192), (8193, 8192), (25601, 8192)]


@pytest.fixture(scope="module")
def K():
    import _dip_hip
    return _dip_hip


@pytest.mark.parametrize("rows,cols", GEMV_SHAPES)
def test_int4_gemv(K, rows, cols):
    print(f"gemv rows={rows} cols={cols}", flush=True)
    rng = np.random.default_rng(rows * 7 + cols)
    qw, sc = random_int4(rng, rows, cols)
    x = random_bf16(rng, cols)
    out = host_bf16(K.int4_gemv(dev(qw), dev_bf16(sc), dev_bf16(x)))
    ref = O.gemv_f64(qw, sc, x)
    assert rel_err(out, ref) < 1e-2
    assert_fp32_close(out, ref, gemv_abs_terms(qw, sc, x))


@pytest.mark.parametrize("rows,cols", [(4096, 5120), (1000, 4096), (300, 2560)])
def test_gemv_silu(K, rows, cols):
    rng = np.random.default_rng(rows + cols)
    qw, sc = random_int4(rng, rows, cols)
    x = random_bf16(rng, cols)
    qd, sd, xd = dev(qw), dev_bf16(sc), dev_bf16(x)
    pre = host_bf16(K.int4_gemv(qd, sd, xd))
    g = host_bf16(K.int4_gemv(qd, sd, xd, act=1))
    want = O.silu_bf16(pre)
    d = ulp_diff(g, want)
    assert d.max() <= 1 and (d > 0).mean() < 1e-3


def test_silu_exhaustive(K):
    """Every bf16 pre-activation through the gate epilogue: one-hot x and
    q = 1 make pre = bf16(s) = s exactly for each of the 65536 patterns."""
    n = 1 << 16
    q = np.zeros((n, 128), np.int8)
    q[:, 0] = 1
    sc = np.arange(n, dtype=np.uint32).astype(np.uint16).reshape(n, 1)
    x = np.zeros(128, np.uint16)
    x[0] = 0x3F80
    qw = O.pack_int4(q)
    g = host_bf16(K.int4_gemv(dev(qw), dev_bf16(sc), dev_bf16(x), act=1))
    # pre as the reference computes it: (q*s)*x summed, so an inf scale times
    # the zero weights of its group gives NaN, as in int4_gemv.cu:71-72
    pre = O.gemv_bf16(qw, sc, x)
    nonzero_finite = np.isfinite(O.bf16_to_f32(sc[:, 0])) & (O.bf16_to_f32(sc[:, 0]) != 0)
    assert np.array_equal(pre[nonzero_finite], sc[nonzero_finite, 0])
    want = O.silu_bf16(pre)
    fw, fg = O.bf16_to_f32(want), O.bf16_to_f32(g)
    both_nan = np.isnan(fw) & np.isnan(fg)
    same = (g == want) | both_nan
    d = ulp_diff(g[~same], want[~same])
    assert np.all(np.isnan(fg) == np.isnan(fw)), np.nonzero(np.isnan(fg) != np.isnan(fw))[0][:8]
    assert d.max(initial=0) <= 1 and (~same).sum() <= 64, int((~same).sum())


def test_quantize_kernel_bit_exact(K):
    """HIP quantizer vs the oracle restatement of scripts/quantize.py, fp32 and
    bf16 inputs, including a zero group and exact half-way ratios."""
    from quantize import quantize_tensor_int4_groupwise
    rng = np.random.default_rng(31)
    w = (rng.standard_normal((300, 1024)) * 0.02).astype(np.float32)
    w[5, :128] = 0.0
    w[6, :6] = [7.0, 2.5, -3.5, 0.5, 1.5, -7.0]
    w[6, 6:128] = 0.0
    qw, sc = quantize_tensor_int4_groupwise(torch.from_numpy(w).cuda())
    oq, osc = O.quantize_int4_groupwise(w)
    assert np.array_equal(qw.cpu().numpy(), oq) and np.array_equal(host_bf16(sc), osc)
    wb = torch.from_numpy(w).to(torch.bfloat16)
    qw, sc = quantize_tensor_int4_groupwise(wb.cuda())
    oq, osc = O.quantize_int4_groupwise(wb.float().numpy())
    assert np.array_equal(qw.cpu().numpy(), oq) and np.array_equal(host_bf16(sc), osc)


def test_transpose_down_kernel_bit_exact(K):
    rng = np.random.default_rng(32)
    down = (rng.standard_normal((512, 1536)) * 0.02).astype(np.float32)
    dq, ds = O.quantize_int4_groupwise(down)
    tq, ts = K.transpose_down_int4(dev(dq), dev_bf16(ds))
    oq, osc = O.transpose_down_to_int4(dq, ds)
    assert np.array_equal(tq.cpu().numpy(), oq) and np.array_equal(host_bf16(ts), osc)


def test_gather_gemv_reference_shape(K):
    """kernels/int4_gather/test_gather.py:29-55 shape: out=4096, in=5120,
    k = int(4096*0.6) sorted random rows."""
    rng = np.random.default_rng(0)
    qw, sc = random_int4(rng, 4096, 5120)
    x = random_bf16(rng, 5120)
    idx = np.sort(rng.permutation(4096)[: int(4096 * 0.6)]).astype(np.int32)
    out = host_bf16(K.int4_gather_gemv(dev(qw), dev_bf16(sc), dev_bf16(x), dev(idx)))
    ref = O.gemv_f64(qw, sc, x, rows=idx)
    assert rel_err(out, ref) < 1e-2
    assert_fp32_close(out, ref, gemv_abs_terms(qw, sc, x, rows=idx))


def test_up_gather_h_is_bf16_of_g_times_u(K):
    rng = np.random.default_rng(1)
    qw, sc = random_int4(rng, 2048, 4096)
    x = random_bf16(rng, 4096)
    g = random_bf16(rng, 2048, 0.5)
    idx = rng.permutation(2048)[:1229].astype(np.int32)
    qd, sd, xd, idd = dev(qw), dev_bf16(sc), dev_bf16(x), dev(idx)
    u = host_bf16(K.int4_gather_gemv(qd, sd, xd, idd))
    h = host_bf16(K.up_gather_h(qd, sd, xd, idd, dev_bf16(g)))
    assert np.array_equal(h, O.h_bf16(g[idx], u))


def test_gather_down_reference_shape(K):
    """kernels/int4_down/test_down.py:31-54 shape: k=15360 rows, out=5120."""
    rng = np.random.default_rng(2)
    k, out_f = 15360, 5120
    qw, sc = random_int4(rng, k, out_f)
    h = random_bf16(rng, k)
    y = host_bf16(K.int4_gather_down(dev(qw), dev_bf16(sc), dev_bf16(h)))
    ref = O.down_f64(qw, sc, h)
    assert rel_err(y, ref) < 1e-2
    assert_fp32_close(y, ref, down_abs_terms(qw, sc, h))


@pytest.mark.parametrize("rows,k,out_f", [(25600, 15360, 5120), (12288, 7373, 4096),
                                          (1024, 100, 2560), (300, 3, 128), (64, 64, 256),
                                          (40000, 33000, 384)])
def test_gather_down_indexed(K, rows, k, out_f):
    rng = np.random.default_rng(rows + k)
    qw, sc = random_int4(rng, rows, out_f)
    idx = rng.permutation(rows)[:k].astype(np.int32)
    h = random_bf16(rng, k)
    y = host_bf16(K.int4_gather_down(dev(qw), dev_bf16(sc), dev_bf16(h), dev(idx)))
    ref = O.down_f64(qw, sc, h, rows=idx)
    assert rel_err(y, ref) < 1e-2
    assert_fp32_close(y, ref, down_abs_terms(qw, sc, h, rows=idx))


def test_down_deterministic(K):
    rng = np.random.default_rng(3)
    qw, sc = random_int4(rng, 25600, 5120)
    idx = rng.permutation(25600)[:15360].astype(np.int32)
    h = random_bf16(rng, 15360)
    a = [host_bf16(K.int4_gather_down(dev(qw), dev_bf16(sc), dev_bf16(h), dev(idx)))
         for _ in range(3)]
    assert np.array_equal(a[0], a[1]) and np.array_equal(a[1], a[2])


@pytest.mark.parametrize("mode", [0, 1])
def test_dequant_rows_bit_exact(K, mode):
    rng = np.random.default_rng(4)
    q = rng.integers(-8, 8, size=(77, 384)).astype(np.int8)
    q[0, :16] = np.arange(-8, 8)
    sc = O.f32_to_bf16(rng.standard_normal((77, 3)).astype(np.float32))
    sc[1, 0] = 0x3F81   # 1.0078125: bf16(3 * s) is a rounding tie
    qw = O.pack_int4(q)
    idx = rng.permutation(77)[:50].astype(np.int32)
    out = K.dequant_rows(dev(qw), dev_bf16(sc), dev(idx), mode=mode)
    if mode == 0:
        assert np.array_equal(out.cpu().numpy(), O.dequant_f32(qw, sc)[idx])
    else:
        assert np.array_equal(host_bf16(out), O.dequantize(qw, sc)[idx])


def _topk_cases():
    rng = np.random.default_rng(20)
    cases = []
    for n, k in [(25600, 15360), (25600, 7680), (25600, 25600), (25600, 1), (12288, 7373),
                 (12288, 3686), (1000, 999), (65536, 30000), (5, 2), (1, 1), (7, 0)]:
        cases.append((random_bf16(rng, n, 0.7), k))
    # gate-like values: silu of a GEMV output, heavy ties at the boundary
    pre = O.f32_to_bf16((rng.standard_normal(25600) * 1.3).astype(np.float32))
    g = O.silu_bf16(pre)
    cases += [(g, 15360), (g, 7680), (g, 25599)]
    t = O.f32_to_bf16(rng.integers(-3, 4, size=4000).astype(np.float32))
    cases += [(t, 1500), (t, 2999), (np.zeros(300, np.uint16), 10)]
    sp = random_bf16(rng, 1000)
    sp[::7] = 0x7FC0
    sp[3] = 0x7F80
    sp[5] = 0xFF80
    sp[11::13] = 0x0001
    sp[12::17] = 0x8000
    cases += [(sp, 50), (sp, 900), (sp, 999)]
    big = np.full(64, 0x7F7F, np.uint16)
    big[::2] = 0x7F70
    tiny = np.full(64, 0x0090, np.uint16)
    tiny[::3] = 0x0100
    cases += [(big, 20), (tiny, 10), (tiny, 30)]
    # magnitudes spread over every bf16 exponent (zero to +inf, either sign):
    # the select's scan then gives each thread 32 bins and the rank walks
    # across many of them
    wide = (rng.integers(0, 0x7F81, size=25600) | (rng.integers(0, 2, size=25600) << 15))
    wide = wide.astype(np.uint16)
    cases += [(wide, 1), (wide, 700), (wide, 12800), (wide, 25000)]
    return cases


def test_topk_bit_exact(K):
    for i, (s, k) in enumerate(_topk_cases()):
        print(f"topk case {i} n={s.size} k={k}", flush=True)
        got = K.topk_select(dev_bf16(s), k).cpu().numpy()
        want = O.topk_select(s, k)
        assert np.array_equal(got, want), (i, s.size, k)
        meta = K.topk_meta()
        lo, hi = O.topk_bisect(s, k)
        if k > 0:
            assert np.float32(meta["t_lo"]) == lo and np.float32(meta["t_strict"]) == hi, i


def test_topk_repeatable(K):
    rng = np.random.default_rng(21)
    s = dev_bf16(O.silu_bf16(random_bf16(rng, 25600, 1.3)))
    a = [K.topk_select(s, 15360).cpu() for _ in range(5)]
    assert all(torch.equal(a[0], b) for b in a[1:])


def test_gate_silu_topk_fused_matches_unfused(K):
    rng = np.random.default_rng(22)
    qw, sc = random_int4(rng, 25600, 5120)
    x = random_bf16(rng, 5120)
    qd, sd, xd = dev(qw), dev_bf16(sc), dev_bf16(x)
    for k in (15360, 7680, 0, 25600):
        g, idx = K.gate_silu_topk(qd, sd, xd, k)
        g2 = K.int4_gemv(qd, sd, xd, act=1)
        assert torch.equal(g, g2)
        assert np.array_equal(idx.cpu().numpy(), O.topk_select(host_bf16(g), k))


def test_gate_silu_topk_across_shapes(K):
    """The fused gate + top-k and the standalone top-k, alternating on one
    workspace over shapes whose select grids have 1 to 13 workgroups."""
    rng = np.random.default_rng(24)
    layers = []
    for rows, cols in ((25600, 5120), (3072, 1024), (12288, 4096), (100 * 128, 128)):
        qw, sc = random_int4(rng, rows, cols)
        layers.append((dev(qw), dev_bf16(sc), dev_bf16(random_bf16(rng, cols))))
    for rep in range(2):
        for i, (qd, sd, xd) in enumerate(layers):
            rows = qd.shape[0]
            for k in (rows * 3 // 5, 1, rows):
                print(f"rep {rep} layer {i} rows={rows} k={k}", flush=True)
                g, idx = K.gate_silu_topk(qd, sd, xd, k)
                want = O.topk_select(host_bf16(g), k)
                assert np.array_equal(idx.cpu().numpy(), want), (rep, i, k)
                s = dev_bf16(random_bf16(rng, rows))
                got = K.topk_select(s, k).cpu().numpy()
                assert np.array_equal(got, O.topk_select(host_bf16(s), k)), (rep, i, k)


def test_ca_assemble(K):
    rng = np.random.default_rng(23)
    inter, k, cache_n = 25600, 15360, 7680
    hot = np.sort(rng.choice(inter, cache_n, replace=False))
    id2slot = np.full(inter, -1, np.int64)
    id2slot[hot] = np.arange(cache_n)
    idx = O.topk_select(random_bf16(rng, inter), k)
    comb, src, row, miss, counts = K.ca_assemble(dev(id2slot), dev(idx))
    c2, s2, r2, n_hit, m2 = O.ca_split(idx, id2slot)
    assert counts.cpu().tolist() == [n_hit, k - n_hit]
    assert np.array_equal(comb.cpu().numpy(), c2)
    assert np.array_equal(src.cpu().numpy(), s2)
    assert np.array_equal(row.cpu().numpy(), r2)
    assert np.array_equal(miss.cpu().numpy()[: k - n_hit], m2)


def test_ca_fused_gemv_reference_shape(K):
    """kernels/ca_fused/test_ca_fused.py:27-79: in=5120, k=15360,
    cache_n=7680, n_hit=5855."""
    rng = np.random.default_rng(24)
    in_f, k, cache_n, n_hit = 5120, 15360, 7680, 5855
    q_full = rng.integers(-8, 8, size=(k, in_f)).astype(np.int8)
    sc_full = O.f32_to_bf16(rng.random((k, in_f // 128), dtype=np.float32) * 0.01 + 0.001)
    x = random_bf16(rng, in_f)
    res_q = np.zeros((cache_n, in_f), np.int8)
    res_q[:n_hit] = q_full[:n_hit]
    res_s = np.zeros((cache_n, in_f // 128), np.uint16)
    res_s[:n_hit] = sc_full[:n_hit]
    str_q = np.zeros((k, in_f), np.int8)
    str_q[: k - n_hit] = q_full[n_hit:]
    str_s = np.zeros((k, in_f // 128), np.uint16)
    str_s[: k - n_hit] = sc_full[n_hit:]
    src = np.r_[np.zeros(n_hit), np.ones(k - n_hit)].astype(np.int32)
    row = np.r_[np.arange(n_hit), np.arange(k - n_hit)].astype(np.int32)
    out = host_bf16(K.ca_fused_gemv(dev(O.pack_int4(res_q)), dev_bf16(res_s),
                                    dev(O.pack_int4(str_q)), dev_bf16(str_s), dev_bf16(x),
                                    dev(src), dev(row)))
    ref = O.gemv_f64(O.pack_int4(q_full), sc_full, x)
    assert rel_err(out, ref) < 1e-2
    assert_fp32_close(out, ref, gemv_abs_terms(O.pack_int4(q_full), sc_full, x))


def test_ca_down_matches_gather_down(K):
    rng = np.random.default_rng(25)
    inter, out_f, k = 4096, 2048, 2458
    qw, sc = random_int4(rng, inter, out_f)
    idx = rng.permutation(inter)[:k].astype(np.int32)
    hot = np.sort(rng.choice(inter, 1200, replace=False))
    id2slot = np.full(inter, -1, np.int64)
    id2slot[hot] = np.arange(1200)
    comb, src, row, n_hit, miss = O.ca_split(idx, id2slot)
    h = random_bf16(rng, k)
    y = host_bf16(K.ca_down(dev(qw[hot]), dev_bf16(sc[hot]), dev(qw[miss]), dev_bf16(sc[miss]),
                            dev_bf16(h), dev(src), dev(row)))
    ref = O.down_f64(qw, sc, h, rows=comb)
    assert rel_err(y, ref) < 1e-2
    assert_fp32_close(y, ref, down_abs_terms(qw, sc, h, rows=comb))


def test_bad_row_ids_poison_instead_of_faulting(K):
    rng = np.random.default_rng(26)
    qw, sc = random_int4(rng, 64, 256)
    x = random_bf16(rng, 256)
    idx = np.array([3, 64, 5, -1], np.int32)   # 64 and -1 are out of range
    out = host_bf16(K.int4_gather_gemv(dev(qw), dev_bf16(sc), dev_bf16(x), dev(idx)))
    assert out[1] == 0x7FC0 and out[3] == 0x7FC0
    assert out[0] != 0x7FC0 and out[2] != 0x7FC0
    # cache-aware fused h: channel ids outside g poison h instead of reading past g
    g = random_bf16(rng, 40)
    src = np.zeros(4, np.int32)
    row = np.array([1, 2, 3, 4], np.int32)
    gid = np.array([0, 40, 39, -5], np.int32)   # 40 and -5 are outside g
    h = host_bf16(K.ca_fused_gemv(dev(qw), dev_bf16(sc), dev(qw), dev_bf16(sc), dev_bf16(x),
                                  dev(src), dev(row), g=dev_bf16(g), gid=dev(gid)))
    assert h[1] == 0x7FC0 and h[3] == 0x7FC0
    assert h[0] != 0x7FC0 and h[2] != 0x7FC0


def test_gather_down_by_channel(K):
    """dip_int4_gather_down_by_channel: h indexed by channel (the decode
    step's form), h_out[j] = h_full[idx[j]], y against the fp64 sum."""
    rng = np.random.default_rng(28)
    rows, k, out_f = 12288, 7373, 4096
    qw, sc = random_int4(rng, rows, out_f)
    idx = np.sort(rng.permutation(rows)[:k]).astype(np.int32)
    h_full = random_bf16(rng, rows)
    h_out = torch.empty(k, dtype=torch.bfloat16, device="cuda")
    y = host_bf16(K.int4_gather_down_by_channel(dev(qw), dev_bf16(sc), dev_bf16(h_full), dev(idx),
                                                h_out=h_out))
    assert np.array_equal(host_bf16(h_out), h_full[idx])
    ref = O.down_f64(qw, sc, h_full[idx], rows=idx)
    assert rel_err(y, ref) < 1e-2
    assert_fp32_close(y, ref, down_abs_terms(qw, sc, h_full[idx], rows=idx))
