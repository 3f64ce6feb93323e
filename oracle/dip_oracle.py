"""CPU oracle for the DIP decode MLP path — TEST INFRASTRUCTURE ONLY.

This module restates, on the CPU, what the reference computes on its decode
path (int4 g128 format, gate GEMV + SiLU, the threshold top-k, the up-row
gather GEMV, h = g[idx] * u, the transposed-down gather, and the cache-aware
hit/miss split).  It exists so that tests, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` can check / time the HIP product path
against it.  Nothing in the product path may import it: the product raises if
its HIP library is missing instead of falling back here.

Representation: bf16 tensors are carried as ``numpy.uint16`` bit patterns so
that every rounding step is explicit; fp32 math uses ``numpy.float32``.  The
only third-party arithmetic the reference itself delegates to is torch's
``F.silu`` on a bf16 tensor (dip_stream_predispatch.py:182); ``silu_bf16``
calls exactly that op on the CPU, and ``silu_bf16_np`` restates it in numpy
so the two can pin each other.

Every function cites the reference file:line it follows.  Parity pinning:
every public function is checked in tests/test_oracle.py against
known-answer vectors, closed forms, invariants, brute force or an
independent second route (the PyTorch restatement of qlinear.py against the
numpy one, the C top-k against the numpy top-k); the test docstrings say
which.  No function is left parity unpinned.
"""
from __future__ import annotations

import numpy as np

GROUP_SIZE = 128          # qlinear.py:25, scripts/quantize.py:28
QMAX = 7                  # scripts/quantize.py:29
BISECT_STEPS = 25         # kernels/topk_select/topk_select.cu:150


# ---------------------------------------------------------------------------
# bf16 <-> fp32 (torch / c10 semantics: round-to-nearest-even, NaN -> 0x7FC0)
# ---------------------------------------------------------------------------
def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns -> float32 (exact widening)."""
    b = np.asarray(bits, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(a) -> np.ndarray:
    """float32 -> bf16 bits, round-to-nearest-even, NaN -> 0x7FC0.

    Same rule as c10::BFloat16's round_to_nearest_even, i.e. what
    ``tensor.to(torch.bfloat16)`` and ``__float2bfloat16_rn`` do
    (qlinear.py:64, int4_gemv.cu:85)."""
    f = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    u = f.view(np.uint32).astype(np.uint64)
    r = ((u + (((u >> 16) & 1) + 0x7FFF)) >> 16).astype(np.uint16)
    nan = np.isnan(f)
    if nan.any():
        r = r.copy()
        r[nan] = 0x7FC0
    return r


# ---------------------------------------------------------------------------
# int4 g128 format  (qlinear.py:25-64, scripts/quantize.py:32-64,
#                    dip_stream_predispatch.py:77-120)
# ---------------------------------------------------------------------------
def unpack_int4(qweight: np.ndarray) -> np.ndarray:
    """int8 [R, C/2] -> int8 [R, C]; low nibble = even column, high = odd,
    each sign-extended from 4 bits (qlinear.py:28-50)."""
    q = np.asarray(qweight).view(np.uint8)
    lo = (q & 0x0F).astype(np.int8)
    hi = ((q >> 4) & 0x0F).astype(np.int8)
    lo = np.where(lo >= 8, lo - 16, lo).astype(np.int8)
    hi = np.where(hi >= 8, hi - 16, hi).astype(np.int8)
    out = np.empty((q.shape[0], q.shape[1] * 2), dtype=np.int8)
    out[:, 0::2] = lo
    out[:, 1::2] = hi
    return out


def pack_int4(q: np.ndarray) -> np.ndarray:
    """int8 [R, C] in [-8, 7] -> packed int8 [R, C/2]
    (dip_stream_predispatch.py:93-97, scripts/quantize.py:57-61)."""
    q = np.asarray(q, dtype=np.int8)
    lo = (q[:, 0::2].view(np.uint8) & 0x0F)
    hi = (q[:, 1::2].view(np.uint8) & 0x0F)
    return (lo | (hi << 4)).astype(np.uint8).view(np.int8)


def dequant_f32(qweight: np.ndarray, scales_bits: np.ndarray) -> np.ndarray:
    """Exact fp32 value q * s the CUDA kernels multiply with
    (int4_gemv.cu:71-72: ``(lo * s_even)`` in fp32)."""
    q = unpack_int4(qweight).astype(np.float32)
    R, C = q.shape
    s = bf16_to_f32(scales_bits).reshape(R, C // GROUP_SIZE, 1)
    return (q.reshape(R, C // GROUP_SIZE, GROUP_SIZE) * s).reshape(R, C)


def dequantize(qweight: np.ndarray, scales_bits: np.ndarray) -> np.ndarray:
    """qlinear.dequantize: bf16 bits of q*s (qlinear.py:53-64)."""
    return f32_to_bf16(dequant_f32(qweight, scales_bits))


def quantize_int4_groupwise(w: np.ndarray):
    """scripts/quantize.py:32-64.  w: float [out, in] -> (packed int8
    [out, in/2], scales bf16 bits [out, in/128]).

    s = clamp(max|w_g| / 7, min=1e-8) in fp32; q = clamp(round_half_even(w / s),
    -8, 7) computed with the fp32 s; the stored scale is bf16(s) afterwards."""
    w = np.asarray(w, dtype=np.float32)
    out_f, in_f = w.shape
    assert in_f % GROUP_SIZE == 0 and in_f % 2 == 0
    wg = w.reshape(out_f, in_f // GROUP_SIZE, GROUP_SIZE)
    max_abs = np.abs(wg).max(axis=2, keepdims=True)
    s = np.maximum(max_abs / np.float32(QMAX), np.float32(1e-8)).astype(np.float32)
    q = np.clip(np.rint(wg / s), -8, 7).astype(np.int8).reshape(out_f, in_f)
    return pack_int4(q), f32_to_bf16(s[..., 0])


def transpose_down_to_int4(down_qw: np.ndarray, down_sc: np.ndarray):
    """dip_stream_predispatch.py:100-120: down [out, inter] int4 ->
    bf16 dequant -> transpose -> fp32 -> re-quantize g128 along `out`.
    Returns (down_t_qw int8 [inter, out/2], down_t_sc bf16 bits [inter, out/128])."""
    wt = bf16_to_f32(dequantize(down_qw, down_sc)).T.copy()
    return quantize_int4_groupwise(wt)


# ---------------------------------------------------------------------------
# GEMV pieces (int4_gemv.cu:39-87, int4_gather_gemv.cu:39-85,
#              int4_gather_down.cu:41-75, ca_fused_gemv.cu:44-85)
# ---------------------------------------------------------------------------
def gemv_f64(qweight, scales_bits, x_bits, rows=None) -> np.ndarray:
    """sum_c (q*s)[r, c] * x[c] for rows `rows` (all rows if None), with the
    exact fp32 products summed in float64.  The reference sums the same
    products in fp32 in a block-reduction order; that order is not part of
    the contract, so callers compare with a tolerance."""
    if rows is not None:
        qweight = np.asarray(qweight)[rows]
        scales_bits = np.asarray(scales_bits)[rows]
    w = dequant_f32(qweight, scales_bits).astype(np.float64)
    return w @ bf16_to_f32(x_bits).astype(np.float64)


def gemv_bf16(qweight, scales_bits, x_bits, rows=None) -> np.ndarray:
    """out = bf16_rn(dot) (int4_gemv.cu:85, int4_gather_gemv.cu:83)."""
    return f32_to_bf16(gemv_f64(qweight, scales_bits, x_bits, rows).astype(np.float32))


def silu_bf16_np(pre_bits: np.ndarray) -> np.ndarray:
    """bf16(silu(float(pre))) with silu(v) = v / (1 + exp(-v)) in fp32 —
    the op-math torch applies for ``F.silu`` on a bf16 tensor
    (dip_stream_predispatch.py:182)."""
    v = bf16_to_f32(pre_bits)
    with np.errstate(over="ignore", invalid="ignore"):
        s = (v / (np.float32(1.0) + np.exp(-v, dtype=np.float32))).astype(np.float32)
    return f32_to_bf16(s)


def silu_bf16(pre_bits: np.ndarray) -> np.ndarray:
    """torch.nn.functional.silu on a CPU bf16 tensor (the library call the
    reference makes at dip_stream_predispatch.py:182 / dip_ca.py:133)."""
    import torch
    import torch.nn.functional as F
    t = torch.from_numpy(np.ascontiguousarray(pre_bits, dtype=np.uint16).view(np.int16))
    out = F.silu(t.view(torch.bfloat16))
    return out.view(torch.int16).numpy().view(np.uint16).copy()


def h_bf16(g_bits: np.ndarray, u_bits: np.ndarray) -> np.ndarray:
    """h = bf16(float(g) * float(u)) (dip_stream_predispatch.py:201:
    ``(g[idx] * up_sel.to(xdt)).to(torch.bfloat16)``).  The fp32 product of
    two bf16 values is exact, so only the final rounding matters."""
    return f32_to_bf16(bf16_to_f32(g_bits) * bf16_to_f32(u_bits))


def down_f64(down_t_qw, down_t_sc, h_bits, rows=None) -> np.ndarray:
    """y[o] = sum_j h[j] * (q*s)[row_j, o] in float64
    (int4_gather_down.cu:56-62; rows = 0..k-1 of the staged copy there)."""
    if rows is not None:
        down_t_qw = np.asarray(down_t_qw)[rows]
        down_t_sc = np.asarray(down_t_sc)[rows]
    w = dequant_f32(down_t_qw, down_t_sc).astype(np.float64)
    return bf16_to_f32(h_bits).astype(np.float64) @ w


# ---------------------------------------------------------------------------
# top-k  (kernels/topk_select/topk_select.cu:30-164, topk_kernel.py:29-40)
# ---------------------------------------------------------------------------
def _flushed_abs(s_bits: np.ndarray) -> np.ndarray:
    """|s| as the reference kernels see it: ``fabsf(__bfloat162float(s))``
    compiled with --use_fast_math (kernels/topk_select/setup_topk.py), so a
    bf16 subnormal magnitude flushes to +0.  NaN stays NaN."""
    a = np.asarray(s_bits, dtype=np.uint16) & np.uint16(0x7FFF)
    a = np.where(a < 0x0080, np.uint16(0), a).astype(np.uint16)
    return bf16_to_f32(a)


def topk_bisect(s_bits: np.ndarray, k: int):
    """The host bisection of topk_select_impl (topk_select.cu:141-158).

    hi = max|s| (max_abs_kernel, NaN ignored by fmaxf, floor 0), lo = 0,
    t = 0.5f*(lo+hi); 25 times: c = #{|s| > t}; c > k ? lo = t : hi = t;
    t = 0.5f*(lo+hi).  All arithmetic in fp32.  Returns (t_lo, t_strict)."""
    v = _flushed_abs(s_bits)
    valid = v[~np.isnan(v)]
    hi = np.float32(valid.max()) if valid.size else np.float32(0.0)
    hi = max(hi, np.float32(0.0))
    lo = np.float32(0.0)
    half = np.float32(0.5)
    with np.errstate(over="ignore"):
        t = np.float32(half * np.float32(lo + hi))
        for _ in range(BISECT_STEPS):
            c = int(np.count_nonzero(valid > t))
            if c > k:
                lo = t
            else:
                hi = t
            t = np.float32(half * np.float32(lo + hi))
    return np.float32(lo), np.float32(hi)


def topk_select(s_bits: np.ndarray, k: int) -> np.ndarray:
    """int32 [k] exactly as topk_ops::topk_select returns it
    (topk_select.cu:134-164): tier A = {|s| > t_strict} in ascending index,
    then tier B = {t_lo < |s| <= t_strict} in ascending index until k are
    emitted (parallel_compact_kernel, :64-132); unfilled slots stay 0
    (torch::zeros at :160)."""
    s_bits = np.asarray(s_bits, dtype=np.uint16).reshape(-1)
    t_lo, t_strict = topk_bisect(s_bits, k)
    v = _flushed_abs(s_bits)
    with np.errstate(invalid="ignore"):
        tier_a = np.nonzero(v > t_strict)[0]
        tier_b = np.nonzero((v > t_lo) & (v <= t_strict))[0]
    out = np.zeros(k, dtype=np.int32)
    sel = np.concatenate([tier_a, tier_b])[:k]
    out[: sel.size] = sel
    return out


def topk_key_order(s_bits: np.ndarray, k: int) -> np.ndarray:
    """Closed form the bisection converges to on ordinary data: the k
    channels with the largest |s|, ties broken by lower channel id, emitted
    as ascending ids of {|s| > a_k} followed by the lowest ids of {|s| == a_k}
    (a_k = k-th largest).  Valid when the final bisection band holds a single
    distinct value; used to pin topk_select."""
    s_bits = np.asarray(s_bits, dtype=np.uint16).reshape(-1)
    v = _flushed_abs(s_bits)
    order = np.lexsort((np.arange(v.size), -v))   # |s| desc, id asc
    chosen = order[:k]
    a_k = v[chosen[-1]]
    if np.count_nonzero(v >= a_k) == k:            # no tie across the boundary
        return np.sort(chosen).astype(np.int32)
    gt = np.sort(chosen[v[chosen] > a_k])
    eq = np.sort(chosen[v[chosen] == a_k])
    return np.concatenate([gt, eq]).astype(np.int32)


# ---------------------------------------------------------------------------
# Module-level forwards (dip_stream_predispatch.py:176-215, dip_ca.py:127-196)
# ---------------------------------------------------------------------------
def keep_count(inter: int, keep_ratio: float) -> int:
    """k = max(1, int(round(I * keep))) (dip_stream_predispatch.py:248;
    Python round() is half-to-even)."""
    return max(1, int(round(inter * keep_ratio)))


def dip_forward(gate_qw, gate_sc, up_qw, up_sc, down_t_qw, down_t_sc, x_bits, k,
                idx=None):
    """StreamingDIPMlp.forward decode path (dip_stream_predispatch.py:176-204).

    Returns dict with pre, g (bf16 bits), idx (int32), u, h (bf16 bits) and
    y_f64 (float64, before the final bf16 rounding) and y (bf16 bits).
    `idx` may be supplied to evaluate the tail for a given selection (tests
    pass the device's idx so the comparison isolates each stage)."""
    pre = gemv_bf16(gate_qw, gate_sc, x_bits)
    g = silu_bf16(pre)
    if idx is None:
        idx = topk_select(g, k)
    idx = np.asarray(idx, dtype=np.int64)
    u = gemv_bf16(up_qw, up_sc, x_bits, rows=idx)
    h = h_bf16(g[idx], u)
    y64 = down_f64(down_t_qw, down_t_sc, h, rows=idx)
    return dict(pre=pre, g=g, idx=idx.astype(np.int32), u=u, h=h, y_f64=y64,
                y=f32_to_bf16(y64.astype(np.float32)))


def dense_forward(gate_qw, gate_sc, up_qw, up_sc, down_t_qw, down_t_sc, x_bits):
    """The DIP computation over every channel in channel order: dip_forward
    with k = I and idx = 0..I-1, i.e. the kernels' exact fp32 q*s weights for
    up and down.  This is NOT the reference's keep >= 0.999 route, which
    multiplies by bf16-rounded weights (dense_literal_forward)."""
    inter = np.asarray(up_qw).shape[0]
    return dip_forward(gate_qw, gate_sc, up_qw, up_sc, down_t_qw, down_t_sc, x_bits,
                       inter, idx=np.arange(inter, dtype=np.int32))


def dense_literal_forward(gate_qw, gate_sc, up_qw, up_sc, down_t_qw, down_t_sc, x_bits):
    """StreamingDIPMlp._dense for one decode token, literally
    (dip_stream_predispatch.py:177-179 route keep >= 0.999 here; :206-215):

      g    = silu(_gate(x))            _gate takes the int4 GEMV kernel for a
                                       decode token (:166-171): exact q*s
      up_w = dequantize(up)            bf16(q*s) (qlinear.py:53-64)
      u    = bf16(F.linear(x, up_w))   fp32 sum of x * bf16(q*s)
      h    = bf16(g * u)
      dn_t = dequantize(down_t)        bf16(q*s)
      y    = bf16(h @ dn_t)            fp32 sum of h * bf16(q*s)

    Sums are taken in float64 (the library GEMMs' fp32 summation order is
    not part of the contract).  Returns the dict of dip_forward (idx = all
    channels)."""
    inter = np.asarray(up_qw).shape[0]
    pre = gemv_bf16(gate_qw, gate_sc, x_bits)
    g = silu_bf16(pre)
    xf = bf16_to_f32(x_bits).astype(np.float64)
    up_w = bf16_to_f32(dequantize(up_qw, up_sc)).astype(np.float64)
    u = f32_to_bf16((up_w @ xf).astype(np.float32))
    h = h_bf16(g, u)
    dn_w = bf16_to_f32(dequantize(down_t_qw, down_t_sc)).astype(np.float64)
    y64 = bf16_to_f32(h).astype(np.float64) @ dn_w
    return dict(pre=pre, g=g, idx=np.arange(inter, dtype=np.int32), u=u, h=h, y_f64=y64,
                y=f32_to_bf16(y64.astype(np.float32)))


def ca_split(idx: np.ndarray, id2slot: np.ndarray):
    """CADIPMlp.forward hit/miss assembly (dip_ca.py:137-171).

    Returns (combined_ids, src, row, n_hit, miss_ids): order [hits..., misses...]
    with each part in idx order; src 0 = resident hit, 1 = streamed miss;
    row = resident slot for hits and 0..n_miss-1 for misses."""
    idx = np.asarray(idx, dtype=np.int64)
    slots = np.asarray(id2slot, dtype=np.int64)[idx]
    hit = slots >= 0
    hit_ids, miss_ids = idx[hit], idx[~hit]
    n_hit, n_miss = hit_ids.size, miss_ids.size
    combined = np.concatenate([hit_ids, miss_ids])
    src = np.concatenate([np.zeros(n_hit, np.int32), np.ones(n_miss, np.int32)])
    row = np.concatenate([slots[hit].astype(np.int32), np.arange(n_miss, dtype=np.int32)])
    return combined, src, row, n_hit, miss_ids


def hot_set(counts: np.ndarray, cache_n: int):
    """calibrate_cache + set_cache (dip_ca.py:305-308, 107-113): order channels
    by key = cnt*I - id descending (frequency desc, id asc), keep the first
    cache_n, sort them ascending; id2slot[hot[s]] = s, -1 elsewhere.
    Returns (hot_ids int64 ascending, id2slot int64 [I])."""
    cnt = np.asarray(counts, dtype=np.int64)
    inter = cnt.size
    key = cnt * inter - np.arange(inter, dtype=np.int64)
    order = np.argsort(-key, kind="stable")
    hot = np.sort(order[:cache_n])
    id2slot = np.full(inter, -1, dtype=np.int64)
    id2slot[hot] = np.arange(hot.size)
    return hot, id2slot


def ca_forward(gate_qw, gate_sc, up_qw, up_sc, down_t_qw, down_t_sc, id2slot, x_bits,
               k, idx=None):
    """CADIPMlp.forward (dip_ca.py:127-188).  Mathematically the same rows as
    dip_forward but summed in [hits..., misses...] order; returns the same
    dict plus the split."""
    pre = gemv_bf16(gate_qw, gate_sc, x_bits)
    g = silu_bf16(pre)
    if idx is None:
        idx = topk_select(g, k)
    combined, src, row, n_hit, miss_ids = ca_split(idx, id2slot)
    u = gemv_bf16(up_qw, up_sc, x_bits, rows=combined)
    h = h_bf16(g[combined], u)
    y64 = down_f64(down_t_qw, down_t_sc, h, rows=combined)
    return dict(pre=pre, g=g, idx=np.asarray(idx, np.int32), combined=combined,
                src=src, row=row, n_hit=n_hit, miss_ids=miss_ids, u=u, h=h,
                y_f64=y64, y=f32_to_bf16(y64.astype(np.float32)))


# ---------------------------------------------------------------------------
# Synthetic layers (N(0, 0.02) weights, int4 g128)
# ---------------------------------------------------------------------------
def make_layer(hidden: int, inter: int, seed: int):
    """Draw gate/up [I, H] and down [H, I] ~ N(0, 0.02) with torch's CPU
    generator seeded `seed`, quantize per scripts/quantize.py:32-64 and
    transpose down per dip_stream_predispatch.py:100-120.  Returns numpy
    arrays (int8 packed / uint16 bf16 bits)."""
    import torch
    gen = torch.Generator().manual_seed(seed)
    gate = (torch.randn(inter, hidden, generator=gen) * 0.02).numpy()
    up = (torch.randn(inter, hidden, generator=gen) * 0.02).numpy()
    down = (torch.randn(hidden, inter, generator=gen) * 0.02).numpy()
    gq, gs = quantize_int4_groupwise(gate)
    uq, us = quantize_int4_groupwise(up)
    dq, ds = quantize_int4_groupwise(down)
    dtq, dts = transpose_down_to_int4(dq, ds)
    return dict(gate_qw=gq, gate_sc=gs, up_qw=uq, up_sc=us, down_qw=dq, down_sc=ds,
                down_t_qw=dtq, down_t_sc=dts)


def make_x(hidden: int, seed: int) -> np.ndarray:
    """x ~ N(0, 1) drawn in fp32 then cast to bf16 (bits)."""
    import torch
    gen = torch.Generator().manual_seed(seed)
    return f32_to_bf16(torch.randn(hidden, generator=gen).numpy())


# ---------------------------------------------------------------------------
# The reference's forward run literally with PyTorch CPU ops (cpu_baseline leg
# of bench.py): dequantize per call as QuantLinear / _dense do
# (qlinear.py:86-88), F.linear, F.silu, the top-k, index_select of the
# selected rows, dequantize, h and the down matmul
# (dip_stream_predispatch.py:176-204).
# ---------------------------------------------------------------------------
def torch_unpack_int4(qweight):
    """qlinear.py:28-50 with torch ops."""
    import torch
    q = qweight.view(torch.uint8)
    low = (q & 0x0F).to(torch.int8)
    high = ((q >> 4) & 0x0F).to(torch.int8)
    low = torch.where(low >= 8, low - 16, low)
    high = torch.where(high >= 8, high - 16, high)
    return torch.stack((low, high), dim=-1).reshape(q.shape[0], q.shape[1] * 2)


def torch_dequantize(qweight, scales):
    """qlinear.py:53-64 with torch ops."""
    import torch
    q = torch_unpack_int4(qweight)
    out_f, in_f = q.shape
    qf = q.float().reshape(out_f, in_f // GROUP_SIZE, GROUP_SIZE)
    s = scales.float().reshape(out_f, in_f // GROUP_SIZE, 1)
    return (qf * s).reshape(out_f, in_f).to(torch.bfloat16)


def torch_cpu_forward(gate_qw, gate_sc, up_qw, up_sc, down_t_qw, down_t_sc, x, k,
                      return_all=False):
    """One DIP decode step on host torch tensors (bf16 x [H]); returns y bf16
    [1, H], or with return_all the dict (g, idx, u, h, y) of torch tensors.

    The gate runs through dequantize + F.linear as QuantLinear.forward does
    (qlinear.py:86-88), so its weights are bf16(q*s) where the reference's
    decode gate kernel uses the exact q*s (int4_gemv.cu:71-72); g may
    therefore differ from the kernel route's by a rounding, and the top-k is
    taken on this route's own g."""
    import torch
    import torch.nn.functional as F
    xb = x.reshape(1, -1)
    g = F.silu(F.linear(xb, torch_dequantize(gate_qw, gate_sc))).reshape(-1)
    g_bits = g.view(torch.int16).numpy().view(np.uint16)
    idx = torch.from_numpy(topk_select(g_bits, k).astype(np.int64))
    up_w = torch_dequantize(torch.index_select(up_qw, 0, idx), torch.index_select(up_sc, 0, idx))
    u = F.linear(xb, up_w).reshape(-1)
    h = (g[idx] * u).to(torch.bfloat16)
    dn = torch_dequantize(torch.index_select(down_t_qw, 0, idx),
                          torch.index_select(down_t_sc, 0, idx))
    y = h.reshape(1, -1) @ dn
    if return_all:
        return dict(g=g, idx=idx, u=u, h=h, y=y.reshape(-1))
    return y
