// dip_tiles.h — device building blocks shared by the row-dot kernels (gate,
// up, the speculative up rows of the top-k launch) and the down kernel.
//
// Row dot (one output per weight row, reduced across the row):
//   LPR lanes ("a row group") own one row at a time; lane l of the group owns
//   chunks l, l+LPR, ..., l+(CH-1)*LPR of the row (16 bytes = 32 columns
//   each), so every load instruction covers LPR*16 contiguous bytes of the
//   row.  x is pre-paired for v_dot2_f32_bf16 with a per-chunk bias term (see
//   dip_common.h); a workgroup stages the pairs of all chunks in LDS once and
//   each lane then copies its own CH chunks into VGPRs.
//
// Down (outputs along the row, reduced across rows):
//   LPR lanes ("a slot") each own one 16-byte chunk (32 outputs) of every row
//   the slot walks; a block of 256 threads holds 256/LPR slots that walk the
//   LPR rows j = j0 + slot + i*(256/LPR).  Lane l of a slot resolves the id,
//   h and scales of the slot's row l; the slot's ids and coefficients reach
//   its lanes through a per-wave LDS exchange.  All LPR rows of a slot are
//   loaded before any is consumed.
#pragma once

#include "dip_common.h"
#include "dip_internal.h"

namespace dip {

constexpr uint32_t kBadRow = 0xFFFFFFFFu;  // out-of-range id: the output becomes NaN
constexpr uint32_t kPadRow = 0xFFFFFFFEu;  // down position past k: contributes 0
constexpr uint32_t kSrcB = 0x80000000u;    // dual-source row id: bit 31 selects matrix B

// ---------------------------------------------------------------------------
// Row dot
// ---------------------------------------------------------------------------

// Row id for output j (j < nrows): bit 31 selects matrix B (kDual); kBadRow
// if the id is out of range.  Branch-free (the id loads are unconditional).
template <int SRC>
DIP_DEV uint32_t resolve_row(const RowdotArgs& a, int j) {
  if (SRC == kContig) return (uint32_t)j;
  if (SRC == kGather) {
    const int r = a.sel[j];
    return (unsigned)r < (unsigned)a.rows_a ? (uint32_t)r : kBadRow;
  }
  const int r = a.sel2[j];
  const bool b = a.sel[j] != 0;
  const bool ok = b ? (unsigned)r < (unsigned)a.rows_b : (unsigned)r < (unsigned)a.rows_a;
  return ok ? ((uint32_t)r | (b ? kSrcB : 0u)) : kBadRow;
}

template <int CH>
struct RowRegs {
  uint4 w[CH];
  uint32_t s[CH];
};

// Unconditional loads of CH chunks (lane l owns chunks l + LPR*c) and their
// scales of row r of one matrix.
template <int LPR, int CH>
DIP_DEV void load_row_at(const int8_t* qw, const uint16_t* sc, uint32_t r, int l,
                         size_t row_bytes, int ngroups, RowRegs<CH>& R) {
  const uint4* wr = reinterpret_cast<const uint4*>(qw + (size_t)r * row_bytes);
  const uint16_t* sr = sc + (size_t)r * ngroups;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int chunk = l + LPR * c;
    R.w[c] = ldg_nt(wr + chunk);
    R.s[c] = sr[chunk / kChunksPerGroup];
  }
}

// The same for a resolved row id (a bad id reads row 0 of the safe matrix).
template <int LPR, int CH, int SRC>
DIP_DEV void load_row(const RowdotArgs& a, uint32_t rid, int l, size_t row_bytes, int ngroups,
                      RowRegs<CH>& R) {
  const bool bad = rid == kBadRow;
  const bool isb = SRC == kDual && !bad && (rid & kSrcB);
  const int8_t* qw = bad ? a.qw_safe : (isb ? a.qw_b : a.qw_a);
  const uint16_t* sc = bad ? a.sc_safe : (isb ? a.sc_b : a.sc_a);
  load_row_at<LPR, CH>(qw, sc, bad ? 0u : (rid & ~kSrcB), l, row_bytes, ngroups, R);
}

// x pairs + bias for one chunk (32 columns starting at 32*chunk), from the
// four 128-bit words of x that cover it.
DIP_DEV void pairs_of(const uint4 X[4], uint32_t xp[4][4], float& bias) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    make_xpairs(X[i].x, X[i].y, X[i].z, X[i].w, xp[i]);
    s += bf16_to_f32(X[i].x & 0xFFFFu) + bf16_to_f32(X[i].x >> 16) +
         bf16_to_f32(X[i].y & 0xFFFFu) + bf16_to_f32(X[i].y >> 16) +
         bf16_to_f32(X[i].z & 0xFFFFu) + bf16_to_f32(X[i].z >> 16) +
         bf16_to_f32(X[i].w & 0xFFFFu) + bf16_to_f32(X[i].w >> 16);
  }
  bias = -kPairBias * s;
}

// LDS bytes for the staged x pairs of a row of `in_features` columns.
constexpr size_t x_pairs_lds_bytes(int in_features) {
  return (size_t)(in_features / kChunkCols) * 17 * sizeof(uint32_t);
}

// x loads for the staging step: thread t < nchunks loads chunk t (four
// 128-bit words; the index is clamped so every thread loads).
DIP_DEV void load_x_chunk(const uint16_t* x, int nchunks, uint4 xs[4]) {
  const int c = min((int)threadIdx.x, nchunks - 1);
  const uint4* src = reinterpret_cast<const uint4*>(x) + c * 4;
#pragma unroll
  for (int i = 0; i < 4; ++i) xs[i] = src[i];
}

// Stage the pairs of every chunk in LDS: the four 128-bit pair words of chunk
// l + LPR*c sit at 16-byte slot (c*4 + q)*LPR + l, so the LPR lanes of a
// group read consecutive 16 B (no bank conflicts; the other groups of the
// wave read the same addresses, a broadcast); then [nchunks] biases.
// Needs nchunks <= blockDim.x; ends with a block barrier (BARRIER false:
// the caller's next barrier publishes the pairs).
template <int LPR, bool BARRIER = true>
DIP_DEV void stage_x_pairs(const uint4 xs[4], uint32_t* xlds, int nchunks) {
  if ((int)threadIdx.x < nchunks) {
    uint32_t p[4][4];
    float b;
    pairs_of(xs, p, b);
    const int lc = threadIdx.x % LPR, cc = threadIdx.x / LPR;
    uint4* dst = reinterpret_cast<uint4*>(xlds);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      dst[(cc * 4 + i) * LPR + lc] = make_uint4(p[i][0], p[i][1], p[i][2], p[i][3]);
    reinterpret_cast<float*>(xlds + nchunks * 16)[threadIdx.x] = b;
  }
  if constexpr (BARRIER) __syncthreads();
}

// ---------------------------------------------------------------------------
// RMSNorm prologue of the norm-fused GEMVs, spread over every thread of the
// workgroup: thread t handles the 8-value units t, t + blockDim, ... (unit u
// is word u % 4 of chunk u / 4) of h, of the residual addend and of the norm
// weight, so the four units of a chunk sit on four consecutive lanes.
// ---------------------------------------------------------------------------
template <int UPT>
DIP_DEV void load_x_units(const uint16_t* p, int nunits, uint4 v[UPT]) {
  const uint4* src = reinterpret_cast<const uint4*>(p);
#pragma unroll
  for (int j = 0; j < UPT; ++j) v[j] = src[min((int)(threadIdx.x + j * blockDim.x), nunits - 1)];
}

// v = bf16(h + add) and x = bf16(w * bf16(v * rsqrt(mean(v^2) + eps))) (the
// rounding of transformers' Qwen3RMSNorm), the block's sum of squares through
// red (4 floats of LDS, one barrier); workgroup 0 writes v to h_out and x to
// x_out (when given).  Then the pairs and chunk biases of x are staged in LDS
// exactly as stage_x_pairs stages them (the same pairs, each chunk's bias
// summed in the same order as pairs_of), ending with a block barrier.
template <int LPR, int UPT>
DIP_DEV void norm_stage_x(const uint4 hs[UPT], const uint4 as[UPT], const uint4 ws[UPT],
                          int nchunks, float eps, uint16_t* h_out, uint16_t* x_out, float* red,
                          uint32_t* xlds) {
  const int nunits = nchunks * 4;
  uint4 v[UPT];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < UPT; ++j) {
    const bool mine = (int)(threadIdx.x + j * blockDim.x) < nunits;
    const uint32_t hw[4] = {hs[j].x, hs[j].y, hs[j].z, hs[j].w};
    const uint32_t aw[4] = {as[j].x, as[j].y, as[j].z, as[j].w};
    uint32_t vw[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      vw[e] = f32x2_to_bf16x2(bf16_to_f32(hw[e] & 0xFFFFu) + bf16_to_f32(aw[e] & 0xFFFFu),
                              bf16_to_f32(hw[e] >> 16) + bf16_to_f32(aw[e] >> 16));
      const float a = bf16_to_f32(vw[e] & 0xFFFFu), b = bf16_to_f32(vw[e] >> 16);
      ss += mine ? a * a + b * b : 0.f;
    }
    v[j] = make_uint4(vw[0], vw[1], vw[2], vw[3]);
  }
  ss = group_sum<64>(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
  for (int w = 0; w < (int)(blockDim.x >> 6); ++w) tot += red[w];
  const float r = rsqrtf(tot * (1.0f / (float)(nchunks * kChunkCols)) + eps);
  uint4* dst = reinterpret_cast<uint4*>(xlds);
  float* bias = reinterpret_cast<float*>(xlds + nchunks * 16);
#pragma unroll
  for (int j = 0; j < UPT; ++j) {
    const int u = (int)(threadIdx.x + j * blockDim.x);
    const bool mine = u < nunits;
    const uint32_t vw[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
    const uint32_t ww[4] = {ws[j].x, ws[j].y, ws[j].z, ws[j].w};
    uint32_t xw[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t t = f32x2_to_bf16x2(bf16_to_f32(vw[e] & 0xFFFFu) * r,
                                         bf16_to_f32(vw[e] >> 16) * r);
      xw[e] = f32x2_to_bf16x2(bf16_to_f32(ww[e] & 0xFFFFu) * bf16_to_f32(t & 0xFFFFu),
                              bf16_to_f32(ww[e] >> 16) * bf16_to_f32(t >> 16));
    }
    if (blockIdx.x == 0 && mine) {
      if (h_out) reinterpret_cast<uint4*>(h_out)[u] = v[j];
      if (x_out) reinterpret_cast<uint4*>(x_out)[u] = make_uint4(xw[0], xw[1], xw[2], xw[3]);
    }
    uint32_t p[4];
    make_xpairs(xw[0], xw[1], xw[2], xw[3], p);
    // this word's sum in the order of pairs_of, then the chunk's four words'
    // sums added in word order on the chunk's first lane
    const float part = bf16_to_f32(xw[0] & 0xFFFFu) + bf16_to_f32(xw[0] >> 16) +
                       bf16_to_f32(xw[1] & 0xFFFFu) + bf16_to_f32(xw[1] >> 16) +
                       bf16_to_f32(xw[2] & 0xFFFFu) + bf16_to_f32(xw[2] >> 16) +
                       bf16_to_f32(xw[3] & 0xFFFFu) + bf16_to_f32(xw[3] >> 16);
    const float p1 = dpp_mov<0x55>(part);  // quad_perm [1,1,1,1]
    const float p2 = dpp_mov<0xAA>(part);  // quad_perm [2,2,2,2]
    const float p3 = dpp_mov<0xFF>(part);  // quad_perm [3,3,3,3]
    if (mine) {
      const int c = u >> 2, i = u & 3;
      dst[((c / LPR) * 4 + i) * LPR + c % LPR] = make_uint4(p[0], p[1], p[2], p[3]);
      if (i == 0) {
        float s = 0.f;
        s += part;
        s += p1;
        s += p2;
        s += p3;
        bias[c] = -kPairBias * s;
      }
    }
  }
  __syncthreads();
}

// Lane l's CH chunks of staged pairs and biases, into VGPRs.
template <int LPR, int CH>
DIP_DEV void x_pairs_to_regs(const uint32_t* xlds, int nchunks, int l, uint32_t xp[CH][4][4],
                             float bias[CH]) {
  const uint4* src = reinterpret_cast<const uint4*>(xlds);
#pragma unroll
  for (int c = 0; c < CH; ++c) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint4 v = src[(c * 4 + q) * LPR + l];
      xp[c][q][0] = v.x;
      xp[c][q][1] = v.y;
      xp[c][q][2] = v.z;
      xp[c][q][3] = v.w;
    }
    bias[c] = reinterpret_cast<const float*>(xlds + nchunks * 16)[l + LPR * c];
  }
}

// One chunk's contribution: acc + 16*s*(bias + sum of its 32 (1.5 + q/16)*x).
DIP_DEV float chunk_dot(const uint4& w, const uint32_t xp[4][4], float bias, uint32_t s,
                        float acc) {
  float t = bias;
  t = dot8_nibbles(w.x, xp[0], t);
  t = dot8_nibbles(w.y, xp[1], t);
  t = dot8_nibbles(w.z, xp[2], t);
  t = dot8_nibbles(w.w, xp[3], t);
  return fmaf(bf16_to_f32(s), kPairScale * t, acc);
}

// The lane's part of one row's dot product with x pairs in VGPRs (not yet
// reduced across the row group).
template <int CH>
DIP_DEV float row_dot_part(const RowRegs<CH>& R, const uint32_t xp[CH][4][4],
                           const float bias[CH]) {
  float acc = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) acc = chunk_dot(R.w[c], xp[c], bias[c], R.s[c], acc);
  return acc;
}

// The same with the pairs read from the staged LDS copy chunk by chunk (the
// same operations in the same order, so the result is bit-identical).
template <int LPR, int CH>
DIP_DEV float row_dot_lds(const RowRegs<CH>& R, const uint32_t* xlds, int nchunks, int l) {
  const uint4* src = reinterpret_cast<const uint4*>(xlds);
  const float* bias = reinterpret_cast<const float*>(xlds + nchunks * 16);
  float acc = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    uint32_t xp[4][4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint4 v = src[(c * 4 + q) * LPR + l];
      xp[q][0] = v.x;
      xp[q][1] = v.y;
      xp[q][2] = v.z;
      xp[q][3] = v.w;
    }
    acc = chunk_dot(R.w[c], xp, bias[l + LPR * c], R.s[c], acc);
  }
  return acc;
}

// h = bf16(g * bf16(u)) from the reduced up dot product u (dip_stream_predispatch.py:198-199).
DIP_DEV uint32_t h_of(uint32_t g_bits, float u) {
  return f32_to_bf16(bf16_to_f32(g_bits) * bf16_to_f32(f32_to_bf16(u)));
}

// ---------------------------------------------------------------------------
// Down
// ---------------------------------------------------------------------------
constexpr int kDownThreads = 256;
// The down workspace starts with the XCD-local reduce's arrival counters, one
// per column block on its own 256 bytes (no two XCDs' L2s hold one line).
constexpr size_t kDownCounterStride = 256;
constexpr size_t kDownCounterBytes = 8192;  // 32 column blocks: out_features <= 8192
constexpr int kDownAcc = kChunkCols;  // outputs per lane: one 16-byte chunk

// Row id for position j (j < k); kBadRow if out of range.  Branch-free.
template <int SRC>
DIP_DEV uint32_t down_row(const DownArgs& a, int j) {
  if (SRC == kContig) return (unsigned)j < (unsigned)a.rows_a ? (uint32_t)j : kBadRow;
  if (SRC == kGather) {
    const int r = a.sel[j];
    return (unsigned)r < (unsigned)a.rows_a ? (uint32_t)r : kBadRow;
  }
  const int r = a.sel2[j];
  const bool b = a.sel[j] != 0;
  const bool ok = b ? (unsigned)r < (unsigned)a.rows_b : (unsigned)r < (unsigned)a.rows_a;
  return ok ? ((uint32_t)r | (b ? kSrcB : 0u)) : kBadRow;
}

struct DownRow {
  uint4 w;  // the lane's 16-byte chunk of the row
};

// Unconditional load of a lane's chunk cc0 of one row (bad and padding ids
// read row 0 of the safe matrix).
template <int SRC>
DIP_DEV void load_down_row(const DownArgs& a, uint32_t rid, int cc0, size_t row_bytes,
                           DownRow& R) {
  const bool bad = rid >= kPadRow;
  const bool isb = SRC == kDual && !bad && (rid & kSrcB);
  const int8_t* qw = bad ? a.qw_safe : (isb ? a.qw_b : a.qw_a);
  const uint32_t r = bad ? 0u : (rid & ~kSrcB);
  R.w = ldg_nt(reinterpret_cast<const uint4*>(qw + (size_t)r * row_bytes) + cc0);
}

// The NG bf16 scales of groups g0 .. g0 + NG - 1 of row rid (a slot's LPR
// chunks span NG = LPR / 4 groups).  Issued by the lane that owns the row,
// once per tile, instead of one scale load per row by every lane.
// Scale layouts of the down kernel: kScRow, the reference's [rows][groups]
// one 16-bit load per group; kScRow4, the same with the NG == 2 pair as one
// 32-bit load (scale rows 4-byte aligned, g0 even); kScGm, A's scales
// group-major [groups][rows_a] (sc_gm): the rows of a tile then read
// neighbouring words of one group row instead of a few bytes of every row's
// own scale line.
enum DownScales : int { kScRow = 0, kScRow4 = 1, kScGm = 2 };

template <int SRC, int NG, int SL>
DIP_DEV void load_down_scales(const DownArgs& a, uint32_t rid, int g0, int ngroups,
                              uint32_t s[NG]) {
  const bool bad = rid >= kPadRow;
  const bool isb = SRC == kDual && !bad && (rid & kSrcB);
  const uint16_t* sc = bad ? a.sc_safe : (isb ? a.sc_b : a.sc_a);
  const uint32_t r = bad ? 0u : (rid & ~kSrcB);
  if constexpr (SL == kScGm) {
    static_assert(SRC != kDual, "group-major scales: one matrix");
#pragma unroll
    for (int i = 0; i < NG; ++i) s[i] = a.sc_gm[(size_t)(g0 + i) * a.rows_a + r];
  } else if constexpr (SL == kScRow4 && NG == 2) {
    const uint32_t p = *reinterpret_cast<const uint32_t*>(sc + (size_t)r * ngroups + g0);
    s[0] = p & 0xFFFFu;
    s[1] = p >> 16;
  } else {
#pragma unroll
    for (int i = 0; i < NG; ++i) s[i] = sc[(size_t)r * ngroups + g0 + i];
  }
}

// The row's coefficients 16*h*s per group (padding row: 0, bad id: NaN),
// computed as (h*s)*16 in fp32 (exact: two 8-bit significands).  Integer
// selects on the bits keep this branch-free.
template <int NG>
DIP_DEV void down_coef(uint32_t rid, uint32_t h, const uint32_t s[NG], float f[NG]) {
#pragma unroll
  for (int i = 0; i < NG; ++i) {
    uint32_t fb = __float_as_uint(bf16_to_f32(h) * bf16_to_f32(s[i]) * 16.0f);
    fb = rid == kPadRow ? 0u : fb;
    fb = rid == kBadRow ? 0x7FC00000u : fb;
    f[i] = __uint_as_float(fb);
  }
}

// acc[0..7] += (q/16) * f for the 8 nibbles of w: the low nibble of byte b
// goes to acc[2b], the high one to acc[2b+1].  v_cvt_off_f32_i4 with an SDWA
// byte select gives q/16 exactly for the low nibble of a byte (high nibbles
// after one shift), so a weight costs one convert and one FMA.  The block is
// one asm statement so that every convert stays next to its FMA: written as
// separate operations, the compiler computes every convert of a row (or of
// several rows) first and holds them all in registers (over 140 VGPRs for
// one tile, spills for two).
DIP_DEV void down_word(uint32_t w, float f, float* acc) {
  const uint32_t hq = w >> 4;
  float t0, t1;
  asm volatile(
      "v_cvt_off_f32_i4_sdwa %[t0], %[w] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0\n\t"
      "v_cvt_off_f32_i4_sdwa %[t1], %[h] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0\n\t"
      "v_fmac_f32 %[a0], %[t0], %[f]\n\t"
      "v_fmac_f32 %[a1], %[t1], %[f]\n\t"
      "v_cvt_off_f32_i4_sdwa %[t0], %[w] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1\n\t"
      "v_cvt_off_f32_i4_sdwa %[t1], %[h] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1\n\t"
      "v_fmac_f32 %[a2], %[t0], %[f]\n\t"
      "v_fmac_f32 %[a3], %[t1], %[f]\n\t"
      "v_cvt_off_f32_i4_sdwa %[t0], %[w] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2\n\t"
      "v_cvt_off_f32_i4_sdwa %[t1], %[h] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2\n\t"
      "v_fmac_f32 %[a4], %[t0], %[f]\n\t"
      "v_fmac_f32 %[a5], %[t1], %[f]\n\t"
      "v_cvt_off_f32_i4_sdwa %[t0], %[w] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3\n\t"
      "v_cvt_off_f32_i4_sdwa %[t1], %[h] dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3\n\t"
      "v_fmac_f32 %[a6], %[t0], %[f]\n\t"
      "v_fmac_f32 %[a7], %[t1], %[f]"
      : [a0] "+v"(acc[0]), [a1] "+v"(acc[1]), [a2] "+v"(acc[2]), [a3] "+v"(acc[3]),
        [a4] "+v"(acc[4]), [a5] "+v"(acc[5]), [a6] "+v"(acc[6]), [a7] "+v"(acc[7]),
        [t0] "=&v"(t0), [t1] "=&v"(t1)
      : [w] "v"(w), [h] "v"(hq), [f] "v"(f));
}

// acc[m] += (q/16)[row i, 32*cc0 + m] * f[i] over the slot's LPR rows, in
// row order (f[i] = 16*h*s of row i for this lane's column group).
template <int LPR>
DIP_DEV void down_accumulate(const DownRow ring[LPR], const float f[LPR], float acc[kDownAcc]) {
#pragma unroll
  for (int i = 0; i < LPR; ++i) {
    down_word(ring[i].w.x, f[i], acc);
    down_word(ring[i].w.y, f[i], acc + 8);
    down_word(ring[i].w.z, f[i], acc + 16);
    down_word(ring[i].w.w, f[i], acc + 24);
  }
}

// v_permlane{16,32}_swap_b32 on two registers: swaps the odd rows (of 16 /
// 32 lanes) of a with the even rows of b (inline asm: see row_pair_sum16).
DIP_DEV void permlane16_swap(float& a, float& b) {
  uint32_t x = __builtin_bit_cast(uint32_t, a), y = __builtin_bit_cast(uint32_t, b);
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(x), "+v"(y));
  a = __builtin_bit_cast(float, x);
  b = __builtin_bit_cast(float, y);
}
DIP_DEV void permlane32_swap(float& a, float& b) {
  uint32_t x = __builtin_bit_cast(uint32_t, a), y = __builtin_bit_cast(uint32_t, b);
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(x), "+v"(y));
  a = __builtin_bit_cast(float, x);
  b = __builtin_bit_cast(float, y);
}

// Floats of LDS for the cross-wave step of down_block_partial.
template <int LPR>
constexpr int down_red_floats() {
  return (kDownThreads / 64) * LPR * kDownAcc;
}

// Sum the block's slots in a fixed order and store the block's LPR*32
// partial sums to out[0 .. LPR*32).  The slots of a wave (lanes l + LPR*s
// hold the same 32 columns) are summed in registers:
//   1. within rows of 16 lanes by DPP rotations (lane l + 8 for LPR = 8;
//      l + 4, then l + 8 for LPR = 4), every lane of the row receiving the
//      row's sum;
//   2. across the row pairs (0,1), (2,3) by v_permlane16_swap of two
//      accumulators m, m + 16 followed by one add: rows 0 and 2 keep column
//      m, rows 1 and 3 column m + 16 (16 registers left);
//   3. across the wave halves by v_permlane32_swap of m, m + 8: lanes 0-31
//      keep m, lanes 32-63 m + 8 (8 registers left).
// Register m' of lane i (i % 16 < LPR) then holds column 32*(i % LPR) + m' +
// 8*(i / 32) + 16*((i / 16) % 2) of the block, summed over the wave's
// slots; the waves' sums meet in LDS (red: down_red_floats floats) and are
// added in wave order.
template <int LPR>
DIP_DEV void down_block_partial(float acc[kDownAcc], float* red, float* out) {
  static_assert(LPR == 4 || LPR == 8, "slot width");
  constexpr int kCols = LPR * kDownAcc;
  constexpr int kWaves = kDownThreads / 64;
#pragma unroll
  for (int m = 0; m < kDownAcc; ++m) {
    if constexpr (LPR == 4) acc[m] += dpp_mov<0x124>(acc[m]);  // row_ror:4
    acc[m] += dpp_mov<0x128>(acc[m]);                          // row_ror:8
  }
  float t[16];
#pragma unroll
  for (int m = 0; m < 16; ++m) {
    permlane16_swap(acc[m], acc[m + 16]);
    t[m] = acc[m] + acc[m + 16];
  }
  float u[8];
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    permlane32_swap(t[m], t[m + 8]);
    u[m] = t[m] + t[m + 8];
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if ((lane & 15) < LPR) {
    float* dst = red + wave * kCols + 32 * (lane % LPR) + 8 * (lane >> 5) + 16 * ((lane >> 4) & 1);
    *reinterpret_cast<float4*>(dst) = make_float4(u[0], u[1], u[2], u[3]);
    *reinterpret_cast<float4*>(dst + 4) = make_float4(u[4], u[5], u[6], u[7]);
  }
  __syncthreads();
  for (int c = threadIdx.x; c < kCols; c += kDownThreads) {
    float s = red[c];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) s += red[w * kCols + c];
    out[c] = s;
  }
}

}  // namespace dip
