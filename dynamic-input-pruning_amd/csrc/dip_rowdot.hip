// dip_rowdot.hip — int4 g128 row-dot kernels: gate GEMV (+SiLU), up-row gather GEMV (+ fused h = g[idx] * u) and the cache-aware
// dual-source variant.
//
// Mapping (one design for every row source):
//   * LPR lanes ("a row group", a power of two dividing 64) own one row at a
//     time; lane l of the group owns chunks l, l+LPR, ..., l+(CH-1)*LPR of the
//     row, so a row of in_features/2 bytes = LPR*CH*16 bytes is read with CH
//     128-bit loads per lane, each instruction covering LPR*16 contiguous
//     bytes per group (fully coalesced).
//   * Because a lane always sees the same columns, its slice of x lives in
//     VGPRs for the whole kernel, pre-paired for v_dot2_f32_bf16, together
//     with the per-chunk bias term (see dip_common.h).
//   * Row groups stride over the outputs; U rows per group are in flight per
//     iteration to keep HBM busy.
//   * The group reduction is an xor-butterfly; lane 0 of the group applies the
//     epilogue and stores one bf16.
#include "dip_common.h"
#include "dip_internal.h"

namespace dip {

namespace {

constexpr uint32_t kBadRow = 0xFFFFFFFFu;
constexpr uint32_t kSrcB = 0x80000000u;

// Row id for output j: bit 31 selects matrix B (kDual); kBadRow if out of range.
template <int SRC>
DIP_DEV uint32_t resolve_row(const RowdotArgs& a, int j) {
  if (SRC == kContig) return (uint32_t)j;
  if (SRC == kGather) {
    const int r = a.sel[j];
    return (unsigned)r < (unsigned)a.rows_a ? (uint32_t)r : kBadRow;
  }
  const int r = a.sel2[j];
  if (a.sel[j] != 0) return (unsigned)r < (unsigned)a.rows_b ? ((uint32_t)r | kSrcB) : kBadRow;
  return (unsigned)r < (unsigned)a.rows_a ? (uint32_t)r : kBadRow;
}

template <int LPR, int CH>
struct RowRegs {
  uint4 w[CH];
  uint32_t s[CH];
};

template <int LPR, int CH, int SRC>
DIP_DEV void load_row(const RowdotArgs& a, uint32_t rid, int l, size_t row_bytes, int ngroups,
                      RowRegs<LPR, CH>& R) {
  if (rid == kBadRow) return;
  const int8_t* qw = a.qw_a;
  const uint16_t* sc = a.sc_a;
  if (SRC == kDual && (rid & kSrcB)) {
    qw = a.qw_b;
    sc = a.sc_b;
  }
  const uint32_t r = rid & ~kSrcB;
  const uint4* wr = reinterpret_cast<const uint4*>(qw + (size_t)r * row_bytes);
  const uint16_t* sr = sc + (size_t)r * ngroups;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int chunk = l + LPR * c;
    R.w[c] = ldg_nt(wr + chunk);
    R.s[c] = sr[chunk / kChunksPerGroup];
  }
}

}  // namespace

// x pairs + bias for one chunk (32 columns starting at 32*chunk).
DIP_DEV void chunk_pairs(const uint16_t* __restrict__ x, int chunk, uint32_t xp[4][4],
                         float& bias) {
  const uint4* xs = reinterpret_cast<const uint4*>(x) + chunk * 4;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint4 X = xs[i];
    make_xpairs(X.x, X.y, X.z, X.w, xp[i]);
    s += bf16_to_f32(X.x & 0xFFFFu) + bf16_to_f32(X.x >> 16) + bf16_to_f32(X.y & 0xFFFFu) +
         bf16_to_f32(X.y >> 16) + bf16_to_f32(X.z & 0xFFFFu) + bf16_to_f32(X.z >> 16) +
         bf16_to_f32(X.w & 0xFFFFu) + bf16_to_f32(X.w >> 16);
  }
  bias = -kPairBias * s;
}

// Row group = LPR lanes; group g handles outputs j = g + i*ngrp for
// i < cnt <= LPR (the launcher sizes the grid so).  Lane l of the group
// fetches the id of the group's l-th row once; each row's id is shuffled to
// the group when it comes up.  D rows of loads stay in flight: the loads of
// row i+D are issued into the ring slot of row i right after row i's dot
// product.  Lane l keeps the reduced sum of row l, and the epilogue (bf16
// round, SiLU or h) runs once at the end with every lane finishing one row.
// XL = 0: each lane keeps its x pairs in VGPRs;
// XL = 1: the workgroup stages all x pairs in LDS once and lanes read their
//         chunk's 64 bytes per row (fewer VGPRs, more waves per SIMD).
template <int LPR, int CH, int SRC, int EPI, int XL, int D>
__global__ __launch_bounds__(256) void rowdot_kernel(RowdotArgs a) {
  extern __shared__ uint32_t xlds[];  // XL: [chunks][16] pairs, then [chunks] bias
  const int l = threadIdx.x % LPR;
  const int lane = threadIdx.x & 63;
  const int gbase = lane - l;  // first lane of my group within the wave
  const size_t row_bytes = (size_t)(a.in_features >> 1);
  const int ngroups = a.in_features >> 7;
  const int nchunks = a.in_features / kChunkCols;
  const int grp = blockIdx.x * (256 / LPR) + threadIdx.x / LPR;
  const int ngrp = gridDim.x * (256 / LPR);
  const int cnt = grp < a.nrows ? (a.nrows - 1 - grp) / ngrp + 1 : 0;  // <= LPR

  const uint32_t rid_lane = l < cnt ? resolve_row<SRC>(a, grp + l * ngrp) : kBadRow;
  RowRegs<LPR, CH> ring[D];
#pragma unroll
  for (int d = 0; d < D; ++d)
    if (d < cnt) load_row<LPR, CH, SRC>(a, __shfl(rid_lane, gbase + d, 64), l, row_bytes, ngroups,
                                        ring[d]);

  uint32_t xp[XL ? 1 : CH][4][4];
  float bias[XL ? 1 : CH];
  if (XL) {
    float* lbias = reinterpret_cast<float*>(xlds + nchunks * 16);
    for (int c = threadIdx.x; c < nchunks; c += 256) {
      uint32_t p[4][4];
      float b;
      chunk_pairs(a.x, c, p, b);
      uint4* dst = reinterpret_cast<uint4*>(xlds + c * 16);
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[i] = make_uint4(p[i][0], p[i][1], p[i][2], p[i][3]);
      lbias[c] = b;
    }
    __syncthreads();
  } else {
#pragma unroll
    for (int c = 0; c < (XL ? 1 : CH); ++c) chunk_pairs(a.x, l + LPR * c, xp[c], bias[c]);
  }

  float mine = 0.f;  // reduced dot product of row l
  for (int i0 = 0; i0 < cnt; i0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int i = i0 + d;
      if (i < cnt) {
        const uint32_t rid = __shfl(rid_lane, gbase + i, 64);
        float acc = 0.f;
        if (rid != kBadRow) {
#pragma unroll
          for (int c = 0; c < CH; ++c) {
            float t;
            if (XL) {
              const int chunk = l + LPR * c;
              const uint4* src = reinterpret_cast<const uint4*>(xlds + chunk * 16);
              uint32_t p[4][4];
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                const uint4 v = src[q];
                p[q][0] = v.x; p[q][1] = v.y; p[q][2] = v.z; p[q][3] = v.w;
              }
              t = reinterpret_cast<const float*>(xlds + nchunks * 16)[chunk];
              t = dot8_nibbles(ring[d].w[c].x, p[0], t);
              t = dot8_nibbles(ring[d].w[c].y, p[1], t);
              t = dot8_nibbles(ring[d].w[c].z, p[2], t);
              t = dot8_nibbles(ring[d].w[c].w, p[3], t);
            } else {
              t = bias[XL ? 0 : c];
              t = dot8_nibbles(ring[d].w[c].x, xp[XL ? 0 : c][0], t);
              t = dot8_nibbles(ring[d].w[c].y, xp[XL ? 0 : c][1], t);
              t = dot8_nibbles(ring[d].w[c].z, xp[XL ? 0 : c][2], t);
              t = dot8_nibbles(ring[d].w[c].w, xp[XL ? 0 : c][3], t);
            }
            acc = fmaf(bf16_to_f32(ring[d].s[c]), kPairScale * t, acc);
          }
        }
        acc = group_sum<LPR>(acc);
        if (l == i) mine = acc;
        if (i + D < cnt)
          load_row<LPR, CH, SRC>(a, __shfl(rid_lane, gbase + i + D, 64), l, row_bytes, ngroups,
                                 ring[d]);
      }
    }
  }

  if (l < cnt) {
    const int j = grp + l * ngrp;
    uint32_t v;
    if (rid_lane == kBadRow) {
      v = 0x7FC0u;
    } else {
      v = f32_to_bf16(mine);
      if (EPI == kSilu) {
        const float f = bf16_to_f32(v);
        v = f32_to_bf16(f / (1.0f + expf(-f)));
      } else if (EPI == kH) {
        const int ch = (SRC == kGather) ? (int)rid_lane : a.gid[j];
        v = f32_to_bf16(bf16_to_f32(a.g[ch]) * bf16_to_f32(v));
      }
    }
    a.out[j] = (uint16_t)v;
  }
}

// ---------------------------------------------------------------------------
// Host dispatch
// ---------------------------------------------------------------------------
namespace {

template <int LPR, int CH, int SRC, int EPI, int XL, int D>
void launch_variant(const RowdotArgs& a, int blocks, hipStream_t stream) {
  const size_t lds = XL ? (size_t)(a.in_features / kChunkCols) * 17 * sizeof(uint32_t) : 0;
  hipLaunchKernelGGL((rowdot_kernel<LPR, CH, SRC, EPI, XL, D>), dim3(blocks), dim3(256), lds,
                     stream, a);
}

template <int LPR, int CH, int SRC, int EPI>
int launch_one(const RowdotArgs& a, hipStream_t stream) {
  // Every row group gets the same number of rows (within one), at most LPR,
  // and the grid aims at ~`wgs_per_cu` workgroups per CU.
  const int groups_per_block = 256 / LPR;
  const int target = device_cus() * tuning(DIP_TUNE_ROWDOT_WGS_PER_CU);
  int per = (a.nrows + target * groups_per_block - 1) / (target * groups_per_block);
  if (per > LPR) per = LPR;
  if (per < 1) per = 1;
  int blocks = (a.nrows + per * groups_per_block - 1) / (per * groups_per_block);
  if (blocks < 1) blocks = 1;
  const int xl = tuning(DIP_TUNE_ROWDOT_X_LDS);
  const int depth = tuning(DIP_TUNE_ROWDOT_DEPTH);
  constexpr bool hot = (LPR == 32 && (CH == 5 || CH == 4)) || (LPR == 16 && CH == 5);
  if constexpr (hot) {
    if (xl) {
      if (depth == 2) launch_variant<LPR, CH, SRC, EPI, 1, 2>(a, blocks, stream);
      else if (depth == 4) launch_variant<LPR, CH, SRC, EPI, 1, 4>(a, blocks, stream);
      else launch_variant<LPR, CH, SRC, EPI, 1, 3>(a, blocks, stream);
    } else {
      if (depth == 3) launch_variant<LPR, CH, SRC, EPI, 0, 3>(a, blocks, stream);
      else launch_variant<LPR, CH, SRC, EPI, 0, 2>(a, blocks, stream);
    }
  } else {
    launch_variant<LPR, CH, SRC, EPI, 0, 2>(a, blocks, stream);
  }
  return hip_status(hipGetLastError());
}

template <int SRC, int EPI>
int dispatch_layout(const RowdotArgs& a, hipStream_t stream) {
  const int chunks = a.in_features / kChunkCols;
#define DIP_TRY(LPR, CH) \
  if (chunks == (LPR) * (CH)) return launch_one<LPR, CH, SRC, EPI>(a, stream);
  DIP_TRY(32, 5)   // 5120 (Qwen3-14B/32B)
  DIP_TRY(32, 4)   // 4096 (Qwen3-8B)
  DIP_TRY(16, 5)   // 2560 (Qwen3-4B)
  DIP_TRY(32, 2)   // 2048
  DIP_TRY(32, 3)   // 3072
  DIP_TRY(32, 6)   // 6144
  DIP_TRY(32, 8)   // 8192
  DIP_TRY(32, 1)   // 1024
  DIP_TRY(16, 3)   // 1536
  DIP_TRY(16, 1)   // 512
  DIP_TRY(8, 1)    // 256
  DIP_TRY(4, 1)    // 128
#undef DIP_TRY
  return DIP_ERR_UNSUPPORTED;
}

}  // namespace

int launch_rowdot(int src, int epi, const RowdotArgs& a, hipStream_t stream) {
  if (a.nrows == 0) return DIP_OK;
#define DIP_CASE(S, E) \
  if (src == (S) && epi == (E)) return dispatch_layout<S, E>(a, stream);
  DIP_CASE(kContig, kRaw)
  DIP_CASE(kContig, kSilu)
  DIP_CASE(kGather, kRaw)
  DIP_CASE(kGather, kH)
  DIP_CASE(kDual, kRaw)
  DIP_CASE(kDual, kH)
#undef DIP_CASE
  return DIP_ERR_ARG;
}

}  // namespace dip

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
using namespace dip;

namespace {

int check_matrix(const int8_t* qw, const uint16_t* sc, int64_t rows, int64_t cols) {
  if (!qw || !sc) return DIP_ERR_NULL;
  if (rows < 0 || cols <= 0 || cols % kGroupSize != 0) return DIP_ERR_SHAPE;
  if (rows > INT32_MAX || cols > (int64_t)1 << 20) return DIP_ERR_SHAPE;
  if (!aligned16(qw)) return DIP_ERR_ALIGN;
  return DIP_OK;
}

RowdotArgs base_args(const int8_t* qw, const uint16_t* sc, const uint16_t* x, uint16_t* out,
                     int64_t n, int64_t cols) {
  RowdotArgs a{};
  a.qw_a = qw;
  a.sc_a = sc;
  a.x = x;
  a.out = out;
  a.nrows = (int)n;
  a.in_features = (int)cols;
  a.rows_a = (int)n;
  return a;
}

}  // namespace

extern "C" int dip_int4_gemv(const int8_t* qweight, const uint16_t* scales, const uint16_t* x,
                             uint16_t* out, int64_t out_features, int64_t in_features, int act,
                             void* stream) {
  int st = check_matrix(qweight, scales, out_features, in_features);
  if (st) return st;
  if (!x || !out) return DIP_ERR_NULL;
  if (!aligned16(x)) return DIP_ERR_ALIGN;
  if (act != DIP_ACT_NONE && act != DIP_ACT_SILU) return DIP_ERR_ARG;
  RowdotArgs a = base_args(qweight, scales, x, out, out_features, in_features);
  return launch_rowdot(kContig, act == DIP_ACT_SILU ? kSilu : kRaw, a, (hipStream_t)stream);
}

extern "C" int dip_int4_gather_gemv(const int8_t* qweight, const uint16_t* scales,
                                    const uint16_t* x, const int32_t* indices, uint16_t* out,
                                    int64_t rows, int64_t in_features, int64_t k,
                                    void* stream) {
  int st = check_matrix(qweight, scales, rows, in_features);
  if (st) return st;
  if (k < 0 || k > INT32_MAX) return DIP_ERR_SHAPE;
  if (k == 0) return DIP_OK;
  if (!x || !out || !indices) return DIP_ERR_NULL;
  if (!aligned16(x)) return DIP_ERR_ALIGN;
  RowdotArgs a = base_args(qweight, scales, x, out, k, in_features);
  a.sel = indices;
  a.rows_a = (int)rows;
  return launch_rowdot(kGather, kRaw, a, (hipStream_t)stream);
}

extern "C" int dip_up_gather_h(const int8_t* qweight, const uint16_t* scales, const uint16_t* x,
                               const int32_t* indices, const uint16_t* g, uint16_t* h,
                               int64_t rows, int64_t in_features, int64_t k, void* stream) {
  int st = check_matrix(qweight, scales, rows, in_features);
  if (st) return st;
  if (k < 0 || k > INT32_MAX) return DIP_ERR_SHAPE;
  if (k == 0) return DIP_OK;
  if (!x || !h || !indices || !g) return DIP_ERR_NULL;
  if (!aligned16(x)) return DIP_ERR_ALIGN;
  RowdotArgs a = base_args(qweight, scales, x, h, k, in_features);
  a.sel = indices;
  a.g = g;
  a.rows_a = (int)rows;
  return launch_rowdot(kGather, kH, a, (hipStream_t)stream);
}

extern "C" int dip_ca_fused_gemv(const int8_t* res_qw, const uint16_t* res_sc,
                                 const int8_t* str_qw, const uint16_t* str_sc, const uint16_t* x,
                                 const int32_t* src, const int32_t* row, const uint16_t* g,
                                 const int32_t* gid, uint16_t* out, int64_t res_rows,
                                 int64_t str_rows, int64_t in_features, int64_t k,
                                 void* stream) {
  int st = check_matrix(res_qw, res_sc, res_rows, in_features);
  if (st) return st;
  st = check_matrix(str_qw, str_sc, str_rows, in_features);
  if (st) return st;
  if (k < 0 || k > INT32_MAX) return DIP_ERR_SHAPE;
  if (k == 0) return DIP_OK;
  if (!x || !out || !src || !row) return DIP_ERR_NULL;
  if (g && !gid) return DIP_ERR_NULL;
  if (!aligned16(x)) return DIP_ERR_ALIGN;
  RowdotArgs a = base_args(res_qw, res_sc, x, out, k, in_features);
  a.qw_b = str_qw;
  a.sc_b = str_sc;
  a.sel = src;
  a.sel2 = row;
  a.g = g;
  a.gid = gid;
  a.rows_a = (int)res_rows;
  a.rows_b = (int)str_rows;
  return launch_rowdot(kDual, g ? kH : kRaw, a, (hipStream_t)stream);
}
