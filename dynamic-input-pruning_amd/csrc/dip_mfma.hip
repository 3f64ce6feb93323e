// dip_mfma.hip — contiguous int4 g128 GEMV (the gate) on int8 MFMA.
//
// out[r] = sum_c x[c] * q[r][c] * s[r][c/128]  (kernels/int4_gemv/int4_gemv.cu:
// 44-76 computes the same sum with fp32 products), evaluated exactly in
// integers per 128-column group:
//   * weights: each byte of packed nibbles gives two int8 values 16*q with
//     two bit operations ((w << 4) & 0xF0F0F0F0 for the even columns,
//     w & 0xF0F0F0F0 for the odd ones), 3 VALU operations per 8 weights;
//   * x: per group t with largest bf16 exponent field E_t, every x is split
//     exactly into four signed base-128 digits,
//         x = 2^(E_t - 133) * sum_n d_n 128^-n,  |d_n| <= 127,
//     (x below 2^-20 of the group's largest magnitude keeps its top bits
//     only), held in the MFMA's N columns 0..3 (columns 4..15 are zero);
//   * v_mfma_i32_16x16x32_i8 sums 16 rows x 32 columns exactly in int32; a
//     group is four of them, D[row][n] = sum_c 16 q d_n;
//   * the row's total is sum_t sum_n s[r][t] * 2^(E_t - 137 - 7n) * D_t[r][n]
//     in fp32 (D is exact in fp32, one rounding per product and per add).
// Non-finite x in a group makes that group's contribution NaN.
//
// Status: exact and tested, but slower than the row-dot gate on the
// Qwen3-32B shape (24.5 us against 15.2 us; a copy with the MFMAs replaced by
// a register sink takes as long, so the load pattern is the cost: every load
// instruction of the MFMA operand layout touches 16 rows x 64 B, where the
// row-dot kernel's touches 2 rows x 512 B).  Opt-in (DIP_TUNE_GATE_MFMA);
// loading rows contiguously and reshaping them into operands through LDS is
// the next step.
//
// Mapping: a wave owns 16-row tiles (lane l: row l%16, chunk l/16 of every
// group it loads; its four dwords feed the group's four MFMAs).  Tiles go to
// the waves of the whole grid round-robin, so with 2 workgroups per CU every
// CU gets the same share.  Each workgroup stages the x digits (in the MFMA B
// layout) and per-group powers of two in LDS; each wave stages its tile's
// scales.  Weight loads run PF groups ahead of the MFMAs.
#include <algorithm>

#include "dip_tiles.h"

namespace dip {

namespace {

constexpr int kMThreads = 256;
constexpr int kMWaves = kMThreads / 64;
constexpr int kPF = 8;  // groups of weight loads in flight per wave

typedef int v4i __attribute__((ext_vector_type(4)));

DIP_DEV long i8x8(uint32_t lo, uint32_t hi) {
  return (long)(((uint64_t)hi << 32) | (uint64_t)lo);
}

// Signed base-128 digits of one bf16 x relative to its group's largest
// exponent field eg (eg < 255): I = |x| * 2^(153 - eg) truncated, < 2^28.
DIP_DEV void x_digits(uint32_t bits, uint32_t eg, int d[4]) {
  const uint32_t e = (bits >> 7) & 0xFFu;
  const uint32_t m = (bits & 0x7Fu) | (e ? 0x80u : 0u);
  const int sh = 20 + (int)(e ? e : 1u) - (int)eg;
  uint32_t I = sh >= 0 ? (m << sh) : (sh > -31 ? (m >> (-sh)) : 0u);
  const bool neg = (bits & 0x8000u) != 0;
  const int v0 = (int)(I >> 21), v1 = (int)((I >> 14) & 127u), v2 = (int)((I >> 7) & 127u),
            v3 = (int)(I & 127u);
  d[0] = neg ? -v0 : v0;
  d[1] = neg ? -v1 : v1;
  d[2] = neg ? -v2 : v2;
  d[3] = neg ? -v3 : v3;
}

}  // namespace

// One 128-column group: four MFMAs over the lane's 16 weight bytes and the
// group's digits, then acc[r] += D[r] * s[r] * 2^(E_t - 137 - 7n).
DIP_DEV void mfma_group(const uint4& wv, const uint8_t* bsrc, const uint16_t* srow, float p,
                        float acc[4]) {
  const uint4 b01 = *reinterpret_cast<const uint4*>(bsrc);
  const uint4 b23 = *reinterpret_cast<const uint4*>(bsrc + 16);
  const uint32_t wq[4] = {wv.x, wv.y, wv.z, wv.w};
  const long bop[4] = {i8x8(b01.x, b01.y), i8x8(b01.z, b01.w), i8x8(b23.x, b23.y),
                       i8x8(b23.z, b23.w)};
  v4i d = {0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < 4; ++i)
    d = __builtin_amdgcn_mfma_i32_16x16x32_i8(i8x8((wq[i] << 4) & 0xF0F0F0F0u, wq[i] & 0xF0F0F0F0u),
                                              bop[i], d, 0, 0, 0);
  const uint2 sv = *reinterpret_cast<const uint2*>(srow);
  const float s4[4] = {bf16_to_f32(sv.x & 0xFFFFu), bf16_to_f32(sv.x >> 16),
                       bf16_to_f32(sv.y & 0xFFFFu), bf16_to_f32(sv.y >> 16)};
#pragma unroll
  for (int r = 0; r < 4; ++r) acc[r] = fmaf((float)d[r], s4[r] * p, acc[r]);
  // keep each group's operand reads next to its MFMAs (left free, the
  // scheduler hoists many groups' LDS reads and runs out of registers)
  __builtin_amdgcn_sched_barrier(0);
}

// LDS: digits [NG][4 chunks][4 digits][4 dwords][8 B] + a 32 B zero block,
// powers [NG][16] fp32, per-wave scales [4][NG][16] bf16, group exponents.
template <int NG, int EPI>
__global__ __launch_bounds__(kMThreads) void mfma_gemv_kernel(RowdotArgs a, int ntiles) {
  __shared__ __align__(16) uint8_t dig[NG * 512 + 32];
  __shared__ __align__(16) float pw[NG * 16];
  __shared__ __align__(16) uint16_t scl[kMWaves][NG * 16];
  __shared__ uint32_t gexp[NG];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  static_assert(NG % kPF == 0, "groups per row");
  const int H = NG * kGroupSize;
  if (a.rotate && blockIdx.x == 0 && tid == 0) a.rotate[0] = a.rotate[1];

  const int m = lane & 15;   // A row / D column
  const int kb = lane >> 4;  // A chunk within a group / D row block
  const int nwaves = gridDim.x * kMWaves;
  const size_t row_bytes = (size_t)(H >> 1);
  constexpr int kSclPer = (16 * NG + 63) / 64;  // a tile's scales per lane

  // The first tile's weight and scale loads go out before x is staged (the
  // staging takes its own memory round trip).
  int tile = blockIdx.x + gridDim.x * wave;
  uint4 ring[kPF];
  uint32_t sreg[kSclPer];
  const uint4* wrow = nullptr;
  auto issue_tile = [&](int tl) {
    const int r0 = tl * 16;
    wrow = reinterpret_cast<const uint4*>(a.qw_a + (size_t)min(r0 + m, a.nrows - 1) * row_bytes) +
           kb;
#pragma unroll
    for (int u = 0; u < kPF; ++u) ring[u] = ldg_nt(wrow + 4 * u);
#pragma unroll
    for (int j = 0; j < kSclPer; ++j) {
      const int e = min(lane + 64 * j, 16 * NG - 1);
      sreg[j] = a.sc_a[(size_t)min(r0 + e / NG, a.nrows - 1) * NG + e % NG];
    }
  };
  if (tile < ntiles) issue_tile(tile);

  // ---- x digits -----------------------------------------------------------
  constexpr int kOct = NG * 16;                       // 8-column octets of x
  constexpr int kOctPer = (kOct + kMThreads - 1) / kMThreads;
  uint4 xo[kOctPer];
  if (tid < NG) gexp[tid] = 0;
#pragma unroll
  for (int j = 0; j < kOctPer; ++j) {
    const int o = min(tid + j * kMThreads, kOct - 1);
    xo[j] = reinterpret_cast<const uint4*>(a.x)[o];
  }
  if (tid < 8) reinterpret_cast<uint32_t*>(dig + NG * 512)[tid] = 0;  // zero block
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kOctPer; ++j) {
    const int o = tid + j * kMThreads;
    if (o < kOct) {
      const uint32_t w[4] = {xo[j].x, xo[j].y, xo[j].z, xo[j].w};
      uint32_t em = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        em = max(em, max((w[q] >> 7) & 0xFFu, (w[q] >> 23) & 0xFFu));
      atomicMax(&gexp[o >> 4], em);
    }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kOctPer; ++j) {
    const int o = tid + j * kMThreads;
    if (o < kOct) {
      const int t = o >> 4, b = (o >> 2) & 3, i = o & 3;
      const uint32_t eg = gexp[t];
      const uint32_t w[4] = {xo[j].x, xo[j].y, xo[j].z, xo[j].w};
      uint32_t lo[4] = {0, 0, 0, 0}, hi[4] = {0, 0, 0, 0};  // per digit: K bytes 0-3, 4-7
      if (eg < 0xFFu) {
#pragma unroll
        for (int p = 0; p < 8; ++p) {  // column p of the octet -> K byte (0,4,1,5,2,6,3,7)
          const uint32_t bits = (p & 1) ? (w[p >> 1] >> 16) : (w[p >> 1] & 0xFFFFu);
          int d[4];
          x_digits(bits, eg, d);
          const int sh = 8 * (p >> 1);
#pragma unroll
          for (int n = 0; n < 4; ++n) {
            if (p & 1) hi[n] |= ((uint32_t)d[n] & 0xFFu) << sh;
            else lo[n] |= ((uint32_t)d[n] & 0xFFu) << sh;
          }
        }
      }
#pragma unroll
      for (int n = 0; n < 4; ++n)
        *reinterpret_cast<uint2*>(dig + (((t * 4 + b) * 4 + n) * 4 + i) * 8) = make_uint2(lo[n], hi[n]);
    }
  }
  for (int e = tid; e < NG * 16; e += kMThreads) {
    const int t = e >> 4, n = e & 15;
    const uint32_t eg = gexp[t];
    float v = 0.f;
    if (n < 4) v = eg >= 0xFFu ? __uint_as_float(0x7FC00000u) : ldexpf(1.0f, (int)eg - 137 - 7 * n);
    pw[e] = v;
  }
  __syncthreads();

  // ---- row tiles ------------------------------------------------------------
  uint16_t* my_scl = scl[wave];
  const uint8_t* bsrc = (m < 4) ? dig + (kb * 4 + m) * 32 : dig + NG * 512;  // + t*512 if m < 4
  const int bstride = (m < 4) ? 512 : 0;
  for (; tile < ntiles; tile += nwaves) {
    const int r0 = tile * 16;
    // this tile's scales, transposed to [group][row] (same-wave LDS order)
#pragma unroll
    for (int j = 0; j < kSclPer; ++j) {
      const int e = lane + 64 * j;
      if (e < 16 * NG) my_scl[(e % NG) * 16 + e / NG] = (uint16_t)sreg[j];
    }
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    // NG is a multiple of kPF: the last kPF groups are peeled so that every
    // load in the loop body is unconditional
#pragma unroll 1
    for (int t0 = 0; t0 < NG - kPF; t0 += kPF) {
#pragma unroll
      for (int u = 0; u < kPF; ++u) {
        const uint4 wv = ring[u];
        ring[u] = ldg_nt(wrow + 4 * (t0 + u + kPF));
        mfma_group(wv, bsrc + (t0 + u) * bstride, my_scl + (t0 + u) * 16 + 4 * kb,
                   pw[(t0 + u) * 16 + m], acc);
      }
    }
    uint4 last[kPF];
#pragma unroll
    for (int u = 0; u < kPF; ++u) last[u] = ring[u];
    if (tile + nwaves < ntiles) issue_tile(tile + nwaves);  // the next tile's loads
#pragma unroll
    for (int u = 0; u < kPF; ++u) {
      const int tt = NG - kPF + u;
      mfma_group(last[u], bsrc + tt * bstride, my_scl + tt * 16 + 4 * kb, pw[tt * 16 + m], acc);
    }
    // sum the four digit columns (lanes m = 0..3 of each 16-lane row)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      acc[r] += dpp_mov<0xB1>(acc[r]);  // lane ^ 1
      acc[r] += dpp_mov<0x4E>(acc[r]);  // lane ^ 2
    }
    if (m == 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int orow = r0 + 4 * kb + r;
        if (orow < a.nrows) {
          uint32_t v = f32_to_bf16(acc[r]);
          if (EPI == kSilu) {
            const float f = bf16_to_f32(v);
            v = f32_to_bf16(f / (1.0f + expf(-f)));
          }
          a.out[orow] = (uint16_t)v;
        }
      }
    }
  }
}

namespace {

template <int NG>
int launch_ng(int epi, const RowdotArgs& a, int blocks, int ntiles, hipStream_t stream) {
  if (epi == kSilu)
    hipLaunchKernelGGL((mfma_gemv_kernel<NG, kSilu>), dim3(blocks), dim3(kMThreads), 0, stream, a,
                       ntiles);
  else
    hipLaunchKernelGGL((mfma_gemv_kernel<NG, kRaw>), dim3(blocks), dim3(kMThreads), 0, stream, a,
                       ntiles);
  return hip_status(hipGetLastError());
}

}  // namespace

// The contiguous GEMV on MFMA when the width has an instantiation and the
// rows give every CU's waves at least one 16-row tile each (else
// DIP_ERR_UNSUPPORTED: the caller runs the row-dot kernel).
int launch_mfma_gemv(int epi, const RowdotArgs& a, hipStream_t stream) {
  if (epi != kSilu && epi != kRaw) return DIP_ERR_UNSUPPORTED;
  const int ng = a.in_features / kGroupSize;
  const int ntiles = (a.nrows + 15) / 16;
  const int wgs = device_cus() * tuning(DIP_TUNE_ROWDOT_WGS_PER_CU);
  if (a.nrows <= 0 || ntiles < wgs * 2) return DIP_ERR_UNSUPPORTED;
  const int blocks = wgs;  // tiles go to the grid's waves round-robin
  if (ng == 40) return launch_ng<40>(epi, a, blocks, ntiles, stream);
  if (ng == 32) return launch_ng<32>(epi, a, blocks, ntiles, stream);
  return DIP_ERR_UNSUPPORTED;
}

}  // namespace dip
