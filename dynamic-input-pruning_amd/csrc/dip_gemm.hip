// dip_gemm.hip — int4 g128 GEMM for prompts (more than one token) on bf16
// MFMA: out[M, N] = bf16( x[M, K] . W[N, K]^T ), W in the reference's Linear
// layout (qweight int8 [N, K/2], scales bf16 [N, K/128]).
//
// The reference computes this as dequantize + F.linear (qlinear.py:86-88,
// dip_stream_predispatch.py:206-215 for gate and up): it writes a bf16 copy
// of W and reads it back in a GEMM.  Here each weight is read once, as
// packed nibbles, and turned into an MFMA operand in registers:
//   * a nibble u (two's complement q) becomes the bf16 value 136 + q, exact:
//     0x4300 | (u ^ 8) is 128 + (q + 8), so 8 nibbles need a few bit ops;
//   * v_mfma_f32_16x16x32_bf16 sums (136 + q) * x over one 128-column group
//     in fp32; subtracting 136 * sum(x) of the group leaves sum(q * x),
//     which is scaled by the group's scale and added to the fp32 total.
// So the weights enter exactly as q * s in fp32 (the reference rounds q * s
// to bf16 first); the output is rounded to bf16 once.
//
// Tiling: a wave owns RW tiles of 16 weight rows and 16 * TM tokens, so each
// x operand it loads feeds RW row tiles (x comes from L2, and with one row
// tile per wave its re-reads, not the weights, bounded the kernel: the
// 32-token 25600 x 5120 product took 91 us with RW = 1, 46 us with RW = 4);
// the 136 * sum(x) term is computed once per x operand.  A workgroup is 4
// waves on RT such row super-tiles; the 4 / RT waves of one super-tile
// split the K groups between them (wave ks takes groups ks, ks + KS, ...)
// and add their partial sums through LDS at the end, in a fixed order.
// Nothing else is shared: each lane loads its own 16 bytes of nibbles per
// row tile and 64 bytes of x per group, weights and scales PW groups ahead
// and x two groups ahead, so no barrier sits in the main loop.  RW is 4 for
// at least 8192 rows, else 2 (fewer, larger tiles leave CUs idle there).  Inside a 32-column MFMA slice the k
// order is permuted identically for both operands (lane quarter kb holds
// columns 32 kb .. 32 kb + 31 and slice j uses its 8 columns 8j .. 8j + 7),
// so a lane's nibbles are one contiguous 16-byte load.  The offset term
// 136 * sum(x) comes from the same MFMA with a constant operand.
#include <algorithm>

#include "dip_common.h"
#include "dip_internal.h"

namespace dip {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kGemmThreads = 256;
constexpr uint32_t kOffsetPair = 0x43084308u;  // bf16 136.0, twice

// 8 nibbles (element p = nibble p of w) -> the 8 bf16 values 136 + q.
DIP_DEV bf16x8_t offset_bf16x8(uint32_t w) {
  const uint32_t t = w ^ 0x88888888u;  // q + 8 in every nibble
  u32x4_t p;
  p.x = 0x43004300u | (t & 0xFu) | ((t & 0xF0u) << 12);
  p.y = 0x43004300u | ((t >> 8) & 0xFu) | ((t & 0xF000u) << 4);
  p.z = 0x43004300u | ((t >> 16) & 0xFu) | ((t >> 4) & 0xF0000u);
  p.w = 0x43004300u | ((t >> 24) & 0xFu) | ((t >> 12) & 0xF0000u);
  return __builtin_bit_cast(bf16x8_t, p);
}

DIP_DEV bf16x8_t as_bf16x8(const uint4& v) {
  return __builtin_bit_cast(bf16x8_t, u32x4_t{v.x, v.y, v.z, v.w});
}

template <int TM, int RT, int PW, int RW>
__global__ __launch_bounds__(kGemmThreads) void int4_gemm_kernel(
    const int8_t* __restrict__ qw, const uint16_t* __restrict__ sc, const uint16_t* __restrict__ x,
    uint16_t* __restrict__ out, int M, int N, int K) {
  static_assert(PW % 2 == 0, "x ring of 2 inside the weight ring");
  constexpr int KS = 4 / RT;  // waves per row super-tile (K split)
  __shared__ float red[KS > 1 ? 4 : 1][RW][TM][4][64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int rt = wave / KS, ks = wave % KS;
  // this wave's RW 16-row tiles: rows row0 + 16 u + ...
  const int row0 = (blockIdx.x * RT + rt) * (16 * RW);
  const int tok0 = blockIdx.y * TM * 16;
  const int ngroups = K >> 7;
  const int ng = ngroups > ks ? (ngroups - ks + KS - 1) / KS : 0;  // this wave's groups
  const int kb = lane >> 4, l16 = lane & 15;

  // A operand: weight row l16 of tile u, columns 32 kb .. 32 kb + 31 of each group
  const uint4* wp[RW];
  // D: token l16, rows 4 kb + r of tile u; their scales
  const uint16_t* sp[RW][4];
#pragma unroll
  for (int u = 0; u < RW; ++u) {
    wp[u] = reinterpret_cast<const uint4*>(qw + (size_t)min(row0 + 16 * u + l16, N - 1) *
                                                     (K >> 1)) + kb;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      sp[u][r] = sc + (size_t)min(row0 + 16 * u + 4 * kb + r, N - 1) * ngroups;
  }
  // B operand: token l16 of each 16-token tile, the same columns
  const uint4* xp[TM];
#pragma unroll
  for (int t = 0; t < TM; ++t)
    xp[t] = reinterpret_cast<const uint4*>(x + (size_t)min(tok0 + t * 16 + l16, M - 1) * K) +
            4 * kb;

  uint4 wq[PW][RW];
  uint32_t sq[PW][RW][4];
  uint4 xq[2][TM][4];
#pragma unroll
  for (int p = 0; p < PW; ++p) {
    if (p < ng) {
      const int g = ks + p * KS;
#pragma unroll
      for (int u = 0; u < RW; ++u) {
        wq[p][u] = wp[u][4 * g];
#pragma unroll
        for (int r = 0; r < 4; ++r) sq[p][u][r] = sp[u][r][g];
      }
    }
  }
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    if (p < ng) {
      const int g = ks + p * KS;
#pragma unroll
      for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) xq[p][t][v] = xp[t][16 * g + v];
    }
  }

  const bf16x8_t c136 = __builtin_bit_cast(
      bf16x8_t, u32x4_t{kOffsetPair, kOffsetPair, kOffsetPair, kOffsetPair});
  floatx4 acc[RW][TM];
#pragma unroll
  for (int u = 0; u < RW; ++u)
#pragma unroll
    for (int t = 0; t < TM; ++t) acc[u][t] = floatx4{0.f, 0.f, 0.f, 0.f};

  for (int i0 = 0; i0 < ng; i0 += PW) {
#pragma unroll
    for (int p = 0; p < PW; ++p) {
      const int i = i0 + p;
      if (i < ng) {
        // 136 * (sum of the group's x) per token: shared by the RW row tiles
        floatx4 d1[TM];
#pragma unroll
        for (int t = 0; t < TM; ++t) {
          d1[t] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int v = 0; v < 4; ++v)
            d1[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(c136, as_bf16x8(xq[p & 1][t][v]),
                                                            d1[t], 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < RW; ++u) {
          const bf16x8_t a0 = offset_bf16x8(wq[p][u].x), a1 = offset_bf16x8(wq[p][u].y);
          const bf16x8_t a2 = offset_bf16x8(wq[p][u].z), a3 = offset_bf16x8(wq[p][u].w);
          float s4[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) s4[r] = bf16_to_f32(sq[p][u][r]);
#pragma unroll
          for (int t = 0; t < TM; ++t) {
            floatx4 d = {0.f, 0.f, 0.f, 0.f};
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, as_bf16x8(xq[p & 1][t][0]), d, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, as_bf16x8(xq[p & 1][t][1]), d, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, as_bf16x8(xq[p & 1][t][2]), d, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a3, as_bf16x8(xq[p & 1][t][3]), d, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r)
              acc[u][t][r] = fmaf(s4[r], d[r] - d1[t][r], acc[u][t][r]);
          }
        }
        if (i + PW < ng) {
          const int g = ks + (i + PW) * KS;
#pragma unroll
          for (int u = 0; u < RW; ++u) {
            wq[p][u] = wp[u][4 * g];
#pragma unroll
            for (int r = 0; r < 4; ++r) sq[p][u][r] = sp[u][r][g];
          }
        }
        if (i + 2 < ng) {
          const int g = ks + (i + 2) * KS;
#pragma unroll
          for (int t = 0; t < TM; ++t)
#pragma unroll
            for (int v = 0; v < 4; ++v) xq[p & 1][t][v] = xp[t][16 * g + v];
        }
      }
    }
  }

  if constexpr (KS > 1) {
#pragma unroll
    for (int u = 0; u < RW; ++u)
#pragma unroll
      for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave][u][t][r][lane] = acc[u][t][r];
    __syncthreads();
    if (ks != 0) return;
#pragma unroll
    for (int w = 1; w < KS; ++w)
#pragma unroll
      for (int u = 0; u < RW; ++u)
#pragma unroll
        for (int t = 0; t < TM; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[u][t][r] += red[wave + w][u][t][r][lane];
  }
#pragma unroll
  for (int t = 0; t < TM; ++t) {
    const int tok = tok0 + t * 16 + l16;
    if (tok >= M) continue;
#pragma unroll
    for (int u = 0; u < RW; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = row0 + 16 * u + 4 * kb + r;
        if (row < N) out[(size_t)tok * N + row] = (uint16_t)f32_to_bf16(acc[u][t][r]);
      }
  }
}

template <int TM, int PW, int RW>
void launch_gemm(const int8_t* qw, const uint16_t* sc, const uint16_t* x, uint16_t* out, int M,
                 int N, int K, hipStream_t s) {
  // 16 * RW rows per wave; 16 * RW * RT rows per workgroup: as many rows as
  // keep at least two workgroups per CU, the rest of the 4 waves splitting K
  const int cus = device_cus();
  const unsigned gy = (unsigned)((M + 16 * TM - 1) / (16 * TM));
  const long long tile = 16LL * RW;
  if ((long long)N >= tile * 4 * 2 * cus)
    hipLaunchKernelGGL((int4_gemm_kernel<TM, 4, PW, RW>), dim3((N + tile * 4 - 1) / (tile * 4), gy),
                       dim3(kGemmThreads), 0, s, qw, sc, x, out, M, N, K);
  else if ((long long)N >= tile * 2 * 2 * cus)
    hipLaunchKernelGGL((int4_gemm_kernel<TM, 2, PW, RW>), dim3((N + tile * 2 - 1) / (tile * 2), gy),
                       dim3(kGemmThreads), 0, s, qw, sc, x, out, M, N, K);
  else
    hipLaunchKernelGGL((int4_gemm_kernel<TM, 1, PW, RW>), dim3((N + tile - 1) / tile, gy),
                       dim3(kGemmThreads), 0, s, qw, sc, x, out, M, N, K);
}

// The token tiling for M tokens, RW row tiles per wave; the weight prefetch
// depth shrinks as RW grows so the wave stays within 256 VGPRs.
template <int RW>
void launch_tokens(const int8_t* qw, const uint16_t* sc, const uint16_t* x, uint16_t* out, int M,
                   int N, int K, hipStream_t s) {
  constexpr int kPW8 = 8 / RW >= 2 ? 8 / RW : 2, kPW4 = 4 / RW >= 2 ? 4 / RW : 2;
  if (M <= 16)
    launch_gemm<1, kPW8, RW>(qw, sc, x, out, M, N, K, s);
  else if (M <= 32)
    launch_gemm<2, kPW8, RW>(qw, sc, x, out, M, N, K, s);
  else
    launch_gemm<4, kPW4, RW>(qw, sc, x, out, M, N, K, s);
}

// ---------------------------------------------------------------------------
// Transposed layout: out[M, N] = bf16( x[M, K] . W[K, N] ) with W stored as
// rows of K (qweight int8 [K, N/2], scales bf16 [K, N/128]): the transposed
// down matrix down_t of the dense route's h @ down_t
// (dip_stream_predispatch.py:213-215).  The scale varies along k here, so
// each weight becomes the reference's bf16(q * s) (qlinear.dequantize's
// rounding, exact to it) on its way into LDS:
//   * a workgroup owns 64 output columns x 16 * TM tokens and a K range
//     (the K ranges of a split are added by int4_gemm_t_reduce_kernel, in
//     a fixed order);
//   * per 128-row step the 256 threads read 128 rows x 32 bytes of nibbles
//     (thread t: rows 2 (t / 4) and 2 (t / 4) + 1, 16 columns) and their
//     scales, and write the dequantised values transposed into LDS
//     [column][k], one 32-bit word (the two rows) per column: each pair is
//     one v_cvt_pk_bf16_f32 (double-buffered, one barrier per step);
//     nibbles and scales run kGemmTPrefetch steps ahead in registers;
//   * wave w reads A = 16 columns x 8 consecutive k (one 16-byte LDS read
//     per slice) and B = x[token][k .. k + 7] straight from L2, and
//     accumulates on v_mfma_f32_16x16x32_bf16.
constexpr int kGemmTStep = 128;     // K rows per step
constexpr int kGemmTStride = 128 + 8;  // LDS row of one column: 128 k + 16 B of padding
constexpr int kGemmTPrefetch = 4;

template <int TM>
__global__ __launch_bounds__(kGemmThreads) void int4_gemm_t_kernel(
    const int8_t* __restrict__ qw, const uint16_t* __restrict__ sc, const uint16_t* __restrict__ x,
    uint16_t* __restrict__ out, float* __restrict__ part, int M, int N, int K, int kchunk) {
  __shared__ __align__(16) uint16_t wt[2][64][kGemmTStride];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int kb = lane >> 4, l16 = lane & 15;
  const int n0 = blockIdx.x * 64;
  const int tok0 = blockIdx.y * TM * 16;
  const int k0 = blockIdx.z * kchunk;
  const int k1 = min(K, k0 + kchunk);
  const int nsteps = (k1 - k0 + kGemmTStep - 1) / kGemmTStep;
  const int ngroups_n = N >> 7;

  // staging role: rows sr, sr + 1 of the step, columns n0 + scol .. + 15
  const int sr = 2 * (threadIdx.x >> 2), scol = 16 * (threadIdx.x & 3);
  const bool col_ok = n0 + scol < N;
  struct WPair {
    uint2 w0, w1;   // 16 nibbles of each row
    uint32_t s01;   // the two rows' scales (row sr low)
  };
  auto load_w = [&](int step, WPair& wp) {
    const int row = k0 + step * kGemmTStep + sr;
    const size_t off = (size_t)((n0 + scol) >> 1);
    const int g = (n0 + scol) >> 7;
    wp.w0 = make_uint2(0, 0);
    wp.w1 = make_uint2(0, 0);
    wp.s01 = 0u;
    if (row < k1 && col_ok) {
      wp.w0 = *reinterpret_cast<const uint2*>(qw + (size_t)row * (N >> 1) + off);
      wp.s01 = sc[(size_t)row * ngroups_n + g];
    }
    if (row + 1 < k1 && col_ok) {
      wp.w1 = *reinterpret_cast<const uint2*>(qw + (size_t)(row + 1) * (N >> 1) + off);
      wp.s01 |= (uint32_t)sc[(size_t)(row + 1) * ngroups_n + g] << 16;
    }
  };
  // bf16(q * s) of both rows for each of the 16 columns, as one word per
  // column: the signed nibble is one bit-field extract, and the pair of
  // roundings one f32x2_to_bf16x2 (f32_to_bf16's bits, NaN included).
  auto stage = [&](int buf, const WPair& wp) {
    const float s0 = bf16_to_f32(wp.s01 & 0xFFFFu), s1 = bf16_to_f32(wp.s01 >> 16);
    const uint32_t a4[2] = {wp.w0.x, wp.w0.y}, b4[2] = {wp.w1.x, wp.w1.y};
    // word k/2 of column c sits at (k/2) ^ (16 * ((c / 16) & 3)): the four
    // 16-column groups written by one instruction land in different banks
    uint32_t* dst = reinterpret_cast<uint32_t*>(&wt[buf][scol][0]) + ((sr >> 1) ^ (scol & 48));
    constexpr int kColWords = kGemmTStride / 2;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        const float va = (float)(int)__builtin_amdgcn_sbfe(a4[i], 4 * b, 4) * s0;
        const float vb = (float)(int)__builtin_amdgcn_sbfe(b4[i], 4 * b, 4) * s1;
        dst[(8 * i + b) * kColWords] = f32x2_to_bf16x2(va, vb);
      }
    }
  };
  // B operand: token l16 of each tile, k .. k + 7 at column quarter kb
  const uint16_t* xrow[TM];
#pragma unroll
  for (int t = 0; t < TM; ++t) xrow[t] = x + (size_t)min(tok0 + t * 16 + l16, M - 1) * K;

  // x operands of one step: slice j, token tile t (zeros past the K range)
  auto load_x = [&](int step, uint4 (&dst)[kGemmTStep / 32][TM]) {
#pragma unroll
    for (int j = 0; j < kGemmTStep / 32; ++j) {
      const int kk = k0 + step * kGemmTStep + 32 * j + 8 * kb;
#pragma unroll
      for (int t = 0; t < TM; ++t)
        dst[j][t] = (step < nsteps && kk < k1) ? *reinterpret_cast<const uint4*>(xrow[t] + kk)
                                               : make_uint4(0, 0, 0, 0);
    }
  };
  // x one step ahead in registers for up to 32 tokens; the 64-token tiling
  // loads it in place (the extra registers would cost it occupancy)
  constexpr bool kXAhead = TM <= 2;
  [[maybe_unused]] uint4 xc[kGemmTStep / 32][TM];
  if constexpr (kXAhead) load_x(0, xc);

  WPair wq[kGemmTPrefetch];
#pragma unroll
  for (int p = 0; p < kGemmTPrefetch; ++p) {
    if (p < nsteps) load_w(p, wq[p]);
  }
  floatx4 acc[TM];
#pragma unroll
  for (int t = 0; t < TM; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
  if (nsteps > 0) stage(0, wq[0]);
  if (kGemmTPrefetch < nsteps) load_w(kGemmTPrefetch, wq[0]);
  __syncthreads();

  for (int i0 = 0; i0 < nsteps; i0 += kGemmTPrefetch) {
#pragma unroll
    for (int p = 0; p < kGemmTPrefetch; ++p) {
      const int i = i0 + p;
      if (i < nsteps) {
        const int buf = i & 1;
        // stage step i + 1 into the other buffer while this one is read
        if (i + 1 < nsteps) {
          const int pn = (p + 1) % kGemmTPrefetch;
          stage(buf ^ 1, wq[pn]);
          if (i + 1 + kGemmTPrefetch < nsteps) load_w(i + 1 + kGemmTPrefetch, wq[pn]);
        }
        if constexpr (kXAhead) {
          // the next step's x operands, in flight while this step multiplies
          uint4 xn[kGemmTStep / 32][TM];
          load_x(i + 1, xn);
#pragma unroll
          for (int j = 0; j < kGemmTStep / 32; ++j) {
            const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(
                &wt[buf][16 * wave + l16][(32 * j + 8 * kb) ^ (32 * (wave & 3))]);
#pragma unroll
            for (int t = 0; t < TM; ++t)
              acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, as_bf16x8(xc[j][t]), acc[t], 0,
                                                               0, 0);
          }
#pragma unroll
          for (int j = 0; j < kGemmTStep / 32; ++j)
#pragma unroll
            for (int t = 0; t < TM; ++t) xc[j][t] = xn[j][t];
        } else {
          const int kbase = k0 + i * kGemmTStep;
#pragma unroll
          for (int j = 0; j < kGemmTStep / 32; ++j) {
            const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(
                &wt[buf][16 * wave + l16][(32 * j + 8 * kb) ^ (32 * (wave & 3))]);
            const int kk = kbase + 32 * j + 8 * kb;
#pragma unroll
            for (int t = 0; t < TM; ++t) {
              uint4 bv = make_uint4(0, 0, 0, 0);
              if (kk < k1) bv = *reinterpret_cast<const uint4*>(xrow[t] + kk);
              acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, as_bf16x8(bv), acc[t], 0, 0, 0);
            }
          }
        }
        __syncthreads();
      }
    }
  }

#pragma unroll
  for (int t = 0; t < TM; ++t) {
    const int tok = tok0 + t * 16 + l16;
    if (tok >= M) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int col = n0 + 16 * wave + 4 * kb + r;
      if (col >= N) continue;
      if (part)
        part[((size_t)blockIdx.z * M + tok) * N + col] = acc[t][r];
      else
        out[(size_t)tok * N + col] = (uint16_t)f32_to_bf16(acc[t][r]);
    }
  }
}

// Sum of the K split's fp32 partials in split order, rounded to bf16.
__global__ __launch_bounds__(256) void int4_gemm_t_reduce_kernel(const float* __restrict__ part,
                                                                 uint16_t* __restrict__ out,
                                                                 size_t mn, int splits) {
  for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < mn; e += (size_t)gridDim.x * 256) {
    float v = 0.f;
    for (int z = 0; z < splits; ++z) v += part[(size_t)z * mn + e];
    out[e] = (uint16_t)f32_to_bf16(v);
  }
}

}  // namespace
}  // namespace dip

using namespace dip;

extern "C" int dip_int4_gemm(const int8_t* qweight, const uint16_t* scales, const uint16_t* x,
                             uint16_t* out, int64_t m, int64_t out_features,
                             int64_t in_features, void* stream) {
  if (!qweight || !scales) return DIP_ERR_NULL;
  if (m < 0 || out_features <= 0 || in_features <= 0 || in_features % kGroupSize != 0 ||
      out_features > INT32_MAX || in_features > (1 << 20) || m > 64 * 65535 ||
      m * out_features > ((int64_t)1 << 40))
    return DIP_ERR_SHAPE;
  if (m == 0) return DIP_OK;  // x and out may be NULL then
  if (!x || !out) return DIP_ERR_NULL;
  if (!aligned16(qweight) || !aligned16(x)) return DIP_ERR_ALIGN;
  const int M = (int)m, N = (int)out_features, K = (int)in_features;
  hipStream_t s = (hipStream_t)stream;
  if (N >= 8192)
    launch_tokens<4>(qweight, scales, x, out, M, N, K, s);
  else
    launch_tokens<2>(qweight, scales, x, out, M, N, K, s);
  return hip_status(hipGetLastError());
}

namespace {
// K split of dip_int4_gemm_t: about two workgroups per CU over the
// (64-column, 16*TM-token) tiles, at most 16 ranges, whole 128-row steps.
int gemm_t_splits(int64_t m, int64_t n, int64_t k) {
  const int64_t tm = m <= 16 ? 1 : (m <= 32 ? 2 : 4);
  const int64_t tiles = ((n + 63) / 64) * ((m + 16 * tm - 1) / (16 * tm));
  const int64_t want = (2LL * device_cus() + tiles - 1) / tiles;
  const int64_t max_split = (k + kGemmTStep - 1) / kGemmTStep;
  return (int)std::max<int64_t>(1, std::min<int64_t>(std::min<int64_t>(want, 16), max_split));
}
}  // namespace

extern "C" size_t dip_int4_gemm_t_workspace_size(int64_t m, int64_t out_features,
                                                 int64_t in_features) {
  if (m <= 0 || out_features <= 0 || in_features <= 0) return 0;
  const int splits = gemm_t_splits(m, out_features, in_features);
  return splits > 1 ? (size_t)splits * (size_t)m * (size_t)out_features * sizeof(float) : 0;
}

extern "C" int dip_int4_gemm_t(const int8_t* qweight_t, const uint16_t* scales_t,
                               const uint16_t* x, uint16_t* out, int64_t m, int64_t out_features,
                               int64_t in_features, void* workspace, size_t ws_bytes,
                               void* stream) {
  if (!qweight_t || !scales_t) return DIP_ERR_NULL;
  if (m < 0 || out_features <= 0 || in_features <= 0 || out_features % kGroupSize != 0 ||
      in_features % 8 != 0 || out_features > (1 << 20) || in_features > INT32_MAX / 2 ||
      m > 64 * 65535 || m * out_features > ((int64_t)1 << 40))
    return DIP_ERR_SHAPE;
  if (m == 0) return DIP_OK;
  if (!x || !out) return DIP_ERR_NULL;
  if (!aligned16(qweight_t) || !aligned16(x)) return DIP_ERR_ALIGN;
  const int M = (int)m, N = (int)out_features, K = (int)in_features;
  const int TM = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  const int gy = (M + 16 * TM - 1) / (16 * TM);
  const int gx = (N + 63) / 64;
  int splits = gemm_t_splits(m, out_features, in_features);
  const size_t need = splits > 1 ? (size_t)splits * (size_t)M * (size_t)N * sizeof(float) : 0;
  if (need > 0 && (!workspace || ws_bytes < need)) return DIP_ERR_WORKSPACE;
  if (splits > 1 && !aligned16(workspace)) return DIP_ERR_ALIGN;
  const int kchunk = ((K + splits - 1) / splits + kGemmTStep - 1) / kGemmTStep * kGemmTStep;
  splits = (K + kchunk - 1) / kchunk;
  float* part = splits > 1 ? static_cast<float*>(workspace) : nullptr;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid(gx, gy, splits);
  if (TM == 1)
    hipLaunchKernelGGL(int4_gemm_t_kernel<1>, grid, dim3(kGemmThreads), 0, s, qweight_t, scales_t,
                       x, out, part, M, N, K, kchunk);
  else if (TM == 2)
    hipLaunchKernelGGL(int4_gemm_t_kernel<2>, grid, dim3(kGemmThreads), 0, s, qweight_t, scales_t,
                       x, out, part, M, N, K, kchunk);
  else
    hipLaunchKernelGGL(int4_gemm_t_kernel<4>, grid, dim3(kGemmThreads), 0, s, qweight_t, scales_t,
                       x, out, part, M, N, K, kchunk);
  if (splits > 1) {
    const size_t mn = (size_t)M * N;
    const unsigned blocks = (unsigned)std::min<size_t>((mn + 255) / 256, 2048);
    hipLaunchKernelGGL(int4_gemm_t_reduce_kernel, dim3(blocks), dim3(256), 0, s, part, out, mn,
                       splits);
  }
  return hip_status(hipGetLastError());
}
