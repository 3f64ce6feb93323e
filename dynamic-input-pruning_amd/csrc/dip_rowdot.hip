// dip_rowdot.hip — int4 g128 row-dot kernels: gate GEMV (+SiLU), up-row gather
// GEMV (+ fused h = g[idx] * u) and the cache-aware dual-source variant.
//
// Mapping (one design for every row source; the row-group layout and the x
// pairs are described in dip_tiles.h):
//   * A workgroup holds 256/LPR groups of LPR lanes; a group
//     handles ROWS outputs j = grp + i*ngrp (i < ROWS), ROWS a compile-time
//     constant, so the row loop is straight-line code: every load is
//     unconditional (row indices past the end are clamped, bad row ids read a
//     designated safe row and are poisoned in the epilogue) and the compiler
//     can wait for exactly the row it consumes (s_waitcnt vmcnt(N) with N > 0)
//     while the next row stays in flight.  Loads under data-dependent
//     branches would make it wait for everything.
//   * Workgroups are 256 threads (plan_rowdot): a Qwen3-32B gate runs exactly
//     2 per CU, 512 workgroups of 8 groups, split over two tiers (the first
//     256 workgroups 9 rows per group, the rest 3-4: row_tier_rows; the
//     Qwen3-8B gate and the Qwen3-32B q|k|v and o GEMVs likewise); its up
//     gather 480 of 8 groups x 4 rows.
//   * x pairs: XS (the hot widths): the workgroup stages all pairs once in LDS
//     and each lane copies its CH chunks' pairs into VGPRs, so the row loop
//     touches no LDS; otherwise each lane builds its own pairs from global
//     memory.  The x loads are issued before the row loads.
//   * The group reduction is DPP + permlane swaps (group_sum); lane l keeps
//     the sum of row l and runs the epilogue for it.
#include <algorithm>

#include "dip_tiles.h"

namespace dip {

#ifdef DIP_WG_STAMPS
__device__ dip_wg_stamps g_stamps_rowdot;
int timeline_read_rowdot(dip_wg_stamps* dst) {
  return hip_status(hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_stamps_rowdot), sizeof(dip_wg_stamps), 0,
                                        hipMemcpyDeviceToHost));
}
#else
int timeline_read_rowdot(dip_wg_stamps*) { return DIP_ERR_UNSUPPORTED; }
#endif

constexpr int kRowdotMaxThreads = 256;

// Rows row_base + grp + i*ngrp (i < ROWS) below row_end, for group grp.
template <int LPR, int CH, int SRC, int EPI, bool XS, int ROWS, bool NORM>
__device__ __forceinline__ void rowdot_rows(const RowdotArgs& a, const int grp, const int ngrp,
                                            const int row_base, const int row_end) {
  constexpr int D = ROWS < 2 ? ROWS : 2;  // rows of loads in flight per group
  static_assert(ROWS <= LPR, "rows per group");
  extern __shared__ __align__(16) uint32_t xlds[];
  const int l = threadIdx.x % LPR;
  const int lane = threadIdx.x & 63;
  const int gbase = lane - l;  // first lane of my group within the wave
  const size_t row_bytes = (size_t)(a.in_features >> 1);
  const int ngroups = a.in_features >> 7;
  const int nchunks = a.in_features / kChunkCols;

  // 1. x loads first (XS: one chunk per thread, index clamped; NORM: h, the
  // residual addend and the norm weight in 8-value units spread over all
  // threads)
  constexpr int UPT = NORM ? (LPR * CH * 4 + kRowdotMaxThreads - 1) / kRowdotMaxThreads : 1;
  uint4 xs[XS ? 4 : CH * 4];
  [[maybe_unused]] uint4 nh[UPT], na[UPT], nw[UPT];
  if constexpr (NORM) {
    load_x_units<UPT>(a.x, nchunks * 4, nh);
    load_x_units<UPT>(a.norm_w, nchunks * 4, nw);
    if (a.norm_add) {
      load_x_units<UPT>(a.norm_add, nchunks * 4, na);
    } else {
#pragma unroll
      for (int j = 0; j < UPT; ++j) na[j] = make_uint4(0, 0, 0, 0);
    }
  } else if constexpr (XS) {
    load_x_chunk(a.x, nchunks, xs);
  } else {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const uint4* src = reinterpret_cast<const uint4*>(a.x) + (l + LPR * c) * 4;
#pragma unroll
      for (int i = 0; i < 4; ++i) xs[4 * c + i] = src[i];
    }
  }

  // (the x loads stay ahead of the row loads: staging x then waits only for
  // them, not for the first rows as well)
  __builtin_amdgcn_sched_barrier(0);

  // 2. row ids: lane l resolves row l of the group (clamped, unconditional)
  const long long jl = row_base + grp + (long long)l * ngrp;
  const bool valid_l = l < ROWS && jl < row_end;
  const uint32_t rid_lane = resolve_row<SRC>(a, (int)min(jl, (long long)row_end - 1));

  // 3. first D rows of loads
  RowRegs<CH> ring[D];
#pragma unroll
  for (int d = 0; d < D; ++d)
    load_row<LPR, CH, SRC>(a, __shfl(rid_lane, gbase + d, 64), l, row_bytes, ngroups, ring[d]);

  // 3b. Workgroup 0's rotation of the decode step's next speculation key
  // into the slot in use (stored at the end).  Loaded after x and the first
  // rows, so that waiting for those never waits for it; read at a
  // lane-dependent offset that is always 0 (in_features < 2^30), since as a
  // uniform value the compiler would move it to a scalar register right after
  // the load and wait for it there.
  const uint32_t zero = threadIdx.x & ((uint32_t)a.in_features >> 30);
  const bool rot = a.rotate && blockIdx.x == 0 && threadIdx.x == 0;
  const uint32_t rot1 = rot ? a.rotate[1 + zero] : 0u;

  // 4. x pairs into VGPRs
  uint32_t xp[CH][4][4];
  float bias[CH];
  if constexpr (XS) {
    if constexpr (NORM)
      norm_stage_x<LPR, UPT>(nh, na, nw, nchunks, a.norm_eps, a.norm_h_out, a.norm_x_out,
                             reinterpret_cast<float*>(xlds + x_pairs_lds_bytes(a.in_features) / 4),
                             xlds);
    else
      stage_x_pairs<LPR>(xs, xlds, nchunks);
    x_pairs_to_regs<LPR, CH>(xlds, nchunks, l, xp, bias);
  } else {
#pragma unroll
    for (int c = 0; c < CH; ++c) pairs_of(&xs[4 * c], xp[c], bias[c]);
  }

  // 5. rows
  float mine = 0.f;  // reduced dot product of row l
#pragma unroll
  for (int i = 0; i < ROWS; ++i) {
    RowRegs<CH>& R = ring[i % D];
    float acc = row_dot_part<CH>(R, xp, bias);
    // the slot's registers are free once its products are taken: reload it
    // before the cross-lane reduction, so the next row is in flight sooner
    if (i + D < ROWS)
      load_row<LPR, CH, SRC>(a, __shfl(rid_lane, gbase + i + D, 64), l, row_bytes, ngroups, R);
    acc = group_sum<LPR>(acc);
    mine = l == i ? acc : mine;
  }

  // 6. epilogue: lane l finishes row l
  uint32_t v = 0;
  if (valid_l) {
    if (rid_lane == kBadRow) {
      v = 0x7FC0u;
    } else {
      v = f32_to_bf16(mine);
      if (EPI == kSilu) {
        const float f = bf16_to_f32(v);
        v = f32_to_bf16(f / (1.0f + expf(-f)));
      } else if (EPI == kH) {
        // a gathered row id is already range-checked against g (rows = channels)
        const int ch = (SRC == kGather) ? (int)rid_lane : a.gid[(int)jl];
        if (SRC != kGather && (unsigned)ch >= (unsigned)a.g_len)
          v = 0x7FC0u;
        else
          v = f32_to_bf16(bf16_to_f32(a.g[ch]) * bf16_to_f32(v));
      }
    }
    a.out[(int)jl] = (uint16_t)v;
  }
  if (rot) a.rotate[0] = rot1;
}

// R1 > 0: two tiers of workgroups, ROWS rows per group in the first
// (blockIdx < a.tier_wgs, rows [0, a.tier_rows)) and R1 in the second.
template <int LPR, int CH, int SRC, int EPI, bool XS, int ROWS, bool NORM = false, int R1 = 0>
__global__ __launch_bounds__(kRowdotMaxThreads) void rowdot_kernel(RowdotArgs a) {
  static_assert(!NORM || XS, "the RMSNorm prologue needs the staged x");
  DIP_STAMP_START(g_stamps_rowdot);
  constexpr int G = kRowdotMaxThreads / LPR;
  const int b = (int)blockIdx.x;
  const int gw = (int)threadIdx.x / LPR;
  if constexpr (R1 > 0) {
    const int ngrp = a.tier_wgs * G;  // groups per tier
    if (b < a.tier_wgs)
      rowdot_rows<LPR, CH, SRC, EPI, XS, ROWS, NORM>(a, b * G + gw, ngrp, 0, a.tier_rows);
    else
      rowdot_rows<LPR, CH, SRC, EPI, XS, R1, NORM>(a, (b - a.tier_wgs) * G + gw, ngrp,
                                                   a.tier_rows, a.nrows);
  } else {
    rowdot_rows<LPR, CH, SRC, EPI, XS, ROWS, NORM>(a, b * G + gw, a.ngrp, 0, a.nrows);
  }
  DIP_STAMP_END(g_stamps_rowdot);
}

// ---------------------------------------------------------------------------
// Host dispatch
// ---------------------------------------------------------------------------
namespace {

struct RowdotPlan {
  int rows;    // per group
  int groups;  // per workgroup
  int blocks;
};

// The grid for nrows outputs.  Contiguous rows (the gate): exactly
// CUs * wgs_per_cu 256-thread workgroups whenever at most 8 rows per group
// cover the outputs, so every CU gets the same number of workgroups; a group
// handles ROWS = ceil(rows per group) outputs, the groups past
// nrows - (ROWS-1)*ngrp one fewer.  (On the Qwen3-32B gate, 512 workgroups of
// 6-7 rows per group took 15.2 us against 16.2 us for 400 workgroups of 8:
// with 1.56 workgroups per CU, 144 CUs carried twice the rows of the other
// 112.  Three workgroups per CU of 4-5 rows took 15.9 us.)  Gathered rows
// keep the fewest of 1, 2, 4, 8 rows per group that hold the grid near
// wgs_per_cu per CU (the 15360-row up gather: 480 x 8 x 4 rows, 9.9 us,
// against 10.1 us for 512 x 8 x 3-4 rows).
RowdotPlan plan_rowdot(int nrows, int lpr, bool balanced, int wgs_per_cu) {
  const int groups = 256 / lpr;
  const long long wgs = (long long)device_cus() * wgs_per_cu;
  const long long need = (nrows + wgs * groups - 1) / (wgs * groups);
  if (need <= 1)  // one row per group: no more workgroups than the rows fill
    return RowdotPlan{1, groups, (int)std::max(1LL, std::min(wgs, (nrows + groups - 1LL) / groups))};
  if (balanced && need <= 8) return RowdotPlan{(int)need, groups, (int)wgs};
  int rows = 1;
  while (rows < 8 && rows < lpr && (long long)rows * wgs * groups < nrows) rows *= 2;
  return RowdotPlan{rows, groups, (nrows + rows * groups - 1) / (rows * groups)};
}

// Workgroups of the SiLU gate instance for `rows` rows per group that fit a
// CU at once (cached per instance).
template <int LPR, int CH>
int gate_occupancy(int rows) {
  static int cache[9] = {};
  if (rows < 1 || rows > 8) return 0;
  if (!cache[rows]) {
    const void* f = nullptr;
    switch (rows) {
#define DIP_ROWS(R) \
      case R: f = reinterpret_cast<const void*>(&rowdot_kernel<LPR, CH, kContig, kSilu, true, R>); break;
      DIP_ROWS(1) DIP_ROWS(2) DIP_ROWS(3) DIP_ROWS(4) DIP_ROWS(5) DIP_ROWS(6) DIP_ROWS(7)
#undef DIP_ROWS
      default: f = reinterpret_cast<const void*>(&rowdot_kernel<LPR, CH, kContig, kSilu, true, 8>); break;
    }
    const size_t lds = x_pairs_lds_bytes(LPR * CH * kChunkCols);
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, f, kRowdotMaxThreads, lds) != hipSuccess)
      nb = 0;
    cache[rows] = nb + 1;
  }
  return cache[rows] - 1;
}

// Contiguous row-dot GEMVs at two workgroups per CU, split over two tiers.
// The first workgroup each CU receives (blockIdx < CUs) wins its SIMDs'
// issue arbitration over the second: on the Qwen3-32B gate at an even split
// (6-7 rows per lane group in both) the first tier ends at about 9.7 us and
// the second at about 12 us.  Giving the first tier more of the rows ends
// them together (rows per group-column = nrows / groups per tier):
//   * the Qwen3-32B SiLU gate (hidden 5120, 12.5 per group-column on 256
//     CUs): 9 and 3.5 rows, 13.5 -> 12.9-13.2 us per launch (8, 8.5, 9.5,
//     10 or 10.5 rows in the first tier gained less or lost);
//   * the Qwen3-8B SiLU gate (hidden 4096, 6 per group-column): 5 and 1
//     rows at two workgroups per CU instead of 2 rows in each of three,
//     7.3-7.6 -> 6.5-6.7 us (4 : 2 gave 7.0-7.1 us, one workgroup per CU
//     with 6 rows 6.9-7.0; 3.5 : 2.5, 4.5 : 1.5 and 5.5 : 0.5, whose second
//     tier ends on a partly clamped row, were slower);
//   * the Qwen3-32B q|k|v GEMV (10240 rows x 5120, 5 per group-column) and
//     o projection (5120 rows x 8192, 64-lane groups, 5 per group-column):
//     4 and 1 rows each, the whole-model decode 223.5-223.7 -> 228.8 tok/s
//     (each alone 226.2-226.3).
// Every row is still one group's dot product in the same order, so the
// output is bit for bit the even split's.  Returns the rows per group of
// the first tier for a GEMV of `chunks` 32-column chunks with `lpr`-lane
// groups and epilogue `epi`, 0 where no split was measured.
int row_tier_rows(int nrows, int lpr, int chunks, int epi) {
  if (!tuning(DIP_TUNE_ROW_TIERS) || lpr <= 0) return 0;
  const long long g = (long long)device_cus() * (kRowdotMaxThreads / lpr);  // groups per tier
  // the SiLU gate, and the up rows with h over every channel (the dense
  // step's up launch: the gate's shape, rows gathered through idx)
  const bool gate_like = epi == kSilu || epi == kH;
  if (gate_like && lpr == 32 && chunks == 160 && nrows > 12 * g && nrows <= 13 * g) return 9;
  if (gate_like && lpr == 32 && chunks == 128 && nrows == 6 * g) return 5;
  if (epi == kRaw && lpr == 32 && chunks == 160 && nrows == 5 * g) return 4;
  if (epi == kRaw && lpr == 64 && chunks == 256 && nrows == 5 * g) return 4;
  return 0;
}

// Workgroups per CU of a row-dot grid: the tuning knob when set, else for
// the SiLU gate two where a two-tier split applies (row_tier_rows, above),
// three where the instance three workgroups per CU would pick still fits
// three at once (the Qwen3-8B gate with its tiers off: 2 rows per group, 97
// VGPRs; 8.0 -> 7.4 us against an even split at two), else two (the
// Qwen3-32B gate would need 5 rows per group at 231 VGPRs, two waves per
// SIMD: 13.5 -> 17.2 us); every other grid two.
// The gate with the RMSNorm prologue keeps two: every workgroup normalises
// x itself, and a third per CU cost more than it gained (the whole Qwen3-8B
// model: 477 against 487 tok/s).
int rowdot_wpc(int nrows, int chunks, bool gate, bool norm) {
  const int t = tuning(DIP_TUNE_ROWDOT_WGS_PER_CU);
  if (t > 0) return t;
  if (!gate || norm) return 2;
  if (row_tier_rows(nrows, chunks == 80 ? 16 : 32, chunks, kSilu)) return 2;
  int lpr = 0, occ = 0;
  if (chunks == 160) lpr = 32;
  else if (chunks == 128) lpr = 32;
  else if (chunks == 80) lpr = 16;
  else return 2;
  const int rows = plan_rowdot(nrows, lpr, true, 3).rows;
  if (chunks == 160) occ = gate_occupancy<32, 5>(rows);
  else if (chunks == 128) occ = gate_occupancy<32, 4>(rows);
  else occ = gate_occupancy<16, 5>(rows);
  return occ >= 3 ? 3 : 2;
}

template <int LPR, int CH, int SRC, int EPI, bool XS, int ROWS, bool NORM = false>
void launch_variant(RowdotArgs a, const RowdotPlan& p, hipStream_t stream) {
  a.ngrp = p.blocks * p.groups;
  const size_t lds = XS ? x_pairs_lds_bytes(a.in_features) + (NORM ? 16 : 0) : 0;
  // the two-tier splits, instantiated for the measured shapes only (with or
  // without the folded RMSNorm where the width has it; the gathered up + h
  // rows take the gate's split whatever grid their own plan chose)
  if constexpr (XS &&
                ((SRC == kContig &&
                  ((EPI == kSilu && LPR == 32 && (CH == 5 || CH == 4)) ||
                   (EPI == kRaw && ((LPR == 32 && CH == 5) || (LPR == 64 && CH == 4))))) ||
                 (SRC == kGather && EPI == kH && !NORM && LPR == 32 && (CH == 5 || CH == 4)))) {
    constexpr int R0 = EPI == kRaw ? 4 : (CH == 5 ? 9 : 5);
    constexpr int R1 = EPI == kRaw ? 1 : (CH == 5 ? 4 : 1);
    const int cus = device_cus();
    if ((SRC == kGather || p.blocks == 2 * cus) && p.groups * LPR == kRowdotMaxThreads &&
        row_tier_rows(a.nrows, LPR, LPR * CH, EPI) == R0) {
      a.tier_wgs = cus;
      a.tier_rows = R0 * cus * p.groups;
      a.ngrp = 2 * cus * p.groups;
      hipLaunchKernelGGL((rowdot_kernel<LPR, CH, SRC, EPI, XS, R0, NORM, R1>), dim3(2 * cus),
                         dim3(p.groups * LPR), lds, stream, a);
      return;
    }
  }
  hipLaunchKernelGGL((rowdot_kernel<LPR, CH, SRC, EPI, XS, ROWS, NORM>), dim3(p.blocks),
                     dim3(p.groups * LPR), lds, stream, a);
}

template <int LPR, int CH, int SRC, int EPI, bool NORM = false>
int launch_one(const RowdotArgs& a, hipStream_t stream) {
  // the widths of Qwen3-4B/8B/14B/32B (hidden and, at 8192, the 32B o
  // projection's input) stage x through LDS; every ROWS the plan can pick
  // is instantiated
  constexpr bool hot = (LPR == 32 && (CH == 5 || CH == 4)) || (LPR == 16 && CH == 5) ||
                       (LPR == 64 && CH == 4);
  if constexpr (hot) {
    const RowdotPlan p = plan_rowdot(a.nrows, LPR, SRC == kContig,
                                     rowdot_wpc(a.nrows, LPR * CH, SRC == kContig && EPI == kSilu,
                                                NORM));
    if constexpr (SRC == kContig) {  // balanced plan: any rows per group up to 8
      switch (p.rows) {
        case 1: launch_variant<LPR, CH, SRC, EPI, true, 1, NORM>(a, p, stream); break;
        case 2: launch_variant<LPR, CH, SRC, EPI, true, 2, NORM>(a, p, stream); break;
        case 3: launch_variant<LPR, CH, SRC, EPI, true, 3, NORM>(a, p, stream); break;
        case 4: launch_variant<LPR, CH, SRC, EPI, true, 4, NORM>(a, p, stream); break;
        case 5: launch_variant<LPR, CH, SRC, EPI, true, 5, NORM>(a, p, stream); break;
        case 6: launch_variant<LPR, CH, SRC, EPI, true, 6, NORM>(a, p, stream); break;
        case 7: launch_variant<LPR, CH, SRC, EPI, true, 7, NORM>(a, p, stream); break;
        default: launch_variant<LPR, CH, SRC, EPI, true, 8, NORM>(a, p, stream); break;
      }
    } else {  // power-of-two plan: 1, 2, 4 or 8
      switch (p.rows) {
        case 1: launch_variant<LPR, CH, SRC, EPI, true, 1, NORM>(a, p, stream); break;
        case 2: launch_variant<LPR, CH, SRC, EPI, true, 2, NORM>(a, p, stream); break;
        case 4: launch_variant<LPR, CH, SRC, EPI, true, 4, NORM>(a, p, stream); break;
        default: launch_variant<LPR, CH, SRC, EPI, true, 8, NORM>(a, p, stream); break;
      }
    }
  } else {
    static_assert(!NORM, "the RMSNorm prologue is built for the staged widths only");
    const int rows = LPR >= 4 ? 4 : LPR;
    const int groups = 256 / LPR;
    const RowdotPlan p{rows, groups, (a.nrows + rows * groups - 1) / (rows * groups)};
    launch_variant<LPR, CH, SRC, EPI, false, (LPR >= 4 ? 4 : LPR)>(a, p, stream);
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
  DIP_TRY(64, 4)   // 8192 (Qwen3-32B o_proj: 64 heads x 128)
  DIP_TRY(32, 1)   // 1024
  DIP_TRY(16, 3)   // 1536
  DIP_TRY(16, 1)   // 512
  DIP_TRY(8, 1)    // 256
  DIP_TRY(4, 1)    // 128
#undef DIP_TRY
  return DIP_ERR_UNSUPPORTED;
}

}  // namespace

int rowdot_contig_blocks(int64_t nrows, int64_t in_features, bool norm) {
  const int64_t chunks = in_features / kChunkCols;
  const int lpr = (chunks == 80 || chunks == 48 || chunks == 16) ? 16 : (chunks == 256 ? 64 : 32);
  return plan_rowdot((int)nrows, lpr, true, rowdot_wpc((int)nrows, (int)chunks, true, norm)).blocks;
}

bool rowdot_norm_supported(int64_t in_features) {
  const int64_t chunks = in_features / kChunkCols;
  return in_features % kChunkCols == 0 && (chunks == 160 || chunks == 128 || chunks == 80);
}

template <int EPI>
int launch_norm_epi(const RowdotArgs& a, hipStream_t stream) {
  const int chunks = a.in_features / kChunkCols;
  if (chunks == 160) return launch_one<32, 5, kContig, EPI, true>(a, stream);
  if (chunks == 128) return launch_one<32, 4, kContig, EPI, true>(a, stream);
  if (chunks == 80) return launch_one<16, 5, kContig, EPI, true>(a, stream);
  return DIP_ERR_UNSUPPORTED;
}

int launch_rowdot_norm(int epi, const RowdotArgs& a, hipStream_t stream) {
  if (a.nrows == 0) return DIP_OK;
  if (epi == kRaw) return launch_norm_epi<kRaw>(a, stream);
  if (epi == kSilu) return launch_norm_epi<kSilu>(a, stream);
  return DIP_ERR_ARG;
}

int launch_spec_after_gate(const uint16_t* g, int64_t inter, int64_t hidden, int64_t k,
                           int32_t* idx, uint16_t* h_full, const int8_t* up_qw,
                           const uint16_t* up_sc, const uint16_t* x, void* workspace,
                           void* state, hipStream_t stream) {
  SpecArgs sp{};
  sp.up_qw = up_qw;
  sp.up_sc = up_sc;
  sp.x = x;
  sp.h_full = h_full;
  sp.state = static_cast<uint32_t*>(state);
  sp.hidden = (int)hidden;
  return launch_topk_spec(g, inter, k, idx, workspace, sp, stream);
}

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
  a.qw_safe = qw;
  a.sc_safe = sc;
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

extern "C" int dip_int4_gemv_rmsnorm(const int8_t* qweight, const uint16_t* scales,
                                     const uint16_t* h, const uint16_t* add,
                                     const uint16_t* norm_w, float eps, uint16_t* h_out,
                                     uint16_t* out, int64_t out_features, int64_t in_features,
                                     void* stream) {
  int st = check_matrix(qweight, scales, out_features, in_features);
  if (st) return st;
  if (!h || !norm_w || !out) return DIP_ERR_NULL;
  if (!rowdot_norm_supported(in_features)) return DIP_ERR_UNSUPPORTED;
  if (!(eps >= 0.f)) return DIP_ERR_ARG;
  if (!aligned16(h) || !aligned16(norm_w) || (add && !aligned16(add)) ||
      (h_out && !aligned16(h_out)))
    return DIP_ERR_ALIGN;
  if (h_out && (h_out == h || h_out == add)) return DIP_ERR_ARG;  // read while written
  RowdotArgs a = base_args(qweight, scales, h, out, out_features, in_features);
  a.norm_w = norm_w;
  a.norm_add = add;
  a.norm_h_out = h_out;
  a.norm_eps = eps;
  return launch_rowdot_norm(kRaw, a, (hipStream_t)stream);
}

extern "C" int dip_gate_silu_topk(const int8_t* gate_qw, const uint16_t* gate_sc,
                                  const uint16_t* x, uint16_t* g, int32_t* idx, int64_t inter,
                                  int64_t hidden, int64_t k, void* workspace, size_t ws_bytes,
                                  void* stream) {
  int st = check_matrix(gate_qw, gate_sc, inter, hidden);
  if (st) return st;
  if (!x || !g) return DIP_ERR_NULL;
  if (!aligned16(x) || !aligned16(g)) return DIP_ERR_ALIGN;
  if (inter > kTopkMaxN || k < 0 || k > INT32_MAX) return DIP_ERR_SHAPE;
  if (k > 0 && !idx) return DIP_ERR_NULL;
  if (!workspace || ws_bytes < dip_topk_workspace_size(inter)) return DIP_ERR_WORKSPACE;
  if (!aligned16(workspace)) return DIP_ERR_ALIGN;
  RowdotArgs a = base_args(gate_qw, gate_sc, x, g, inter, hidden);
  st = launch_rowdot(kContig, kSilu, a, (hipStream_t)stream);
  if (st || k == 0) return st;
  return launch_topk_select(g, inter, k, idx, workspace, (hipStream_t)stream);
}

extern "C" size_t dip_mlp_state_size(void) { return kMlpStateWords * sizeof(uint32_t); }

extern "C" int dip_gate_silu_topk_spec(const int8_t* gate_qw, const uint16_t* gate_sc,
                                       const int8_t* up_qw, const uint16_t* up_sc,
                                       const uint16_t* x, uint16_t* g, int32_t* idx,
                                       uint16_t* h_full, int64_t inter, int64_t hidden,
                                       int64_t k, void* workspace, size_t ws_bytes, void* state,
                                       void* stream) {
  int st = check_matrix(gate_qw, gate_sc, inter, hidden);
  if (st) return st;
  st = check_matrix(up_qw, up_sc, inter, hidden);
  if (st) return st;
  if (!x || !g || !idx || !h_full || !state) return DIP_ERR_NULL;
  if (!aligned16(x) || !aligned16(g) || (reinterpret_cast<uintptr_t>(state) & 3u))
    return DIP_ERR_ALIGN;
  if (inter > kTopkMaxN || k < 1 || k > inter) return DIP_ERR_SHAPE;
  if (!topk_spec_supported(hidden)) return DIP_ERR_UNSUPPORTED;
  if (!workspace || ws_bytes < dip_topk_workspace_size(inter)) return DIP_ERR_WORKSPACE;
  if (!aligned16(workspace)) return DIP_ERR_ALIGN;
  RowdotArgs a = base_args(gate_qw, gate_sc, x, g, inter, hidden);
  a.rotate = static_cast<uint32_t*>(state);
  st = launch_rowdot(kContig, kSilu, a, (hipStream_t)stream);
  if (st) return st;
  return launch_spec_after_gate(g, inter, hidden, k, idx, h_full, up_qw, up_sc, x, workspace,
                                state, (hipStream_t)stream);
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
  if (rows == 0) return DIP_ERR_SHAPE;  // every index would be out of range
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
  if (rows == 0) return DIP_ERR_SHAPE;  // every index would be out of range
  RowdotArgs a = base_args(qweight, scales, x, h, k, in_features);
  a.sel = indices;
  a.g = g;
  a.rows_a = (int)rows;
  return launch_rowdot(kGather, kH, a, (hipStream_t)stream);
}

extern "C" int dip_ca_fused_gemv(const int8_t* res_qw, const uint16_t* res_sc,
                                 const int8_t* str_qw, const uint16_t* str_sc, const uint16_t* x,
                                 const int32_t* src, const int32_t* row, const uint16_t* g,
                                 const int32_t* gid, int64_t g_len, uint16_t* out,
                                 int64_t res_rows, int64_t str_rows, int64_t in_features,
                                 int64_t k, void* stream) {
  int st = check_matrix(res_qw, res_sc, res_rows, in_features);
  if (st) return st;
  st = check_matrix(str_qw, str_sc, str_rows, in_features);
  if (st) return st;
  if (k < 0 || k > INT32_MAX) return DIP_ERR_SHAPE;
  if (k == 0) return DIP_OK;
  if (!x || !out || !src || !row) return DIP_ERR_NULL;
  if (g && !gid) return DIP_ERR_NULL;
  if (g && (g_len <= 0 || g_len > INT32_MAX)) return DIP_ERR_SHAPE;
  if (!aligned16(x)) return DIP_ERR_ALIGN;
  if (res_rows == 0 && str_rows == 0) return DIP_ERR_SHAPE;
  RowdotArgs a = base_args(res_qw, res_sc, x, out, k, in_features);
  a.qw_b = str_qw;
  a.sc_b = str_sc;
  if (res_rows == 0) {
    a.qw_safe = str_qw;
    a.sc_safe = str_sc;
  }
  a.sel = src;
  a.sel2 = row;
  a.g = g;
  a.gid = gid;
  a.g_len = g ? (int)g_len : 0;
  a.rows_a = (int)res_rows;
  a.rows_b = (int)str_rows;
  return launch_rowdot(kDual, g ? kH : kRaw, a, (hipStream_t)stream);
}
