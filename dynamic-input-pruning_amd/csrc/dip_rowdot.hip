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
//     2 per CU, 512 workgroups of 8 groups x 6-7 rows; its up gather 480 of
//     8 groups x 4 rows.
//   * x pairs: XS (the hot widths): the workgroup stages all pairs once in LDS
//     and each lane copies its CH chunks' pairs into VGPRs, so the row loop
//     touches no LDS; otherwise each lane builds its own pairs from global
//     memory.  The x loads are issued before the row loads.
//   * The group reduction is DPP + permlane swaps (group_sum); lane l keeps
//     the sum of row l and runs the epilogue for it.
#include <algorithm>

#include "dip_tiles.h"

namespace dip {

constexpr int kRowdotMaxThreads = 256;

template <int LPR, int CH, int SRC, int EPI, bool XS, int ROWS, bool NORM = false>
__global__ __launch_bounds__(kRowdotMaxThreads) void rowdot_kernel(RowdotArgs a) {
  static_assert(!NORM || XS, "the RMSNorm prologue needs the staged x");
  constexpr int D = ROWS < 2 ? ROWS : 2;  // rows of loads in flight per group
  static_assert(ROWS <= LPR, "rows per group");
  extern __shared__ __align__(16) uint32_t xlds[];
  const int l = threadIdx.x % LPR;
  const int lane = threadIdx.x & 63;
  const int gbase = lane - l;  // first lane of my group within the wave
  const size_t row_bytes = (size_t)(a.in_features >> 1);
  const int ngroups = a.in_features >> 7;
  const int nchunks = a.in_features / kChunkCols;
  const int grp = blockIdx.x * (blockDim.x / LPR) + threadIdx.x / LPR;
  const int ngrp = a.ngrp;

  // 1. x loads first (XS: one chunk per thread, index clamped)
  uint4 xs[XS ? 4 : CH * 4];
  [[maybe_unused]] uint4 xa[NORM ? 4 : 1], xw[NORM ? 4 : 1];
  if constexpr (XS) {
    load_x_chunk(a.x, nchunks, xs);
    if constexpr (NORM) {
      load_x_chunk(a.norm_w, nchunks, xw);
      if (a.norm_add) {
        load_x_chunk(a.norm_add, nchunks, xa);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) xa[i] = make_uint4(0, 0, 0, 0);
      }
    }
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
  const long long jl = grp + (long long)l * ngrp;
  const bool valid_l = l < ROWS && jl < a.nrows;
  const uint32_t rid_lane = resolve_row<SRC>(a, (int)min(jl, (long long)a.nrows - 1));

  // 3. first D rows of loads
  RowRegs<CH> ring[D];
#pragma unroll
  for (int d = 0; d < D; ++d)
    load_row<LPR, CH, SRC>(a, __shfl(rid_lane, gbase + d, 64), l, row_bytes, ngroups, ring[d]);

  // 3b. The layer state of a decode step: the fused step's speculation key
  // and key band (its finish launch rewrites them, never this launch), and
  // workgroup 0's rotation of the four-launch step's next key into the slot
  // in use (stored at the end).  Loaded after x and the first rows, so that
  // waiting for those never waits for these; read at a lane-dependent offset
  // that is always 0 (in_features < 2^30), since as a uniform value the
  // compiler would move it to a scalar register right after the load and
  // wait for it there.
  const uint32_t zero = threadIdx.x & ((uint32_t)a.in_features >> 30);
  [[maybe_unused]] uint32_t cand_key = 0, band = 0;
  if constexpr (SRC == kContig && EPI == kSilu)
    if (a.cand_count) {
      cand_key = a.spec[1 + zero];
      band = a.spec[2 + zero];
    }
  const bool rot = a.rotate && blockIdx.x == 0 && threadIdx.x == 0;
  const uint32_t rot1 = rot ? a.rotate[1 + zero] : 0u;

  // 4. x pairs into VGPRs
  uint32_t xp[CH][4][4];
  float bias[CH];
  if constexpr (XS) {
    if constexpr (NORM)
      norm_x_chunk(xs, xa, xw, nchunks, a.norm_eps, a.norm_h_out, a.norm_x_out,
                   reinterpret_cast<float*>(xlds + x_pairs_lds_bytes(a.in_features) / 4));
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
  if constexpr (SRC == kContig && EPI == kSilu) {
    if (a.cand_count) {  // uniform: the decode gate of the fused step
      // per wave: candidate / band / above counts and the largest key (one
      // 16-byte LDS record, all read under one wait); then each list gets
      // its entries in lane order, waves in order
      __shared__ uint4 wrec[kRowdotMaxThreads / 64];
      const int wave = threadIdx.x >> 6;
      const uint32_t kk = v & 0x7FFFu;
      const bool ok = valid_l && kk <= 0x7F80u;
      const uint32_t blo = band & 0xFFFFu, bhi = band >> 16;
      const bool cand = ok && kk >= cand_key;
      const bool inb = ok && kk >= blo && kk < bhi;
      const bool abv = ok && bhi != 0u && kk >= bhi;
      const uint64_t m = __ballot(cand), mb = __ballot(inb), ma = __ballot(abv);
      float mk = ok ? bf16_to_f32(kk < 0x80u ? 0u : kk) : -1.f;
      mk = group_max<64>(mk);
      if (lane == 0)
        wrec[wave] = make_uint4((uint32_t)__popcll(m), (uint32_t)__popcll(mb),
                                (uint32_t)__popcll(ma), __float_as_uint(mk));
      __syncthreads();
      uint32_t base = 0, total = 0, bbase = 0, btotal = 0, atotal = 0;
      float bm = -1.f;
      const int nwv = (int)(blockDim.x >> 6);
#pragma unroll
      for (int w = 0; w < kRowdotMaxThreads / 64; ++w) {
        const uint4 r = wrec[w];  // records past the block's waves are not used
        const bool in = w < nwv;
        base += in && w < wave ? r.x : 0u;
        bbase += in && w < wave ? r.y : 0u;
        total += in ? r.x : 0u;
        btotal += in ? r.y : 0u;
        atotal += in ? r.z : 0u;
        bm = in ? fmaxf(bm, __uint_as_float(r.w)) : bm;
      }
      const uint64_t below = (1ull << lane) - 1ull;
      const uint32_t entry = (uint32_t)jl | (v << 16);
      if (cand) a.cand_list[(size_t)blockIdx.x * kCandCap + base + (uint32_t)__popcll(m & below)] = entry;
      const uint32_t bpos = bbase + (uint32_t)__popcll(mb & below);
      if (inb && bpos < (uint32_t)kBandSlot) a.band_list[(size_t)blockIdx.x * kBandSlot + bpos] = entry;
      if (threadIdx.x == 0) {
        a.cand_count[blockIdx.x] = total;
        a.cand_max[blockIdx.x] = bm < 0.f ? 0xFFFFFFFFu : (__float_as_uint(bm) >> 16);
        a.band_count[blockIdx.x] = btotal;
        a.above_count[blockIdx.x] = atotal;
      }
    }
  }
  if (rot) a.rotate[0] = rot1;
}

// ---------------------------------------------------------------------------
// Gate + the workgroup's candidate up rows (the split decode step's first
// launch, dip_internal.h).  The gate half is rowdot_kernel<LPR, CH, kContig,
// kSilu, true, ROWS> (the same loads, arithmetic and order, so g is bit for
// bit the plain gate's).  Then the workgroup's candidates, the rows it just
// computed whose key |g bits| lies in [key, 0x7F80), are listed in LDS (and
// in cand_list when given), and its groups take them in turn (entry e goes to group e
// mod groups, one row of loads in flight): u = up[c] . x with the x pairs
// still in VGPRs (row_dot_part, as dip_up_gather_h computes it), h_full[c] =
// bf16(g[c] * bf16(u)).  The up rows follow the gate rows in the same
// workgroup, so the up stream needs no launch, list or x staging of its own.
// ---------------------------------------------------------------------------
template <int LPR, int CH, int ROWS>
__global__ __launch_bounds__(kRowdotMaxThreads) void gate_spec_kernel(GateSpecArgs a) {
  constexpr int D = ROWS < 2 ? ROWS : 2;  // gate rows of loads in flight per group
  constexpr int kGroups = kRowdotMaxThreads / LPR;
  static_assert(kGroups * ROWS <= kCandCap, "candidate list");
  extern __shared__ __align__(16) uint32_t xlds[];
  __shared__ uint32_t clist[kGroups * ROWS];
  __shared__ uint32_t gcnt[kGroups];
  const int l = threadIdx.x % LPR;
  const int lane = threadIdx.x & 63;
  const int gbase = lane - l;
  const int gw = threadIdx.x / LPR;  // group within the workgroup
  const size_t row_bytes = (size_t)(a.in_features >> 1);
  const int ngroups = a.in_features >> 7;
  const int nchunks = a.in_features / kChunkCols;
  const int grp = blockIdx.x * kGroups + gw;
  const int ngrp = a.ngrp;

  uint4 xs[4];
  load_x_chunk(a.x, nchunks, xs);
  __builtin_amdgcn_sched_barrier(0);
  const long long jl = grp + (long long)l * ngrp;
  const bool valid_l = l < ROWS && jl < a.nrows;
  const uint32_t rid_lane = (uint32_t)min(jl, (long long)a.nrows - 1);
  RowRegs<CH> ring[D];
#pragma unroll
  for (int d = 0; d < D; ++d)
    load_row_at<LPR, CH>(a.qw, a.sc, __shfl(rid_lane, gbase + d, 64), l, row_bytes, ngroups,
                         ring[d]);
  // the key, after the first rows (a lane-dependent offset that is always 0:
  // as a uniform load it would be a scalar load waited for before them)
  const uint32_t zero = threadIdx.x & ((uint32_t)a.in_features >> 30);
  const uint32_t key = a.state[1 + zero];
  const bool rot = blockIdx.x == 0 && threadIdx.x == 0;

  uint32_t xp[CH][4][4];
  float bias[CH];
  stage_x_pairs<LPR>(xs, xlds, nchunks);
  x_pairs_to_regs<LPR, CH>(xlds, nchunks, l, xp, bias);

  float mine = 0.f;
#pragma unroll
  for (int i = 0; i < ROWS; ++i) {
    RowRegs<CH>& R = ring[i % D];
    float acc = row_dot_part<CH>(R, xp, bias);
    if (i + D < ROWS)
      load_row_at<LPR, CH>(a.qw, a.sc, __shfl(rid_lane, gbase + i + D, 64), l, row_bytes,
                           ngroups, R);
    acc = group_sum<LPR>(acc);
    mine = l == i ? acc : mine;
  }
  uint32_t v = 0;
  if (valid_l) {
    v = f32_to_bf16(mine);
    const float f = bf16_to_f32(v);
    v = f32_to_bf16(f / (1.0f + expf(-f)));
    a.g[(int)jl] = (uint16_t)v;
  }

  // the workgroup's candidate list: groups in order, lanes in order
  const uint32_t kk = v & 0x7FFFu;
  const bool cand = valid_l && kk >= key && kk < kKeyInf;
  const uint64_t m = __ballot(cand);
  const uint32_t gm = (uint32_t)(m >> gbase) & (LPR == 32 ? 0xFFFFFFFFu : ((1u << LPR) - 1u));
  if (l == 0) gcnt[gw] = (uint32_t)__popc(gm);
  __syncthreads();
  int base = 0, total = 0;
#pragma unroll
  for (int q = 0; q < kGroups; ++q) {
    base += q < gw ? (int)gcnt[q] : 0;
    total += (int)gcnt[q];
  }
  if (cand) {
    const int e = base + __popc(gm & ((1u << l) - 1u));
    const uint32_t entry = (uint32_t)jl | (v << 16);
    clist[e] = entry;
    if (a.cand_list) a.cand_list[(size_t)blockIdx.x * kCandCap + e] = entry;
  }
  if (a.cand_count && threadIdx.x == 0) a.cand_count[blockIdx.x] = (uint32_t)total;
  if (rot) a.state[0] = key;
  __syncthreads();

  // the candidates' up rows: group gw takes entries gw, gw + kGroups, ...
  const int mycnt = total > gw ? (total - gw + kGroups - 1) / kGroups : 0;
  if (mycnt == 0) return;  // uniform within the group
  RowRegs<CH> ur;
  uint32_t ent = clist[gw];
  load_row_at<LPR, CH>(a.up_qw, a.up_sc, ent & 0xFFFFu, l, row_bytes, ngroups, ur);
#pragma unroll
  for (int i = 0; i < ROWS; ++i) {
    if (i >= mycnt) break;  // uniform within the group
    float acc = row_dot_part<CH>(ur, xp, bias);
    const uint32_t e = ent;
    if (i + 1 < mycnt) {
      ent = clist[gw + kGroups * (i + 1)];
      load_row_at<LPR, CH>(a.up_qw, a.up_sc, ent & 0xFFFFu, l, row_bytes, ngroups, ur);
    }
    acc = group_sum<LPR>(acc);
    if (l == 0) a.h_full[e & 0xFFFFu] = (uint16_t)h_of(e >> 16, acc);
  }
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

// Workgroups per CU of a row-dot grid: the tuning knob when set, else for
// the SiLU gate three where the instance three workgroups per CU would pick
// still fits three at once (the Qwen3-8B gate: 2 rows per group, 97 VGPRs;
// 8.0 -> 7.4 us), else two (the Qwen3-32B gate would need 5 rows per group
// at 231 VGPRs, two waves per SIMD: 13.5 -> 17.2 us); every other grid two.
// The gate with the RMSNorm prologue keeps two: every workgroup normalises
// x itself, and a third per CU cost more than it gained (the whole Qwen3-8B
// model: 477 against 487 tok/s).
int rowdot_wpc(int nrows, int chunks, bool gate, bool norm) {
  const int t = tuning(DIP_TUNE_ROWDOT_WGS_PER_CU);
  if (t > 0) return t;
  if (!gate || norm) return 2;
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

namespace {
// the split step's gate launch: the tuning knob when set, else two
int gate_spec_wpc() {
  const int t = tuning(DIP_TUNE_ROWDOT_WGS_PER_CU);
  return t > 0 ? t : 2;
}
template <int LPR, int CH, int ROWS>
void launch_gate_spec_rows(const GateSpecArgs& a, int blocks, hipStream_t stream) {
  hipLaunchKernelGGL((gate_spec_kernel<LPR, CH, ROWS>), dim3(blocks), dim3(kRowdotMaxThreads),
                     x_pairs_lds_bytes(a.in_features), stream, a);
}
template <int LPR, int CH>
int launch_gate_spec_width(GateSpecArgs a, hipStream_t stream) {
  const RowdotPlan p = plan_rowdot(a.nrows, LPR, true, gate_spec_wpc());
  if (p.groups * LPR != kRowdotMaxThreads || p.rows < 1 || p.rows > 8) return DIP_ERR_UNSUPPORTED;
  a.ngrp = p.blocks * p.groups;
  switch (p.rows) {
    case 1: launch_gate_spec_rows<LPR, CH, 1>(a, p.blocks, stream); break;
    case 2: launch_gate_spec_rows<LPR, CH, 2>(a, p.blocks, stream); break;
    case 3: launch_gate_spec_rows<LPR, CH, 3>(a, p.blocks, stream); break;
    case 4: launch_gate_spec_rows<LPR, CH, 4>(a, p.blocks, stream); break;
    case 5: launch_gate_spec_rows<LPR, CH, 5>(a, p.blocks, stream); break;
    case 6: launch_gate_spec_rows<LPR, CH, 6>(a, p.blocks, stream); break;
    case 7: launch_gate_spec_rows<LPR, CH, 7>(a, p.blocks, stream); break;
    default: launch_gate_spec_rows<LPR, CH, 8>(a, p.blocks, stream); break;
  }
  return hip_status(hipGetLastError());
}
}  // namespace

// Workgroups of the split step's gate launch (0: the width or the row count
// is not supported).
int gate_spec_blocks(int64_t nrows, int64_t in_features) {
  const int64_t chunks = in_features / kChunkCols;
  const int lpr = chunks == 80 ? 16 : 32;
  if (!(chunks == 160 || chunks == 128 || chunks == 80) || nrows < 1) return 0;
  const RowdotPlan p = plan_rowdot((int)nrows, lpr, true, gate_spec_wpc());
  if (p.rows < 1 || p.rows > 8 || (long long)p.blocks > kMaxCandWgs) return 0;
  return p.blocks;
}

int launch_gate_spec(GateSpecArgs a, hipStream_t stream) {
  const int chunks = a.in_features / kChunkCols;
  if (chunks == 160) return launch_gate_spec_width<32, 5>(a, stream);
  if (chunks == 128) return launch_gate_spec_width<32, 4>(a, stream);
  if (chunks == 80) return launch_gate_spec_width<16, 5>(a, stream);
  return DIP_ERR_UNSUPPORTED;
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

extern "C" size_t dip_mlp_state_size(void) { return kStepStateWords * sizeof(uint32_t); }

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
