// dip_topk.hip — bit-exact restatement of the reference's threshold top-k
// (kernels/topk_select/topk_select.cu:30-164) without host round trips.
//
// The reference computes hi = max|s|, lo = 0 and runs 25 fp32 bisection
// steps, each launching a counting kernel and reading c = #{|s| > t} back to
// the host (26 syncs), then compacts {|s| > hi} and {lo < |s| <= hi} in index
// order.  Each step only asks "c > k", and
//     #{|s| > t} > k   <=>   a_{k+1} > t
// where a_{k+1} is the (k+1)-th largest |s| (NaN never counts, fewer than k+1
// values means "never").  So the whole bisection is a function of two
// numbers, max|s| and a_{k+1}, which a 32768-bin histogram of the 15-bit
// magnitudes gives exactly; the steps are then replayed with the same fp32
// arithmetic.
//
// One launch of ceil(n / 2048) workgroups of 1024 threads writes idx.  Every
// workgroup redundantly
//   1. loads all n values into registers and builds the histogram in its LDS
//      (a global histogram would need device-scope atomics, and the many
//      channels that share a bf16 magnitude serialise those), reducing the
//      range [kmin, kmax] of the valid keys on the way;
//   2. takes max|s| = kmax and finds a_{k+1} by a prefix over per-thread
//      sums of consecutive bins of that range (only the thread holding rank
//      k+1 walks its bins);
//   3. replays the 25 bisection steps on one lane -> the two key cuts;
//   4. takes the tier totals from the histogram and counts the tiers of the
//      values on the shorter side of its slice (before or after it);
// and then places the ids of its own slice of 2048 values (2 per thread, one
// block scan) at their final positions in idx.  The workgroups never wait for
// each other.
//
// Magnitudes are used unflushed: bf16 subnormals (|bits| 1..0x7F) are 0 under
// the reference's --use_fast_math, so histogram bins below 0x80 all mean 0
// and both cuts are clamped to >= 0x80; NaN and padding (0xFFFF) land in bins
// above 0x7F80, which the search ignores and the tier ranges exclude.
#include <algorithm>

#include "dip_tiles.h"

namespace dip {

namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int kSlice = 2 * kThreads;  // values placed per select workgroup
constexpr uint32_t kNoKey = 0xFFFFFFFFu;
constexpr uint32_t kMaxValidKey = kKeyInf;  // 0x7F80: +inf
constexpr uint32_t kMinNormalKey = 0x0080u;

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// Per 16-bit half: 1 if d < span1 (unsigned), else 0.  Saturating packed
// subtract then min with 1, as two VOP3P instructions (written as asm so the
// compiler keeps them packed instead of splitting into per-half compares).
DIP_DEV uint32_t in_span2(uint32_t d, uint32_t span1_2, uint32_t ones) {
  uint32_t r;
  asm("v_pk_sub_u16 %0, %1, %2 clamp\n\tv_pk_min_u16 %0, %0, %3"
      : "=&v"(r)
      : "v"(span1_2), "v"(d), "v"(ones));
  return r;
}

DIP_DEV uint32_t pk_sub(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, a) - __builtin_bit_cast(u16x2, b));
}
DIP_DEV uint32_t pk_add(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, a) + __builtin_bit_cast(u16x2, b));
}

// Tier counts of 8 raw values (4 dwords): returns (count A) | (count B) << 16.
// tier A: cut_a <= b <= 0x7F80;  tier B: cut_b <= b < cut_a   (b = |bits|)
DIP_DEV uint32_t tier_counts8(const uint32_t w[4], uint32_t cut_a2, uint32_t span_a2,
                              uint32_t cut_b2, uint32_t span_b2) {
  const uint32_t ones = 0x00010001u;
  uint32_t acc_a = 0, acc_b = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t k2 = w[i] & 0x7FFF7FFFu;
    acc_a = pk_add(acc_a, in_span2(pk_sub(k2, cut_a2), span_a2, ones));
    acc_b = pk_add(acc_b, in_span2(pk_sub(k2, cut_b2), span_b2, ones));
  }
  return ((acc_a & 0xFFFFu) + (acc_a >> 16)) | (((acc_b & 0xFFFFu) + (acc_b >> 16)) << 16);
}

// Maximum over the 64 lanes of a wave (row_shr 1, 2, 4, 8 within rows of
// 16, then row_bcast:15 / row_bcast:31 across rows; zero fill), returned
// from lane 63 to every lane.
DIP_DEV uint32_t wave_max(uint32_t v) {
  v = max(v, dpp_zero<0x111>(v));
  v = max(v, dpp_zero<0x112>(v));
  v = max(v, dpp_zero<0x114>(v));
  v = max(v, dpp_zero<0x118>(v));
  v = max(v, dpp_zero<0x142, 0xA>(v));
  v = max(v, dpp_zero<0x143, 0xC>(v));
  return lane63(v);
}

// Elements [base, n) of a chunk that straddles n, 2 per dword; the rest read
// 0xFFFF.
DIP_DEV void load_tail8(const uint16_t* __restrict__ s, int n, int base, uint32_t out[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t lo = base + 2 * i < n ? s[base + 2 * i] : 0xFFFFu;
    const uint32_t hi = base + 2 * i + 1 < n ? s[base + 2 * i + 1] : 0xFFFFu;
    out[i] = lo | (hi << 16);
  }
}

// 8 raw values at [base, base+8): whole chunks by a predicated 128-bit load
// (no else branch), a chunk straddling n element by element, past n 0xFFFF.
DIP_DEV void load_chunk8(const uint16_t* __restrict__ s, int n, int base, uint32_t out[4]) {
  uint4 v = make_uint4(0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu);
  if (base + 8 <= n) v = *reinterpret_cast<const uint4*>(s + base);
  out[0] = v.x;
  out[1] = v.y;
  out[2] = v.z;
  out[3] = v.w;
}


// Tier ranges of the 15-bit keys b = |bits|:
//   tier A: cut_a <= b <= 0x7F80      tier B: cut_b <= b < cut_a
struct Cuts {
  uint32_t cut_a2, span_a2, cut_b2, span_b2;  // packed in both 16-bit halves
  uint32_t cut_a, span_a, cut_b, span_b;
};

DIP_DEV Cuts make_cuts(uint32_t cut_a, uint32_t cut_b) {
  Cuts c;
  c.cut_a = cut_a;
  c.cut_b = cut_b;
  c.span_a = kMaxValidKey + 1u - cut_a;
  c.span_b = cut_a - cut_b;
  c.cut_a2 = cut_a * 0x10001u;
  c.cut_b2 = cut_b * 0x10001u;
  c.span_a2 = c.span_a * 0x10001u;
  c.span_b2 = c.span_b * 0x10001u;
  return c;
}

}  // namespace

// ---------------------------------------------------------------------------
// Speculative up rows.  h for a channel c is bf16(g[c] * bf16(up[c] . x)),
// computed with the same row-dot code and order as dip_up_gather_h, so every
// h below is bit-identical to the one that entry point would produce.
// ---------------------------------------------------------------------------

// h of the residual channels of a select workgroup (list entries: channel |
// g bits << 16): row group i takes entries i, i + groups, ... one row at a
// time (the residual is a handful of rows in steady state).
template <int LPR, int CH>
DIP_DEV void residual_rows(const SpecArgs& sp, const uint32_t* rlist, int rcount,
                           uint32_t* xlds) {
  const int nchunks = sp.hidden / kChunkCols;
  uint4 xs[4];
  load_x_chunk(sp.x, nchunks, xs);
  stage_x_pairs<LPR>(xs, xlds, nchunks);
  const int l = threadIdx.x % LPR;
  const size_t row_bytes = (size_t)(sp.hidden >> 1);
  const int ngr = sp.hidden >> 7;
  for (int e = threadIdx.x / LPR; e < rcount; e += kThreads / LPR) {
    const uint32_t ent = rlist[e];
    RowRegs<CH> R;
    load_row_at<LPR, CH>(sp.up_qw, sp.up_sc, ent & 0xFFFFu, l, row_bytes, ngr, R);
    const float u = group_sum<LPR>(row_dot_lds<LPR, CH>(R, xlds, nchunks, l));
    if (l == 0) sp.h_full[ent & 0xFFFFu] = (uint16_t)h_of(ent >> 16, u);
  }
}

// Speculation workgroup u: h for every channel c in [u*C, min((u+1)*C, n))
// whose magnitude key |bits| is at or above the speculation key state[0]
// (C = chan_per_wg <= kThreads).  The channels are compacted into an LDS
// list (channel | g bits << 16); row group i takes entries i, i + groups, ...
// with D rows in flight.
template <int LPR, int CH>
DIP_DEV void spec_rows(const uint16_t* __restrict__ g, int n, const SpecArgs& sp, int u,
                       uint32_t* lds, TopkMeta* __restrict__ meta, int stamps, int nspec) {
  constexpr int kGroups = kThreads / LPR;
  // rows in flight per group (16-lane groups: twice the groups, and more
  // rows in flight spill registers)
  constexpr int D = LPR >= 32 ? 3 : 1;
  __shared__ uint32_t lcount;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nchunks = sp.hidden / kChunkCols;
  const int c0 = u * sp.chan_per_wg;
  const int c1 = min(c0 + sp.chan_per_wg, n);
  const int sw = (u == 0) ? 0 : (u == nspec / 2 ? 1 : -1);
  const bool stamp = stamps && sw >= 0 && tid == 0;
  if (stamp) meta->spec_stamp[sw][0] = wall_clock64();

  // x first, then g and the key: staging x's pairs then waits for x alone
  uint4 xs[4];
  load_x_chunk(sp.x, nchunks, xs);
  __builtin_amdgcn_sched_barrier(0);
  const int c = c0 + tid;
  const uint32_t gb = c < c1 ? (uint32_t)g[c] : 0u;
  // the speculation key at a lane-dependent offset that is always 0 (hidden
  // < 2^30): a uniform load would be a scalar load, waited for before the
  // load of g is even issued; this way both are in flight together
  const uint32_t sk = sp.state[threadIdx.x & ((uint32_t)sp.hidden >> 30)];
  __builtin_amdgcn_sched_barrier(0);
  // the list's length, zero before any wave claims its part
  if (tid == 0) lcount = 0u;
  __syncthreads();
  // x pairs are staged before any row load is issued (with the whole chip
  // streaming, issuing a wave's row loads stalls until data drains, and
  // compute must be able to start as soon as the first rows arrive), and
  // while g is still in flight: the barrier after the list publishes them
  uint32_t* xlds = lds + kThreads;  // after the list
  stage_x_pairs<LPR, false>(xs, xlds, nchunks);
  const bool f = c < c1 && (gb & 0x7FFFu) >= sk;
  const uint64_t m = __ballot(f);
  if (stamp) meta->spec_stamp[sw][1] = wall_clock64();
  // each wave claims its part of the list with one LDS atomic, in whatever
  // order the waves get there: which group computes which channel's h then
  // varies from call to call, the h values do not (each is one row's dot
  // product in a fixed order)
  uint32_t wbase = 0;
  if (lane == 0 && m) wbase = atomicAdd(&lcount, (uint32_t)__popcll(m));
  wbase = __shfl(wbase, 0, 64);
  if (f) lds[wbase + __popcll(m & ((1ull << lane) - 1ull))] = (uint32_t)c | (gb << 16);
  __syncthreads();  // publishes the list and x's pairs
  const int total = (int)lcount;
  if (stamp) meta->spec_stamp[sw][2] = wall_clock64();
  if (total == 0) return;  // workgroup-uniform

  const int grp = tid / LPR;
  const int l = tid % LPR;
  const size_t row_bytes = (size_t)(sp.hidden >> 1);
  const int ngr = sp.hidden >> 7;
  const int rounds = (total + kGroups - 1) / kGroups;
  RowRegs<CH> ring[D];
  uint32_t ent[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {  // entries past the end re-read the last row
    ent[d] = lds[min(grp + d * kGroups, total - 1)];
    load_row_at<LPR, CH>(sp.up_qw, sp.up_sc, ent[d] & 0xFFFFu, l, row_bytes, ngr, ring[d]);
  }
  const uint4* xsrc = reinterpret_cast<const uint4*>(xlds);
  const float* xbias = reinterpret_cast<const float*>(xlds + nchunks * 16);
  for (int i0 = 0; i0 < rounds; i0 += D) {
    // The D rows in flight share each chunk's x pairs (one LDS read for all
    // of them); a group skips its rows past the end of the list.  Each row
    // still accumulates its chunks in order, as row_dot_part does.
    bool live[D];
    float acc[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
      live[d] = i0 + d < rounds && grp + (i0 + d) * kGroups < total;
      acc[d] = 0.f;
    }
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      uint32_t xp[4][4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint4 v = xsrc[(c * 4 + q) * LPR + l];
        xp[q][0] = v.x;
        xp[q][1] = v.y;
        xp[q][2] = v.z;
        xp[q][3] = v.w;
      }
      const float b = xbias[l + LPR * c];
#pragma unroll
      for (int d = 0; d < D; ++d)
        if (live[d]) acc[d] = chunk_dot(ring[d].w[c], xp, b, ring[d].s[c], acc[d]);
    }
#pragma unroll
    for (int d = 0; d < D; ++d) {
      if (live[d]) {  // uniform within the group
        const float uu = group_sum<LPR>(acc[d]);
        if (l == 0) sp.h_full[ent[d] & 0xFFFFu] = (uint16_t)h_of(ent[d] >> 16, uu);
      }
      if (i0 + d + D < rounds) {  // workgroup-uniform
        ent[d] = lds[min(grp + (i0 + d + D) * kGroups, total - 1)];
        load_row_at<LPR, CH>(sp.up_qw, sp.up_sc, ent[d] & 0xFFFFu, l, row_bytes, ngr,
                             ring[d]);
      }
    }
  }
  if (stamps && sw >= 0) {  // when the last wave of the workgroup is done
    __syncthreads();
    if (stamp) meta->spec_stamp[sw][3] = wall_clock64();
  }
}

// ---------------------------------------------------------------------------
// Select: R rounds of one 8-value chunk per thread cover n <= 8192 R values;
// workgroup w places values [2048 w, 2048 (w + 1)).
// ---------------------------------------------------------------------------
// The select body, run by workgroups 0 .. nblk-1 of a launch.  MODE
// kSelSpec (the decode step with speculative up rows): also records the
// magnitude key at rank k + margin for the next call and computes h for the
// selected channels that the speculation workgroups skip (residual_rows).
enum SelMode : int { kSelPlain = 0, kSelSpec = 1 };

template <int R, int MODE, int LPR, int CH>
DIP_DEV void topk_body(const uint16_t* __restrict__ s, int n, int k, int32_t* __restrict__ idx,
                       TopkMeta* __restrict__ meta, int stamps, int nblk, const SpecArgs& sp,
                       uint32_t* hist) {
  constexpr bool SPEC = MODE != kSelPlain;
  __shared__ uint32_t wtot[kWaves];
  __shared__ uint32_t wsum_a[kWaves], wsum_b[kWaves], wside[kWaves], wown[kWaves];
  __shared__ uint32_t wlo[kWaves], whi[kWaves];
  __shared__ uint32_t sh_a, sh_cut_a, sh_cut_b, sh_spec, sh_rcount;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int slice0 = blockIdx.x * kSlice;
  const bool stamp = stamps && blockIdx.x == 0 && tid == 0;
  const uint32_t sk = SPEC ? sp.state[0] : 0u;  // read early: used after placement
  if (stamp) {
    meta->stamp[0] = wall_clock64();
    meta->cycles[0] = clock64();
  }

  // ---- 1. values into registers; clear the histogram meanwhile -----------
  // thread t holds chunks t, t + 1024, ... (8 values each)
  uint32_t key[R][4];
#pragma unroll
  for (int r = 0; r < R; ++r) load_chunk8(s, n, (tid + kThreads * r) * 8, key[r]);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int base = (tid + kThreads * r) * 8;
    if (base < n && base + 8 > n) load_tail8(s, n, base, key[r]);
  }
  const int my = slice0 + 2 * tid;  // my two values to place (even index: one aligned dword)
  uint32_t mine = 0xFFFFFFFFu;
  if (my + 1 < n) mine = *reinterpret_cast<const uint32_t*>(s + my);
  else if (my < n) mine = (uint32_t)s[my] | 0xFFFF0000u;
  {
    uint4* h4 = reinterpret_cast<uint4*>(hist);
#pragma unroll
    for (int i = 0; i < kFineBins / 4 / kThreads; ++i)
      h4[tid + i * kThreads] = make_uint4(0, 0, 0, 0);
  }
  if (tid == 0) {
    sh_a = kNoKey;
    sh_spec = kNoKey;
    sh_rcount = 0;
  }
  __syncthreads();

  // ---- 2. histogram of every magnitude, and the range of the valid keys ---
  // (NaN and padding keys, above 0x7F80, land in bins the search never reads)
  {
    uint32_t lo = kNoKey, hi1 = 0;  // smallest valid key, largest + 1
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if ((tid + kThreads * r) * 8 < n) {  // chunks wholly past n would pile onto one bin
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t b0 = key[r][i] & 0x7FFFu, b1 = (key[r][i] >> 16) & 0x7FFFu;
          atomicAdd(&hist[b0], 1u);
          atomicAdd(&hist[b1], 1u);
          const bool v0 = b0 <= kMaxValidKey, v1 = b1 <= kMaxValidKey;
          lo = v0 ? min(lo, b0) : lo;
          hi1 = v0 ? max(hi1, b0 + 1u) : hi1;
          lo = v1 ? min(lo, b1) : lo;
          hi1 = v1 ? max(hi1, b1 + 1u) : hi1;
        }
      }
    }
    lo = ~wave_max(~lo);
    hi1 = wave_max(hi1);
    if (lane == 0) {
      wlo[wave] = lo;
      whi[wave] = hi1;
    }
  }
  __syncthreads();
  if (stamp) meta->stamp[1] = wall_clock64();
  // Only the bins [kmin, kmax1) can hold valid values: magnitudes span a few
  // thousand keys in practice, so the scan below reads those and not all
  // 32768.
  uint32_t kmin = kNoKey, kmax1 = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    kmin = min(kmin, wlo[w]);
    kmax1 = max(kmax1, whi[w]);
  }
  const int span = kmax1 > kmin ? (int)(kmax1 - kmin) : 0;  // 0: no valid value

  // ---- 3. a_{k+1} (and the key of rank k+margin) ---------------------------
  // Thread t sums the m = ceil(span / 1024) bins [top_t - m, top_t) counted
  // down from kmax1 (top_t = kmax1 - t m), so an exclusive prefix over t
  // counts the values above its bins; the thread whose bins hold a rank walks
  // them.  max|s| is kmax1 - 1.
  const int m = (span + kThreads - 1) / kThreads;
  const int top = (int)kmax1 - tid * m;           // my bins: [bot, top)
  const int bot = max(top - m, (int)kmin);
  uint32_t mysum = 0;
  for (int b = top - 1; b >= bot; --b) mysum += hist[b];
  uint32_t nvalid = 0, above = 0;
  {
    const uint32_t incl = wave_prefix(mysum);
    if (lane == 63) wtot[wave] = incl;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      above += w < wave ? wtot[w] : 0u;
      nvalid += wtot[w];
    }
    above += incl - mysum;
  }
  const uint32_t need = (uint32_t)k + 1u;
  const uint32_t need_s = SPEC && blockIdx.x == 0 ? (uint32_t)k + (uint32_t)sp.margin : 0u;
  if (above < need && above + mysum >= need) {
    uint32_t run = above;
    for (int b = top - 1; b >= bot; --b) {
      run += hist[b];
      if (run >= need) {
        sh_a = (uint32_t)b;
        break;
      }
    }
  }
  if (above < need_s && above + mysum >= need_s) {
    uint32_t run = above;
    for (int b = top - 1; b >= bot; --b) {
      run += hist[b];
      if (run >= need_s) {
        sh_spec = (uint32_t)b;
        break;
      }
    }
  }
  __syncthreads();
  const uint32_t key_max = span > 0 ? kmax1 - 1u : kNoKey;
  if (stamp) meta->stamp[2] = wall_clock64();

  // ---- 4. replay the 25 fp32 bisection steps (topk_select.cu:141-158) -----
  if (tid == 0) {
    uint32_t ka = sh_a, km = key_max;
    if (ka != kNoKey && ka < kMinNormalKey) ka = 0;  // subnormal -> 0
    if (km != kNoKey && km < kMinNormalKey) km = 0;
    // with fewer than k+1 values "c > k" never holds: a = 0 never exceeds t >= 0
    const float a = ka == kNoKey ? 0.f : bf16_to_f32(ka);
    float hi = km == kNoKey ? 0.f : bf16_to_f32(km);
    float lo = 0.f;
    float t = 0.5f * (lo + hi);
#pragma unroll
    for (int step = 0; step < 25; ++step) {
      const bool gt = a > t;
      lo = gt ? t : lo;
      hi = gt ? hi : t;
      t = 0.5f * (lo + hi);
    }
    // |s| > v for a bf16 magnitude b  <=>  b >= (bits(v) >> 16) + 1  (v >= 0);
    // subnormal magnitudes never qualify, so the cuts start at 0x80.
    sh_cut_a = max((__float_as_uint(hi) >> 16) + 1u, kMinNormalKey);
    sh_cut_b = max((__float_as_uint(lo) >> 16) + 1u, kMinNormalKey);
    if (SPEC && blockIdx.x == 0)  // fewer than k + margin values: speculate on all
      sp.state[1] = sh_spec == kNoKey ? 0u : sh_spec;
    if (blockIdx.x == 0) {
      meta->lo = lo;
      meta->hi = hi;
      meta->key_a = ka;
      meta->key_max = km;
      meta->n_valid = (int32_t)nvalid;
    }
  }
  __syncthreads();
  if (stamp) meta->stamp[3] = wall_clock64();
  const Cuts c = make_cuts(sh_cut_a, sh_cut_b);

  // ---- 5. tier totals from the histogram, tier counts of one side ----------
  // Totals: #{b >= cut} over my bins [bot, top), whole when the cut is at or
  // below them, bin by bin when it splits them.
  uint32_t ge_a = 0, ge_b = 0;
  {
    const int ca = (int)c.cut_a, cb = (int)c.cut_b;
    ge_a = bot >= ca ? mysum : 0u;
    ge_b = bot >= cb ? mysum : 0u;
    if ((bot < ca && top > ca) || (bot < cb && top > cb)) {
      for (int b = top - 1; b >= bot; --b) {
        const uint32_t h = hist[b];
        ge_a += bot < ca && b >= ca ? h : 0u;
        ge_b += bot < cb && b >= cb ? h : 0u;
      }
    }
  }
  // The tier counts before my slice: count whichever side of the slice is
  // shorter (values before it, or after it) and derive the other.
  const int slice1 = min(slice0 + kSlice, n);
  const bool count_before = slice0 <= n - slice1;
  uint32_t side = 0;  // packed (A | B << 16); at most 8R values per thread
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int base = (tid + kThreads * r) * 8;
    const bool in_side = count_before ? base < slice0 : (base >= slice1 && base < n);
    if (in_side) side += tier_counts8(key[r], c.cut_a2, c.span_a2, c.cut_b2, c.span_b2);
  }
  // my two values: tier flags, counts packed (A | B << 16)
  const uint32_t b0 = mine & 0x7FFFu, b1 = (mine >> 16) & 0x7FFFu;
  const uint32_t a0 = b0 - c.cut_a < c.span_a, a1 = b1 - c.cut_a < c.span_a;
  const uint32_t q0 = b0 - c.cut_b < c.span_b, q1 = b1 - c.cut_b < c.span_b;
  const uint32_t own = (a0 + a1) | ((q0 + q1) << 16);
  const uint32_t incl = wave_prefix(own);
  {
    const uint32_t ta = lane63(wave_prefix(ge_a));
    const uint32_t tb = lane63(wave_prefix(ge_b));
    const uint32_t ts = lane63(wave_prefix(side));
    if (lane == 63) wown[wave] = incl;
    if (lane == 0) {
      wsum_a[wave] = ta;
      wsum_b[wave] = tb;
      wside[wave] = ts;
    }
  }
  __syncthreads();
  if (stamp) meta->stamp[4] = wall_clock64();

  uint32_t tot_a = 0, tot_ge_b = 0, side_a = 0, side_b = 0, own_tot = 0, before = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    tot_a += wsum_a[w];
    tot_ge_b += wsum_b[w];
    side_a += wside[w] & 0xFFFFu;
    side_b += wside[w] >> 16;
    own_tot += wown[w];   // packed: a slice holds at most 2048 values
    before += w < wave ? wown[w] : 0u;
  }
  const uint32_t tot_b = tot_ge_b - tot_a;
  // tier counts of the values before my slice
  const uint32_t pre_a = count_before ? side_a : tot_a - side_a - (own_tot & 0xFFFFu);
  const uint32_t pre_b = count_before ? side_b : tot_b - side_b - (own_tot >> 16);

  // ---- 6. place my slice ---------------------------------------------------
  const uint32_t ex = before + incl - own;
  const uint32_t uk = (uint32_t)k;
  const uint32_t pa0 = pre_a + (ex & 0xFFFFu);
  const uint32_t pb0 = tot_a + pre_b + (ex >> 16);
  const uint32_t pos0 = a0 ? pa0 : pb0;
  const uint32_t pos1 = a1 ? pa0 + a0 : pb0 + q0;
  // unfilled slots (fewer than k values qualify) are 0, as in the reference
  const uint32_t filled = min(uk, tot_a + tot_b);
  int rcount = 0;
  if constexpr (MODE == kSelSpec) {
    // Residual h: selected channels whose key is below the speculation key
    // (the speculation workgroups compute every channel at or above it), and
    // channel 0 when unfilled slots point at it.  The histogram is no longer
    // read: its LDS holds the list and then the x pairs.  The list is
    // published before the idx stores, so this barrier does not wait for them.
    const bool r0 = (((a0 | q0) && pos0 < uk) || (my == 0 && filled < uk)) && b0 < sk;
    const bool r1 = (a1 | q1) && pos1 < uk && b1 < sk;
    const uint64_t m0 = __ballot(r0), m1 = __ballot(r1);
    const uint64_t below = (1ull << lane) - 1ull;
    const uint32_t n0 = (uint32_t)__popcll(m0), nw = n0 + (uint32_t)__popcll(m1);
    uint32_t base = 0;
    if (lane == 0 && nw) base = atomicAdd(&sh_rcount, nw);
    base = (uint32_t)__shfl((int)base, 0, 64);
    const uint32_t gpair = mine;
    if (r0) hist[base + __popcll(m0 & below)] = (uint32_t)my | (gpair << 16);
    if (r1) hist[base + n0 + __popcll(m1 & below)] = (uint32_t)(my + 1) | (gpair & 0xFFFF0000u);
    __syncthreads();
    rcount = (int)sh_rcount;
  }
  if ((a0 | q0) && pos0 < uk) idx[pos0] = my;
  if ((a1 | q1) && pos1 < uk) idx[pos1] = my + 1;
  for (uint32_t p = filled + (uint32_t)(blockIdx.x * kThreads + tid); p < uk;
       p += (uint32_t)nblk * kThreads)
    idx[p] = 0;
  if (blockIdx.x == 0 && tid == 0) {
    meta->count_a = (int32_t)tot_a;
    meta->count_b = (int32_t)tot_b;
  }
  if constexpr (MODE == kSelSpec) {
    if (rcount > 0) residual_rows<LPR, CH>(sp, hist, rcount, hist + kSlice);
  }
  if (stamp) {
    meta->stamp[5] = wall_clock64();
    meta->cycles[1] = clock64();
  }
}

template <int R>
__global__ __launch_bounds__(kThreads) void topk_select_kernel(
    const uint16_t* __restrict__ s, int n, int k, int32_t* __restrict__ idx,
    TopkMeta* __restrict__ meta, int stamps) {
  // 16-byte aligned: the histogram is cleared and scanned with 128-bit LDS
  // accesses, which are slow when misaligned
  extern __shared__ __align__(16) uint32_t hist[];  // kFineBins bins
  const SpecArgs none{};
  topk_body<R, kSelPlain, 32, 5>(s, n, k, idx, meta, stamps, (int)gridDim.x, none, hist);
}

// Top-k + speculative up rows in one launch: workgroups [0, sp.ntopk) run
// the select (and the residual rows), the rest compute h for the channels at
// or above the speculation key.  No workgroup waits for another.
#ifdef DIP_WG_STAMPS
__device__ dip_wg_stamps g_stamps_topk;
int timeline_read_topk(dip_wg_stamps* dst) {
  return hip_status(hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_stamps_topk), sizeof(dip_wg_stamps), 0,
                                        hipMemcpyDeviceToHost));
}
#else
int timeline_read_topk(dip_wg_stamps*) { return DIP_ERR_UNSUPPORTED; }
#endif

template <int R, int LPR, int CH>
__global__ __launch_bounds__(kThreads) void topk_spec_kernel(
    const uint16_t* __restrict__ s, int n, int k, int32_t* __restrict__ idx,
    TopkMeta* __restrict__ meta, int stamps, SpecArgs sp) {
  extern __shared__ __align__(16) uint32_t lds[];  // 128-bit LDS accesses: keep aligned
  DIP_STAMP_START(g_stamps_topk);
  if ((int)blockIdx.x < sp.ntopk)
    topk_body<R, kSelSpec, LPR, CH>(s, n, k, idx, meta, stamps, sp.ntopk, sp, lds);
  else
    spec_rows<LPR, CH>(s, n, sp, (int)blockIdx.x - sp.ntopk, lds, meta, stamps,
                       (int)gridDim.x - sp.ntopk);
  DIP_STAMP_END(g_stamps_topk);
}

int launch_topk_select(const uint16_t* s, int64_t n, int64_t k, int32_t* idx, void* ws,
                       hipStream_t stream) {
  static const bool lds_ok = [] {
    const int bytes = kFineBins * (int)sizeof(uint32_t);
    return hipFuncSetAttribute(reinterpret_cast<const void*>(&topk_select_kernel<4>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, bytes) == hipSuccess &&
           hipFuncSetAttribute(reinterpret_cast<const void*>(&topk_select_kernel<8>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, bytes) == hipSuccess;
  }();
  if (!lds_ok) return hip_status(hipGetLastError());
  TopkMeta* meta = reinterpret_cast<TopkMeta*>(ws);
  const unsigned blocks = (unsigned)(n > 0 ? (n + kSlice - 1) / kSlice : 1);
  const int stamps = tuning(DIP_TUNE_TOPK_STAMPS);
  const size_t lds = kFineBins * sizeof(uint32_t);
  if (n <= 4 * 8 * kThreads)
    hipLaunchKernelGGL((topk_select_kernel<4>), dim3(blocks), dim3(kThreads), lds, stream, s,
                       (int)n, (int)k, idx, meta, stamps);
  else
    hipLaunchKernelGGL((topk_select_kernel<8>), dim3(blocks), dim3(kThreads), lds, stream, s,
                       (int)n, (int)k, idx, meta, stamps);
  return hip_status(hipGetLastError());
}

namespace {

template <int R, int LPR, int CH>
int launch_spec_variant(const uint16_t* s, int n, int k, int32_t* idx, TopkMeta* meta,
                        const SpecArgs& sp, int blocks, hipStream_t stream) {
  static const bool lds_ok =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&topk_spec_kernel<R, LPR, CH>),
                          hipFuncAttributeMaxDynamicSharedMemorySize,
                          kFineBins * (int)sizeof(uint32_t)) == hipSuccess;
  if (!lds_ok) return hip_status(hipGetLastError());
  hipLaunchKernelGGL((topk_spec_kernel<R, LPR, CH>), dim3(blocks), dim3(kThreads),
                     kFineBins * sizeof(uint32_t), stream, s, n, k, idx, meta,
                     tuning(DIP_TUNE_TOPK_STAMPS), sp);
  return hip_status(hipGetLastError());
}

template <int LPR, int CH>
int launch_spec_width(const uint16_t* s, int n, int k, int32_t* idx, TopkMeta* meta,
                      const SpecArgs& sp, int blocks, hipStream_t stream) {
  if (n <= 4 * 8 * kThreads) return launch_spec_variant<4, LPR, CH>(s, n, k, idx, meta, sp, blocks, stream);
  return launch_spec_variant<8, LPR, CH>(s, n, k, idx, meta, sp, blocks, stream);
}

}  // namespace

bool topk_spec_supported(int64_t hidden) {
  const int64_t chunks = hidden / kChunkCols;
  return hidden % kGroupSize == 0 && (chunks == 160 || chunks == 128 || chunks == 80);
}

int launch_topk_spec(const uint16_t* g, int64_t n, int64_t k, int32_t* idx, void* ws,
                     SpecArgs sp, hipStream_t stream) {
  if (n <= 0 || k <= 0 || k > n || n > kTopkMaxN) return DIP_ERR_SHAPE;
  if (!topk_spec_supported(sp.hidden)) return DIP_ERR_UNSUPPORTED;
  const int ntopk = (int)((n + kSlice - 1) / kSlice);
  const int min_spec = (int)((n + kThreads - 1) / kThreads);
  const int nspec = std::max(std::max(device_cus() - ntopk, min_spec), 1);
  sp.ntopk = ntopk;
  sp.chan_per_wg = (int)((n + nspec - 1) / nspec);
  sp.margin = (int)(n * (int64_t)tuning(DIP_TUNE_SPEC_MARGIN) / 1024);
  TopkMeta* meta = reinterpret_cast<TopkMeta*>(ws);
  const int blocks = ntopk + nspec;
  const int chunks = sp.hidden / kChunkCols;
  if (chunks == 160) return launch_spec_width<32, 5>(g, (int)n, (int)k, idx, meta, sp, blocks, stream);
  if (chunks == 128) return launch_spec_width<32, 4>(g, (int)n, (int)k, idx, meta, sp, blocks, stream);
  return launch_spec_width<16, 5>(g, (int)n, (int)k, idx, meta, sp, blocks, stream);
}

}  // namespace dip

using namespace dip;

namespace {

int check_topk(const uint16_t* s, int32_t* idx, int64_t n, int64_t k, void* ws,
               size_t ws_bytes) {
  if (n < 0 || k < 0 || n > kTopkMaxN || k > INT32_MAX) return DIP_ERR_SHAPE;
  if (k > 0 && !idx) return DIP_ERR_NULL;
  if (n > 0 && !s) return DIP_ERR_NULL;
  if (n > 0 && (reinterpret_cast<uintptr_t>(s) & 15u)) return DIP_ERR_ALIGN;
  if (!ws || ws_bytes < dip_topk_workspace_size(n)) return DIP_ERR_WORKSPACE;
  if (reinterpret_cast<uintptr_t>(ws) & 15u) return DIP_ERR_ALIGN;
  return DIP_OK;
}

}  // namespace

static_assert(sizeof(TopkMeta) <= kTopkWorkspace, "top-k workspace");

extern "C" size_t dip_topk_workspace_size(int64_t n) {
  (void)n;
  return kTopkWorkspace;  // the last call's thresholds and tier sizes (TopkMeta)
}

extern "C" int64_t dip_topk_max_n(void) { return kTopkMaxN; }

extern "C" int dip_topk_select(const uint16_t* s, int32_t* idx, int64_t n, int64_t k,
                               void* workspace, size_t ws_bytes, void* stream) {
  int st = check_topk(s, idx, n, k, workspace, ws_bytes);
  if (st) return st;
  if (k == 0) return DIP_OK;
  return launch_topk_select(s, n, k, idx, workspace, (hipStream_t)stream);
}

extern "C" int dip_topk_meta(const void* workspace, void* meta_out, void* stream) {
  if (!workspace || !meta_out) return DIP_ERR_NULL;
  return hip_status(hipMemcpyAsync(meta_out, workspace, 16, hipMemcpyDeviceToDevice,
                                   (hipStream_t)stream));
}
