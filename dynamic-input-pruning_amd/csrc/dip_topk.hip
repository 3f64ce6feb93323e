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
  __shared__ uint32_t wcnt[kWaves];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nchunks = sp.hidden / kChunkCols;
  const int c0 = u * sp.chan_per_wg;
  const int c1 = min(c0 + sp.chan_per_wg, n);
  const int sw = (u == 0) ? 0 : (u == nspec / 2 ? 1 : -1);
  const bool stamp = stamps && sw >= 0 && tid == 0;
  if (stamp) meta->spec_stamp[sw][0] = wall_clock64();

  uint4 xs[4];
  load_x_chunk(sp.x, nchunks, xs);
  const int c = c0 + tid;
  const uint32_t gb = c < c1 ? (uint32_t)g[c] : 0u;
  // the speculation key at a lane-dependent offset that is always 0 (hidden
  // < 2^30): a uniform load would be a scalar load, waited for before the
  // load of g is even issued; this way both are in flight together
  const uint32_t sk = sp.state[threadIdx.x & ((uint32_t)sp.hidden >> 30)];
  const bool f = c < c1 && (gb & 0x7FFFu) >= sk;
  const uint64_t m = __ballot(f);
  if (lane == 0) wcnt[wave] = (uint32_t)__popcll(m);
  __syncthreads();
  int base = 0, total = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const int v = (int)wcnt[w];
    base += w < wave ? v : 0;
    total += v;
  }
  if (f) lds[base + __popcll(m & ((1ull << lane) - 1ull))] = (uint32_t)c | (gb << 16);
  if (stamp) meta->spec_stamp[sw][1] = wall_clock64();
  // x pairs are staged before any row load is issued: with the whole chip
  // streaming, issuing a wave's row loads stalls until data drains, and
  // compute must be able to start as soon as the first rows arrive.
  uint32_t* xlds = lds + kThreads;  // after the list
  stage_x_pairs<LPR>(xs, xlds, nchunks);  // its barrier also publishes the list
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
// MODE kSelSplit (the split step's second launch): the same key, then
// split_select_tail.
enum SelMode : int { kSelPlain = 0, kSelSpec = 1, kSelSplit = 2 };
template <int LPR, int CH>
DIP_DEV void split_select_tail(const SelDownArgs& a, int my, uint32_t mine, bool s0, bool s1,
                               uint32_t pos0, uint32_t pos1, uint32_t uk, uint32_t filled,
                               uint32_t sk, uint32_t* lds);

template <int R, int MODE, int LPR, int CH>
DIP_DEV void topk_body(const uint16_t* __restrict__ s, int n, int k, int32_t* __restrict__ idx,
                       TopkMeta* __restrict__ meta, int stamps, int nblk, const SpecArgs& sp,
                       uint32_t* hist, const SelDownArgs* sd = nullptr) {
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
  if constexpr (MODE == kSelSplit) {
    __syncthreads();  // every wave is past the histogram reads: its LDS is reused
    split_select_tail<LPR, CH>(*sd, my, mine, (a0 | q0) && pos0 < uk, (a1 | q1) && pos1 < uk,
                               pos0, pos1, uk, filled, sk, hist, stamps);
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
template <int R, int LPR, int CH>
__global__ __launch_bounds__(kThreads) void topk_spec_kernel(
    const uint16_t* __restrict__ s, int n, int k, int32_t* __restrict__ idx,
    TopkMeta* __restrict__ meta, int stamps, SpecArgs sp) {
  extern __shared__ __align__(16) uint32_t lds[];  // 128-bit LDS accesses: keep aligned
  if ((int)blockIdx.x < sp.ntopk)
    topk_body<R, kSelSpec, LPR, CH>(s, n, k, idx, meta, stamps, sp.ntopk, sp, lds);
  else
    spec_rows<LPR, CH>(s, n, sp, (int)blockIdx.x - sp.ntopk, lds, meta, stamps,
                       (int)gridDim.x - sp.ntopk);
}


// ---------------------------------------------------------------------------
// The split decode step's second launch (dip_internal.h): select workgroups
// [0, ntopk) and down workgroups after them.  No workgroup waits for another.
// ---------------------------------------------------------------------------
namespace {
constexpr int kSubThreads = 128;                  // a down sub-tile: two waves
constexpr int kSubTiles = kThreads / kSubThreads; // per down workgroup
constexpr int kTilePos = kSubThreads;             // list positions per pass of a down sub-tile
constexpr int kSubSlots = kSubThreads / 8;        // 8-lane slots of a sub-tile
constexpr int kSlotRows = 8;                      // rows per slot and pass (one per lane)
static_assert(kSelectSlice == kSlice, "one fix-up row per select workgroup");
constexpr int kRangeMax = 512;                    // channels per range at most (4 per thread)
constexpr int kFixGroups = 4;                     // entry groups of the fix-up row
constexpr int kFixLdsWord = 12288;                // the fix-up groups' sums: past the x pairs
constexpr int kRangeTarget = 224;                 // candidates per range aimed at (two passes)

// Wave-ordered exclusive prefix of per-thread counts c (< 2^16 in total):
// returns my offset and sets *total; scratch: kWaves words of LDS.  Ends with
// a block barrier.
DIP_DEV uint32_t block_offset(uint32_t c, uint32_t* scratch, uint32_t* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t incl = wave_prefix(c);
  if (lane == 63) scratch[wave] = incl;
  __syncthreads();
  uint32_t before = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const uint32_t v = scratch[w];
    before += w < wave ? v : 0u;
    tot += v;
  }
  *total = tot;
  __syncthreads();  // scratch may be reused
  return before + incl - c;
}

// acc[m] += (q/16)[row, columns 8t .. 8t+7] * f for the dword t of the row.
DIP_DEV void fix_accumulate(uint32_t w, float f, float acc[8]) {
  const uint32_t hq = w >> 4;
  acc[0] = fmaf(cvt_nibble_div16<0>(w), f, acc[0]);
  acc[1] = fmaf(cvt_nibble_div16<0>(hq), f, acc[1]);
  acc[2] = fmaf(cvt_nibble_div16<1>(w), f, acc[2]);
  acc[3] = fmaf(cvt_nibble_div16<1>(hq), f, acc[3]);
  acc[4] = fmaf(cvt_nibble_div16<2>(w), f, acc[4]);
  acc[5] = fmaf(cvt_nibble_div16<2>(hq), f, acc[5]);
  acc[6] = fmaf(cvt_nibble_div16<3>(w), f, acc[6]);
  acc[7] = fmaf(cvt_nibble_div16<3>(hq), f, acc[7]);
}

// scale of (row ch, group g) of the down matrix, group-major copy if given
DIP_DEV uint32_t down_scale(const SelDownArgs& a, uint32_t ch, int g) {
  return a.dn_sc_gm ? a.dn_sc_gm[(size_t)g * a.n + ch]
                    : a.dn_sc[(size_t)ch * (a.sp.hidden >> 7) + g];
}
}  // namespace

// After the placement of a select workgroup's slice (values my, my + 1; s0
// / s1: selected at pos0 / pos1): candidates are the values whose raw key
// lies in [sk, 0x7F80) (the gate launch computed their h).
//   * residual channels: selected non-candidates, and channel 0 when it
//     fills unfilled slots without being a candidate: h from their up rows
//     (h_full, and h_out for the selected ones);
//   * h_out of the selected candidates from h_full; the unfilled slots
//     (workgroup 0) get channel 0's h;
//   * one fix-up partial row: + the selected residual rows, - the rows of
//     candidates that were not selected, + channel 0 once per unfilled slot
//     (workgroup 0), each as h * (q/16) * 16 s with the products of the down
//     tiles; entries in a fixed order (residual then margin, each in slice
//     order) split over fixed thread groups, so the row is deterministic.
template <int LPR, int CH>
DIP_DEV void split_select_tail(const SelDownArgs& a, int my, uint32_t mine, bool s0, bool s1,
                               uint32_t pos0, uint32_t pos1, uint32_t uk, uint32_t filled,
                               uint32_t sk, uint32_t* lds, int stamps) {
  __shared__ uint32_t scratch[kWaves];
  const bool stamp = stamps && blockIdx.x == 0 && threadIdx.x == 0;
  if (stamp) a.meta->spec_stamp[1][0] = wall_clock64();
  __shared__ uint32_t sh_c0, sh_e0;
  const int tid = threadIdx.x;
  const SpecArgs& sp = a.sp;
  const int hidden = sp.hidden;
  // LDS (the histogram's, free): residual entries | their aux (pos | sel <<
  // 31) | their h | margin entries (h already signed) | staged x pairs
  uint32_t* rlist = lds;
  uint32_t* raux = lds + kSlice;
  uint32_t* rh = lds + 2 * kSlice;
  uint32_t* mlist = lds + 3 * kSlice;
  uint32_t* xlds = lds + 4 * kSlice;
  const uint32_t b0 = mine & 0x7FFFu, b1 = (mine >> 16) & 0x7FFFu;
  const bool c0 = b0 >= sk && b0 < kKeyInf;  // padding (0x7FFF) never qualifies
  const bool c1 = b1 >= sk && b1 < kKeyInf;
  const bool fill = my == 0 && filled < uk;
  const bool r0 = (s0 || fill) && !c0, r1 = s1 && !c1;
  const bool m0 = c0 && !s0, m1 = c1 && !s1;
  if (tid == 0 && blockIdx.x == 0) sh_c0 = c0;
  uint32_t nr, nm;
  const uint32_t ro = block_offset((uint32_t)r0 + (uint32_t)r1, scratch, &nr);
  const uint32_t mo = block_offset((uint32_t)m0 + (uint32_t)m1, scratch, &nm);
  if (r0) {
    rlist[ro] = (uint32_t)my | (mine << 16);
    raux[ro] = s0 ? (pos0 | 0x80000000u) : 0u;
    if (fill) sh_e0 = ro;
  }
  if (r1) {
    rlist[ro + r0] = (uint32_t)(my + 1) | (mine & 0xFFFF0000u);
    raux[ro + r0] = pos1 | 0x80000000u;
  }
  if (m0) mlist[mo] = (uint32_t)my;
  if (m1) mlist[mo + m0] = (uint32_t)(my + 1);
  if (stamp) a.meta->spec_stamp[1][1] = wall_clock64();

  // residual h: one row group per entry (x pairs staged in LDS)
  const int nchunks = hidden / kChunkCols;
  if (nr > 0) {  // workgroup-uniform
    uint4 xs[4];
    load_x_chunk(sp.x, nchunks, xs);
    stage_x_pairs<LPR>(xs, xlds, nchunks);  // its barrier also publishes the lists
    const int l = tid % LPR;
    const size_t row_bytes = (size_t)(hidden >> 1);
    const int ngr = hidden >> 7;
    for (int e = tid / LPR; e < (int)nr; e += kThreads / LPR) {
      const uint32_t ent = rlist[e];
      RowRegs<CH> Rr;
      load_row_at<LPR, CH>(sp.up_qw, sp.up_sc, ent & 0xFFFFu, l, row_bytes, ngr, Rr);
      const float u = group_sum<LPR>(row_dot_lds<LPR, CH>(Rr, xlds, nchunks, l));
      if (l == 0) {
        const uint32_t h = h_of(ent >> 16, u);
        rh[e] = h;
        sp.h_full[ent & 0xFFFFu] = (uint16_t)h;
        const uint32_t aux = raux[e];
        if (aux >> 31) a.h_out[aux & 0x7FFFFFFFu] = (uint16_t)h;
      }
    }
  }
  __syncthreads();
  if (stamp) a.meta->spec_stamp[1][2] = wall_clock64();
  // channel 0's h for the unfilled slots (workgroup 0)
  uint32_t h0 = 0;
  if (blockIdx.x == 0 && filled < uk) {  // workgroup-uniform
    h0 = sh_c0 ? (uint32_t)sp.h_full[0] : rh[sh_e0];
    for (uint32_t p = filled + (uint32_t)tid; p < uk; p += kThreads) a.h_out[p] = (uint16_t)h0;
  }

  // the fix-up row: ng groups of hidden / 16 threads; thread (grp, d) owns
  // columns 16 d .. 16 d + 15 and takes entries grp, grp + ng, ... B at a
  // time (one round of loads for the few dozen entries of a steady-state
  // token), and the groups' sums are added in group order through LDS
  const int nd = hidden >> 4;
  const int ng = min(kThreads / nd, kFixGroups);
  const int grp = tid / nd, d = tid % nd;
  float* gsum = reinterpret_cast<float*>(lds + kFixLdsWord);  // [ng][hidden]
  if (grp < ng) {
    const int gcol = (16 * d) >> 7;  // the scale group of my columns
    const int nfl = (int)(nr + nm);
    float acc[16];
#pragma unroll
    for (int m = 0; m < 16; ++m) acc[m] = 0.f;
    constexpr int B = 12;  // entries in flight per thread
    for (int e0 = grp; e0 < nfl; e0 += B * ng) {
      uint2 w[B];
      uint32_t sc[B], hb[B];
      int sgn[B];  // +1 residual, -1 margin, 0 none
#pragma unroll
      for (int u = 0; u < B; ++u) {
        // branch-free: every load is issued, from clamped indices, and the
        // entry kind picks the values (loads under branches serialise)
        const int e = e0 + u * ng;
        const bool isr = e < (int)nr, ism = !isr && e < nfl;
        const int er = isr ? e : 0, em = ism ? e - (int)nr : 0;
        const uint32_t rent = rlist[er], raux_e = raux[er], rhe = rh[er];
        const uint32_t ment = mlist[em];
        const uint32_t ch = isr ? (rent & 0xFFFFu) : (ism ? ment : 0u);
        sgn[u] = isr ? ((raux_e >> 31) ? 1 : 0) : (ism ? -1 : 0);  // fill-only entry: skipped
        w[u] = reinterpret_cast<const uint2*>(a.dn_qw + (size_t)ch * (hidden >> 1))[d];
        sc[u] = down_scale(a, ch, gcol);
        const uint32_t hg = sp.h_full[ch];
        hb[u] = isr ? rhe : (hg ^ 0x8000u);  // margin: the gate launch's h, negated
      }
#pragma unroll
      for (int u = 0; u < B; ++u) {
        const float f = sgn[u] ? bf16_to_f32(hb[u]) * bf16_to_f32(sc[u]) * 16.0f : 0.f;
        fix_accumulate(w[u].x, f, acc);
        fix_accumulate(w[u].y, f, acc + 8);
      }
    }
    if (grp == 0 && blockIdx.x == 0 && filled < uk) {  // channel 0 once per unfilled slot
      const uint2 w = reinterpret_cast<const uint2*>(a.dn_qw)[d];
      const float f = bf16_to_f32(h0) * bf16_to_f32(down_scale(a, 0u, gcol)) * 16.0f;
      for (uint32_t u = filled; u < uk; ++u) {
        fix_accumulate(w.x, f, acc);
        fix_accumulate(w.y, f, acc + 8);
      }
    }
    float4* dst = reinterpret_cast<float4*>(gsum + (size_t)grp * hidden + 16 * d);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      dst[i] = make_float4(acc[4 * i], acc[4 * i + 1], acc[4 * i + 2], acc[4 * i + 3]);
  }
  __syncthreads();
  {
    float* out = a.partial + (size_t)(a.ranges + (int)blockIdx.x) * hidden;
    const float4* g4 = reinterpret_cast<const float4*>(gsum);
    for (int c4 = tid; c4 < hidden / 4; c4 += kThreads) {
      float4 v = g4[c4];
      for (int q = 1; q < ng; ++q) {
        const float4 u = g4[(size_t)q * (hidden / 4) + c4];
        v.x += u.x;
        v.y += u.y;
        v.z += u.z;
        v.w += u.w;
      }
      reinterpret_cast<float4*>(out)[c4] = v;
    }
  }
  // h_out of the selected candidates (the gate launch's h), after the
  // fix-up so that no barrier above waits for these loads
  if (s0 && c0) a.h_out[pos0] = sp.h_full[my];
  if (s1 && c1) a.h_out[pos1] = sp.h_full[my + 1];
  if (stamp) a.meta->spec_stamp[1][3] = wall_clock64();
}

// Down workgroup w of the split step: tiles (channel range r, column block
// cb), tile t = r * col_blocks + cb on sub-tile t / ndown of workgroup t %
// ndown (split_layout keeps the tiles within one round).  A sub-tile (128
// threads: 16 slots of 8 lanes) loads g and h_full of its range's channels at
// once, lists the candidates (the gate launch's key test) in channel order,
// and walks them 128 positions per pass: slot s takes positions 128 pass + s
// + 16 i (i < 8; lane l holds row l), all loaded before any is used;
// positions past the count contribute 0.  The slot sums are reduced as
// in the down kernel into partial row r, block cb.
template <int SL>
DIP_DEV void range_down_role(const SelDownArgs& a, int w, uint32_t* lds, int stamps) {
  constexpr int kPer = kRangeMax / kSubThreads;  // channels per thread
  __shared__ uint32_t wcnt[kSubTiles][kPer][2];   // candidates per sub-tile, pass q, wave
  const int tid = threadIdx.x;
  const bool stamp = stamps && w == 0 && tid == 0;
  if (stamp) a.meta->spec_stamp[0][0] = wall_clock64();
  const int hidden = a.sp.hidden;
  const int sub = tid / kSubThreads, st = tid % kSubThreads;
  const int lane = tid & 63, wv = st >> 6;
  const int l = st % 8, slot = st / 8;
  const int gbase = lane - l;
  const int cbs = a.col_blocks;
  const int t = w + sub * a.ndown;
  const bool active = t < a.ranges * cbs;
  const int r = active ? t / cbs : 0, cb = active ? t % cbs : 0;
  const int c0 = r * a.chan_per_range, c1 = min(c0 + a.chan_per_range, a.n);
  uint32_t* list = lds + sub * kRangeMax;
  float* red = reinterpret_cast<float*>(lds + kSubTiles * kRangeMax);  // [sub][wave][256]

  // 1. the range's candidates (key in [state[0], 0x7F80), as the gate
  //    launch tested them); the key is read per lane at an offset that is
  //    always 0, so that it is in flight with g instead of a scalar load
  const uint32_t zero = (uint32_t)tid & ((uint32_t)hidden >> 30);
  const uint32_t sk = a.sp.state[zero];
  uint32_t gv[kPer], hv[kPer];
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int c = min(c0 + st + kSubThreads * q, a.n - 1);
    gv[q] = a.g[c];
    hv[q] = a.sp.h_full[c];
  }
  bool f[kPer];
  uint64_t m[kPer];
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int c = c0 + st + kSubThreads * q;
    const uint32_t key = gv[q] & 0x7FFFu;
    f[q] = active && c < c1 && key >= sk && key < kKeyInf;
    m[q] = __ballot(f[q]);
    if (lane == 0) wcnt[sub][q][wv] = (uint32_t)__popcll(m[q]);
  }
  __syncthreads();
  int total = 0, base[kPer];
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int n0 = (int)wcnt[sub][q][0];
    base[q] = total + (wv ? n0 : 0);
    total += n0 + (int)wcnt[sub][q][1];
  }
  const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
  for (int q = 0; q < kPer; ++q)
    if (f[q])
      list[base[q] + __popcll(m[q] & below)] =
          (uint32_t)(c0 + st + kSubThreads * q) | (hv[q] << 16);
  __syncthreads();
  if (stamp) a.meta->spec_stamp[0][1] = wall_clock64();

  // 2. their down rows, 256 positions per pass
  const size_t row_bytes = (size_t)(hidden >> 1);
  const int ngroups = hidden >> 7;
  DownArgs da{};  // the fields load_down_scales / load_down_row read
  da.qw_a = a.dn_qw;
  da.sc_a = a.dn_sc;
  da.sc_gm = a.dn_sc_gm;
  da.qw_safe = a.dn_qw;
  da.sc_safe = a.dn_sc;
  da.rows_a = a.n;
  float acc[kDownAcc];
#pragma unroll
  for (int i = 0; i < kDownAcc; ++i) acc[i] = 0.f;
  const int passes = (total + kTilePos - 1) / kTilePos;  // uniform within the sub-tile
  for (int pass = 0; pass < passes; ++pass) {
    // lane l: the id, h and scales of its slot's row l
    const int p = pass * kTilePos + slot + kSubSlots * l;
    const uint32_t ent = list[min(p, total - 1)];
    const uint32_t rid = p < total ? (ent & 0xFFFFu) : kPadRow;
    uint32_t sv[2];
    load_down_scales<kGather, 2, SL>(da, rid, 2 * cb, ngroups, sv);
    DownRow ring[kSlotRows];
#pragma unroll
    for (int i = 0; i < kSlotRows; ++i)
      load_down_row<kGather>(da, __shfl(rid, gbase + i, 64), cb * 8 + l, row_bytes, ring[i]);
    if (stamp && pass == 0) a.meta->spec_stamp[0][2] = wall_clock64();
    float fc[2];
    down_coef<2>(rid, ent >> 16, sv, fc);
    down_accumulate<kSlotRows, 2>(ring, fc, l >= 4, gbase, acc);
  }

  // 3. the slots of each wave in registers, the sub-tile's two waves via LDS
#pragma unroll
  for (int i = 0; i < kDownAcc; ++i) acc[i] += dpp_mov<0x128>(acc[i]);  // row_ror:8
  float t16[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    permlane16_swap(acc[i], acc[i + 16]);
    t16[i] = acc[i] + acc[i + 16];
  }
  float u8[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    permlane32_swap(t16[i], t16[i + 8]);
    u8[i] = t16[i] + t16[i + 8];
  }
  float* rs = red + sub * (2 * 256);
  if ((lane & 15) < 8) {
    float* dst = rs + wv * 256 + 32 * (lane % 8) + 8 * (lane >> 5) + 16 * ((lane >> 4) & 1);
    *reinterpret_cast<float4*>(dst) = make_float4(u8[0], u8[1], u8[2], u8[3]);
    *reinterpret_cast<float4*>(dst + 4) = make_float4(u8[4], u8[5], u8[6], u8[7]);
  }
  __syncthreads();
  if (active) {
    float* out = a.partial + (size_t)r * hidden + (size_t)cb * 256;
    for (int c = st; c < 256; c += kSubThreads) out[c] = rs[c] + rs[256 + c];
  }
  if (stamp) a.meta->spec_stamp[0][3] = wall_clock64();
}

template <int R, int LPR, int CH, int SL>
__global__ __launch_bounds__(kThreads) void select_down_kernel(SelDownArgs a, int stamps) {
  extern __shared__ __align__(16) uint32_t lds[];
  if ((int)blockIdx.x < a.sp.ntopk)
    topk_body<R, kSelSplit, LPR, CH>(a.g, a.n, a.k, a.idx, a.meta, stamps, a.sp.ntopk, a.sp, lds,
                                     &a);
  else
    range_down_role<SL>(a, (int)blockIdx.x - a.sp.ntopk, lds, stamps);
}


// ---------------------------------------------------------------------------
// Finish of the fused decode step (after dip_step.hip's launch), one launch of
// two kinds of workgroups:
//   * workgroups [0, ny): y[o] = bf16(sum of the step workgroups' partial
//     rows), the rows in a fixed order (four interleaved ascending splits,
//     added in order);
//   * workgroups [ny, ny + ceil(n/2048)): idx and h_out for one slice of
//     2048 channels.  The step recorded the bisection's lo / hi (so the tier
//     cuts) and the tier totals; each workgroup counts the tiers of the
//     channels before its slice (packed 16-bit counting), places its slice's
//     selected channels at their positions — tier A in ascending id, then
//     tier B in ascending id up to k (topk_select.cu:64-132) — and copies
//     each one's h from h_full.  The first one also fills the unfilled slots
//     with channel 0 (topk_select.cu:160).
// ---------------------------------------------------------------------------
namespace {
constexpr int kFinThreads = 256;
constexpr int kFinOut = 32;                   // outputs per y workgroup
constexpr int kFinSplit = kFinThreads / kFinOut;
constexpr int kFinBatch = 32;                 // partial rows in flight per thread
constexpr int kFinSlice = 2048;               // channels per idx workgroup
constexpr int kFinCountBatch = 16;            // 8-channel chunks in flight per thread
}  // namespace

__global__ __launch_bounds__(kFinThreads) void finish_kernel(FinishArgs a) {
  __shared__ float part[kFinSplit][kFinOut];
  __shared__ uint32_t wtot[kFinThreads / 64][3];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if ((int)blockIdx.x < a.ny) {
    // split p sums rows p, p + kFinSplit, ... (all loads of a batch issued
    // before the adds), then the splits in order
    const int oo = tid % kFinOut, p = tid / kFinOut;
    const int o = min((int)blockIdx.x * kFinOut + oo, a.hidden - 1);
    float s = 0.f;
    for (int r0 = p; r0 < a.rows; r0 += kFinBatch * kFinSplit) {
      float v[kFinBatch];
#pragma unroll
      for (int u = 0; u < kFinBatch; ++u) {
        const int rb = min(r0 + u * kFinSplit, a.rows - 1);
        v[u] = a.partial[(size_t)rb * a.hidden + o];
      }
#pragma unroll
      for (int u = 0; u < kFinBatch; ++u) s = r0 + u * kFinSplit < a.rows ? s + v[u] : s;
    }
    part[p][oo] = s;
    __syncthreads();
    if (p == 0 && (int)blockIdx.x * kFinOut + oo < a.hidden) {
      float t = part[0][oo];
#pragma unroll
      for (int qq = 1; qq < kFinSplit; ++qq) t += part[qq][oo];
      a.y[blockIdx.x * kFinOut + oo] = (uint16_t)f32_to_bf16(t);
    }
    return;
  }
  const int n = a.n;
  const uint32_t uk = (uint32_t)a.k;
  const int slice0 = ((int)blockIdx.x - a.ny) * kFinSlice;
  const uint32_t cut_a = max((__float_as_uint(a.meta->hi) >> 16) + 1u, kMinNormalKey);
  const uint32_t cut_b = max((__float_as_uint(a.meta->lo) >> 16) + 1u, kMinNormalKey);
  const Cuts c = make_cuts(cut_a, cut_b);
  const uint32_t tot_a = (uint32_t)a.meta->count_a, tot_b = (uint32_t)a.meta->count_b;
  // tier counts of the channels before the slice (whole 8-channel chunks:
  // slice0 <= n is a multiple of 8), a batch of chunks in flight at a time
  uint32_t pa = 0, pb = 0;
  for (int base0 = tid * 8; base0 < slice0; base0 += kFinThreads * 8 * kFinCountBatch) {
    uint32_t w[kFinCountBatch][4];
    // unconditional loads (chunk 0 stands in past the slice), masked after
    // all of them are issued
#pragma unroll
    for (int u = 0; u < kFinCountBatch; ++u) {
      const int base = base0 + u * kFinThreads * 8;
      const uint4 v = *reinterpret_cast<const uint4*>(a.g + (base < slice0 ? base : 0));
      w[u][0] = v.x;
      w[u][1] = v.y;
      w[u][2] = v.z;
      w[u][3] = v.w;
    }
#pragma unroll
    for (int u = 0; u < kFinCountBatch; ++u) {
      if (base0 + u * kFinThreads * 8 >= slice0) {
#pragma unroll
        for (int e = 0; e < 4; ++e) w[u][e] = 0xFFFFFFFFu;  // NaN: in no tier
      }
      const uint32_t t = tier_counts8(w[u], c.cut_a2, c.span_a2, c.cut_b2, c.span_b2);
      pa += t & 0xFFFFu;
      pb += t >> 16;
    }
  }
  // my 8 channels of the slice, in order
  const int my = slice0 + tid * 8;
  uint32_t w[4];
  load_chunk8(a.g, n, my, w);
  if (my < n && my + 8 > n) load_tail8(a.g, n, my, w);
  // their h, in one load (h_full spans whole 256-byte blocks past n)
  const uint4 hq = *reinterpret_cast<const uint4*>(a.h_full + (my < n ? my : 0));
  const uint32_t hw[4] = {hq.x, hq.y, hq.z, hq.w};
  uint32_t ta = 0, tb = 0, flags = 0;  // flags: 2 bits per value (1 = A, 2 = B)
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t kk = (w[e >> 1] >> (16 * (e & 1))) & 0x7FFFu;
    const bool ia = kk - c.cut_a < c.span_a;
    const bool ib = kk - c.cut_b < c.span_b;
    ta += ia ? 1u : 0u;
    tb += ib ? 1u : 0u;
    flags |= (ia ? 1u : (ib ? 2u : 0u)) << (2 * e);
  }
  const uint32_t own = ta | (tb << 16);
  const uint32_t incl = wave_prefix(own);
  const uint32_t sa = lane63(wave_prefix(pa)), sb = lane63(wave_prefix(pb));
  if (lane == 63) wtot[wave][0] = incl;
  if (lane == 0) {
    wtot[wave][1] = sa;
    wtot[wave][2] = sb;
  }
  __syncthreads();
  uint32_t before = 0, pre_a = 0, pre_b = 0;
#pragma unroll
  for (int wv = 0; wv < kFinThreads / 64; ++wv) {
    before += wv < wave ? wtot[wv][0] : 0u;
    pre_a += wtot[wv][1];
    pre_b += wtot[wv][2];
  }
  const uint32_t ex = before + incl - own;
  uint32_t pos_a = pre_a + (ex & 0xFFFFu), pos_b = tot_a + pre_b + (ex >> 16);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t f = (flags >> (2 * e)) & 3u;
    const uint32_t pos = f == 1u ? pos_a : pos_b;
    if (f != 0u && pos < uk) {
      a.idx[pos] = my + e;
      a.h_out[pos] = (uint16_t)(hw[e >> 1] >> (16 * (e & 1)));
    }
    pos_a += f == 1u ? 1u : 0u;
    pos_b += f == 2u ? 1u : 0u;
  }
  if (slice0 == 0) {  // unfilled slots: channel 0
    const uint32_t filled = min(uk, tot_a + tot_b);
    for (uint32_t pp = filled + (uint32_t)tid; pp < uk; pp += kFinThreads) {
      a.idx[pp] = 0;
      a.h_out[pp] = a.h_full[0];
    }
    if (a.state && tid == 0) {  // the next call's speculation key and band
      const uint32_t key = a.meta->next_key, band = a.meta->next_band;
      a.state[0] = key;
      a.state[1] = key;
      a.state[2] = band;
      a.state[3] = 0u;
    }
  }
}

int launch_finish(const FinishArgs& args, hipStream_t stream) {
  FinishArgs a = args;
  a.ny = (a.hidden + kFinOut - 1) / kFinOut;
  const int ni = (a.n + kFinSlice - 1) / kFinSlice;
  hipLaunchKernelGGL(finish_kernel, dim3(a.ny + ni), dim3(kFinThreads), 0, stream, a);
  return hip_status(hipGetLastError());
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

namespace {
template <int R, int LPR, int CH, int SL>
int launch_select_down_variant(const SelDownArgs& a, int blocks, hipStream_t stream) {
  static const bool lds_ok =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&select_down_kernel<R, LPR, CH, SL>),
                          hipFuncAttributeMaxDynamicSharedMemorySize,
                          kFineBins * (int)sizeof(uint32_t)) == hipSuccess;
  if (!lds_ok) return hip_status(hipGetLastError());
  hipLaunchKernelGGL((select_down_kernel<R, LPR, CH, SL>), dim3(blocks), dim3(kThreads),
                     kFineBins * sizeof(uint32_t), stream, a, tuning(DIP_TUNE_TOPK_STAMPS));
  return hip_status(hipGetLastError());
}
template <int LPR, int CH, int SL>
int launch_select_down_width(const SelDownArgs& a, int blocks, hipStream_t stream) {
  if (a.n <= 4 * 8 * kThreads) return launch_select_down_variant<4, LPR, CH, SL>(a, blocks, stream);
  return launch_select_down_variant<8, LPR, CH, SL>(a, blocks, stream);
}
template <int SL>
int launch_select_down_sl(const SelDownArgs& a, int blocks, hipStream_t stream) {
  const int chunks = a.sp.hidden / kChunkCols;
  if (chunks == 160) return launch_select_down_width<32, 5, SL>(a, blocks, stream);
  if (chunks == 128) return launch_select_down_width<32, 4, SL>(a, blocks, stream);
  return launch_select_down_width<16, 5, SL>(a, blocks, stream);
}
}  // namespace

bool split_step_supported(int64_t hidden, int64_t inter) {
  // 8-chunk column blocks and an even number of scale groups per row (the
  // down tiles' scale pairs)
  return topk_spec_supported(hidden) && hidden % 256 == 0 && inter >= 1 && inter <= kTopkMaxN &&
         (hidden / kChunkCols) % 8 == 0;
}

bool split_layout(int64_t hidden, int64_t n, int64_t k, int* ranges, int* chan_per_range) {
  if (!split_step_supported(hidden, n) || k < 1 || k > n) return false;
  const int64_t ntopk = (n + kSlice - 1) / kSlice;
  const int64_t ndown = std::max<int64_t>(device_cus() - ntopk, 1);
  const int64_t cbs = hidden / (kChunkCols * 8);
  // ranges of about kRangeTarget candidates in steady state (the k selected
  // plus the margin above them), at most one round of the down tiles
  const int64_t cand = std::min<int64_t>(n, k + n * (int64_t)tuning(DIP_TUNE_SPEC_MARGIN) / 1024);
  const int64_t c = std::min<int64_t>(
      kRangeMax, std::max<int64_t>(kSubThreads, kRangeTarget * n / std::max<int64_t>(cand, 1)));
  const int64_t r = std::min((n + c - 1) / c, kSubTiles * ndown / cbs);
  if (r < 1) return false;
  const int64_t per = (n + r - 1) / r;  // the same ranges, evened out
  if (per > kRangeMax) return false;
  *ranges = (int)((n + per - 1) / per);
  *chan_per_range = (int)per;
  return true;
}

int launch_select_down(SelDownArgs a, hipStream_t stream) {
  if (a.n <= 0 || a.k <= 0 || a.k > a.n || a.n > kTopkMaxN) return DIP_ERR_SHAPE;
  int ranges = 0, per = 0;
  if (!split_layout(a.sp.hidden, a.n, a.k, &ranges, &per)) return DIP_ERR_UNSUPPORTED;
  const int ntopk = (a.n + kSlice - 1) / kSlice;
  a.sp.ntopk = ntopk;
  a.sp.margin = (int)(a.n * (int64_t)tuning(DIP_TUNE_SPEC_MARGIN) / 1024);
  a.ranges = ranges;
  a.chan_per_range = per;
  a.col_blocks = a.sp.hidden / (kChunkCols * 8);
  a.ndown = std::max(device_cus() - ntopk, 1);
  const int blocks = ntopk + a.ndown;
  if (a.dn_sc_gm) return launch_select_down_sl<kScGm>(a, blocks, stream);
  if (((reinterpret_cast<uintptr_t>(a.dn_sc)) & 3u) == 0)
    return launch_select_down_sl<kScRow4>(a, blocks, stream);
  return launch_select_down_sl<kScRow>(a, blocks, stream);
}

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
