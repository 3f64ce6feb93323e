// dip_step.hip — the body of a resident DIP decode step after the gate, in
// one launch: the exact threshold top-k cut of |g| (bit-exact with
// kernels/topk_select/topk_select.cu:134-164), the up rows, h = bf16(g *
// bf16(up . x)) (dip_stream_predispatch.py:199-201) and the transposed-down
// rows (int4_gather_down.cu:41-75) summed into one fp32 partial y per
// workgroup.  A finish launch (dip_topk.hip) sums the partials in a fixed
// order and writes idx and the per-position h.
//
// The layer state carries the speculation key (the previous call's key of
// rank k + margin) and a *key band* around the previous cut.  The gate launch
// left, per gate workgroup, its *candidates* (channels whose magnitude key is
// at or above the speculation key) in a fixed order, its channels inside the
// band and the number above it.
//
// One workgroup of 512 threads per CU.  Each workgroup:
//   A. ranks the candidates by a scan of the per-gate-workgroup counts and
//      takes an even share of them, so every workgroup gets the same number
//      of rows; gathers the whole band (a few hundred channels); pairs x for
//      the up rows;
//   B. sets up its rings of up and down rows (loaded once the cut is known);
//   C. computes the exact cut (every workgroup does, so none waits for
//      another): max|g| from the gate's per-workgroup maxima; the (k+1)-th
//      largest magnitude (and the (k+margin)-th, the next call's speculation
//      key) from a key-by-key histogram of the band on top of the count
//      above it; the reference's 25 fp32 bisection steps replayed; then,
//      from the band's channels, the tied tier B (whose lowest channel ids
//      fill the last slots: ranked through a bitmap of its channels and a
//      scan of the bitmap's popcounts) and the *late* channels (selected but
//      below the speculation key, ranked by id the same way).  When a rank or
//      a tier falls outside the band (or the band is absent or overfull) an
//      exact whole-g path does the same from g staged in LDS.  The late
//      entries (late channels, then the unfilled slots, which the reference
//      leaves at channel 0, topk_select.cu:160) are split across the grid
//      like the candidates;
//   D. splits by wave: the up waves compute h for every entry (by channel to
//      h_full, and with a ready bit to LDS); the down waves stream the
//      entries' down rows (S streams of CHUNKS threads, each thread one
//      16-byte chunk of every row) and, once an entry's h is ready,
//      accumulate it if the entry is selected;
//   E. sums its streams' accumulators through LDS into its partial row.
// Workgroup 0 also stores the cut for the finish launch and the next call's
// speculation key and band (the finish launch moves them to the layer
// state, after every workgroup here has read it).  Which workgroup handles
// which channel depends on the speculation key, so y's fp32 summation order
// (not its value beyond rounding) depends on the state; for a given state
// the step is deterministic, and every state gives the same idx, g and h.
#include <algorithm>

#include "dip_tiles.h"

namespace dip {

namespace {

constexpr int kStepThreads = 512;
constexpr int kStepWaves = kStepThreads / 64;
constexpr int kStepMaxN = 32768;           // channels (ids fit 16 bits)
constexpr int kMaxEnt = 256;               // candidate or late entries per workgroup
constexpr int kWin = 256;                  // widest key band (one histogram bin per key)
static_assert(kWin <= kStepThreads, "one band bin per thread");
static_assert(kStepMaxN / 32 == 2 * kStepThreads, "two bitmap words per thread");
constexpr int kBandMax = 1024;             // band entries the band path takes
constexpr int kL1Bins = 1024;              // slow path: magnitude key >> 5
static_assert(kBandMax <= kL1Bins + 64, "the band entries share LDS with the histogram");
static_assert(kMaxCandWgs <= kStepMaxN / 32, "the band prefixes share LDS with the bits");
constexpr int kDnRing = 8;                 // down rows in flight per down thread
constexpr int kUpRing = 2;                 // up rows in flight per up group
constexpr uint32_t kNoneKey = 0xFFFFFFFFu;
constexpr uint32_t kInfKey = 0x7F80u;
constexpr uint32_t kMinNormal = 0x0080u;
constexpr uint32_t kSpinLimit = 1u << 20;  // bounded waits on LDS flags

// Work split of a width: UPW up waves (groups of LPR lanes), the rest down.
template <int LPR, int CH>
struct StepShape {
  static constexpr int CHUNKS = LPR * CH;                     // 16-byte chunks per row
  static constexpr int DNW = CHUNKS == 128 ? 4 : 5;           // down waves
  static constexpr int UPW = kStepWaves - DNW;                // up waves
  static constexpr int DN = DNW * 64;                         // down threads
  static constexpr int S = DN / CHUNKS;                       // down streams
  static constexpr int GUP = UPW * 64 / LPR;                  // up groups
  static_assert(S * CHUNKS == DN, "down streams tile the down waves");
};

// LDS layout of the step kernel (32-bit words).
template <int CHUNKS, int S>
struct StepLds {
  static constexpr int xpairs = 0;                            // CHUNKS * 17
  static constexpr int ent = xpairs + CHUNKS * 17;            // 2*kMaxEnt entries: ch | g << 16
  static constexpr int sel = ent + 2 * kMaxEnt;               // 1 if the entry is selected
  static constexpr int hl = sel + 2 * kMaxEnt;                // h | 0x10000 once ready
  static constexpr int pre = hl + 2 * kMaxEnt;                // gate-list prefix counts
  static constexpr int whist = pre + kMaxCandWgs + 1;          // kWin band bins
  static constexpr int low = whist + kWin;                    // kStepMaxN / 32 late bits
  static constexpr int bits = low + kStepMaxN / 32;           // kStepMaxN / 32 tier-B bits
                                                              //  (phase A: band prefixes)
  static constexpr int hist = bits + kStepMaxN / 32;          // kL1Bins + 64 (whole-g path;
                                                              //  band path: band entries)
  static constexpr int red = hist + kL1Bins + 64;             // S x CHUNKS x 33 floats
  static constexpr int gl = (red + S * CHUNKS * 33 + 3) & ~3; // g: ceil(n/8) 128-bit words
  static_assert(ent % 4 == 0, "x pairs are read as 128-bit words");
  static size_t bytes(int n) { return (size_t)(gl + (n + 7) / 8 * 4) * sizeof(uint32_t); }
};

// Exclusive prefix over the 512 threads in thread order; *total gets the sum.
// Uses wsum[kStepWaves]; two block barriers.
DIP_DEV uint32_t step_scan(uint32_t v, uint32_t* wsum, uint32_t* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t incl = wave_prefix(v);
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  uint32_t before = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kStepWaves; ++w) {
    const uint32_t s = wsum[w];
    before += w < wave ? s : 0u;
    tot += s;
  }
  __syncthreads();
  *total = tot;
  return before + incl - v;
}

// Sum over the 512 threads; uses wsum; two block barriers.
DIP_DEV uint32_t step_sum(uint32_t v, uint32_t* wsum) {
  uint32_t tot;
  step_scan(v, wsum, &tot);
  return tot;
}

// acc[m] += (q/16)[chunk, m] * f for the 32 nibbles of one 16-byte chunk
// (v_cvt_off_f32_i4 through SDWA: q/16 exactly; f = 16 * h * s).
DIP_DEV void chunk_accumulate(const uint4& w, float f, float acc[kChunkCols]) {
  const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t hq = wv[q] >> 4;
    acc[8 * q + 0] = fmaf(cvt_nibble_div16<0>(wv[q]), f, acc[8 * q + 0]);
    acc[8 * q + 1] = fmaf(cvt_nibble_div16<0>(hq), f, acc[8 * q + 1]);
    acc[8 * q + 2] = fmaf(cvt_nibble_div16<1>(wv[q]), f, acc[8 * q + 2]);
    acc[8 * q + 3] = fmaf(cvt_nibble_div16<1>(hq), f, acc[8 * q + 3]);
    acc[8 * q + 4] = fmaf(cvt_nibble_div16<2>(wv[q]), f, acc[8 * q + 4]);
    acc[8 * q + 5] = fmaf(cvt_nibble_div16<2>(hq), f, acc[8 * q + 5]);
    acc[8 * q + 6] = fmaf(cvt_nibble_div16<3>(wv[q]), f, acc[8 * q + 6]);
    acc[8 * q + 7] = fmaf(cvt_nibble_div16<3>(hq), f, acc[8 * q + 7]);
  }
}

// The lane's part of one up row's dot product with the x pairs read from
// LDS chunk by chunk: row_dot_lds's operations in the same order (so h is
// bit-identical to the other up paths), with a scheduling barrier after each
// chunk so that one chunk's pairs, not all of them, are live at a time.
template <int LPR, int CH>
DIP_DEV float up_dot_lds(const RowRegs<CH>& R, const uint32_t* xlds, int nchunks, int l) {
  const uint4* src = reinterpret_cast<const uint4*>(xlds);
  const float* bias = reinterpret_cast<const float*>(xlds + nchunks * 16);
  float acc = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    uint32_t xp[4][4];
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      const uint4 v = src[(c * 4 + qq) * LPR + l];
      xp[qq][0] = v.x;
      xp[qq][1] = v.y;
      xp[qq][2] = v.z;
      xp[qq][3] = v.w;
    }
    // R.s[c] holds the dword around the scale: its upper half for odd groups
    acc = chunk_dot(R.w[c], xp, bias[l + LPR * c], R.s[c] >> (16 * ((l >> 2) & 1)), acc);
    __builtin_amdgcn_sched_barrier(0);
  }
  return acc;
}

// Loads from a uniform base pointer plus a 32-bit byte offset (every matrix
// here is below 4 GB): the SGPR-base form, one VGPR per address.
DIP_DEV uint4 ldg_nt_off(const void* base, uint32_t off) {
  return ldg_nt(reinterpret_cast<const uint4*>(static_cast<const char*>(base) + off));
}
// The aligned dword holding the 16-bit value at byte offset off (a 32-bit
// load: a 16-bit one is widened where it is loaded, which makes the wave wait
// for it there instead of where it is used).
DIP_DEV uint32_t ld_u16_pair_off(const void* base, uint32_t off) {
  return *reinterpret_cast<const uint32_t*>(static_cast<const char*>(base) + (off & ~3u));
}

// Up row `ch`: lane l's chunks l + LPR*c, and the dwords holding their
// scales (groups l/4 + c*LPR/4; the half is (l/4) & 1 with an even number of
// groups per row), each from one address.
template <int LPR, int CH>
DIP_DEV void load_up_row(const int8_t* qw, const uint16_t* sc, uint32_t ch, int l,
                         uint32_t row_bytes, uint32_t ngroups, RowRegs<CH>& R) {
  const uint32_t wo = ch * row_bytes + 16u * (uint32_t)l;
  const uint32_t so = 2u * (ch * ngroups + (uint32_t)(l >> 2));
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    R.w[c] = ldg_nt_off(qw, wo + 16u * LPR * c);
    R.s[c] = ld_u16_pair_off(sc, so + (uint32_t)(LPR / 2) * c);
  }
}

// Bounded wait for an LDS word to become nonzero.  The producer is an up
// wave of the same workgroup, which never waits for the down waves, so it
// always gets there; the bound only turns a logic error into wrong output
// instead of a hang.
DIP_DEV uint32_t wait_nonzero(uint32_t* p) {
  uint32_t v = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  for (uint32_t i = 0; v == 0 && i < kSpinLimit; ++i) {
    __builtin_amdgcn_s_sleep(1);
    v = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  return v;
}

}  // namespace

template <int LPR, int CH>
__global__ __launch_bounds__(kStepThreads) void step_kernel(StepArgs a) {
  using SS = StepShape<LPR, CH>;
  constexpr int CHUNKS = SS::CHUNKS, S = SS::S, GUP = SS::GUP;
  using L = StepLds<CHUNKS, S>;
  extern __shared__ __align__(16) uint32_t lds[];
  uint32_t* xlds = lds + L::xpairs;
  uint32_t* ent = lds + L::ent;
  uint32_t* sel = lds + L::sel;
  uint32_t* hl = lds + L::hl;
  uint32_t* pre = lds + L::pre;
  uint32_t* whist = lds + L::whist;
  uint32_t* low = lds + L::low;
  uint32_t* bits = lds + L::bits;
  uint32_t* hist = lds + L::hist;
  uint32_t* sub = hist + kL1Bins;
  uint32_t* bpre = bits;   // phase A only: gate band-list prefix counts
  uint32_t* bandl = hist;  // the band path only: the gate's band entries
  uint32_t* lbits = low;   // the late channels' bitmap
  float* red = reinterpret_cast<float*>(lds + L::red);
  uint4* gl = reinterpret_cast<uint4*>(lds + L::gl);
  __shared__ uint32_t wsum[kStepWaves];
  __shared__ uint32_t wsum2[kStepWaves];
  __shared__ float wmaxf[kStepWaves];
  __shared__ uint32_t sh[16];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nw = gridDim.x, wg = blockIdx.x;
  const int n = a.n, k = a.k;
  const bool stamp = a.stamps && wg == 0 && tid == 0;
  if (stamp) a.meta->stamp[0] = wall_clock64();
  const uint32_t sk = a.state[1];    // speculation key (the gate's candidates: key >= sk)
  const uint32_t band = a.state[2];  // key band lo | hi << 16 the gate listed
  const uint32_t rb32 = (uint32_t)(a.hidden >> 1), ng32 = (uint32_t)(a.hidden >> 7);
  const bool up_role = wave < SS::UPW;
  const int dt = tid - SS::UPW * 64;                          // down thread (down waves)
  const int grp = tid / LPR, l = tid % LPR;                   // up group / lane
  const int sd = up_role ? 0 : dt / CHUNKS, q = up_role ? 0 : dt % CHUNKS;
  const uint32_t dsh = 16u * ((uint32_t)(q >> 2) & 1u);      // my down scale's half

  // ---- A. x and the gate lists -----------------------------------------
  uint4 xs[4];
  load_x_chunk(a.x, CHUNKS, xs);
  const uint32_t g0 = a.g[0];  // channel 0's g: the unfilled slots
  const uint32_t blo = band & 0xFFFFu, bhi = band >> 16;
  // gate workgroups b = 2t, 2t+1: candidate and band counts -> prefixes;
  // rows above the band and band overflows -> sums; max keys -> max
  const int ng = a.gate_wgs;
  uint32_t cc[2] = {0u, 0u}, bc[2] = {0u, 0u}, above = 0, ovf = 0, mk = 0;
  bool anymk = false;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int b = 2 * tid + h;
    if (b < ng) {
      cc[h] = a.cand_count[b];
      const uint32_t bn = a.band_count[b];
      bc[h] = min(bn, (uint32_t)kBandSlot);
      ovf += bn > (uint32_t)kBandSlot ? 1u : 0u;
      above += a.above_count[b];
      const uint32_t m = a.cand_max[b];
      if (m != kNoneKey) {
        mk = anymk ? max(mk, m) : m;
        anymk = true;
      }
    }
  }
  // candidate totals fit 16 bits (at most n <= kStepMaxN), clamped band
  // totals too (at most kMaxCandWgs * kBandSlot)
  uint32_t ptot;
  const uint32_t pbefore = step_scan((cc[0] + cc[1]) | ((bc[0] + bc[1]) << 16), wsum, &ptot);
  if (2 * tid < ng) {
    pre[2 * tid] = pbefore & 0xFFFFu;
    bpre[2 * tid] = pbefore >> 16;
  }
  if (2 * tid + 1 < ng) {
    pre[2 * tid + 1] = (pbefore & 0xFFFFu) + cc[0];
    bpre[2 * tid + 1] = (pbefore >> 16) + bc[0];
  }
  {
    const float mf = group_max<64>(anymk ? bf16_to_f32(mk) : -1.f);
    const uint32_t s2 = lane63(wave_prefix(above | (min(ovf, 1u) << 16)));
    if (lane == 0) {
      wmaxf[wave] = mf;
      wsum2[wave] = s2;
    }
  }
  __syncthreads();
  float vmax = -1.f;
  uint32_t s2 = 0;
#pragma unroll
  for (int w = 0; w < kStepWaves; ++w) {
    vmax = fmaxf(vmax, wmaxf[w]);
    s2 += wsum2[w];
  }
  const uint32_t ctot = ptot & 0xFFFFu, nb = ptot >> 16;
  const uint32_t g_hi = s2 & 0xFFFFu;  // valid values with key >= bhi
  // the band path needs a well-formed band whose entries all fit, and every
  // late channel (selected, key below sk) inside it
  bool fast = bhi > blo && blo >= kMinNormal && bhi - blo <= (uint32_t)kWin && (s2 >> 16) == 0u &&
              nb <= (uint32_t)kBandMax && sk <= bhi;
  // my candidate ranks [r0, r1): entry e is rank r0 + e, found in the gate
  // list whose prefix range holds it (the last b with pre[b] <= rank)
  const int r0 = (int)(((uint64_t)wg * ctot) / (uint64_t)nw);
  const int r1 = (int)(((uint64_t)(wg + 1) * ctot) / (uint64_t)nw);
  const int E = r1 - r0;
  auto last_le = [&](const uint32_t* p, uint32_t r) {
    int lo = 0, hi = ng - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (p[mid] <= r) lo = mid;
      else hi = mid - 1;
    }
    return lo;
  };
  if (tid < E) {
    const uint32_t r = (uint32_t)(r0 + tid);
    const int b = last_le(pre, r);
    ent[tid] = a.cand_list[(size_t)b * kCandCap + (r - pre[b])];
  }
  if (fast) {  // uniform: every workgroup holds the whole band
    for (uint32_t j = tid; j < nb; j += kStepThreads) {
      const int b = last_le(bpre, j);
      bandl[j] = a.band_list[(size_t)b * kBandSlot + (j - bpre[b])];
    }
  }
  stage_x_pairs<LPR>(xs, xlds, CHUNKS);  // its barrier also publishes ent and bandl
  if (stamp) a.meta->stamp[1] = wall_clock64();

  // ---- B. the rings ------------------------------------------------------
  // entry e of the (clamped) list: ent[min(e, cnt - 1)], channel 0 if empty
  auto entry = [&](int cnt, int e) -> uint32_t {  // branch-free (one LDS read either way)
    const uint32_t v = ent[max(min(e, cnt - 1), 0)];
    return cnt > 0 ? v : 0u;
  };
  RowRegs<CH> UR[kUpRing];
  uint4 DR[kDnRing];
  uint32_t DS[kDnRing];
  auto load_up = [&](int cnt, int e, RowRegs<CH>& U) {
    load_up_row<LPR, CH>(a.up_qw, a.up_sc, entry(cnt, e) & 0xFFFFu, l, rb32, ng32, U);
  };
  auto load_dn = [&](int cnt, int e, int slot) {
    const uint32_t ch = entry(cnt, e) & 0xFFFFu;
    DR[slot] = ldg_nt_off(a.dn_qw, ch * rb32 + 16u * (uint32_t)q);
    DS[slot] = ld_u16_pair_off(a.dn_sc, 2u * (ch * ng32 + (uint32_t)(q >> 2)));
  };
  // up group grp takes entries grp + GUP*r; down stream sd entries sd + S*i
  // (the rings are first loaded once the cut is known: loads issued before
  // it would hold up the cut's barriers while the memory queues are full)

  // ---- C. the exact cut --------------------------------------------------
  // flushed magnitude keys: NaN (> 0x7F80) invalid, subnormals count as 0
  auto fkey = [](uint32_t b) -> uint32_t {
    const uint32_t kk = b & 0x7FFFu;
    return kk > kInfKey ? kNoneKey : (kk < kMinNormal ? 0u : kk);
  };
  // order-free pass over g: fn(channel, bits) for words tid, tid + 512, ...
  const int nwords = (n + 7) / 8;
  auto scan_g = [&](auto&& fn) {
    for (int wi = tid; wi < nwords; wi += kStepThreads) {
      const uint4 v = gl[wi];
      const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) fn(8 * wi + e, (wv[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
    }
  };
  const uint32_t need_a = (uint32_t)k + 1u;               // the cut
  const uint32_t need_s = (uint32_t)k + (uint32_t)a.margin;  // the next speculation key
  // the next band: ranks k + 2 margin down to k + 1 - margin
  const uint32_t need_l = need_s + (uint32_t)a.margin;
  const uint32_t need_h = need_a > (uint32_t)a.margin + 1u ? need_a - (uint32_t)a.margin : 1u;
  // replay of the 25 fp32 bisection steps (topk_select.cu:141-158): each
  // step asks #{|s| > t} > k, i.e. a_{k+1} > t (every thread, same arithmetic)
  float hi_f = 0.f, lo_f = 0.f;
  auto bisect = [&](uint32_t key_a) {
    const float av = key_a == kNoneKey ? 0.f : bf16_to_f32(key_a);
    float hi = vmax < 0.f ? 0.f : vmax;
    float lo = 0.f;
    float t = 0.5f * (lo + hi);
#pragma unroll
    for (int step = 0; step < 25; ++step) {
      const bool gt = av > t;
      lo = gt ? t : lo;
      hi = gt ? hi : t;
      t = 0.5f * (lo + hi);
    }
    hi_f = hi;
    lo_f = lo;
  };
  // |s| > v for a bf16 magnitude b  <=>  b >= (bits(v) >> 16) + 1 (v >= 0);
  // tier A: cut_a <= key <= 0x7F80; tier B: cut_b <= key < cut_a (key = |bits|)
  auto cut_of = [](float v) { return max((__float_as_uint(v) >> 16) + 1u, kMinNormal); };
  uint32_t ka = kNoneKey, ks = 0, kl = kNoneKey, kh = kNoneKey;
  uint32_t cut_a = 0, cut_b = 0, tot_a = 0, tot_b = 0;
  if (fast) {  // uniform: the band's keys, one bin each, above g_hi values
    for (int i = tid; i < kWin; i += kStepThreads) whist[i] = 0;
    if (tid == 0) {
      sh[1] = kNoneKey;
      sh[2] = kNoneKey;
      sh[3] = kNoneKey;
      sh[4] = kNoneKey;
    }
    __syncthreads();
    for (uint32_t j = tid; j < nb; j += kStepThreads) {
      const uint32_t d = ((bandl[j] >> 16) & 0x7FFFu) - blo;
      if (d < (uint32_t)kWin) atomicAdd(&whist[d], 1u);
    }
    __syncthreads();
    // thread t < kWin holds the bin of key blo + kWin-1-t, so the prefix in
    // thread order counts the band values above its key
    const int bin = kWin - 1 - tid;
    const uint32_t hb = tid < kWin ? whist[max(bin, 0)] : 0u;
    uint32_t btot;
    const uint32_t gt = g_hi + step_scan(hb, wsum, &btot);  // values with a larger key
    if (tid < kWin) {
      whist[bin] = gt + hb;  // from here on: values with key >= blo + bin (up to bhi)
      const uint32_t key = blo + (uint32_t)bin;
      if (gt < need_a && gt + hb >= need_a) sh[1] = key;
      if (gt < need_s && gt + hb >= need_s) sh[2] = key;
      if (gt < need_l && gt + hb >= need_l) sh[3] = key;
      if (gt < need_h && gt + hb >= need_h) sh[4] = key;
    }
    __syncthreads();
    ka = sh[1];
    ks = sh[2];
    kl = sh[3];
    kh = sh[4];
    fast = ka != kNoneKey && ks != kNoneKey;  // else: a rank outside the band
    if (fast) {
      bisect(ka);
      cut_a = cut_of(hi_f);
      cut_b = cut_of(lo_f);
      fast = cut_b >= blo && cut_a <= bhi;  // both tiers inside the band
      if (fast) {
        tot_a = cut_a >= bhi ? g_hi : whist[cut_a - blo];
        tot_b = (cut_b >= bhi ? g_hi : whist[cut_b - blo]) - tot_a;
      }
    }
  }
  if (stamp) a.meta->spec_stamp[0][0] = wall_clock64();
  if (!fast) {  // uniform: g into LDS, whole-g histogram (1024 bins of key >> 5, then 32 keys)
    __syncthreads();  // the band path's last reads of bandl (it shares LDS with hist)
    for (int i = tid; i < nwords; i += kStepThreads) {
      uint4 v;
      if (8 * i + 8 <= n) {
        v = *reinterpret_cast<const uint4*>(a.g + 8 * i);
      } else {  // the word straddling n: values past n read 0xFFFF (never valid)
        uint32_t wv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t lo = 8 * i + 2 * e < n ? a.g[8 * i + 2 * e] : 0xFFFFu;
          const uint32_t hi = 8 * i + 2 * e + 1 < n ? a.g[8 * i + 2 * e + 1] : 0xFFFFu;
          wv[e] = lo | (hi << 16);
        }
        v = make_uint4(wv[0], wv[1], wv[2], wv[3]);
      }
      gl[i] = v;
    }
    for (int i = tid; i < kL1Bins + 64; i += kStepThreads) hist[i] = 0;
    __syncthreads();
    scan_g([&](int, uint32_t b) {
      const uint32_t f = fkey(b);
      if (f != kNoneKey) atomicAdd(&hist[f >> 5], 1u);
    });
    __syncthreads();
    const uint32_t h0 = hist[2 * tid], h1 = hist[2 * tid + 1];
    uint32_t nvalid;
    const uint32_t before = step_scan(h0 + h1, wsum, &nvalid);
    const uint32_t abv = nvalid - before - h0 - h1;  // bins > 2t+1
    const uint32_t ge1 = abv + h1, ge0 = ge1 + h0;
    if (tid == 0) {
      sh[4] = kNoneKey;
      sh[6] = kNoneKey;
    }
    __syncthreads();
    if (abv < need_a && ge1 >= need_a) {
      sh[4] = 2 * tid + 1;
      sh[5] = abv;
    } else if (ge1 < need_a && ge0 >= need_a) {
      sh[4] = 2 * tid;
      sh[5] = ge1;
    }
    if (abv < need_s && ge1 >= need_s) {
      sh[6] = 2 * tid + 1;
      sh[7] = abv;
    } else if (ge1 < need_s && ge0 >= need_s) {
      sh[6] = 2 * tid;
      sh[7] = ge1;
    }
    __syncthreads();
    const uint32_t bin_a = sh[4], bin_s = sh[6];
    scan_g([&](int, uint32_t b) {
      const uint32_t f = fkey(b);
      if (f == kNoneKey) return;
      if ((f >> 5) == bin_a) atomicAdd(&sub[f & 31u], 1u);
      if ((f >> 5) == bin_s) atomicAdd(&sub[32 + (f & 31u)], 1u);
    });
    __syncthreads();
    if (tid == 0) {
      uint32_t xa = kNoneKey, xs2 = kNoneKey;
      if (bin_a != kNoneKey) {
        uint32_t run = sh[5];
        for (int j = 31; j >= 0 && xa == kNoneKey; --j) {
          run += sub[j];
          if (run >= need_a) xa = (bin_a << 5) | (uint32_t)j;
        }
      }
      if (bin_s != kNoneKey) {
        uint32_t run = sh[7];
        for (int j = 31; j >= 0 && xs2 == kNoneKey; --j) {
          run += sub[32 + j];
          if (run >= need_s) xs2 = (bin_s << 5) | (uint32_t)j;
        }
      }
      sh[1] = xa;
      sh[2] = xs2 == kNoneKey ? 0u : xs2;  // fewer than k + margin values: all
    }
    __syncthreads();
    ka = sh[1];
    ks = sh[2];
    bisect(ka);
    cut_a = cut_of(hi_f);
    cut_b = cut_of(lo_f);
    uint32_t na = 0, nbb = 0;
    scan_g([&](int, uint32_t b) {
      const uint32_t kk = b & 0x7FFFu;
      na += (kk <= kInfKey && kk >= cut_a) ? 1u : 0u;
      nbb += (kk <= kInfKey && kk >= cut_b && kk < cut_a) ? 1u : 0u;
    });
    tot_a = step_sum(na, wsum);
    tot_b = step_sum(nbb, wsum);
  }
  if (stamp) a.meta->spec_stamp[0][1] = wall_clock64();
  const uint32_t fillb = (uint32_t)k - min((uint32_t)k, tot_a);  // tier-B slots
  const uint32_t filled = min((uint32_t)k, tot_a + tot_b);
  // The channels that can be tier B or late: the band's on the band path,
  // all of g otherwise.  fn(channel, g bits).
  auto each_channel = [&](auto&& fn) {
    if (fast) {
      for (uint32_t j = tid; j < nb; j += kStepThreads) {
        const uint32_t e = bandl[j];
        fn(e & 0xFFFFu, e >> 16);
      }
    } else {
      scan_g([&](int c, uint32_t b) { fn((uint32_t)c, b); });
    }
  };
  // Tier B is selected up to its fillb lowest channel ids: its channels go
  // into a bitmap, a scan of the bitmap's popcounts ranks them, and the
  // thread holding rank fillb - 1 names the last selected channel.  (NaN
  // keys lie above cut_a <= 0x7F81, so never in tier B.)
  if (tid == 0) sh[9] = kNoneKey;
  __syncthreads();  // bpre (shares LDS with bits) is dead
  for (int i = tid; i < kStepMaxN / 32; i += kStepThreads) {
    bits[i] = 0;
    lbits[i] = 0;
  }
  __syncthreads();
  each_channel([&](uint32_t c, uint32_t b) {
    const uint32_t kk = b & 0x7FFFu;
    if (kk >= cut_b && kk < cut_a) atomicOr(&bits[c >> 5], 1u << (c & 31));
  });
  __syncthreads();
  {
    const uint32_t w0 = bits[2 * tid], w1 = bits[2 * tid + 1];  // channels 64t .. 64t+63
    const uint32_t p0 = __popc(w0), p1 = __popc(w1);
    uint32_t ntb;
    const uint32_t rb0 = step_scan(p0 + p1, wsum, &ntb);
    if (fillb > 0u && rb0 < fillb && rb0 + p0 + p1 >= fillb) {
      uint32_t r = fillb - 1u - rb0, w = w0, base = 64u * (uint32_t)tid;
      if (r >= p0) {
        r -= p0;
        w = w1;
        base += 32u;
      }
      for (uint32_t i = 0; i < r; ++i) w &= w - 1u;  // drop the r lowest set bits
      sh[9] = base + (uint32_t)__ffs(w) - 1u;
    }
  }
  __syncthreads();
  // tier-B channels below cend are selected
  const uint32_t cend = fillb == 0u ? 0u : (sh[9] == kNoneKey ? kNoneKey : sh[9] + 1u);
  auto selected = [&](uint32_t c, uint32_t kk) -> bool {
    return kk <= kInfKey && (kk >= cut_a || (kk >= cut_b && c < cend));
  };
  // late channels (selected, key below sk: not candidates) exist only when
  // sk > cut_b: their bitmap, then per-word ranks into pre (dead since A)
  uint32_t res_total = 0;
  if (sk > cut_b) {  // uniform
    each_channel([&](uint32_t c, uint32_t b) {
      const uint32_t kk = b & 0x7FFFu;
      if (kk < sk && selected(c, kk)) atomicOr(&lbits[c >> 5], 1u << (c & 31));
    });
    __syncthreads();
    const uint32_t v0 = lbits[2 * tid], v1 = lbits[2 * tid + 1];
    const uint32_t lr = step_scan(__popc(v0) + __popc(v1), wsum, &res_total);
    pre[2 * tid] = lr;
    pre[2 * tid + 1] = lr + __popc(v0);
    __syncthreads();
  }
  if (stamp) a.meta->spec_stamp[0][2] = wall_clock64();
  for (int e = tid; e < E; e += kStepThreads) {
    const uint32_t ev = ent[e];
    sel[e] = selected(ev & 0xFFFFu, (ev >> 16) & 0x7FFFu) ? 1u : 0u;
    hl[e] = 0;
  }
  // late entries: late channels (by id), then the unfilled slots (channel 0)
  const uint32_t nlate = res_total + (uint32_t)k - filled;
  const int q0 = (int)(((uint64_t)wg * nlate) / (uint64_t)nw);
  const int q1 = (int)(((uint64_t)(wg + 1) * nlate) / (uint64_t)nw);
  const int EL = q1 - q0;
  if (q0 < (int)res_total) {  // uniform: my share includes late channels
    each_channel([&](uint32_t c, uint32_t b) {
      const uint32_t kk = b & 0x7FFFu;
      if (kk < sk && selected(c, kk)) {
        const uint32_t w = c >> 5;
        const int rank = (int)(pre[w] + __popc(lbits[w] & ((1u << (c & 31)) - 1u)));
        if (rank >= q0 && rank < q1) ent[E + rank - q0] = c | (b << 16);
      }
    });
  }
  for (int r = max(q0, (int)res_total) + tid; r < q1; r += kStepThreads) ent[E + r - q0] = g0 << 16;
  for (int e = E + tid; e < E + EL; e += kStepThreads) {
    sel[e] = 1;
    hl[e] = 0;
  }
  if (stamp) a.meta->spec_stamp[0][3] = wall_clock64();
  if (wg == 0 && tid == 0) {
    // the next call's band: ranks k + 2 margin to k + 1 - margin where the
    // band saw them (else its own ends); after the whole-g path, the
    // cut-to-key distance on either side
    uint32_t nband = 0;
    if (ka != kNoneKey && ka >= kMinNormal) {
      uint32_t lo2, hi2;
      if (fast) {
        lo2 = kl == kNoneKey ? blo : kl;
        hi2 = kh == kNoneKey ? bhi : kh + 1u;
      } else {
        const uint32_t d = ka - min(ks, ka);
        lo2 = ks > d + kMinNormal ? ks - d : kMinNormal;
        hi2 = ka + 1u + d;
        if (hi2 - lo2 > (uint32_t)kWin) {  // a quarter of the span above the cut
          const uint32_t top = ka + 1u + (uint32_t)kWin / 4u;
          if (top > (uint32_t)kWin) lo2 = max(lo2, top - (uint32_t)kWin);
          hi2 = lo2 + (uint32_t)kWin;
        }
      }
      lo2 = max(lo2, kMinNormal);
      hi2 = min(hi2, kInfKey + 1u);
      if (hi2 > lo2) nband = lo2 | (hi2 << 16);
    }
    a.meta->next_key = ks;
    a.meta->next_band = nband;
    a.meta->lo = lo_f;
    a.meta->hi = hi_f;
    a.meta->key_a = ka;
    a.meta->key_max = vmax < 0.f ? kNoneKey : (__float_as_uint(vmax) >> 16);
    a.meta->count_a = (int32_t)tot_a;
    a.meta->count_b = (int32_t)tot_b;
    a.meta->n_valid = fast ? 1 : 0;            // diagnostics: the band path was taken
    a.meta->pad = (int32_t)res_total;          // diagnostics: late channels
  }
  __syncthreads();  // ent, sel, hl published
  if (stamp) a.meta->stamp[2] = wall_clock64();

  // ---- D. up waves: h for every entry; down waves: accumulate --------------
  // Each role's ring slot is consumed, then reloaded with the entry kUpRing
  // (kDnRing) further on, so that many rows stay in flight.
  const int ET = E + EL;
  float acc[kChunkCols];
#pragma unroll
  for (int m = 0; m < kChunkCols; ++m) acc[m] = 0.f;
  if (up_role) {
#pragma unroll
    for (int d = 0; d < kUpRing; ++d) load_up(ET, grp + GUP * d, UR[d]);
    // rounds of kUpRing rows; every round but the last reloads its slots
    // with the next round's rows (clamped past the end), the last only
    // drains, so no load is left in flight at the end
    const int rounds = (ET + GUP - 1) / GUP;
    const int nring = (rounds + kUpRing - 1) / kUpRing;
    auto up_slot = [&](int r, int d, bool reload) {
      const int e = grp + GUP * r;
      const float u = group_sum<LPR>(up_dot_lds<LPR, CH>(UR[d], xlds, CHUNKS, l));
      if (l == 0 && e < ET) {
        const uint32_t ev = ent[e];
        const uint32_t h = h_of(ev >> 16, u);
        a.h_full[ev & 0xFFFFu] = (uint16_t)h;
        __hip_atomic_store(&hl[e], h | 0x10000u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
      // the reload issues before the next slot's arithmetic (which would
      // otherwise wait for that slot's rows first)
      __builtin_amdgcn_sched_barrier(0);
      if (reload) load_up(ET, grp + GUP * (r + kUpRing), UR[d]);
      __builtin_amdgcn_sched_barrier(0);
    };
    for (int q0 = 0; q0 + 1 < nring; ++q0) {
#pragma unroll
      for (int d = 0; d < kUpRing; ++d) up_slot(q0 * kUpRing + d, d, true);
    }
    if (nring > 0) {
#pragma unroll
      for (int d = 0; d < kUpRing; ++d) up_slot((nring - 1) * kUpRing + d, d, false);
    }
  } else {
    // the down waves share SIMDs with the up waves: issue first, so that
    // they keep up with the h the up waves produce (they sleep while
    // waiting for it)
    __builtin_amdgcn_s_setprio(2);
#pragma unroll
    for (int d = 0; d < kDnRing; ++d) load_dn(ET, sd + S * d, d);
    // rounds of kDnRing rows, the last one draining (as for the up rows)
    const int rows = (ET - sd + S - 1) / S;
    const int nring = (rows + kDnRing - 1) / kDnRing;
    auto dn_slot = [&](int i, int d, bool reload) {
      const int e = sd + S * i;
      if (i < rows) {
        const uint32_t hv = wait_nonzero(&hl[e]);
        float f = bf16_to_f32(hv & 0xFFFFu) * bf16_to_f32(DS[d] >> dsh) * 16.0f;
        f = sel[e] ? f : 0.f;
        chunk_accumulate(DR[d], f, acc);
      }
      if (reload) load_dn(ET, e + S * kDnRing, d);  // clamped past the end
      __builtin_amdgcn_sched_barrier(0);
    };
    for (int q0 = 0; q0 + 1 < nring; ++q0) {
#pragma unroll
      for (int d = 0; d < kDnRing; ++d) dn_slot(q0 * kDnRing + d, d, true);
    }
    if (nring > 0) {
#pragma unroll
      for (int d = 0; d < kDnRing; ++d) dn_slot((nring - 1) * kDnRing + d, d, false);
    }
  }
  __builtin_amdgcn_s_setprio(0);
  if (stamp) a.meta->stamp[3] = wall_clock64();

  // ---- E. the workgroup's partial row --------------------------------------
  // red[s][q][m] (rows of 33: conflict-free both ways), then a fixed-order
  // sum over the streams in output order
  if (!up_role) {
    float* mine = red + (sd * CHUNKS + q) * 33;
#pragma unroll
    for (int m = 0; m < kChunkCols; ++m) mine[m] = acc[m];
  }
  __syncthreads();
  float* out = a.partial + (size_t)wg * a.hidden;
  for (int o = tid; o < a.hidden; o += kStepThreads) {
    const int qq = o >> 5, mm = o & 31;
    float s = 0.f;
#pragma unroll
    for (int st = 0; st < S; ++st) s += red[(st * CHUNKS + qq) * 33 + mm];
    out[o] = s;
  }
  if (stamp) a.meta->stamp[4] = wall_clock64();
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
namespace {

template <int LPR, int CH>
int launch_step_width(const StepArgs& a, int blocks, hipStream_t stream) {
  using SS = StepShape<LPR, CH>;
  using L = StepLds<SS::CHUNKS, SS::S>;
  static const bool lds_ok =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&step_kernel<LPR, CH>),
                          hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)L::bytes(kStepMaxN)) == hipSuccess;
  if (!lds_ok) return hip_status(hipGetLastError());
  hipLaunchKernelGGL((step_kernel<LPR, CH>), dim3(blocks), dim3(kStepThreads), L::bytes(a.n),
                     stream, a);
  return hip_status(hipGetLastError());
}

}  // namespace

int step_grid() { return std::min(device_cus(), kStepMaxWorkgroups); }

bool step_supported(int64_t hidden, int64_t inter) {
  const int64_t chunks = hidden / kChunkCols;
  // an even number of scale groups per row (scales are read as aligned dwords)
  if (hidden % (2 * kGroupSize) != 0 || !(chunks == 160 || chunks == 128 || chunks == 80))
    return false;
  if (inter <= 0 || inter > kStepMaxN) return false;
  // every workgroup's share of candidates and late entries fits its lists
  return (inter + step_grid() - 1) / step_grid() <= kMaxEnt;
}

int step_max_gate_wgs() { return kMaxCandWgs; }

size_t step_partial_bytes(int64_t hidden) {
  return (size_t)kStepMaxWorkgroups * (size_t)std::max<int64_t>(hidden, 0) * sizeof(float);
}

int launch_step(const StepArgs& args, hipStream_t stream) {
  if (!step_supported(args.hidden, args.n) || args.k < 1 || args.k > args.n ||
      args.gate_wgs < 1 || args.gate_wgs > kMaxCandWgs)
    return DIP_ERR_UNSUPPORTED;
  StepArgs a = args;
  a.margin = (int)(a.n * (int64_t)tuning(DIP_TUNE_SPEC_MARGIN) / 1024);
  a.stamps = tuning(DIP_TUNE_TOPK_STAMPS);
  const int blocks = step_grid();
  const int chunks = a.hidden / kChunkCols;
  if (chunks == 160) return launch_step_width<32, 5>(a, blocks, stream);
  if (chunks == 128) return launch_step_width<32, 4>(a, blocks, stream);
  return launch_step_width<16, 5>(a, blocks, stream);
}

}  // namespace dip
