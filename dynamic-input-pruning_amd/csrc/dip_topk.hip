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
// numbers, max|s| and a_{k+1}, which a 32768-bin histogram of the 15-bit |s|
// keys gives exactly.  The steps are then replayed in registers with the same
// fp32 arithmetic, and the compaction runs once over keys staged in LDS.
//
//   pass 1 (many workgroups, or fused into the gate GEMV epilogue):
//       fine[key]++, coarse[key >> 7]++ with device-scope atomics
//   pass 2 (one workgroup of 1024 threads):
//       coarse suffix scan -> bin of a_{k+1} and of max; fine scan inside
//       those bins -> exact keys; 25 bisection steps -> (lo, hi); per-thread
//       tier counts -> block scan -> scatter of ascending ids; zero the
//       histogram bins it used so the workspace is clean for the next call.
#include "dip_common.h"
#include "dip_internal.h"

namespace dip {

namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr uint32_t kNoKey = 0xFFFFFFFFu;

// Inclusive suffix sum across the 64 lanes of a wave: lane L gets
// sum_{L' >= L} v_{L'}.
DIP_DEV uint32_t wave_suffix(uint32_t v, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    uint32_t t = __shfl_down(v, d, 64);
    if (lane + d < 64) v += t;
  }
  return v;
}

// Inclusive prefix sum across the 64 lanes of a wave (64-bit payload).
DIP_DEV uint64_t wave_prefix64(uint64_t v, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    uint64_t t = __shfl_up(v, d, 64);
    if (lane >= d) v += t;
  }
  return v;
}

// Highest lane whose predicate holds, or -1.
DIP_DEV int highest_lane(bool p) {
  const unsigned long long m = __ballot(p);
  return m ? 63 - __clzll(m) : -1;
}

}  // namespace

// Keys of 8 consecutive bf16 values from one 128-bit load, packed 2 per
// dword; positions past n get 0xFFFF (never counted, never selected).
DIP_DEV void load_keys8(const uint16_t* __restrict__ s, int n, int c, uint32_t out[4]) {
  const int base = c * 8;
  uint32_t w[4];
  if (base + 8 <= n) {
    const uint4 v = *reinterpret_cast<const uint4*>(s + base);
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = base + 2 * i < n ? s[base + 2 * i] : 0xFFFFu;
      const uint32_t hi = base + 2 * i + 1 < n ? s[base + 2 * i + 1] : 0xFFFFu;
      w[i] = lo | (hi << 16);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t lo = w[i] & 0xFFFFu, hi = w[i] >> 16;
    const uint32_t klo = lo == 0xFFFFu && base + 2 * i >= n ? 0xFFFFu : topk_key(lo);
    const uint32_t khi = hi == 0xFFFFu && base + 2 * i + 1 >= n ? 0xFFFFu : topk_key(hi);
    out[i] = klo | (khi << 16);
  }
}

// One workgroup of 1024 threads; dynamic LDS = 32768 u32 histogram bins.
// Thread t owns 8-element chunks t, t+1024, ... (kRounds of them, n <=
// kRounds * 8192) in registers, and histogram bins [32t, 32t+32).
template <int kRounds>
__global__ __launch_bounds__(kThreads) void topk_kernel(const uint16_t* __restrict__ s, int n,
                                                        int k, int32_t* __restrict__ idx,
                                                        TopkMeta* __restrict__ meta) {
  extern __shared__ uint32_t hist[];
  __shared__ uint32_t wsum[kWaves];
  __shared__ uint32_t wround[kWaves][kRounds];
  __shared__ int wmax[kWaves];
  __shared__ uint32_t sh_a, sh_max, sh_nvalid, sh_cut_a, sh_cut_b, sh_tot_a;
  __shared__ float sh_lo, sh_hi;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nchunks = (n + 7) >> 3;
  if (tid == 0 && meta) meta->stamp[0] = wall_clock64();

  // ---- keys into registers (loads issued before the LDS clear) ----------
  uint32_t key[kRounds][4];
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int c = tid + r * kThreads;
    if (c < nchunks) {
      load_keys8(s, n, c, key[r]);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) key[r][i] = 0xFFFFFFFFu;
    }
  }
  {
    uint4* h4 = reinterpret_cast<uint4*>(hist);
#pragma unroll
    for (int i = 0; i < kFineBins / 4 / kThreads; ++i) h4[tid + i * kThreads] = make_uint4(0, 0, 0, 0);
  }
  if (tid == 0) {
    sh_a = kNoKey;
    sh_max = kNoKey;
  }
  __syncthreads();
  if (tid == 0 && meta) meta->stamp[1] = wall_clock64();

  // ---- LDS histogram of valid keys ---------------------------------------
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = key[r][i] & 0xFFFFu, hi = key[r][i] >> 16;
      if (lo <= kKeyInf) atomicAdd(&hist[lo], 1u);
      if (hi <= kKeyInf) atomicAdd(&hist[hi], 1u);
    }
  }
  __syncthreads();
  if (tid == 0 && meta) meta->stamp[2] = wall_clock64();

  // ---- block suffix scan of my 32 bins' sums -----------------------------
  const uint4* my_bins = reinterpret_cast<const uint4*>(hist) + tid * 8;
  uint32_t tsum = 0;
  int top = -1;  // highest nonempty bin of mine
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint4 v = my_bins[i];
    tsum += v.x + v.y + v.z + v.w;
    if (v.x) top = 4 * i;
    if (v.y) top = 4 * i + 1;
    if (v.z) top = 4 * i + 2;
    if (v.w) top = 4 * i + 3;
  }
  const uint32_t wincl = wave_suffix(tsum, lane);      // within the wave, from my lane up
  int wtop = top >= 0 ? tid * 32 + top : -1;
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) wtop = max(wtop, __shfl_xor(wtop, d, 64));
  if (lane == 0) {
    wsum[wave] = wincl;   // lane 0 holds the whole wave's sum
    wmax[wave] = wtop;
  }
  __syncthreads();
  uint32_t above_waves = 0;
  int gmax = -1;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    if (w > wave) above_waves += wsum[w];
    gmax = max(gmax, wmax[w]);
  }
  const uint32_t suf_me = wincl + above_waves;   // valid keys in bins >= 32*tid
  const uint32_t suf_next = suf_me - tsum;       // valid keys in bins >= 32*(tid+1)
  const uint32_t need = (uint32_t)k + 1u;
  if (suf_me >= need && suf_next < need) {
    // a_{k+1} lies in my bins: walk them from the top
    uint32_t run = suf_next;
    uint32_t a = kNoKey;
    for (int b = 31; b >= 0 && a == kNoKey; --b) {
      run += hist[tid * 32 + b];
      if (run >= need) a = tid * 32 + b;
    }
    sh_a = a;
  }
  if (tid == 0) {
    sh_max = gmax < 0 ? kNoKey : (uint32_t)gmax;
    sh_nvalid = suf_me;
  }
  __syncthreads();

  // ---- replay the 25 fp32 bisection steps (topk_select.cu:141-158) --------
  if (tid == 0) {
    if (meta) meta->stamp[3] = wall_clock64();
    const uint32_t ka = sh_a, km = sh_max;
    const float a = ka == kNoKey ? 0.f : bf16_to_f32(ka);
    float hi = km == kNoKey ? 0.f : bf16_to_f32(km);
    float lo = 0.f;
    float t = 0.5f * (lo + hi);
#pragma unroll 1
    for (int step = 0; step < 25; ++step) {
      if (ka != kNoKey && a > t) lo = t; else hi = t;
      t = 0.5f * (lo + hi);
    }
    // |s| > v for a bf16 key b  <=>  b >= (bits(v) >> 16) + 1   (v >= 0)
    sh_cut_a = (__float_as_uint(hi) >> 16) + 1u;
    sh_cut_b = (__float_as_uint(lo) >> 16) + 1u;
    sh_lo = lo;
    sh_hi = hi;
    sh_tot_a = 0;
  }
  __syncthreads();
  if (tid == 0 && meta) meta->stamp[4] = wall_clock64();
  const uint32_t cut_a = sh_cut_a, cut_b = sh_cut_b;
  // tier-A size from the histogram: valid keys >= cut_a
  if (cut_a >= 32u * tid && cut_a < 32u * (tid + 1)) {
    uint32_t c = suf_next;
    for (uint32_t b = cut_a; b < 32u * (tid + 1); ++b) c += hist[b];
    sh_tot_a = c;
  }

  // ---- compaction: per-round block scans of (tier A, tier B) counts -------
  uint32_t cnt[kRounds];
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    uint32_t ca = 0, cb = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = key[r][i] & 0xFFFFu, hi = key[r][i] >> 16;
      ca += (lo <= kKeyInf && lo >= cut_a) + (hi <= kKeyInf && hi >= cut_a);
      cb += (lo <= kKeyInf && lo >= cut_b && lo < cut_a) + (hi <= kKeyInf && hi >= cut_b && hi < cut_a);
    }
    cnt[r] = ca | (cb << 16);
  }
  uint32_t incl[kRounds];
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    uint32_t v = cnt[r];
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const uint32_t t = __shfl_up(v, d, 64);
      if (lane >= d) v += t;
    }
    incl[r] = v;
    if (lane == 63) wround[wave][r] = v;
  }
  __syncthreads();
  const uint32_t tot_a = sh_tot_a;
  uint32_t base_a = 0, base_b = 0;   // counts before this round
  uint32_t pos_a[kRounds], pos_b[kRounds];
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    uint32_t before = 0, round_tot = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const uint32_t v = wround[w][r];
      if (w < wave) before += v;
      round_tot += v;
    }
    const uint32_t ex = before + incl[r] - cnt[r];
    pos_a[r] = base_a + (ex & 0xFFFFu);
    pos_b[r] = tot_a + base_b + (ex >> 16);
    base_a += round_tot & 0xFFFFu;
    base_b += round_tot >> 16;
  }
  const uint32_t uk = (uint32_t)k;
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    uint32_t pa = pos_a[r], pb = pos_b[r];
    const int c = tid + r * kThreads;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t kv = (key[r][i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
      if (kv > kKeyInf) continue;
      if (kv >= cut_a) {
        if (pa < uk) idx[pa] = c * 8 + i;
        ++pa;
      } else if (kv >= cut_b) {
        if (pb < uk) idx[pb] = c * 8 + i;
        ++pb;
      }
    }
  }
  const uint32_t filled = min(uk, tot_a + base_b);
  for (uint32_t p = filled + tid; p < uk; p += kThreads) idx[p] = 0;
  if (tid == 0 && meta) {
    meta->stamp[5] = wall_clock64();
    meta->lo = sh_lo;
    meta->hi = sh_hi;
    meta->count_a = (int32_t)tot_a;
    meta->count_b = (int32_t)base_b;
    meta->key_a = sh_a;
    meta->key_max = sh_max;
    meta->n_valid = (int32_t)sh_nvalid;
  }
}

template <int R>
int launch_topk_r(const uint16_t* s, int64_t n, int64_t k, int32_t* idx, TopkMeta* meta,
                  hipStream_t stream) {
  static const bool lds_ok = [] {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(&topk_kernel<R>),
                               hipFuncAttributeMaxDynamicSharedMemorySize,
                               kFineBins * (int)sizeof(uint32_t)) == hipSuccess;
  }();
  if (!lds_ok) return hip_status(hipGetLastError());
  hipLaunchKernelGGL(topk_kernel<R>, dim3(1), dim3(kThreads), kFineBins * sizeof(uint32_t),
                     stream, s, (int)n, (int)k, idx, meta);
  return hip_status(hipGetLastError());
}

int launch_topk(const uint16_t* s, int64_t n, int64_t k, int32_t* idx, TopkMeta* meta,
                hipStream_t stream) {
  if (n <= 2 * kThreads * 8) return launch_topk_r<2>(s, n, k, idx, meta, stream);
  if (n <= 4 * kThreads * 8) return launch_topk_r<4>(s, n, k, idx, meta, stream);
  return launch_topk_r<8>(s, n, k, idx, meta, stream);
}

}  // namespace dip

using namespace dip;

namespace {

TopkMeta* meta_of(void* ws) { return reinterpret_cast<TopkMeta*>(ws); }

int check_topk(const uint16_t* s, int32_t* idx, int64_t n, int64_t k, void* ws,
               size_t ws_bytes) {
  if (n < 0 || k < 0 || n > kTopkMaxN || k > INT32_MAX) return DIP_ERR_SHAPE;
  if (k > 0 && !idx) return DIP_ERR_NULL;
  if (n > 0 && !s) return DIP_ERR_NULL;
  if (n > 0 && (reinterpret_cast<uintptr_t>(s) & 15u)) return DIP_ERR_ALIGN;
  if (!ws || ws_bytes < dip_topk_workspace_size(n)) return DIP_ERR_WORKSPACE;
  return DIP_OK;
}

}  // namespace

extern "C" size_t dip_topk_workspace_size(int64_t n) {
  (void)n;
  return 256;  // holds the last call's thresholds (TopkMeta)
}

extern "C" int64_t dip_topk_max_n(void) { return kTopkMaxN; }

extern "C" int dip_topk_select(const uint16_t* s, int32_t* idx, int64_t n, int64_t k,
                               void* workspace, size_t ws_bytes, void* stream) {
  int st = check_topk(s, idx, n, k, workspace, ws_bytes);
  if (st) return st;
  if (k == 0) return DIP_OK;
  return launch_topk(s, n, k, idx, meta_of(workspace), (hipStream_t)stream);
}

extern "C" int dip_topk_meta(const void* workspace, void* meta_out, void* stream) {
  if (!workspace || !meta_out) return DIP_ERR_NULL;
  return hip_status(hipMemcpyAsync(meta_out, workspace, 16, hipMemcpyDeviceToDevice,
                                   (hipStream_t)stream));
}
