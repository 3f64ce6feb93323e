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
// Two kernels:
//   analysis (one workgroup of 1024 threads): all n values into VGPRs
//     (wave w holds the R*512 consecutive values [w*512R, (w+1)*512R)),
//     LDS histogram, max and a_{k+1} (only the waves holding those ranks
//     search their bins), the 25 bisection steps, then per-wave tier counts
//     -> TopkShare in the workspace;
//   scatter (kTopkSlices workgroups of 256 threads): workgroup w re-reads
//     slice w (the values wave w held), takes its starting positions from
//     the earlier slices' counts, runs one block scan and writes its ids
//     through LDS with coalesced stores.
//
// Magnitudes are used unflushed: bf16 subnormals (|bits| 1..0x7F) are 0 under
// the reference's --use_fast_math, so histogram bins below 0x80 all mean 0
// and both cuts are clamped to >= 0x80; NaN and padding (0xFFFF) land in bins
// above 0x7F80, which the search ignores and the tier ranges exclude.
#include "dip_common.h"
#include "dip_internal.h"

namespace dip {

namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
static_assert(kWaves == kTopkSlices, "one scatter slice per analysis wave");
constexpr int kScatterThreads = 256;
constexpr uint32_t kNoKey = 0xFFFFFFFFu;
constexpr uint32_t kMaxValidKey = kKeyInf;  // 0x7F80: +inf
constexpr uint32_t kMinNormalKey = 0x0080u;

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// DPP move with zero fill: lanes whose source is outside the row (or whose
// row is masked off) read 0.
template <int CTRL, int ROW_MASK = 0xF>
DIP_DEV uint32_t dpp_zero(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xF, true);
}

// Inclusive prefix sum over the 64 lanes of a wave: Hillis-Steele within
// rows of 16 (row_shr 1, 2, 4, 8), then row_bcast:15 / row_bcast:31 carry
// the row totals into the later rows.
DIP_DEV uint32_t wave_prefix(uint32_t v) {
  v += dpp_zero<0x111>(v);        // row_shr:1
  v += dpp_zero<0x112>(v);        // row_shr:2
  v += dpp_zero<0x114>(v);        // row_shr:4
  v += dpp_zero<0x118>(v);        // row_shr:8
  v += dpp_zero<0x142, 0xA>(v);   // row_bcast:15 -> rows 1, 3
  v += dpp_zero<0x143, 0xC>(v);   // row_bcast:31 -> rows 2, 3
  return v;
}

DIP_DEV uint32_t lane63(uint32_t v) { return (uint32_t)__builtin_amdgcn_readlane((int)v, 63); }

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

}  // namespace

// ---------------------------------------------------------------------------
// Analysis: R rounds of 8 values per lane, n <= 16 waves * 64 lanes * 8R.
// ---------------------------------------------------------------------------
template <int R>
__global__ __launch_bounds__(kThreads) void topk_analysis_kernel(
    const uint16_t* __restrict__ s, int n, int k, TopkMeta* __restrict__ meta,
    TopkShare* __restrict__ share, int stamps) {
  extern __shared__ uint32_t hist[];  // kFineBins bins
  __shared__ uint32_t wtot[kWaves];
  __shared__ uint32_t sh_a, sh_max, sh_cut_a, sh_cut_b;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  // Phase stamps (diagnostics, off by default: each store makes the storing
  // wave wait for its completion at the next vmcnt wait).
  const bool stamp = stamps && tid == 0;
  if (stamp) {
    meta->stamp[0] = wall_clock64();
    meta->cycles[0] = clock64();
  }

  // ---- 1. values into registers; clear the histogram meanwhile -----------
  uint32_t key[R][4];
#pragma unroll
  for (int r = 0; r < R; ++r) load_chunk8(s, n, (wave * 64 * R + 64 * r + lane) * 8, key[r]);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int base = (wave * 64 * R + 64 * r + lane) * 8;
    if (base < n && base + 8 > n) load_tail8(s, n, base, key[r]);
  }
  {
    uint4* h4 = reinterpret_cast<uint4*>(hist);
#pragma unroll
    for (int i = 0; i < kFineBins / 4 / kThreads; ++i)
      h4[tid + i * kThreads] = make_uint4(0, 0, 0, 0);
  }
  if (tid == 0) {
    sh_a = kNoKey;
    sh_max = kNoKey;
  }
  __syncthreads();
  if (stamp) meta->stamp[1] = wall_clock64();

  // ---- 2. histogram of every magnitude (NaN / padding bins ignored later) --
  // (rounds wholly past n are skipped: their padding would pile onto one bin)
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if ((wave * 64 * R + 64 * r + lane) * 8 < n) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        atomicAdd(&hist[key[r][i] & 0x7FFFu], 1u);
        atomicAdd(&hist[(key[r][i] >> 16) & 0x7FFFu], 1u);
      }
    }
  }
  __syncthreads();
  if (stamp) meta->stamp[2] = wall_clock64();

  // ---- 3. max and a_{k+1} ------------------------------------------------
  // Wave w reads its 2048 bins as eight 256-bin rows j; lane L holds bins
  // 2048w + 256j + 4L .. +3 (consecutive lanes, consecutive 16 B: no bank
  // conflicts).  Wave totals first; only a wave that holds rank 1 or rank
  // k+1 (counting from the top bin) scans its rows.
  uint32_t nvalid = 0;
  {
    const uint4* h4 = reinterpret_cast<const uint4*>(hist);
    uint4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = h4[512 * wave + 64 * j + lane];
    if (wave == kWaves - 1) {
      // bins above +inf (NaN magnitudes, padding) do not exist
      const uint32_t b0 = 2048u * wave + 256u * 7 + 4u * lane;
      if (b0 + 0 > kMaxValidKey) v[7].x = 0;
      if (b0 + 1 > kMaxValidKey) v[7].y = 0;
      if (b0 + 2 > kMaxValidKey) v[7].z = 0;
      if (b0 + 3 > kMaxValidKey) v[7].w = 0;
    }
    uint32_t sum4[8];
    uint32_t lsum = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      sum4[j] = v[j].x + v[j].y + v[j].z + v[j].w;
      lsum += sum4[j];
    }
    const uint32_t wsum = lane63(wave_prefix(lsum));
    if (lane == 0) wtot[wave] = wsum;
    __syncthreads();
    uint32_t above = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      above += w > wave ? wtot[w] : 0u;
      nvalid += wtot[w];
    }
    const uint32_t need = (uint32_t)k + 1u;
    const bool own1 = above < 1u && wsum >= 1u;
    const bool ownk = above < need && above + wsum >= need;
    if (own1 || ownk) {  // wave-uniform
      uint32_t carry = above;
#pragma unroll
      for (int j = 7; j >= 0; --j) {
        const uint32_t p = wave_prefix(sum4[j]);
        const uint32_t t = lane63(p);
        const uint32_t ge = carry + t - p + sum4[j];  // valid values in bins >= my first bin
        const uint32_t gt = ge - sum4[j];             // ... in bins >= my first bin + 4
        carry += t;
        const uint32_t b0 = 2048u * wave + 256u * j + 4u * lane;
        const uint32_t cnt[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
        if (own1 && gt < 1u && ge >= 1u) {
          uint32_t run = gt, b = kNoKey;
#pragma unroll
          for (int e = 3; e >= 0; --e) {
            run += cnt[e];
            if (b == kNoKey && run >= 1u) b = b0 + e;
          }
          sh_max = b;
        }
        if (ownk && gt < need && ge >= need) {
          uint32_t run = gt, b = kNoKey;
#pragma unroll
          for (int e = 3; e >= 0; --e) {
            run += cnt[e];
            if (b == kNoKey && run >= need) b = b0 + e;
          }
          sh_a = b;
        }
      }
    }
  }
  __syncthreads();
  if (stamp) meta->stamp[3] = wall_clock64();

  // ---- 4. replay the 25 fp32 bisection steps (topk_select.cu:141-158) -----
  if (tid == 0) {
    uint32_t ka = sh_a, km = sh_max;
    if (ka != kNoKey && ka < kMinNormalKey) ka = 0;  // subnormal -> 0
    if (km != kNoKey && km < kMinNormalKey) km = 0;
    const float a = ka == kNoKey ? 0.f : bf16_to_f32(ka);
    float hi = km == kNoKey ? 0.f : bf16_to_f32(km);
    float lo = 0.f;
    float t = 0.5f * (lo + hi);
#pragma unroll 1
    for (int step = 0; step < 25; ++step) {
      if (ka != kNoKey && a > t) lo = t; else hi = t;
      t = 0.5f * (lo + hi);
    }
    // |s| > v for a bf16 magnitude b  <=>  b >= (bits(v) >> 16) + 1  (v >= 0);
    // subnormal magnitudes never qualify, so the cuts start at 0x80.
    sh_cut_a = max((__float_as_uint(hi) >> 16) + 1u, kMinNormalKey);
    sh_cut_b = max((__float_as_uint(lo) >> 16) + 1u, kMinNormalKey);
    meta->lo = lo;
    meta->hi = hi;
    meta->key_a = ka;
    meta->key_max = km;
    meta->n_valid = (int32_t)nvalid;
  }
  __syncthreads();
  if (stamp) meta->stamp[4] = wall_clock64();

  // ---- 5. tier counts of each wave's values -------------------------------
  const uint32_t cut_a = sh_cut_a, cut_b = sh_cut_b;
  const uint32_t cut_a2 = cut_a * 0x10001u, cut_b2 = cut_b * 0x10001u;
  const uint32_t span_a2 = (kMaxValidKey + 1u - cut_a) * 0x10001u;  // b - cut_a < span_a
  const uint32_t span_b2 = (cut_a - cut_b) * 0x10001u;              // b - cut_b < span_b
  uint32_t la = 0, lb = 0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint32_t c = tier_counts8(key[r], cut_a2, span_a2, cut_b2, span_b2);
    la += c & 0xFFFFu;
    lb += c >> 16;
  }
  // packed: a wave's counts stay below 2^16 (at most 512R values)
  const uint32_t wt = lane63(wave_prefix(la | (lb << 16)));
  if (lane == 0) {
    share->slice_a[wave] = wt & 0xFFFFu;
    share->slice_b[wave] = wt >> 16;
  }
  if (tid == 0) {
    share->cut_a = cut_a;
    share->cut_b = cut_b;
    if (stamps) {
      meta->stamp[5] = wall_clock64();
      meta->cycles[1] = clock64();
    }
  }
}

// ---------------------------------------------------------------------------
// Scatter: workgroup w handles slice w = values [w*512R, (w+1)*512R); thread t
// holds the 2R consecutive values at w*512R + 2R*t.
// ---------------------------------------------------------------------------
template <int R>
__global__ __launch_bounds__(kScatterThreads) void topk_scatter_kernel(
    const uint16_t* __restrict__ s, int n, int k, int32_t* __restrict__ idx,
    const TopkShare* __restrict__ share, TopkMeta* __restrict__ meta) {
  constexpr int kPer = 2 * R;           // values per thread
  constexpr int kSlice = 512 * R;       // values per slice
  __shared__ uint32_t stage[kSlice];
  __shared__ uint32_t wsum[kScatterThreads / 64];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int w = blockIdx.x;
  const int base = w * kSlice + tid * kPer;

  uint32_t key[kPer / 8][4];
#pragma unroll
  for (int c = 0; c < kPer / 8; ++c) load_chunk8(s, n, base + 8 * c, key[c]);
#pragma unroll
  for (int c = 0; c < kPer / 8; ++c)
    if (base + 8 * c < n && base + 8 * c + 8 > n) load_tail8(s, n, base + 8 * c, key[c]);

  const uint32_t cut_a = share->cut_a, cut_b = share->cut_b;
  uint32_t pre_a = 0, pre_b = 0, tot_a = 0, tot_b = 0;
#pragma unroll
  for (int q = 0; q < kTopkSlices; ++q) {
    const uint32_t xa = share->slice_a[q], xb = share->slice_b[q];
    pre_a += q < w ? xa : 0u;
    pre_b += q < w ? xb : 0u;
    tot_a += xa;
    tot_b += xb;
  }
  const uint32_t my_a = share->slice_a[w];

  const uint32_t cut_a2 = cut_a * 0x10001u, cut_b2 = cut_b * 0x10001u;
  const uint32_t span_a = kMaxValidKey + 1u - cut_a, span_b = cut_a - cut_b;
  uint32_t cnt = 0;
#pragma unroll
  for (int c = 0; c < kPer / 8; ++c)
    cnt += tier_counts8(key[c], cut_a2, span_a * 0x10001u, cut_b2, span_b * 0x10001u);
  // block exclusive scan of the packed (A | B << 16) counts (slice totals < 2^16)
  const uint32_t incl = wave_prefix(cnt);
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  uint32_t before = 0;
#pragma unroll
  for (int q = 0; q < kScatterThreads / 64; ++q) before += q < wave ? wsum[q] : 0u;
  const uint32_t ex = before + incl - cnt;
  // stage: the slice's tier-A ids at [0, my_a), its tier-B ids after them
  uint32_t pa = ex & 0xFFFFu;
  uint32_t pb = my_a + (ex >> 16);
#pragma unroll
  for (int c = 0; c < kPer / 8; ++c) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t b = (key[c][i >> 1] >> (16 * (i & 1))) & 0x7FFFu;
      const bool in_a = b - cut_a < span_a;
      const bool in_b = b - cut_b < span_b;
      if (in_a | in_b) stage[in_a ? pa : pb] = (uint32_t)(base + 8 * c + i);
      pa += in_a;
      pb += in_b;
    }
  }
  __syncthreads();
  // copy out: tier A to [pre_a, pre_a + my_a), tier B to tot_a + pre_b + ...,
  // both capped at k
  const uint32_t uk = (uint32_t)k;
  const uint32_t my_b = share->slice_b[w];
  for (uint32_t i = tid; i < my_a + my_b; i += kScatterThreads) {
    const uint32_t pos = i < my_a ? pre_a + i : tot_a + pre_b + (i - my_a);
    if (pos < uk) idx[pos] = (int32_t)stage[i];
  }
  // unfilled slots (fewer than k values qualify) are 0, as in the reference
  const uint32_t filled = min(uk, tot_a + tot_b);
  for (uint32_t p = filled + (uint32_t)(w * kScatterThreads + tid); p < uk;
       p += kTopkSlices * kScatterThreads)
    idx[p] = 0;
  if (w == 0 && tid == 0) {
    meta->count_a = (int32_t)tot_a;
    meta->count_b = (int32_t)tot_b;
  }
}

template <int R>
int launch_topk_r(const uint16_t* s, int64_t n, int64_t k, int32_t* idx, TopkMeta* meta,
                  hipStream_t stream) {
  static const bool lds_ok = [] {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(&topk_analysis_kernel<R>),
                               hipFuncAttributeMaxDynamicSharedMemorySize,
                               kFineBins * (int)sizeof(uint32_t)) == hipSuccess;
  }();
  if (!lds_ok) return hip_status(hipGetLastError());
  TopkShare* share =
      reinterpret_cast<TopkShare*>(reinterpret_cast<char*>(meta) + kTopkShareOffset);
  hipLaunchKernelGGL((topk_analysis_kernel<R>), dim3(1), dim3(kThreads),
                     kFineBins * sizeof(uint32_t), stream, s, (int)n, (int)k, meta, share,
                     tuning(DIP_TUNE_TOPK_STAMPS));
  int st = hip_status(hipGetLastError());
  if (st) return st;
  hipLaunchKernelGGL((topk_scatter_kernel<R>), dim3(kTopkSlices), dim3(kScatterThreads), 0,
                     stream, s, (int)n, (int)k, idx, share, meta);
  return hip_status(hipGetLastError());
}

int launch_topk(const uint16_t* s, int64_t n, int64_t k, int32_t* idx, TopkMeta* meta,
                hipStream_t stream) {
  if (n <= 4 * 8 * kThreads) return launch_topk_r<4>(s, n, k, idx, meta, stream);
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

static_assert(sizeof(TopkMeta) <= kTopkShareOffset, "TopkMeta overlaps TopkShare");
static_assert(kTopkShareOffset + sizeof(TopkShare) <= 512, "top-k workspace");

extern "C" size_t dip_topk_workspace_size(int64_t n) {
  (void)n;
  return 512;  // the last call's thresholds (TopkMeta) and cuts / tier counts (TopkShare)
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
