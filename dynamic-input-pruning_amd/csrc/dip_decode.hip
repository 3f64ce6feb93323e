// dip_decode.hip — the one-token decode steps of a Qwen3 decoder layer around
// the DIP MLP: residual add + RMSNorm, q/k RMSNorm + rotary embedding + key /
// value cache write, and grouped-query attention of the token over the cache.
//
// The reference runs these steps through transformers' Qwen3 modules with
// PyTorch ops (the model its loader builds, dip_stream_predispatch.py:218-289;
// transformers' modeling_qwen3: Qwen3RMSNorm.forward, apply_rotary_pos_emb,
// Qwen3Attention.forward, Qwen3DecoderLayer.forward).  Where those modules
// round to bf16 these kernels round at the same points:
//   RMSNorm   y = bf16(w * bf16(x * rsqrt(mean(x^2) + eps)))  (fp32 mean)
//   residual  h = bf16(h + a)
//   rotary    q' = bf16(bf16(q * cos) + bf16(rotate_half(q) * sin))
// The attention keeps scores, softmax and the weighted value sum in fp32 and
// rounds its output once (torch's fused attention kernels round in between,
// so the two agree to bf16 rounding, not bit for bit).
//
// Every kernel here is latency-bound (a few KB per token, except attention
// over a long cache); each is one launch of a handful of workgroups.
#include "dip_common.h"
#include "dip_internal.h"

namespace dip {
namespace {

constexpr int kNormThreads = 256;
constexpr int kNormVecs = 4;              // 16-byte vectors per thread: n <= 8192
constexpr int kHeadDim = 128;
constexpr int kAttnChunk = 32;            // cache positions per attention workgroup
constexpr int kPartFloats = 2 + kHeadDim; // m, l, acc[128] per (kv head, chunk, query head)

// Wave-wide reductions on DPP / permlane exchanges (no LDS round trips).
DIP_DEV float wave_sum(float v) { return group_sum<64>(v); }
DIP_DEV float wave_max(float v) { return group_max<64>(v); }

DIP_DEV float round_bf16(float v) { return bf16_to_f32(f32_to_bf16(v)); }

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

DIP_DEV bf16x8_t as_bf16x8(const uint4& v) {
  return __builtin_bit_cast(bf16x8_t, u32x4_t{v.x, v.y, v.z, v.w});
}

// h = bf16(h + add) when add is given; out = RMSNorm(h) * w.  One workgroup;
// thread t owns the 16-byte vectors t, t + 256, ... (8 values each), all
// loaded before anything is stored.
__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_kernel(
    uint16_t* __restrict__ h, const uint16_t* __restrict__ add, const uint16_t* __restrict__ w,
    uint16_t* __restrict__ out, int n, float eps) {
  __shared__ float part[kNormThreads / 64];
  const int nv = n / 8;
  uint4 hv[kNormVecs], av[kNormVecs], wv[kNormVecs];
#pragma unroll
  for (int j = 0; j < kNormVecs; ++j) {
    const int c = threadIdx.x + j * kNormThreads;
    hv[j] = av[j] = wv[j] = make_uint4(0, 0, 0, 0);
    if (c < nv) {
      hv[j] = reinterpret_cast<const uint4*>(h)[c];
      av[j] = add ? reinterpret_cast<const uint4*>(add)[c] : make_uint4(0, 0, 0, 0);
      wv[j] = reinterpret_cast<const uint4*>(w)[c];
    }
  }
  float x[kNormVecs][8];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < kNormVecs; ++j) {
    const int c = threadIdx.x + j * kNormThreads;
    const uint32_t hw[4] = {hv[j].x, hv[j].y, hv[j].z, hv[j].w};
    const uint32_t aw[4] = {av[j].x, av[j].y, av[j].z, av[j].w};
    uint32_t nw[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float lo = bf16_to_f32(hw[e] & 0xFFFFu), hi = bf16_to_f32(hw[e] >> 16);
      if (add) {
        lo = round_bf16(lo + bf16_to_f32(aw[e] & 0xFFFFu));
        hi = round_bf16(hi + bf16_to_f32(aw[e] >> 16));
      }
      nw[e] = f32_to_bf16(lo) | (f32_to_bf16(hi) << 16);
      x[j][2 * e] = lo;
      x[j][2 * e + 1] = hi;
      if (c < nv) ss += lo * lo + hi * hi;
    }
    if (add && c < nv) reinterpret_cast<uint4*>(h)[c] = make_uint4(nw[0], nw[1], nw[2], nw[3]);
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; ++i) tot += part[i];
  const float r = rsqrtf(tot * (1.0f / (float)n) + eps);
#pragma unroll
  for (int j = 0; j < kNormVecs; ++j) {
    const int c = threadIdx.x + j * kNormThreads;
    if (c >= nv) continue;
    const uint32_t ww[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
    uint32_t ow[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t lo = f32_to_bf16(bf16_to_f32(ww[e] & 0xFFFFu) * round_bf16(x[j][2 * e] * r));
      const uint32_t hi =
          f32_to_bf16(bf16_to_f32(ww[e] >> 16) * round_bf16(x[j][2 * e + 1] * r));
      ow[e] = lo | (hi << 16);
    }
    reinterpret_cast<uint4*>(out)[c] = make_uint4(ow[0], ow[1], ow[2], ow[3]);
  }
}

// One workgroup (one wave) per head of the fused q|k|v projection output:
// q heads [0, nh) and k heads [nh, nh + nkv) get RMSNorm over the head and
// the rotary embedding at `pos`; q goes to q_out, k to the key cache; v heads
// [nh + nkv, nh + 2 nkv) are copied to the value cache.  Lane l holds
// dimensions 2l and 2l + 1; rotate_half pairs dimension d with d +- 64, which
// lives in lane l ^ 32.  Cache writes happen only for 0 <= pos < max_len.
__global__ __launch_bounds__(64) void qk_rope_cache_kernel(
    const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ q_w,
    const uint16_t* __restrict__ k_w, const uint16_t* __restrict__ cos_t,
    const uint16_t* __restrict__ sin_t, const int64_t* __restrict__ pos_p,
    uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_cache,
    uint16_t* __restrict__ v_cache, int nh, int nkv, int max_len, float eps) {
  const int head = blockIdx.x;
  const int l = threadIdx.x;
  const int64_t pos = *pos_p;
  const bool pos_ok = pos >= 0 && pos < max_len;
  const uint32_t pair = reinterpret_cast<const uint32_t*>(qkv)[(size_t)head * 64 + l];
  if (head >= nh + nkv) {
    if (pos_ok)
      reinterpret_cast<uint32_t*>(v_cache)[((size_t)(head - nh - nkv) * max_len + pos) * 64 + l] =
          pair;
    return;
  }
  const bool is_q = head < nh;
  const uint32_t wp = reinterpret_cast<const uint32_t*>(is_q ? q_w : k_w)[l];
  const float x0 = bf16_to_f32(pair & 0xFFFFu), x1 = bf16_to_f32(pair >> 16);
  const float ss = wave_sum(x0 * x0 + x1 * x1);
  const float r = rsqrtf(ss * (1.0f / (float)kHeadDim) + eps);
  const uint32_t y0 = f32_to_bf16(bf16_to_f32(wp & 0xFFFFu) * round_bf16(x0 * r));
  const uint32_t y1 = f32_to_bf16(bf16_to_f32(wp >> 16) * round_bf16(x1 * r));
  // rotate_half: dims [0, 64) take -y[d + 64], dims [64, 128) take y[d - 64]
  float r0 = bf16_to_f32(__shfl_xor(y0, 32, 64));
  float r1 = bf16_to_f32(__shfl_xor(y1, 32, 64));
  if (l < 32) {
    r0 = -r0;
    r1 = -r1;
  }
  const size_t trow = (size_t)(pos_ok ? pos : 0) * 64 + l;
  const uint32_t cs = reinterpret_cast<const uint32_t*>(cos_t)[trow];
  const uint32_t sn = reinterpret_cast<const uint32_t*>(sin_t)[trow];
  const uint32_t o0 = f32_to_bf16(round_bf16(bf16_to_f32(y0) * bf16_to_f32(cs & 0xFFFFu)) +
                                  round_bf16(r0 * bf16_to_f32(sn & 0xFFFFu)));
  const uint32_t o1 = f32_to_bf16(round_bf16(bf16_to_f32(y1) * bf16_to_f32(cs >> 16)) +
                                  round_bf16(r1 * bf16_to_f32(sn >> 16)));
  const uint32_t o = o0 | (o1 << 16);
  if (is_q)
    reinterpret_cast<uint32_t*>(q_out)[(size_t)head * 64 + l] = o;
  else if (pos_ok)
    reinterpret_cast<uint32_t*>(k_cache)[((size_t)(head - nh) * max_len + pos) * 64 + l] = o;
}

// Attention, pass 1: workgroup (one wave) = (32-row chunk c, kv head): the
// scores of the G query heads over the chunk's rows up to pos on bf16 MFMA
// (A = 16 cache rows, B = the q heads; exact products, fp32 sums), softmax
// in fp32, the value sum in fp32 on the VALU (lane l: dimensions 2l, 2l + 1).
// Writes per query head the chunk's max score m, sum of exp(s - m) and the
// unnormalised value sum.
template <int G>
__global__ __launch_bounds__(64) void attn_partial_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k_cache,
    const uint16_t* __restrict__ v_cache, const int64_t* __restrict__ pos_p,
    float* __restrict__ part, int max_len, int nchunks, float scale) {
  static_assert(G <= 16, "one MFMA column per query head");
  __shared__ __align__(16) uint32_t qb[16][64 + 4];  // q as bf16 pairs; heads >= G are 0
  __shared__ float ps[G][kAttnChunk];
  __shared__ float cm[G], cl[G];
  const int c = blockIdx.x, kvh = blockIdx.y, l = threadIdx.x;
  const int l16 = l & 15, kb = l >> 4;
  const int64_t pos = *pos_p;
  const int64_t last = pos < (int64_t)max_len ? pos : (int64_t)max_len - 1;
  const int start = c * kAttnChunk;
  if ((int64_t)start > last) return;  // no position of this chunk is attended
  const int npos = (int)((last - start + 1) < kAttnChunk ? (last - start + 1) : kAttnChunk);

  uint4 ka[2][4];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int row = start + 16 * t + l16;
    if ((int64_t)row <= last) {
      const uint4* src = reinterpret_cast<const uint4*>(
          k_cache + ((size_t)kvh * max_len + row) * kHeadDim + 32 * kb);
#pragma unroll
      for (int j = 0; j < 4; ++j) ka[t][j] = src[j];
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) ka[t][j] = make_uint4(0, 0, 0, 0);
    }
  }
  const uint32_t* vcol =
      reinterpret_cast<const uint32_t*>(v_cache + ((size_t)kvh * max_len + start) * kHeadDim) + l;
  uint32_t vv[kAttnChunk];
#pragma unroll
  for (int j = 0; j < kAttnChunk; ++j) vv[j] = j < npos ? vcol[(size_t)j * 64] : 0u;
  const uint32_t* qsrc = reinterpret_cast<const uint32_t*>(q + (size_t)kvh * G * kHeadDim);
  for (int i = l; i < 16 * 64; i += 64) qb[i >> 6][i & 63] = (i >> 6) < G ? qsrc[i] : 0u;
  __syncthreads();

  uint4 bq[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) bq[j] = *reinterpret_cast<const uint4*>(&qb[l16][16 * kb + 4 * j]);
  float sc[2][4];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    floatx4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j)
      d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(ka[t][j]), as_bf16x8(bq[j]), d, 0, 0,
                                                  0);
#pragma unroll
    for (int r = 0; r < 4; ++r) sc[t][r] = 16 * t + 4 * kb + r < npos ? d[r] * scale : -INFINITY;
  }
  float mx = -INFINITY;
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) mx = fmaxf(mx, sc[t][r]);
  mx = row_pair_max32(row_pair_max16(mx));
  float sum = 0.f;
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float e = sc[t][r] == -INFINITY ? 0.f : expf(sc[t][r] - mx);
      sum += e;
      if (l16 < G) ps[l16][16 * t + 4 * kb + r] = e;
    }
  sum = row_pair_sum32(row_pair_sum16(sum));
  if (kb == 0 && l16 < G) {
    cm[l16] = mx;
    cl[l16] = sum;
  }
  __syncthreads();

  float a0[G], a1[G];
#pragma unroll
  for (int g = 0; g < G; ++g) a0[g] = a1[g] = 0.f;
#pragma unroll
  for (int j = 0; j < kAttnChunk; ++j) {
    if (j < npos) {
      const float v0 = bf16_to_f32(vv[j] & 0xFFFFu), v1 = bf16_to_f32(vv[j] >> 16);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        a0[g] = fmaf(ps[g][j], v0, a0[g]);
        a1[g] = fmaf(ps[g][j], v1, a1[g]);
      }
    }
  }
  float* out = part + ((size_t)kvh * nchunks + c) * G * kPartFloats;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float* o = out + g * kPartFloats;
    if (l == 0) {
      o[0] = cm[g];
      o[1] = cl[g];
    }
    o[2 + 2 * l] = a0[g];
    o[3 + 2 * l] = a1[g];
  }
}

// Attention, pass 2: one workgroup per query head merges the chunks
// 0 .. pos/32: wave w takes chunks w, w + 4, ... with a one-pass running
// rescale (max, sum, value sum), then the 4 waves merge through LDS in a
// fixed order and write bf16(sum / l).
__global__ __launch_bounds__(256) void attn_combine_kernel(
    const float* __restrict__ part, const int64_t* __restrict__ pos_p, uint16_t* __restrict__ out,
    int G, int max_len, int nchunks) {
  __shared__ float wm[4], wl[4];
  __shared__ float wa[4][kHeadDim];
  const int qh = blockIdx.x, wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int kvh = qh / G, g = qh % G;
  const int64_t pos = *pos_p;
  const int64_t last = pos < (int64_t)max_len ? pos : (int64_t)max_len - 1;
  const int nc = last < 0 ? 0 : (int)(last / kAttnChunk) + 1;
  const float* base = part + (size_t)kvh * nchunks * G * kPartFloats + (size_t)g * kPartFloats;
  const size_t stride = (size_t)G * kPartFloats;
  float mx = -INFINITY, den = 0.f, a0 = 0.f, a1 = 0.f;
  for (int c = wave; c < nc; c += 4) {
    const float* pc = base + c * stride;
    const float mc = pc[0], lc = pc[1], v0 = pc[2 + 2 * l], v1 = pc[3 + 2 * l];
    const float mn = fmaxf(mx, mc);
    const float fo = expf(mx - mn), fn = expf(mc - mn);
    den = den * fo + lc * fn;
    a0 = a0 * fo + v0 * fn;
    a1 = a1 * fo + v1 * fn;
    mx = mn;
  }
  if (l == 0) {
    wm[wave] = mx;
    wl[wave] = den;
  }
  wa[wave][2 * l] = a0;
  wa[wave][2 * l + 1] = a1;
  __syncthreads();
  if (wave != 0) return;
  float m = -INFINITY;
#pragma unroll
  for (int w = 0; w < 4; ++w) m = fmaxf(m, wm[w]);
  float d = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float f = wl[w] > 0.f ? expf(wm[w] - m) : 0.f;
    d = fmaf(f, wl[w], d);
    o0 = fmaf(f, wa[w][2 * l], o0);
    o1 = fmaf(f, wa[w][2 * l + 1], o1);
  }
  reinterpret_cast<uint32_t*>(out)[(size_t)qh * 64 + l] =
      f32_to_bf16(o0 / d) | (f32_to_bf16(o1 / d) << 16);
}

// Norm + rotary + cache write + attention in one launch, for caches of at
// most kFusedMaxLen rows (4 waves up to 128 rows, 16 beyond, which walk the
// 32-row chunks 16 at a time): workgroup = HPW consecutive query heads of one kv
// head (group = nh / nkv query heads share it).  Every workgroup of a group
// normalises and rotates the group's k itself; only the group's first
// workgroup writes k and v to cache row pos (the others take this token's
// row from their own LDS copy, never from the cache).  One query head per
// workgroup spreads a layer over nh workgroups instead of nkv, which takes
// the per-head norm, rotary, softmax and value sums off one serial chain.
//   0. every load that does not need this token's k and v is issued first:
//      the q heads, k and v, the norm weights and the cos / sin rows into
//      LDS, each wave's first 32-row chunk of the cache into registers;
//   1. RMSNorm + rotary as qk_rope_cache_kernel; q into LDS as bf16, this
//      token's k and v into LDS (and into cache row pos);
//   2. wave w of NW takes the chunks w, w + NW, ...: the scores on bf16 MFMA
//      (v_mfma_f32_16x16x32_bf16, A = 16 cache rows, B = the q heads, exact
//      products, fp32 sums; row pos from LDS, not read back), softmax in
//      fp32, the value sum in fp32 on the VALU, merged into a running (max,
//      sum, value sum) per query head;
//   3. the NW waves' partials are merged through LDS in a fixed order.
// One launch wins over the split path up to about 900 cache rows (64 query /
// 8 kv heads: 11.9 against 15.6 us at 512 rows, 18.3 against 17.3 at 1024);
// beyond, each query head's workgroup re-reading its kv head's rows costs
// more than the split path's extra launches.
constexpr int kFusedMaxLen = 1024;

template <int HPW, int NW>
__global__ __launch_bounds__(NW * 64) void attn_fused_kernel(
    const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ q_w,
    const uint16_t* __restrict__ k_w, const uint16_t* __restrict__ cos_t,
    const uint16_t* __restrict__ sin_t, const int64_t* __restrict__ pos_p,
    uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache, uint16_t* __restrict__ out,
    int nh, int nkv, int max_len, float eps, float scale) {
  static_assert(HPW <= 16, "one MFMA column per query head");
  static_assert(NW >= 4 && NW <= 16, "waves");
  constexpr int kThreads = NW * 64;
  const int group = nh / nkv;           // query heads per kv head
  const int h0 = blockIdx.x * HPW;      // this workgroup's first query head
  const bool writer = h0 % group == 0;  // the group's first workgroup writes the cache
  __shared__ __align__(16) uint32_t qb[16][64 + 4];   // q as bf16 pairs; heads >= HPW are 0
  __shared__ __align__(16) uint32_t kv_new[2][64];
  __shared__ uint32_t heads[HPW + 2][64];  // raw q heads | k | v
  __shared__ uint32_t tabs[4][64];         // q_w, k_w, cos row, sin row
  __shared__ float ps[NW][HPW][kAttnChunk];
  __shared__ float cm[NW][HPW], cl[NW][HPW];
  __shared__ float wm[NW][HPW], wl[NW][HPW];
  __shared__ float wacc[NW][HPW][kHeadDim];
  const int kvh = h0 / group, wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int l16 = l & 15, kb = l >> 4;
  const int64_t pos = *pos_p;
  const bool pos_ok = pos >= 0 && pos < max_len;
  const int64_t last = pos < (int64_t)max_len ? pos : (int64_t)max_len - 1;

  // 0. loads
  for (int i = threadIdx.x; i < (HPW + 2) * 64; i += kThreads) {
    const int hi = i >> 6;
    const int head = hi < HPW ? h0 + hi : (hi == HPW ? nh + kvh : nh + nkv + kvh);
    heads[hi][i & 63] = reinterpret_cast<const uint32_t*>(qkv)[(size_t)head * 64 + (i & 63)];
  }
  for (int i = threadIdx.x + HPW * 64; i < 16 * 64; i += kThreads) qb[i >> 6][i & 63] = 0u;
  if (wave < 4) {
    const size_t trow = (size_t)(pos_ok ? pos : 0) * 64 + l;
    const uint32_t* src = wave == 0 ? reinterpret_cast<const uint32_t*>(q_w) + l
                        : wave == 1 ? reinterpret_cast<const uint32_t*>(k_w) + l
                        : wave == 2 ? reinterpret_cast<const uint32_t*>(cos_t) + trow
                                    : reinterpret_cast<const uint32_t*>(sin_t) + trow;
    tabs[wave][l] = *src;
  }
  int start = wave * kAttnChunk;
  uint4 ka[2][4];       // A operand: cache rows start + 16t + l16, dims 32 kb .. 32 kb + 31
  uint32_t vv[kAttnChunk];  // values: rows start + j, dims 2l, 2l + 1
  auto load_chunk = [&](int st) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int row = st + 16 * t + l16;
      if ((int64_t)row <= last) {
        const uint4* src = reinterpret_cast<const uint4*>(
            k_cache + ((size_t)kvh * max_len + row) * kHeadDim + 32 * kb);
#pragma unroll
        for (int j = 0; j < 4; ++j) ka[t][j] = src[j];
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) ka[t][j] = make_uint4(0, 0, 0, 0);
      }
    }
    const int np = (int)((last - st + 1) < kAttnChunk ? (last - st + 1) : kAttnChunk);
    const uint32_t* vcol =
        reinterpret_cast<const uint32_t*>(v_cache + ((size_t)kvh * max_len + st) * kHeadDim) + l;
#pragma unroll
    for (int j = 0; j < kAttnChunk; ++j) vv[j] = j < np ? vcol[(size_t)j * 64] : 0u;
  };
  if ((int64_t)start <= last) load_chunk(start);
  __syncthreads();

  // 1. RMSNorm + rotary of the q heads and the k head; v and k to the cache
  for (int hi = wave; hi < HPW + 2; hi += NW) {
    const uint32_t pair = heads[hi][l];
    if (hi == HPW + 1) {
      kv_new[1][l] = pair;
      if (pos_ok && writer)
        reinterpret_cast<uint32_t*>(v_cache)[((size_t)kvh * max_len + pos) * 64 + l] = pair;
      continue;
    }
    const uint32_t wp = tabs[hi < HPW ? 0 : 1][l];
    const float x0 = bf16_to_f32(pair & 0xFFFFu), x1 = bf16_to_f32(pair >> 16);
    const float ss = wave_sum(x0 * x0 + x1 * x1);
    const float r = rsqrtf(ss * (1.0f / (float)kHeadDim) + eps);
    const uint32_t y0 = f32_to_bf16(bf16_to_f32(wp & 0xFFFFu) * round_bf16(x0 * r));
    const uint32_t y1 = f32_to_bf16(bf16_to_f32(wp >> 16) * round_bf16(x1 * r));
    float r0 = bf16_to_f32(__shfl_xor(y0, 32, 64));
    float r1 = bf16_to_f32(__shfl_xor(y1, 32, 64));
    if (l < 32) {
      r0 = -r0;
      r1 = -r1;
    }
    const uint32_t cs = tabs[2][l], sn = tabs[3][l];
    const uint32_t o0 = f32_to_bf16(round_bf16(bf16_to_f32(y0) * bf16_to_f32(cs & 0xFFFFu)) +
                                    round_bf16(r0 * bf16_to_f32(sn & 0xFFFFu)));
    const uint32_t o1 = f32_to_bf16(round_bf16(bf16_to_f32(y1) * bf16_to_f32(cs >> 16)) +
                                    round_bf16(r1 * bf16_to_f32(sn >> 16)));
    if (hi < HPW) {
      qb[hi][l] = o0 | (o1 << 16);
    } else {
      kv_new[0][l] = o0 | (o1 << 16);
      if (pos_ok && writer)
        reinterpret_cast<uint32_t*>(k_cache)[((size_t)kvh * max_len + pos) * 64 + l] =
            o0 | (o1 << 16);
    }
  }
  __syncthreads();

  // 2. B operand (q head l16, dims 32 kb .. 32 kb + 31) once; then the chunks
  uint4 bq[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) bq[j] = *reinterpret_cast<const uint4*>(&qb[l16][16 * kb + 4 * j]);
  float m[HPW], lsum[HPW], a0[HPW], a1[HPW];
#pragma unroll
  for (int g = 0; g < HPW; ++g) {
    m[g] = -INFINITY;
    lsum[g] = a0[g] = a1[g] = 0.f;
  }
  for (; (int64_t)start <= last; start += NW * kAttnChunk) {
    const int npos = (int)((last - start + 1) < kAttnChunk ? (last - start + 1) : kAttnChunk);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      if ((int64_t)(start + 16 * t + l16) == pos) {  // this token's row from LDS
#pragma unroll
        for (int j = 0; j < 4; ++j)
          ka[t][j] = *reinterpret_cast<const uint4*>(&kv_new[0][16 * kb + 4 * j]);
      }
    }
    if ((int64_t)start <= pos && pos < (int64_t)start + npos) vv[pos - start] = kv_new[1][l];

    // scores: lane (head l16, rows 4 kb + r of tile t)
    float sc[2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      floatx4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j)
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(ka[t][j]), as_bf16x8(bq[j]), d, 0,
                                                    0, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool ok = 16 * t + 4 * kb + r < npos;
        sc[t][r] = ok ? d[r] * scale : -INFINITY;
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) mx = fmaxf(mx, sc[t][r]);
    mx = row_pair_max32(row_pair_max16(mx));  // over the lanes of head l16
    float sum = 0.f;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float e = sc[t][r] == -INFINITY ? 0.f : expf(sc[t][r] - mx);
        sum += e;
        if (l16 < HPW) ps[wave][l16][16 * t + 4 * kb + r] = e;
      }
    sum = row_pair_sum32(row_pair_sum16(sum));
    if (kb == 0 && l16 < HPW) {
      cm[wave][l16] = mx;
      cl[wave][l16] = sum;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");

    // values: lane l takes dimensions 2l, 2l + 1
    float c0[HPW], c1[HPW];
#pragma unroll
    for (int g = 0; g < HPW; ++g) c0[g] = c1[g] = 0.f;
#pragma unroll
    for (int j = 0; j < kAttnChunk; ++j) {
      if (j < npos) {
        const float v0 = bf16_to_f32(vv[j] & 0xFFFFu), v1 = bf16_to_f32(vv[j] >> 16);
#pragma unroll
        for (int g = 0; g < HPW; ++g) {
          c0[g] = fmaf(ps[wave][g][j], v0, c0[g]);
          c1[g] = fmaf(ps[wave][g][j], v1, c1[g]);
        }
      }
    }
#pragma unroll
    for (int g = 0; g < HPW; ++g) {
      const float mc = cm[wave][g], lc = cl[wave][g];
      const float mn = fmaxf(m[g], mc);
      const float fo = expf(m[g] - mn), fn = expf(mc - mn);
      lsum[g] = lsum[g] * fo + lc * fn;
      a0[g] = a0[g] * fo + c0[g] * fn;
      a1[g] = a1[g] * fo + c1[g] * fn;
      m[g] = mn;
    }
    __builtin_amdgcn_wave_barrier();
    if ((int64_t)(start + NW * kAttnChunk) <= last) load_chunk(start + NW * kAttnChunk);
  }

  // 3. merge the waves in a fixed order
#pragma unroll
  for (int g = 0; g < HPW; ++g) {
    if (l == 0) {
      wm[wave][g] = m[g];
      wl[wave][g] = lsum[g];
    }
    wacc[wave][g][2 * l] = a0[g];
    wacc[wave][g][2 * l + 1] = a1[g];
  }
  __syncthreads();
  for (int g = wave; g < HPW; g += NW) {
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) mx = fmaxf(mx, wm[w][g]);
    float den = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float f = wl[w][g] > 0.f ? expf(wm[w][g] - mx) : 0.f;
      den = fmaf(f, wl[w][g], den);
      o0 = fmaf(f, wacc[w][g][2 * l], o0);
      o1 = fmaf(f, wacc[w][g][2 * l + 1], o1);
    }
    reinterpret_cast<uint32_t*>(out)[((size_t)h0 + g) * 64 + l] =
        f32_to_bf16(o0 / den) | (f32_to_bf16(o1 / den) << 16);
  }
}

template <int G>
void launch_attention(const uint16_t* q, const uint16_t* kc, const uint16_t* vc, const int64_t* pos,
                      uint16_t* out, int nkv, int max_len, int nchunks, float scale, float* part,
                      hipStream_t stream) {
  hipLaunchKernelGGL((attn_partial_kernel<G>), dim3(nchunks, nkv), dim3(64), 0, stream, q, kc, vc,
                     pos, part, max_len, nchunks, scale);
  hipLaunchKernelGGL(attn_combine_kernel, dim3(nkv * G), dim3(256), 0, stream, part, pos, out, G,
                     max_len, nchunks);
}

}  // namespace
}  // namespace dip

using namespace dip;

extern "C" int dip_add_rmsnorm(uint16_t* h, const uint16_t* add, const uint16_t* weight,
                               uint16_t* out, int64_t n, float eps, void* stream) {
  if (!h || !weight || !out) return DIP_ERR_NULL;
  if (n <= 0 || n % 8 != 0 || n > (int64_t)kNormThreads * kNormVecs * 8) return DIP_ERR_SHAPE;
  if (!(eps >= 0.f)) return DIP_ERR_ARG;
  if (!aligned16(h) || !aligned16(weight) || !aligned16(out) || (add && !aligned16(add)))
    return DIP_ERR_ALIGN;
  hipLaunchKernelGGL(add_rmsnorm_kernel, dim3(1), dim3(kNormThreads), 0, (hipStream_t)stream, h,
                     add, weight, out, (int)n, eps);
  return hip_status(hipGetLastError());
}

extern "C" int dip_qk_norm_rope_cache(const uint16_t* qkv, const uint16_t* q_norm_w,
                                      const uint16_t* k_norm_w, const uint16_t* cos_table,
                                      const uint16_t* sin_table, const int64_t* pos,
                                      uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache,
                                      int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                                      int64_t max_len, float eps, void* stream) {
  if (!qkv || !q_norm_w || !k_norm_w || !cos_table || !sin_table || !pos || !q_out || !k_cache ||
      !v_cache)
    return DIP_ERR_NULL;
  if (head_dim != kHeadDim) return DIP_ERR_UNSUPPORTED;
  if (n_heads <= 0 || n_kv_heads <= 0 || n_heads > 4096 || n_kv_heads > 4096 || max_len <= 0 ||
      max_len > INT32_MAX / kHeadDim)
    return DIP_ERR_SHAPE;
  if (!(eps >= 0.f)) return DIP_ERR_ARG;
  if (!aligned16(qkv) || !aligned16(q_out) || !aligned16(k_cache) || !aligned16(v_cache) ||
      !aligned16(cos_table) || !aligned16(sin_table) || !aligned16(q_norm_w) ||
      !aligned16(k_norm_w))
    return DIP_ERR_ALIGN;
  hipLaunchKernelGGL(qk_rope_cache_kernel, dim3((unsigned)(n_heads + 2 * n_kv_heads)), dim3(64), 0,
                     (hipStream_t)stream, qkv, q_norm_w, k_norm_w, cos_table, sin_table, pos,
                     q_out, k_cache, v_cache, (int)n_heads, (int)n_kv_heads, (int)max_len, eps);
  return hip_status(hipGetLastError());
}

extern "C" int64_t dip_decode_attention_fused_max_len(void) { return kFusedMaxLen; }

extern "C" int dip_decode_attention_fused(const uint16_t* qkv, const uint16_t* q_norm_w,
                                          const uint16_t* k_norm_w, const uint16_t* cos_table,
                                          const uint16_t* sin_table, const int64_t* pos,
                                          uint16_t* k_cache, uint16_t* v_cache, uint16_t* out,
                                          int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                                          int64_t max_len, float eps, float scale, void* stream) {
  if (!qkv || !q_norm_w || !k_norm_w || !cos_table || !sin_table || !pos || !k_cache ||
      !v_cache || !out)
    return DIP_ERR_NULL;
  if (head_dim != kHeadDim) return DIP_ERR_UNSUPPORTED;
  if (n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads != 0 || n_heads > 4096 ||
      max_len <= 0 || max_len > kFusedMaxLen)
    return DIP_ERR_SHAPE;
  if (!(eps >= 0.f)) return DIP_ERR_ARG;
  if (!aligned16(qkv) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(out) ||
      !aligned16(cos_table) || !aligned16(sin_table) || !aligned16(q_norm_w) ||
      !aligned16(k_norm_w))
    return DIP_ERR_ALIGN;
  const int nh = (int)n_heads, nkv = (int)n_kv_heads, ml = (int)max_len;
  hipStream_t s = (hipStream_t)stream;
  // one query head per workgroup; 16 waves (chunks 16 at a time) for caches
  // of more than 128 rows
  if (ml <= 128)
    hipLaunchKernelGGL((attn_fused_kernel<1, 4>), dim3(nh), dim3(256), 0, s, qkv, q_norm_w,
                       k_norm_w, cos_table, sin_table, pos, k_cache, v_cache, out, nh, nkv, ml,
                       eps, scale);
  else
    hipLaunchKernelGGL((attn_fused_kernel<1, 16>), dim3(nh), dim3(1024), 0, s, qkv, q_norm_w,
                       k_norm_w, cos_table, sin_table, pos, k_cache, v_cache, out, nh, nkv, ml,
                       eps, scale);
  return hip_status(hipGetLastError());
}

extern "C" size_t dip_decode_attention_workspace_size(int64_t n_heads, int64_t head_dim,
                                                      int64_t max_len) {
  if (n_heads <= 0 || head_dim != kHeadDim || max_len <= 0) return 0;
  const size_t nchunks = (size_t)((max_len + kAttnChunk - 1) / kAttnChunk);
  return nchunks * (size_t)n_heads * kPartFloats * sizeof(float);
}

extern "C" int dip_decode_attention(const uint16_t* q, const uint16_t* k_cache,
                                    const uint16_t* v_cache, const int64_t* pos, uint16_t* out,
                                    int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                                    int64_t max_len, float scale, void* workspace,
                                    size_t ws_bytes, void* stream) {
  if (!q || !k_cache || !v_cache || !pos || !out) return DIP_ERR_NULL;
  if (head_dim != kHeadDim) return DIP_ERR_UNSUPPORTED;
  if (n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads != 0 || n_heads > 4096 ||
      max_len <= 0 || max_len > INT32_MAX / kHeadDim)
    return DIP_ERR_SHAPE;
  if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(out))
    return DIP_ERR_ALIGN;
  if (!workspace || ws_bytes < dip_decode_attention_workspace_size(n_heads, head_dim, max_len))
    return DIP_ERR_WORKSPACE;
  if (!aligned16(workspace)) return DIP_ERR_ALIGN;
  const int nkv = (int)n_kv_heads;
  const int G = (int)(n_heads / n_kv_heads);
  const int nchunks = (int)((max_len + kAttnChunk - 1) / kAttnChunk);
  float* part = static_cast<float*>(workspace);
  hipStream_t s = (hipStream_t)stream;
  const int ml = (int)max_len;
  switch (G) {
    case 1: launch_attention<1>(q, k_cache, v_cache, pos, out, nkv, ml, nchunks, scale, part, s); break;
    case 2: launch_attention<2>(q, k_cache, v_cache, pos, out, nkv, ml, nchunks, scale, part, s); break;
    case 4: launch_attention<4>(q, k_cache, v_cache, pos, out, nkv, ml, nchunks, scale, part, s); break;
    case 5: launch_attention<5>(q, k_cache, v_cache, pos, out, nkv, ml, nchunks, scale, part, s); break;
    case 8: launch_attention<8>(q, k_cache, v_cache, pos, out, nkv, ml, nchunks, scale, part, s); break;
    case 16: launch_attention<16>(q, k_cache, v_cache, pos, out, nkv, ml, nchunks, scale, part, s); break;
    default: return DIP_ERR_UNSUPPORTED;
  }
  return hip_status(hipGetLastError());
}
