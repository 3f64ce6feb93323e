// dip_quantize.hip — the int4 g128 format conversions on the GPU, bit-exact
// with the reference's CPU torch code:
//   * quantize (scripts/quantize.py:32-64): per group of 128 columns,
//     s = max(max|w| / 7, 1e-8) in fp32, q = clamp(rint(w / s), -8, 7) with
//     the fp32 s, stored scale = bf16(s);
//   * down transpose (dip_stream_predispatch.py:100-120): down [out, inter]
//     int4 -> bf16(q*s) -> transpose -> fp32 -> quantize along `out`.
// Divisions are IEEE correctly rounded (hipcc's default for fp32 '/'), and
// rintf rounds half to even, matching torch.round.
#include <algorithm>

#include "dip_common.h"
#include "dip_internal.h"

namespace dip {

namespace {

DIP_DEV float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

// Quantize the 128 values of one group held as 2 per lane (columns 2l, 2l+1)
// and store one packed byte per lane plus the group's scale from lane 0.
DIP_DEV void quantize_group(float v0, float v1, int8_t* qdst, uint16_t* sdst, int lane) {
  const float m = wave_max(fmaxf(fabsf(v0), fabsf(v1)));
  float s = m / 7.0f;
  s = s < 1e-8f ? 1e-8f : s;
  const float q0 = fminf(fmaxf(rintf(v0 / s), -8.0f), 7.0f);
  const float q1 = fminf(fmaxf(rintf(v1 / s), -8.0f), 7.0f);
  const uint32_t b = ((uint32_t)(int)q0 & 0xFu) | (((uint32_t)(int)q1 & 0xFu) << 4);
  qdst[lane] = (int8_t)b;
  if (lane == 0) *sdst = (uint16_t)f32_to_bf16(s);
}

}  // namespace

// One wave per (row, group).
__global__ __launch_bounds__(256) void quantize_kernel(const void* __restrict__ w, int in_bf16,
                                                       int8_t* __restrict__ qw,
                                                       uint16_t* __restrict__ sc, int rows,
                                                       int cols) {
  const int lane = threadIdx.x & 63;
  const int ngroups = cols / kGroupSize;
  const long long total = (long long)rows * ngroups;
  for (long long gidx = ((long long)blockIdx.x * 256 + threadIdx.x) / 64; gidx < total;
       gidx += (long long)gridDim.x * 4) {
    const int r = (int)(gidx / ngroups);
    const int g = (int)(gidx % ngroups);
    const size_t e = (size_t)r * cols + (size_t)g * kGroupSize + 2 * lane;
    float v0, v1;
    if (in_bf16) {
      const uint32_t pair = *reinterpret_cast<const uint32_t*>(
          reinterpret_cast<const uint16_t*>(w) + e);
      v0 = bf16_to_f32(pair & 0xFFFFu);
      v1 = bf16_to_f32(pair >> 16);
    } else {
      const float2 f = *reinterpret_cast<const float2*>(reinterpret_cast<const float*>(w) + e);
      v0 = f.x;
      v1 = f.y;
    }
    quantize_group(v0, v1, qw + (size_t)r * (cols / 2) + (size_t)g * 64,
                   sc + (size_t)r * ngroups + g, lane);
  }
}

// Tile: 128 `out` rows x 64 `inter` columns of down, staged in LDS.  Wave w
// then requantizes inter columns c0 + w, c0 + w + 4, ... each over its 128
// dequantized values (one output group of down_t).
__global__ __launch_bounds__(256) void transpose_down_kernel(
    const int8_t* __restrict__ dqw, const uint16_t* __restrict__ dsc, int8_t* __restrict__ tqw,
    uint16_t* __restrict__ tsc, int out_f, int inter) {
  __shared__ uint8_t tile[128][33];     // 32 packed bytes (64 columns) per out row, padded
  __shared__ uint16_t tscale[128];      // scale of (out row, column group of c0)
  const int n_ctiles = inter / 64;
  const int g = blockIdx.x / n_ctiles;  // output group (128 out rows)
  const int c0 = (blockIdx.x % n_ctiles) * 64;
  const int tid = threadIdx.x;
  const int in_half = inter / 2;
  const int in_groups = inter / kGroupSize;
  for (int e = tid; e < 128 * 32; e += 256) {
    const int o = e / 32, b = e % 32;
    tile[o][b] = (uint8_t)dqw[(size_t)(g * 128 + o) * in_half + c0 / 2 + b];
  }
  if (tid < 128) tscale[tid] = dsc[(size_t)(g * 128 + tid) * in_groups + c0 / kGroupSize];
  __syncthreads();
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int out_groups = out_f / kGroupSize;
  for (int cc = wave; cc < 64; cc += 4) {
    const int c = c0 + cc;
    float v[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int o = 2 * lane + h;
      const uint32_t byte = tile[o][cc / 2];
      const uint32_t nib = (cc & 1) ? (byte >> 4) : (byte & 0xFu);
      const int q = (int)nib - (int)((nib & 8u) << 1);
      // qlinear.dequantize rounds q*s to bf16 before the transpose
      v[h] = bf16_to_f32(f32_to_bf16((float)q * bf16_to_f32(tscale[o])));
    }
    quantize_group(v[0], v[1], tqw + (size_t)c * (out_f / 2) + (size_t)g * 64,
                   tsc + (size_t)c * out_groups + g, lane);
  }
}

// sc_gm[g][r] = sc[r][g]: 64 x 64 tiles through LDS, both sides coalesced.
__global__ __launch_bounds__(256) void scales_group_major_kernel(
    const uint16_t* __restrict__ sc, uint16_t* __restrict__ gm, int rows, int groups) {
  __shared__ uint16_t tile[64][65];
  const int r0 = blockIdx.x * 64, g0 = blockIdx.y * 64;
  for (int e = threadIdx.x; e < 64 * 64; e += 256) {
    const int r = e / 64, g = e % 64;
    if (r0 + r < rows && g0 + g < groups) tile[r][g] = sc[(size_t)(r0 + r) * groups + g0 + g];
  }
  __syncthreads();
  for (int e = threadIdx.x; e < 64 * 64; e += 256) {
    const int g = e / 64, r = e % 64;
    if (r0 + r < rows && g0 + g < groups) gm[(size_t)(g0 + g) * rows + r0 + r] = tile[r][g];
  }
}

}  // namespace dip

using namespace dip;

extern "C" int dip_scales_group_major(const uint16_t* scales, uint16_t* scales_gm, int64_t rows,
                                      int64_t groups, void* stream) {
  if (!scales || !scales_gm) return DIP_ERR_NULL;
  if (rows < 0 || groups <= 0 || rows > INT32_MAX || groups > 65536 ||
      (rows + 63) / 64 > INT32_MAX)
    return DIP_ERR_SHAPE;
  if (rows == 0) return DIP_OK;
  const dim3 grid((unsigned)((rows + 63) / 64), (unsigned)((groups + 63) / 64));
  hipLaunchKernelGGL(scales_group_major_kernel, grid, dim3(256), 0, (hipStream_t)stream, scales,
                     scales_gm, (int)rows, (int)groups);
  return hip_status(hipGetLastError());
}

extern "C" int dip_quantize_int4(const void* w, int w_is_bf16, int8_t* qweight, uint16_t* scales,
                                 int64_t rows, int64_t cols, void* stream) {
  if (!w || !qweight || !scales) return DIP_ERR_NULL;
  if (rows < 0 || cols <= 0 || cols % kGroupSize != 0 || rows > INT32_MAX || cols > (1 << 24))
    return DIP_ERR_SHAPE;
  if ((reinterpret_cast<uintptr_t>(w) & 7u) != 0) return DIP_ERR_ALIGN;
  if (rows == 0) return DIP_OK;
  const long long groups = rows * (cols / kGroupSize);
  const unsigned blocks = (unsigned)std::min<long long>((groups + 3) / 4, 65536);
  hipLaunchKernelGGL(quantize_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, w,
                     w_is_bf16 ? 1 : 0, qweight, scales, (int)rows, (int)cols);
  return hip_status(hipGetLastError());
}

extern "C" int dip_transpose_down_int4(const int8_t* down_qw, const uint16_t* down_sc,
                                       int8_t* down_t_qw, uint16_t* down_t_sc,
                                       int64_t out_features, int64_t inter, void* stream) {
  if (!down_qw || !down_sc || !down_t_qw || !down_t_sc) return DIP_ERR_NULL;
  if (out_features <= 0 || inter <= 0 || out_features % kGroupSize || inter % kGroupSize ||
      out_features > INT32_MAX || inter > INT32_MAX)
    return DIP_ERR_SHAPE;
  const long long blocks = (out_features / kGroupSize) * (inter / 64);
  if (blocks > INT32_MAX) return DIP_ERR_SHAPE;
  hipLaunchKernelGGL(transpose_down_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     (hipStream_t)stream, down_qw, down_sc, down_t_qw, down_t_sc,
                     (int)out_features, (int)inter);
  return hip_status(hipGetLastError());
}
