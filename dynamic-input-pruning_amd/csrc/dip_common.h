// dip_common.h — device helpers shared by the DIP decode kernels (gfx950).
//
// Format (reference qlinear.py:25-64, scripts/quantize.py:32-64):
//   qweight int8 [R, C/2]: byte b of a row holds column 2b in its low nibble
//   and column 2b+1 in its high nibble, two's-complement int4 in [-8, 7];
//   scales bf16 [R, C/128]: one scale per group of 128 columns.
//
// A "chunk" below is 16 bytes of one packed row = 32 columns, always inside a
// single 128-column group (a group is 64 bytes = 4 chunks).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/dip_hip.h"

#define DIP_DEV __device__ __forceinline__

namespace dip {

constexpr int kGroupSize = 128;       // columns per scale
constexpr int kChunkBytes = 16;       // one 128-bit load
constexpr int kChunkCols = 32;        // columns per chunk
constexpr int kChunksPerGroup = 4;    // 128 / 32

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

DIP_DEV float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// Round-to-nearest-even fp32 -> bf16 with NaN -> 0x7FC0; the exact rule of
// c10::BFloat16 / __float2bfloat16_rn, so outputs can be compared bit for bit.
DIP_DEV uint32_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7FC0u;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// Two fp32 values to a packed bf16 pair (lo in bits 0-15) by the rule of
// f32_to_bf16, in one v_cvt_pk_bf16_f32 (round to nearest even) after NaN
// inputs are made the canonical quiet NaN (so they become 0x7FC0).  Checked
// against f32_to_bf16 on all 2^32 fp32 patterns in both halves on gfx950
// (this library keeps fp32 denormals).
DIP_DEV uint32_t f32x2_to_bf16x2(float lo, float hi) {
  lo = lo != lo ? __uint_as_float(0x7FC00000u) : lo;
  hi = hi != hi ? __uint_as_float(0x7FC00000u) : hi;
  uint32_t r;
  asm("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(r) : "v"(lo), "v"(hi));
  return r;
}

// |v| as the bf16 key the top-k orders by: sign dropped, subnormal
// magnitudes flushed to 0 (the reference's top-k kernels are built with
// --use_fast_math, so fabsf flushes them).  NaN keys (> 0x7F80) are kept
// as-is; callers skip them because every comparison with NaN is false.
DIP_DEV uint32_t topk_key(uint32_t bits16) {
  uint32_t a = bits16 & 0x7FFFu;
  return a < 0x0080u ? 0u : a;
}
constexpr uint32_t kKeyInf = 0x7F80u;

// ---------------------------------------------------------------------------
// Nibble expansion for v_dot2_f32_bf16.
//
// For a dword w of 8 nibbles n0..n7 (column c+p for nibble p), flipping bit 3
// of a nibble turns the two's-complement value q into u = q + 8 in [0, 15].
// Placing u in mantissa bits 3..6 of bf16 1.0 (0x3F80 | u << 3) encodes
// 1 + u/16 = 1.5 + q/16 exactly.  For j = 0..3, shifting w so nibble j lands
// on bits 3..6 (and nibble j+4 on bits 19..22), masking with 0x00780078 and
// XOR-ing 0x3FC03FC0 (1.0 in both halves plus the bit-3 flip of u) gives
//     pair_j(w) = bf16x2(1.5 + q_j/16, 1.5 + q_{j+4}/16)
// in one v_bitop3_b32 after the shift.  Then
//     sum_p (1.5 + q_p/16) x_p = 1.5 sum_p x_p + (1/16) sum_p q_p x_p,
// so each chunk's dot2 chain starts at -1.5 * sum(x over the chunk) and the
// result, times 16 * scale, is the chunk's contribution.  Every product is
// exact in fp32, and the running sums stay within a few times the size of
// the signal, which keeps fp32 accumulation error small.
// ---------------------------------------------------------------------------
constexpr uint32_t kPairMask = 0x00780078u;
constexpr uint32_t kPairMagicFlip = 0x3FC03FC0u;
constexpr float kPairBias = 1.5f;
constexpr float kPairScale = 16.0f;

DIP_DEV float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                          __builtin_bit_cast(bf16x2_t, b), c, false);
}

// x pairs for one dword of weights: xp[j] = (x[c+j], x[c+j+4]) as bf16x2,
// from X0 = (x[c], x[c+1]), X1 = (x[c+2], x[c+3]), X2 = (x[c+4], x[c+5]),
// X3 = (x[c+6], x[c+7]).
DIP_DEV void make_xpairs(uint32_t X0, uint32_t X1, uint32_t X2, uint32_t X3, uint32_t xp[4]) {
  xp[0] = (X0 & 0xFFFFu) | (X2 << 16);
  xp[1] = (X0 >> 16) | (X2 & 0xFFFF0000u);
  xp[2] = (X1 & 0xFFFFu) | (X3 << 16);
  xp[3] = (X1 >> 16) | (X3 & 0xFFFF0000u);
}

// acc + sum over the 8 nibbles of w of (1.5 + q_p/16) * x_p.
DIP_DEV float dot8_nibbles(uint32_t w, const uint32_t xp[4], float acc) {
  acc = dot2_bf16(((w << 3) & kPairMask) ^ kPairMagicFlip, xp[0], acc);
  acc = dot2_bf16(((w >> 1) & kPairMask) ^ kPairMagicFlip, xp[1], acc);
  acc = dot2_bf16(((w >> 5) & kPairMask) ^ kPairMagicFlip, xp[2], acc);
  acc = dot2_bf16(((w >> 9) & kPairMask) ^ kPairMagicFlip, xp[3], acc);
  return acc;
}

// ---------------------------------------------------------------------------
// Per-nibble conversions for the down kernel (one output column per nibble).
// ---------------------------------------------------------------------------
// float(byte n of v), n = 0..3 (v_cvt_f32_ubyteN).
template <int N>
DIP_DEV float cvt_ubyte(uint32_t v) {
  float r;
  if (N == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(v));
  if (N == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(v));
  if (N == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(v));
  if (N == 3) asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(v));
  return r;
}

// sext(low nibble of byte n of v) / 16 as fp32, exactly (v_cvt_off_f32_i4
// reading byte n through SDWA).
template <int N>
DIP_DEV float cvt_nibble_div16(uint32_t v) {
  float r;
  if (N == 0)
    asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0"
        : "=v"(r) : "v"(v));
  if (N == 1)
    asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1"
        : "=v"(r) : "v"(v));
  if (N == 2)
    asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2"
        : "=v"(r) : "v"(v));
  if (N == 3)
    asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3"
        : "=v"(r) : "v"(v));
  return r;
}

// Sum over aligned groups of W lanes (W a power of two <= 64), every lane of
// the group receiving the total: DPP within rows of 16 lanes (xor 1, xor 2,
// half-row mirror, row mirror), then v_permlane16_swap / v_permlane32_swap to
// combine rows.  All VALU, no LDS round trips.
template <int CTRL>
DIP_DEV float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL,
                                                            0xF, 0xF, true));
}

// v_permlane{16,32}_swap_b32 a, b swaps the odd rows (of 16 / 32 lanes) of a
// with the even rows of b.  With a = b = v every lane then holds its own row
// in one register and the partner row in the other, so a + b is the sum of
// the row pair in every lane.  Written as inline asm with two distinct
// read-write registers: this toolchain's optimiser folds the second result
// of __builtin_amdgcn_permlane16_swap into the first (both read element 0).
// The s_nop covers the VALU-write -> permlane read hazard.
DIP_DEV float row_pair_sum16(float v) {
  uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}
DIP_DEV float row_pair_sum32(float v) {
  uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}

template <int W>
DIP_DEV float group_sum(float v) {
  static_assert(W == 1 || W == 2 || W == 4 || W == 8 || W == 16 || W == 32 || W == 64, "W");
  if (W >= 2) v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]: lane ^ 1
  if (W >= 4) v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]: lane ^ 2
  if (W >= 8) v += dpp_mov<0x141>(v);  // row_half_mirror: the other quad of 8
  if (W >= 16) v += dpp_mov<0x140>(v); // row_mirror: the other half of 16
  if (W >= 32) v = row_pair_sum16(v);  // rows (0,1) and (2,3)
  if (W >= 64) v = row_pair_sum32(v);  // lanes 0-31 and 32-63
  return v;
}

// Max over aligned groups of W lanes, every lane receiving it: group_sum's
// exchange pattern with fmaxf.
DIP_DEV float row_pair_max16(float v) {
  uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}
DIP_DEV float row_pair_max32(float v) {
  uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}

template <int W>
DIP_DEV float group_max(float v) {
  static_assert(W == 1 || W == 2 || W == 4 || W == 8 || W == 16 || W == 32 || W == 64, "W");
  if (W >= 2) v = fmaxf(v, dpp_mov<0xB1>(v));
  if (W >= 4) v = fmaxf(v, dpp_mov<0x4E>(v));
  if (W >= 8) v = fmaxf(v, dpp_mov<0x141>(v));
  if (W >= 16) v = fmaxf(v, dpp_mov<0x140>(v));
  if (W >= 32) v = row_pair_max16(v);
  if (W >= 64) v = row_pair_max32(v);
  return v;
}

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

// Layer timeline stamps (the timeline build only, DIP_WG_STAMPS; the record
// layout is dip_wg_stamps of dip_hip.h): the first thread of a workgroup
// stamps its start and XCD, lane 0 of every wave its end.
#ifdef DIP_WG_STAMPS
DIP_DEV void stamp_start(dip_wg_stamps* s) {
  if (blockIdx.x < DIP_STAMP_BLOCKS && threadIdx.x == 0) {
    uint32_t xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    s->start[blockIdx.x] = wall_clock64();
    s->xcc[blockIdx.x] = xcc;
    if (blockIdx.x == 0) s->blocks = gridDim.x;
  }
}
DIP_DEV void stamp_end(dip_wg_stamps* s) {
  if (blockIdx.x < DIP_STAMP_BLOCKS && (threadIdx.x & 63) == 0 &&
      (threadIdx.x >> 6) < DIP_STAMP_WAVES)
    s->end[blockIdx.x][threadIdx.x >> 6] = wall_clock64();
}
#define DIP_STAMP_START(sym) ::dip::stamp_start(&(sym))
#define DIP_STAMP_END(sym) ::dip::stamp_end(&(sym))
#else
#define DIP_STAMP_START(sym) ((void)0)
#define DIP_STAMP_END(sym) ((void)0)
#endif

// 128-bit streaming load (weights are read once per call: non-temporal).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
DIP_DEV uint4 ldg_nt(const uint4* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

}  // namespace dip
