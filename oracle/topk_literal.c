/*
 * topk_literal.c — TEST INFRASTRUCTURE: a sequential C restatement of the
 * reference's threshold top-k, used only by tests to pin the numpy oracle
 * (oracle/dip_oracle.py: topk_select) from a second, independent
 * implementation.  Never linked into the product.
 *
 * Follows kernels/topk_select/topk_select.cu:
 *   max_abs_kernel (:30-44)      -> max over fabsf, fmaxf from 0 (NaN ignored)
 *   host bisection (:141-158)    -> 25 fp32 steps of count_gt_kernel (:46-57)
 *   parallel_compact_kernel (:64-132) -> tier A then tier B, ascending index
 * The reference is built with --use_fast_math (setup_topk.py), so fabsf of a
 * bf16 subnormal flushes to zero; flushed_abs() reproduces that.
 * Host arithmetic is plain IEEE fp32 (build without -ffast-math).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float bf16_bits_to_float(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, sizeof f);
  return f;
}

static float flushed_abs(uint16_t b) {
  uint16_t a = (uint16_t)(b & 0x7FFFu);
  if (a < 0x0080u) a = 0;
  return bf16_bits_to_float(a);
}

/* Writes idx[0..k) exactly as topk_ops::topk_select; returns the number of
 * entries the compaction emitted (<= k); *t_lo / *t_strict receive the
 * final bisection bounds. */
int oracle_topk_literal(const uint16_t* s, int n, int k, int32_t* idx, float* t_lo,
                        float* t_strict) {
  float m = 0.0f;
  for (int i = 0; i < n; ++i) m = fmaxf(m, flushed_abs(s[i]));
  float hi = m, lo = 0.0f;
  float thresh = 0.5f * (lo + hi);
  for (int step = 0; step < 25; ++step) {
    int cnt = 0;
    for (int i = 0; i < n; ++i)
      if (flushed_abs(s[i]) > thresh) ++cnt;
    if (cnt > k)
      lo = thresh;
    else
      hi = thresh;
    thresh = 0.5f * (lo + hi);
  }
  for (int j = 0; j < k; ++j) idx[j] = 0;
  int running = 0;
  for (int i = 0; i < n; ++i) {
    if (flushed_abs(s[i]) > hi) {
      if (running < k) idx[running] = i;
      ++running;
    }
  }
  for (int i = 0; i < n && running < k; ++i) {
    const float v = flushed_abs(s[i]);
    if (v > lo && v <= hi) idx[running++] = i;
  }
  if (t_lo) *t_lo = lo;
  if (t_strict) *t_strict = hi;
  return running < k ? running : k;
}
