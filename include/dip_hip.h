/*
 * dip_hip.h — C ABI of libdip_hip.so, the MI355X (gfx950) decode path of
 * Dynamic Input Pruning (DIP) for an int4 g128 SwiGLU MLP.
 *
 * Conventions for every entry point:
 *   - All tensor arguments are DEVICE pointers to contiguous, caller-owned
 *     memory; weight/activation pointers must be 16-byte aligned.
 *   - bf16 values travel as uint16_t bit patterns; packed int4 weights as
 *     int8_t [rows, cols/2] (low nibble = even column, high nibble = odd
 *     column, two's complement), scales as bf16 [rows, cols/128].
 *   - `stream` is a hipStream_t (NULL = legacy default stream).  Calls only
 *     enqueue work: none synchronises the host and none allocates memory.
 *   - Return value: DIP_OK (0), a negative DIP_ERR_* code for an argument
 *     rejected before any launch, or a positive hipError_t from the launch.
 *   - Workspaces are caller-owned device buffers of the size the matching
 *     *_workspace_size() reports.  They must be zero-filled once before their
 *     first use; every call returns the parts that must start at zero
 *     (arrival counters) to zero before it ends, so no clearing is needed
 *     between calls (and none is recorded into a captured graph).  Calls
 *     that share a workspace must be ordered on one stream.
 *
 * Reference interfaces each entry point replaces are cited as
 * <file>:<line> of rohitpotluri/dynamic-input-pruning.
 */
#ifndef DIP_HIP_H_
#define DIP_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  DIP_OK = 0,
  DIP_ERR_NULL = -1,        /* a required pointer is NULL */
  DIP_ERR_SHAPE = -2,       /* a size is negative / inconsistent / too large */
  DIP_ERR_ALIGN = -3,       /* a pointer is not 16-byte aligned */
  DIP_ERR_UNSUPPORTED = -4, /* the shape has no kernel instantiation */
  DIP_ERR_WORKSPACE = -5,   /* workspace missing or smaller than required */
  DIP_ERR_ARG = -6,         /* any other invalid argument */
  DIP_ERR_SCRATCH = -7      /* the shape needs more than the no-alloc scratch holds */
};

enum { DIP_ACT_NONE = 0, DIP_ACT_SILU = 1 };

/* Human-readable text for a status returned by this library. */
const char* dip_status_string(int status);

/*
 * Library version as an integer (major * 10000 + minor * 100 + patch).  The
 * minor number changes whenever an entry point's argument list changes, so
 * a binding written against this header checks dip_version() == DIP_VERSION
 * before its first call.  0.3.4: dip_int4_gather_down_by_channel takes
 * indices == NULL (every row in order; it was an error).  0.3.3 adds the
 * DIP_TUNE_ROW_TIERS knob (no argument list changes).  0.3.2: the down and decode workspaces grow by
 * 8 KB of arrival counters (the sizes functions report it).  0.3.1 adds
 * dip_timeline_read.  0.3.0: the
 * measurement probes and the DIP_TUNE_STEP knob are gone; 0.2.0 added
 * down_t_sc_gm to the decode and gather-down entry points and g_len to
 * dip_ca_fused_gemv.
 */
#define DIP_VERSION 304
int dip_version(void);

/* Highest row count the top-k supports (its keys are staged in LDS). */
int64_t dip_topk_max_n(void);

/*
 * out[r] = bf16( sum_c (q*s)[r,c] * x[c] ), or with act = DIP_ACT_SILU
 * out[r] = bf16( silu( float( bf16(dot) ) ) ).
 * Replaces int4_ops::int4_gemv (kernels/int4_gemv/int4_gemv.cu:89-115,
 * gate_kernel.py:29-33); DIP_ACT_SILU also fuses the separate F.silu of
 * dip_stream_predispatch.py:182.
 */
int dip_int4_gemv(const int8_t* qweight, const uint16_t* scales, const uint16_t* x,
                  uint16_t* out, int64_t out_features, int64_t in_features, int act,
                  void* stream);

/*
 * idx[0:k] int32 = the reference's threshold top-k of |s| (bisection of 25
 * fp32 steps on max|s|, then tier |s| > t_strict in ascending index followed
 * by tier t_lo < |s| <= t_strict in ascending index, unfilled slots 0).
 * Bit-exact with topk_ops::topk_select (kernels/topk_select/topk_select.cu:
 * 134-171, topk_kernel.py:29-40).  n <= dip_topk_max_n(); s 16-byte aligned.
 * No host round trips: one launch of one workgroup per 2048 values; each
 * builds an LDS histogram of the 15-bit magnitudes, finds max|s| and
 * a_{k+1}, replays the 25 bisection steps and writes its 2048-value slice
 * of idx.  The workspace (512 B) keeps the last call's thresholds
 * (dip_topk_meta).
 */
size_t dip_topk_workspace_size(int64_t n);
int dip_topk_select(const uint16_t* s, int32_t* idx, int64_t n, int64_t k,
                    void* workspace, size_t ws_bytes, void* stream);
/* Copy the last top-k's thresholds (fp32 t_lo, t_strict) and tier sizes
 * (int32 count_a, count_b) from the workspace into `meta` (device, 16 B). */
int dip_topk_meta(const void* workspace, void* meta_out, void* stream);

/*
 * Gate GEMV + SiLU + top-k in one call: g = bf16(silu(bf16(gate @ x))) as
 * dip_int4_gemv with DIP_ACT_SILU, then idx[0:k] = dip_topk_select(g).
 * inter <= dip_topk_max_n(); workspace: dip_topk_workspace_size(inter).
 * Replaces gate_gemv + F.silu + select_topk (gate_kernel.py:29-33,
 * dip_stream_predispatch.py:181-185, topk_kernel.py:29-40).
 */
int dip_gate_silu_topk(const int8_t* gate_qw, const uint16_t* gate_sc, const uint16_t* x,
                       uint16_t* g, int32_t* idx, int64_t inter, int64_t hidden, int64_t k,
                       void* workspace, size_t ws_bytes, void* stream);

/*
 * out[j] = bf16( sum_c (q*s)[indices[j], c] * x[c] ), j < k.
 * Replaces int4_gather_ops::int4_gather_gemv
 * (kernels/int4_gather/int4_gather_gemv.cu:87-115).
 */
int dip_int4_gather_gemv(const int8_t* qweight, const uint16_t* scales, const uint16_t* x,
                         const int32_t* indices, uint16_t* out, int64_t rows,
                         int64_t in_features, int64_t k, void* stream);

/*
 * Up-row gather GEMV fused with h: h[j] = bf16( float(g[indices[j]]) *
 * float( bf16( sum_c (q*s)[indices[j], c] * x[c] ) ) ).
 * Replaces int4_gather_gemv + `(g[idx] * up_sel).to(bf16)` at
 * dip_stream_predispatch.py:199-201.
 */
int dip_up_gather_h(const int8_t* qweight, const uint16_t* scales, const uint16_t* x,
                    const int32_t* indices, const uint16_t* g, uint16_t* h, int64_t rows,
                    int64_t in_features, int64_t k, void* stream);

/*
 * y[o] = bf16( sum_{j<k} float(h[j]) * (q*s)[row_j, o] ) over rows of the
 * transposed down matrix down_t [rows, out_features/2]; row_j = indices[j],
 * or j when indices == NULL (the staged-copy layout of the reference).
 * Deterministic: fp32 partial sums over fixed blocks of 256 positions
 * reduced in a fixed order by a second launch, no float atomics.
 * k <= 131072; the workspace holds 8 KB of arrival counters (used by
 * dip_int4_gather_down_by_channel) and ceil(k/256) * out_features fp32
 * partials.
 * Replaces int4_down_ops::int4_gather_down
 * (kernels/int4_down/int4_gather_down.cu:77-102).
 */
size_t dip_gather_down_workspace_size(int64_t k, int64_t out_features);
int dip_int4_gather_down(const int8_t* down_t, const uint16_t* scales, const uint16_t* h,
                         const int32_t* indices, uint16_t* y, int64_t rows,
                         int64_t out_features, int64_t k, void* workspace, size_t ws_bytes,
                         void* stream);

/*
 * Launch tuning, no counterpart in the reference (process-wide, host side;
 * speed only):
 *   DIP_TUNE_ROWDOT_WGS_PER_CU  gate/up grids aim at CUs * this workgroups
 *                               (0, the default: 3 for a gate whose kernel
 *                               then still fits 3 workgroups per CU, else 2)
 *   DIP_TUNE_TOPK_STAMPS        1: the top-k records wall-clock phase stamps
 *                               in its workspace (diagnostics, slower) (0)
 *   DIP_TUNE_SPEC_MARGIN        speculative up rows: the next call speculates
 *                               on the channels at or above the magnitude of
 *                               rank k + inter * this / 1024 (0..1024) (8)
 *   DIP_TUNE_ROW_TIERS          1: a contiguous row-dot GEMV whose shape has a
 *                               measured split runs two workgroups per CU
 *                               and gives the first on each CU more rows per
 *                               lane group than the second: the SiLU gate at
 *                               hidden 5120 with 12 < rows / (8 * CUs) <= 13
 *                               (9 and the rest) and at hidden 4096 with
 *                               rows = 6 * 8 * CUs (5 and 1); the plain GEMV
 *                               at 5120 columns with rows = 5 * 8 * CUs and
 *                               at 8192 columns with rows = 5 * 4 * CUs (4
 *                               and 1); the gathered up rows with h
 *                               (dip_up_gather_h) at the SiLU gate's row
 *                               counts, whatever the grid its own plan
 *                               picks (the split of the gate of that
 *                               width); 0: every group the same rows.  Same
 *                               bits either way. (1)
 * Knob 3 (a removed step-form switch) is not a knob.  dip_set_tuning and
 * dip_get_tuning return DIP_ERR_ARG for an unknown knob, dip_set_tuning also
 * for a value out of range.
 */
enum {
  DIP_TUNE_ROWDOT_WGS_PER_CU = 0,
  DIP_TUNE_TOPK_STAMPS = 1,
  DIP_TUNE_SPEC_MARGIN = 2,
  DIP_TUNE_ROW_TIERS = 4,
  DIP_TUNE_COUNT = 5
};
int dip_set_tuning(int knob, int value);
int dip_get_tuning(int knob);

/*
 * Layer timeline (diagnostics, no counterpart in the reference; for callers
 * that profile the decode step).  In the timeline build of this library,
 * libdip_hip_timeline.so (the same sources compiled with DIP_WG_STAMPS), the
 * decode step's kernels record, per workgroup, the wall clock (s_memrealtime
 * ticks: 100 MHz, one clock for the whole device) when the workgroup's first
 * wave starts and when each of its waves ends, and the XCD it ran on
 * (HW_REG_XCC_ID).  Each launch of a kernel overwrites that kernel's record;
 * a wave that ends early (a padding tile) keeps its last launch's stamp,
 * which is older than the workgroup's start.
 *   DIP_STAMP_GATE    the row-dot kernel (the decode step's gate + SiLU)
 *   DIP_STAMP_TOPK    the top-k + speculative-up launch
 *   DIP_STAMP_DOWN    the decode step's down partials
 *   DIP_STAMP_REDUCE  the down reduce
 * dip_timeline_read copies a kernel's record to host memory after every
 * queued kernel has finished (it synchronises the device).  The product
 * build records nothing and returns DIP_ERR_UNSUPPORTED.
 */
enum { DIP_STAMP_GATE = 0, DIP_STAMP_TOPK = 1, DIP_STAMP_DOWN = 2, DIP_STAMP_REDUCE = 3 };
#define DIP_STAMP_BLOCKS 2048
#define DIP_STAMP_WAVES 16
typedef struct {
  uint64_t start[DIP_STAMP_BLOCKS];
  uint64_t end[DIP_STAMP_BLOCKS][DIP_STAMP_WAVES];
  uint32_t xcc[DIP_STAMP_BLOCKS];
  uint32_t blocks; /* grid size of the kernel's last launch */
  uint32_t pad;
} dip_wg_stamps;
int dip_timeline_read(int kernel, dip_wg_stamps* dst);

/*
 * Cache-aware dual-source up GEMV: row j comes from the resident cache
 * (src[j] == 0, row res[row[j]]) or the streamed staging buffer
 * (src[j] != 0, row str[row[j]]).  Replaces ca_fused_ops::ca_fused_gemv
 * (kernels/ca_fused/ca_fused_gemv.cu:87-112).  If g != NULL the output is
 * h[j] = bf16(g[gid[j]] * bf16(dot)) instead (dip_ca.py:185-186); g holds
 * g_len values, and a channel id gid[j] outside [0, g_len) makes h[j] NaN
 * (0x7FC0) like an out-of-range row id, instead of a read past g.
 */
int dip_ca_fused_gemv(const int8_t* res_qw, const uint16_t* res_sc, const int8_t* str_qw,
                      const uint16_t* str_sc, const uint16_t* x, const int32_t* src,
                      const int32_t* row, const uint16_t* g, const int32_t* gid,
                      int64_t g_len, uint16_t* out, int64_t res_rows, int64_t str_rows,
                      int64_t in_features, int64_t k, void* stream);

/*
 * Cache-aware dual-source down: like dip_int4_gather_down with row j read
 * from the resident cache (src[j] == 0) or the staging buffer (src[j] != 0),
 * replacing the torch.cat assembly + int4_gather_down of dip_ca.py:175-187.
 */
int dip_ca_down(const int8_t* res_qw, const uint16_t* res_sc, const int8_t* str_qw,
                const uint16_t* str_sc, const uint16_t* h, const int32_t* src,
                const int32_t* row, uint16_t* y, int64_t res_rows, int64_t str_rows,
                int64_t out_features, int64_t k, void* workspace, size_t ws_bytes,
                void* stream);

/*
 * Cache-aware hit/miss assembly (dip_ca.py:137-171): from idx[k] and
 * id2slot[inter] (int64, -1 = not resident) write, in the order
 * [hits in idx order, misses in idx order]:
 *   combined[k] channel ids, src[k] (0 hit / 1 miss), row[k] (slot for hits,
 *   0..n_miss-1 for misses), miss_ids[0:n_miss], counts[0] = n_hit,
 *   counts[1] = n_miss.
 */
int dip_ca_assemble(const int64_t* id2slot, const int32_t* idx, int32_t* combined,
                    int32_t* src, int32_t* row, int32_t* miss_ids, int32_t* counts,
                    int64_t inter, int64_t k, void* stream);

/*
 * Dequantize rows: mode 0 -> out float32 [rows, cols] = float(q) * float(s)
 * (the value the reference kernels multiply with, int4_gemv.cu:71-72);
 * mode 1 -> out bf16 [rows, cols] = bf16(q*s) (qlinear.dequantize,
 * qlinear.py:53-64).  Rows are indices[i] (or i when indices == NULL).
 */
int dip_dequant_rows(const int8_t* qweight, const uint16_t* scales, const int32_t* indices,
                     void* out, int64_t n_out_rows, int64_t rows, int64_t cols, int mode,
                     void* stream);

/*
 * Quantize w [rows, cols] (fp32, or bf16 when w_is_bf16) to int4 g128:
 * s = max(max|w_group| / 7, 1e-8) in fp32, q = clamp(round_half_even(w / s),
 * -8, 7), scales = bf16(s).  Bit-exact with quantize_tensor_int4_groupwise
 * (scripts/quantize.py:32-64) run on the CPU.  w 8-byte aligned.
 */
int dip_quantize_int4(const void* w, int w_is_bf16, int8_t* qweight, uint16_t* scales,
                      int64_t rows, int64_t cols, void* stream);

/*
 * down [out_features, inter] int4 -> down_t [inter, out_features] int4 via
 * bf16 dequantize, transpose and re-quantization along out_features; bit-exact
 * with _transpose_down_to_int4 (dip_stream_predispatch.py:100-120).
 */
int dip_transpose_down_int4(const int8_t* down_qw, const uint16_t* down_sc, int8_t* down_t_qw,
                            uint16_t* down_t_sc, int64_t out_features, int64_t inter,
                            void* stream);

/*
 * scales_gm[g][r] = scales[r][g] for a [rows, groups] bf16 scale matrix: the
 * group-major copy of down_t's scales that the decode step's down stage
 * reads when given one (dip_mlp_decode's down_t_sc_gm).  A resident layout
 * of this library with no counterpart in the reference (whose down_t keeps
 * [inter, hidden/128] scales only); 2 * rows * groups bytes per layer.
 */
int dip_scales_group_major(const uint16_t* scales, uint16_t* scales_gm, int64_t rows,
                           int64_t groups, void* stream);

/*
 * The decode step's first half with speculative up rows: no counterpart in
 * the reference (it replaces gate_kernel.py:29-33 + topk_kernel.py:29-40 +
 * the up half of dip_stream_predispatch.py:196-199 by two launches):
 *   1. g = bf16(silu(bf16(gate @ x))) [inter] (as dip_int4_gemv, DIP_ACT_SILU);
 *   2. one launch: idx[0:k] as dip_topk_select(g), and meanwhile
 *      h_full[c] = bf16(g[c] * bf16(up[c] . x)) for the channels c whose
 *      magnitude key (|g| bits) is at or above state[0], then for the
 *      selected channels below it (and channel 0 when slots are unfilled).
 * h_full[idx[j]] is bit-identical to the h of dip_up_gather_h for every j;
 * entries of unselected channels are unspecified.  state: 2 uint32 per layer
 * (dip_mlp_state_size bytes, zero before the first call, then left to these
 * calls): [0] the key in use, [1] the key of rank k + margin of the last call
 * (DIP_TUNE_SPEC_MARGIN), moved to [0] by launch 1 of the next call.  The
 * state only decides which workgroups compute which h, never a value.
 * hidden / 32 must be 160, 128 or 80 (else DIP_ERR_UNSUPPORTED); 1 <= k <=
 * inter <= dip_topk_max_n(); workspace: dip_topk_workspace_size(inter).
 */
size_t dip_mlp_state_size(void);
int dip_gate_silu_topk_spec(const int8_t* gate_qw, const uint16_t* gate_sc,
                            const int8_t* up_qw, const uint16_t* up_sc, const uint16_t* x,
                            uint16_t* g, int32_t* idx, uint16_t* h_full, int64_t inter,
                            int64_t hidden, int64_t k, void* workspace, size_t ws_bytes,
                            void* state, void* stream);

/*
 * dip_int4_gather_down with h indexed by channel: y = sum_j h_full[idx[j]] *
 * down_t[idx[j]] (the down half of dip_stream_predispatch.py:196-203 after
 * dip_gate_silu_topk_spec); h_out[j] = h_full[idx[j]] when h_out != NULL.
 * indices == NULL: idx[j] = j for j < k (k <= rows), the every-row down of
 * the keep >= 0.999 route (dip_stream_predispatch.py:177-179), whose row
 * loads then wait for no id.
 * Same workspace as dip_int4_gather_down.  scales_gm (optional, may be
 * NULL): the same scales group-major, [out_features/128][rows]
 * (dip_scales_group_major); when given the kernel reads the scales there
 * (same values, same y bit for bit) instead of a few bytes of every
 * selected row's own scale line.  With scales_gm, a matrix under 4 GiB,
 * out_features a multiple of 2048 (at most 8192) and a full 256-CU gfx950,
 * the partial sums are reduced inside the same launch: every tile of a
 * column block runs on one XCD and the last one to finish sums them, in the
 * same order as the reduce launch (same y bit for bit, one launch).
 */
int dip_int4_gather_down_by_channel(const int8_t* down_t, const uint16_t* scales,
                                    const uint16_t* scales_gm,
                                    const uint16_t* h_full, const int32_t* indices,
                                    uint16_t* y, uint16_t* h_out, int64_t rows,
                                    int64_t out_features, int64_t k, void* workspace,
                                    size_t ws_bytes, void* stream);

/*
 * One resident-weight DIP MLP decode step (batch 1, seq 1):
 *   g = silu(gate(x)); idx = topk(|g|, k); h = g[idx] * up[idx](x);
 *   y = h @ down_t[idx]
 * i.e. StreamingDIPMlp.forward (dip_stream_predispatch.py:176-204) with all
 * weights resident in HBM.  g_out [inter], idx_out [k], h_out [k] receive
 * the intermediates; y [hidden].  workspace: dip_mlp_workspace_size().
 * layer_state (dip_mlp_state_size bytes per layer, zeroed once, or NULL):
 * when set and the width allows, the step runs as dip_gate_silu_topk_spec +
 * dip_int4_gather_down_by_channel (four launches); otherwise as
 * dip_gate_silu_topk + dip_up_gather_h + dip_int4_gather_down (five).  Both
 * give bit-identical outputs.  down_t_sc_gm (optional, may be NULL): the
 * group-major copy of down_t_sc (dip_scales_group_major), which the down
 * stage then reads instead (same outputs, bit for bit; the opt-in fused
 * step ignores it).
 */
size_t dip_mlp_workspace_size(int64_t hidden, int64_t inter, int64_t k);
int dip_mlp_decode(const int8_t* gate_qw, const uint16_t* gate_sc, const int8_t* up_qw,
                   const uint16_t* up_sc, const int8_t* down_t_qw, const uint16_t* down_t_sc,
                   const uint16_t* down_t_sc_gm, const uint16_t* x, uint16_t* y, uint16_t* g_out, int32_t* idx_out,
                   uint16_t* h_out, int64_t hidden, int64_t inter, int64_t k,
                   void* workspace, size_t ws_bytes, void* layer_state, void* stream);

/*
 * dip_mlp_decode for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference.  Same arguments and outputs as
 * dip_mlp_decode without the workspace: the step's workspace is a
 * DIP_NOALLOC_SCRATCH_BYTES device array the library holds on every GPU it
 * runs on until the process ends (its address is looked up at the first
 * call on a device, with that device current).  A shape whose
 * dip_mlp_workspace_size exceeds it returns DIP_ERR_SCRATCH.  The call
 * allocates nothing.  All calls on one GPU share its array, so calls that
 * overlap on one GPU (other streams or threads) race; calls in stream order
 * do not (nothing in the array is read before the same call writes it).
 */
#define DIP_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)
int dip_mlp_decode_noalloc(const int8_t* gate_qw, const uint16_t* gate_sc,
                           const int8_t* up_qw, const uint16_t* up_sc,
                           const int8_t* down_t_qw, const uint16_t* down_t_sc,
                           const uint16_t* down_t_sc_gm, const uint16_t* x, uint16_t* y,
                           uint16_t* g_out, int32_t* idx_out, uint16_t* h_out, int64_t hidden,
                           int64_t inter, int64_t k, void* layer_state, void* stream);

/*
 * dip_mlp_decode with the post-attention RMSNorm of a decoder layer folded
 * into its gate launch: v = bf16(h + add) (add may be NULL), x = bf16(norm_w
 * * bf16(v * rsqrt(mean(v^2) + eps))); the gate's workgroup 0 writes v to
 * h_res_out (if non-NULL) and x to x_out, which the up rows then read.
 * y, g_out, idx_out and h_out are dip_mlp_decode's on that x, bit for bit.
 * x_out and h_res_out must differ from h and add.  hidden 5120, 4096 or
 * 2560 (else DIP_ERR_UNSUPPORTED).  No counterpart kernel in the reference
 * (its decode runs the norm as separate PyTorch ops before
 * StreamingDIPMlp.forward).
 */
int dip_mlp_decode_rmsnorm(const int8_t* gate_qw, const uint16_t* gate_sc, const int8_t* up_qw,
                           const uint16_t* up_sc, const int8_t* down_t_qw,
                           const uint16_t* down_t_sc, const uint16_t* down_t_sc_gm,
                           const uint16_t* h, const uint16_t* add,
                           const uint16_t* norm_w, float eps, uint16_t* h_res_out,
                           uint16_t* x_out, uint16_t* y, uint16_t* g_out, int32_t* idx_out,
                           uint16_t* h_out, int64_t hidden, int64_t inter, int64_t k,
                           void* workspace, size_t ws_bytes, void* layer_state, void* stream);

/*
 * Host-side row gather for the cache-aware miss path: copies rows
 * src + ids[i] * row_bytes -> dst + i * row_bytes for i < n using up to
 * `threads` host threads (the pinned index_select of dip_ca.py:148-153).
 * Host pointers; returns DIP_OK or a DIP_ERR_* code.
 */
int dip_host_gather_rows(const void* src, const int32_t* ids, void* dst, int64_t n,
                         int64_t row_bytes, int64_t src_rows, int threads);

/*
 * dip_host_gather_rows over several matrices that share the row ids (the
 * four index_selects of one miss set, dip_ca.py:148-153) in one pass:
 * dst[p] + i * row_bytes[p] <- src[p] + ids[i] * row_bytes[p] for every
 * piece p < npieces (at most 64) and i < n.  The threads come from a
 * persistent pool created on first use.  Host pointers; returns DIP_OK or
 * a DIP_ERR_* code.
 */
int dip_host_gather_rows_multi(const void* const* src, void* const* dst,
                               const int64_t* row_bytes, int64_t npieces, const int32_t* ids,
                               int64_t n, int64_t src_rows, int threads);

/*
 * The cache-aware miss stream (dip_ca.py:146-156: pinned index_select, then
 * non_blocking H2D copies on a side stream) as one pipelined call: the ids
 * are taken in chunks (the first ramping up from chunk_rows / 8, doubling,
 * then chunk_rows each); for each chunk the library's host threads gather
 * the rows of every piece into pinned[p] (host, pinned, at least n rows),
 * and the calling thread queues the chunk's copies pinned[p] -> dst[p]
 * (device, at least n rows) as soon as it is gathered, so a chunk's copy
 * runs while the next chunk is gathered.  Pieces [0, npieces/2) are copied
 * on `stream`, the rest on a library-owned second stream of the current
 * device (so two DMA engines share each chunk), which `stream` waits for
 * before the call returns: work queued on `stream` afterwards sees every
 * copy.  Only the calling thread makes HIP calls.  Returns once every copy
 * is queued (not finished).  When copy_ms is non-NULL, each chunk's copies
 * on each stream are bracketed by events, the call waits for them and
 * writes the sum over chunks of the longer stream's copy time, in
 * milliseconds.  Returns DIP_OK, a DIP_ERR_* code or a hipError_t.
 */
int dip_host_stream_rows(const void* const* src, void* const* pinned, void* const* dst,
                         const int64_t* row_bytes, int64_t npieces, const int32_t* ids,
                         int64_t n, int64_t src_rows, int64_t chunk_rows, int threads,
                         void* stream, float* copy_ms);

/*
 * dip_int4_gemv with the input RMSNorm of a decoder layer folded in:
 * v = bf16(h + add) (add may be NULL), x = bf16(norm_w * bf16(v * rsqrt(
 * mean(v^2) + eps))) (transformers' Qwen3RMSNorm, fp32 mean), out = the
 * GEMV of x; v is also written to h_out when h_out is non-NULL (it must not
 * be h or add: every workgroup reads them).  Each workgroup normalises x
 * itself, so the launch replaces an RMSNorm launch before the GEMV.
 * in_features 5120, 4096 or 2560 (else DIP_ERR_UNSUPPORTED).  No
 * counterpart kernel in the reference (its decode runs the norm and the
 * projection as separate PyTorch ops).
 */
int dip_int4_gemv_rmsnorm(const int8_t* qweight, const uint16_t* scales, const uint16_t* h,
                          const uint16_t* add, const uint16_t* norm_w, float eps, uint16_t* h_out,
                          uint16_t* out, int64_t out_features, int64_t in_features, void* stream);

/*
 * out[m, n] = bf16( sum_c (q*s)[n, c] * x[m, c] ) for m < M tokens: the int4
 * projection of a prompt (more than one token) on bf16 MFMA, weights read
 * once as packed nibbles.  x bf16 [M, in_features] row-major, out bf16
 * [M, out_features].  Replaces dequantize + F.linear for prompts
 * (qlinear.py:86-88; the gate and up GEMMs of StreamingDIPMlp._dense,
 * dip_stream_predispatch.py:206-212).  The weights enter as exact fp32 q*s
 * (the reference rounds them to bf16 first); fp32 sums, one bf16 rounding.
 * M <= 64 * 65535; qweight and x 16-byte aligned.
 */
int dip_int4_gemm(const int8_t* qweight, const uint16_t* scales, const uint16_t* x,
                  uint16_t* out, int64_t m, int64_t out_features, int64_t in_features,
                  void* stream);

/*
 * out[m, n] = bf16( sum_c x[m, c] * bf16(q*s)[c, n] ) for W stored as rows
 * of in_features (qweight_t int8 [in_features, out_features/2], scales_t
 * bf16 [in_features, out_features/128]): the dense route's h @ down_t for a
 * prompt (dip_stream_predispatch.py:213-215) on bf16 MFMA, without the bf16
 * copy of down_t.  Each weight enters as the reference's bf16(q*s); fp32
 * sums; one bf16 rounding.  K is split over workgroups when the output has
 * few column tiles; the workspace (dip_int4_gemm_t_workspace_size bytes,
 * 0 when no split is needed) holds their fp32 partials, added in a fixed
 * order by a second launch.  out_features a multiple of 128, in_features a
 * multiple of 8; qweight_t and x 16-byte aligned.
 */
size_t dip_int4_gemm_t_workspace_size(int64_t m, int64_t out_features, int64_t in_features);
int dip_int4_gemm_t(const int8_t* qweight_t, const uint16_t* scales_t, const uint16_t* x,
                    uint16_t* out, int64_t m, int64_t out_features, int64_t in_features,
                    void* workspace, size_t ws_bytes, void* stream);

/*
 * One-token decode steps of a Qwen3 decoder layer around the DIP MLP, for
 * the whole-model decode loop.  The reference has no kernels of its own
 * here: its decode runs these steps through transformers' Qwen3 modules
 * with PyTorch ops (the model built by dip_stream_predispatch.py:218-289 /
 * dip_ca.py:199-269; transformers' modeling_qwen3 Qwen3RMSNorm.forward,
 * apply_rotary_pos_emb, Qwen3Attention.forward,
 * Qwen3DecoderLayer.forward).  bf16 tensors as uint16_t bits; `pos` is a
 * device int64 holding the token's position, so the launches can be
 * captured once and replayed for every token.
 *
 * dip_add_rmsnorm: if `add` is non-NULL, h[i] = bf16(h[i] + add[i]) in place
 * (the residual add); then out = bf16(w * bf16(h * rsqrt(mean(h^2) + eps)))
 * with an fp32 mean.  n a multiple of 8, at most 8192; pointers 16-byte
 * aligned.
 */
int dip_add_rmsnorm(uint16_t* h, const uint16_t* add, const uint16_t* weight, uint16_t* out,
                    int64_t n, float eps, void* stream);

/*
 * dip_qk_norm_rope_cache: `qkv` holds one token's q | k | v projections,
 * (n_heads + 2 n_kv_heads) * head_dim values.  Each q and k head gets
 * RMSNorm over the head (q_norm_w / k_norm_w, head_dim values), then the
 * rotary embedding with row `pos` of the [max_len, head_dim] cos / sin
 * tables (bf16(bf16(x cos) + bf16(rotate_half(x) sin))); q goes to q_out
 * [n_heads, head_dim], k and v to row `pos` of k_cache / v_cache
 * [n_kv_heads, max_len, head_dim].  Cache rows are written only when
 * 0 <= pos < max_len.  head_dim must be 128 (else DIP_ERR_UNSUPPORTED);
 * pointers 16-byte aligned.
 */
int dip_qk_norm_rope_cache(const uint16_t* qkv, const uint16_t* q_norm_w,
                           const uint16_t* k_norm_w, const uint16_t* cos_table,
                           const uint16_t* sin_table, const int64_t* pos, uint16_t* q_out,
                           uint16_t* k_cache, uint16_t* v_cache, int64_t n_heads,
                           int64_t n_kv_heads, int64_t head_dim, int64_t max_len, float eps,
                           void* stream);

/*
 * dip_decode_attention: out[h] = softmax(scale * q[h] . K[j]) V over cache
 * rows j = 0 .. pos of kv head h / (n_heads / n_kv_heads) (grouped-query
 * attention of one token; fp32 scores, softmax and sums, bf16 output).
 * Two launches: per (32-row chunk, kv head) partial sums into the workspace
 * (dip_decode_attention_workspace_size bytes), then one merge per query
 * head.  head_dim 128 and n_heads / n_kv_heads in {1, 2, 4, 5, 8, 16}
 * (else DIP_ERR_UNSUPPORTED).
 */
size_t dip_decode_attention_workspace_size(int64_t n_heads, int64_t head_dim, int64_t max_len);

/*
 * dip_decode_attention_fused: dip_qk_norm_rope_cache followed by
 * dip_decode_attention (q_out not kept) in one launch of one workgroup per
 * query head, for caches of at most dip_decode_attention_fused_max_len()
 * rows (1024; else DIP_ERR_SHAPE) and any n_heads that n_kv_heads divides.
 * The first workgroup of each kv head's group writes the cache row; every
 * workgroup takes the token's own row from its copy, not read back.  Same
 * cache rows bit for bit; the scores are summed on bf16 MFMA (exact
 * products, fp32 sums) and the chunks merged in another order.  No
 * workspace.
 */
int64_t dip_decode_attention_fused_max_len(void);
int dip_decode_attention_fused(const uint16_t* qkv, const uint16_t* q_norm_w,
                               const uint16_t* k_norm_w, const uint16_t* cos_table,
                               const uint16_t* sin_table, const int64_t* pos, uint16_t* k_cache,
                               uint16_t* v_cache, uint16_t* out, int64_t n_heads,
                               int64_t n_kv_heads, int64_t head_dim, int64_t max_len, float eps,
                               float scale, void* stream);
int dip_decode_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                         const int64_t* pos, uint16_t* out, int64_t n_heads, int64_t n_kv_heads,
                         int64_t head_dim, int64_t max_len, float scale, void* workspace,
                         size_t ws_bytes, void* stream);

#ifdef __cplusplus
}  // extern "C"
#endif

#endif  /* DIP_HIP_H_ */
