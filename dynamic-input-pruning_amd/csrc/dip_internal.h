// dip_internal.h — host-side declarations shared by the DIP translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/dip_hip.h"

namespace dip {

// Row source for the row-dot and down kernels.
enum RowSrc : int {
  kContig = 0,  // output j reads row j of matrix A
  kGather = 1,  // output j reads row sel[j] of matrix A
  kDual = 2,    // output j reads row sel2[j] of A (sel[j]==0) or of B (sel[j]!=0)
};

// Epilogue of the row-dot kernel.
enum Epi : int {
  kRaw = 0,       // out[j] = bf16(dot)
  kSilu = 1,      // out[j] = bf16(silu(bf16(dot)))
  kH = 3,         // out[j] = bf16(g[gid[j]] * bf16(dot))
};

struct RowdotArgs {
  const int8_t* qw_a;
  const uint16_t* sc_a;
  const int8_t* qw_b;
  const uint16_t* sc_b;
  const uint16_t* x;
  const int32_t* sel;
  const int32_t* sel2;
  const int32_t* gid;
  const uint16_t* g;
  int g_len;   // kH with kDual: channel ids gid[j] outside [0, g_len) yield NaN
  uint16_t* out;
  const int8_t* qw_safe;   // a matrix with at least one row: read in place of bad rows
  const uint16_t* sc_safe;
  int nrows;
  int in_features;
  int rows_a;  // rows of matrix A (row ids outside [0, rows_a) yield NaN)
  int rows_b;  // rows of matrix B (kDual)
  int ngrp;    // row groups (set by the launcher)
  // two tiers of workgroups (set by the launcher; tier_wgs 0: one tier):
  // workgroups [0, tier_wgs) compute rows [0, tier_rows), the others the rest
  int tier_wgs;
  int tier_rows;
  uint32_t* rotate;  // if set: workgroup 0 copies rotate[1] to rotate[0] (speculation state)
  // RMSNorm prologue (dip_int4_gemv_rmsnorm): x = bf16(w * bf16(v * rsqrt(mean(v^2)
  // + eps))) with v = bf16(x + norm_add); workgroup 0 writes v to norm_h_out
  const uint16_t* norm_w;
  const uint16_t* norm_add;
  uint16_t* norm_h_out;
  uint16_t* norm_x_out;  // workgroup 0 also writes the normalised x here (if set)
  float norm_eps;
};

struct DownArgs {
  const int8_t* qw_a;
  const uint16_t* sc_a;
  const int8_t* qw_b;
  const uint16_t* sc_b;
  const uint16_t* sc_gm;   // optional: A's scales group-major [groups][rows_a] (kContig, kGather)
  const uint16_t* h;
  const int32_t* sel;
  const int32_t* sel2;
  const int8_t* qw_safe;   // a matrix with at least one row: read in place of bad rows
  const uint16_t* sc_safe;
  float* partial;     // [row_blocks, out_features]
  uint16_t* h_out;    // if set: h_out[j] = the h used for position j
  int h_by_row;       // h is indexed by row id (h[sel[j]]) instead of by position
  int rows_a;
  int rows_b;
  int k;
  int out_features;
  int col_blocks;
  int row_blocks;
};

// Top-k: one histogram bin per 15-bit |s| key, held in LDS.
constexpr int kFineBins = 32768;
constexpr int kTopkMaxN = 65536;

struct TopkMeta {
  float lo;
  float hi;
  int32_t count_a;
  int32_t count_b;
  uint32_t key_a;   // (k+1)-th largest magnitude key, 0xFFFFFFFF if fewer than k+1 values
  uint32_t key_max;
  int32_t n_valid;
  int32_t pad;
  uint64_t stamp[6];   // wall_clock64() at the select kernel's phase boundaries (diagnostics)
  uint64_t cycles[2];  // clock64() (shader clock) at the start and end (diagnostics)
  // wall_clock64() in two speculation workgroups (the first and the middle
  // one): start, x staged and the list counted, list published, done
  // (diagnostics)
  uint64_t spec_stamp[2][4];
};

// The top-k workspace holds the last call's TopkMeta.
constexpr size_t kTopkWorkspace = 512;
static_assert(sizeof(TopkMeta) <= kTopkWorkspace, "TopkMeta fits the top-k workspace");

// Top-k + speculative up (one launch): workgroups [0, ntopk) run the select,
// the rest compute h_full[c] = bf16(g[c] * bf16(up[c] . x)) for every channel
// whose magnitude key is at or above state[0]; the select workgroups add the
// selected channels below it.  state[1] receives the key at rank k + margin
// for the next call.
struct SpecArgs {
  const int8_t* up_qw;
  const uint16_t* up_sc;
  const uint16_t* x;
  uint16_t* h_full;   // [n] h by channel (only the selected channels are meaningful)
  uint32_t* state;    // [0] speculation key in use, [1] the next call's key
  int hidden;
  int margin;         // set by the launcher (DIP_TUNE_SPEC_MARGIN)
  int chan_per_wg;    // set by the launcher
  int ntopk;          // set by the launcher
};

// Per-layer state of the decode step with speculative up rows: [0] the
// speculation key in use, [1] the next call's key (the gate launch moves [1]
// to [0]); [2] and [3] are spare.  Zero before the first call.
constexpr int kMlpStateWords = 4;
// The grid (workgroups) launch_rowdot (norm false) / launch_rowdot_norm
// (norm true) use for the SiLU gate of nrows rows of in_features columns.
int rowdot_contig_blocks(int64_t nrows, int64_t in_features, bool norm);
// y[o] = bf16(sum over rows rb < row_blocks of partial[rb][o]) in a fixed order.
int launch_down_reduce(const float* partial, int row_blocks, int out_features, uint16_t* y,
                       hipStream_t stream);

// Launchers (return hipSuccess or a DIP_ERR_* code).
int launch_rowdot(int src, int epi, const RowdotArgs& a, hipStream_t stream);
// Contiguous rows with the RMSNorm prologue (staged-x widths only).
bool rowdot_norm_supported(int64_t in_features);
int launch_rowdot_norm(int epi, const RowdotArgs& a, hipStream_t stream);
// The top-k + speculative up launch that follows the gate in a decode step
// (dip_gate_silu_topk_spec without its gate launch).
int launch_spec_after_gate(const uint16_t* g, int64_t inter, int64_t hidden, int64_t k,
                           int32_t* idx, uint16_t* h_full, const int8_t* up_qw,
                           const uint16_t* up_sc, const uint16_t* x, void* workspace,
                           void* state, hipStream_t stream);
int run_down(int src, const int8_t* qw_a, const uint16_t* sc_a, int64_t rows_a,
             const int8_t* qw_b, const uint16_t* sc_b, int64_t rows_b, const uint16_t* h,
             const int32_t* sel, const int32_t* sel2, int64_t k, int64_t out_features,
             uint16_t* y, void* workspace, size_t ws_bytes, hipStream_t stream,
             int h_by_row = 0, uint16_t* h_out = nullptr, const uint16_t* sc_gm = nullptr);
size_t down_workspace_bytes(int64_t k, int64_t out_features);
int64_t down_max_k();  // largest k the down path accepts
// The top-k select kernel: idx from s (TopkMeta into the workspace).
int launch_topk_select(const uint16_t* s, int64_t n, int64_t k, int32_t* idx, void* ws,
                       hipStream_t stream);
// The top-k + speculative-up launch (hidden widths of topk_spec_supported).
bool topk_spec_supported(int64_t hidden);
int launch_topk_spec(const uint16_t* g, int64_t n, int64_t k, int32_t* idx, void* ws,
                     SpecArgs sp, hipStream_t stream);


// Layer timeline records (the timeline build; DIP_ERR_UNSUPPORTED otherwise).
int timeline_read_rowdot(dip_wg_stamps* dst);
int timeline_read_topk(dip_wg_stamps* dst);
int timeline_read_down(int reduce, dip_wg_stamps* dst);

// Launch tuning (process-wide, host side): see DIP_TUNE_* in dip_hip.h.
int tuning(int knob);
// Compute units of the current device (cached per device).
int device_cus();

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int hip_status(hipError_t e) { return e == hipSuccess ? DIP_OK : (int)e; }

}  // namespace dip
