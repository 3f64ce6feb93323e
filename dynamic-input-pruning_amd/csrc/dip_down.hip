// dip_down.hip — transposed-down gather: y[o] = sum_j h[j] * (q*s)[row_j, o].
//
// down_t is [rows, out/2] packed int4 (row = one intermediate channel), so a
// selected channel is one contiguous row.  The work is tiled two ways:
//   * column block cb: LPR lanes each own one 16-byte chunk (32 outputs) of
//     every row, i.e. 16*LPR contiguous bytes per row per block;
//   * row block rb: 256 consecutive selected positions j.
// A block of 256 threads holds 256/LPR "slots" of LPR lanes; slot s walks the
// LPR rows j = 256*rb + s + i*(256/LPR), i < LPR.  Lane l of a slot fetches
// the id, h and the scales of the slot's column groups (one or two) of the
// slot's l-th row and turns them into the row's coefficients 16*h*s.  The
// ids and coefficients reach the slot's lanes through a per-wave LDS
// exchange (each lane writes its row's, then reads its slot's LPR: two
// 128-bit reads each, no per-row shuffles), so every lane issues one memory
// instruction per row (its 16-byte chunk).  The row loop is straight-line
// code (LPR is a compile-time constant; positions past k are clamped and
// contribute 0), so every load is unconditional and all of a slot's rows are
// in flight at once.  Each lane keeps 32 fp32 accumulators (its outputs).
//
// Dequant: v_cvt_off_f32_i4 with an SDWA byte select gives q/16 exactly for
// the low nibble of any byte (high nibbles after one shift), so each weight
// costs one convert and one FMA: acc += (q/16) * (16*h*s).
//
// Reduction, deterministic and without float atomics:
//   1. the slots of a wave are summed in registers (DPP rotations, then
//      permlane swaps that halve the live accumulators at each step), the
//      four waves' sums are added in wave order through 4 KB of LDS, and the
//      block stores its fp32 partial row segment;
//   2. the row blocks' partials of every output are summed in a fixed order
//      (row blocks rb = p, p + 4, ... ascending for p = 0..3, then the four
//      sums in order of p) and rounded to bf16: by a reduce kernel, or, in
//      the decode step's kernel on a device whose workgroups reach its 8 XCDs
//      round-robin, by the last tile of each column block inside the same
//      launch (down_gm_kernel<true>: every tile of a column block runs on one
//      XCD, so its partials and its arrival counter stay in that XCD's L2).
// (A last-arriving-block reduce with the column blocks of a row block spread
// over every XCD was measured and dropped: the 64 arrivals on each column
// block's device-scope counter serialise and cost more than the second
// launch.)
#include <string.h>

#include "dip_tiles.h"

namespace dip {

namespace {
constexpr int kThreads = kDownThreads;
constexpr int kRowsPerBlock = kThreads;  // 256/LPR slots x LPR rows each
constexpr int kXcds = 8;                 // MI355X: 8 XCDs, workgroups dispatched round-robin
constexpr int kMaxRowBlocks = 512;       // k <= 131072
constexpr int kRedOut = 32;              // outputs per reduce block
constexpr int kRedSplit = 4;             // interleaved row-block splits per output
constexpr int kMaxXcdColBlocks = kDownCounterBytes / kDownCounterStride;
}  // namespace

#ifdef DIP_WG_STAMPS
__device__ dip_wg_stamps g_stamps_down;
__device__ dip_wg_stamps g_stamps_reduce;
int timeline_read_down(int reduce, dip_wg_stamps* dst) {
  return reduce ? hip_status(hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_stamps_reduce),
                                                 sizeof(dip_wg_stamps), 0, hipMemcpyDeviceToHost))
                : hip_status(hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_stamps_down),
                                                 sizeof(dip_wg_stamps), 0, hipMemcpyDeviceToHost));
}
#else
int timeline_read_down(int, dip_wg_stamps*) { return DIP_ERR_UNSUPPORTED; }
#endif

// OFF32 (one matrix below 4 GiB): the exchange carries each row's 32-bit
// byte offset instead of its id, and the row loads add it to the matrix's
// base in a scalar register (one VGPR per address, no 64-bit multiply).
template <int LPR, int SRC, int SL, bool OFF32>
__global__ __launch_bounds__(kThreads) void down_kernel(DownArgs a) {
  static_assert(!OFF32 || SRC != kDual, "32-bit offsets: one matrix");
  static_assert(LPR % kChunksPerGroup == 0 && LPR / kChunksPerGroup <= 2, "groups per slot");
  constexpr int kSlots = kThreads / LPR;
  constexpr int kCols = LPR * kDownAcc;  // outputs per column block
  constexpr int NG = LPR / kChunksPerGroup;
  __shared__ __align__(16) float red[down_red_floats<LPR>()];
  // the per-wave exchange: lane t's row id, and its row's coefficient for
  // each of the slot's column groups (a slot's lanes are all in one wave)
  __shared__ __align__(16) uint32_t xid[kThreads];
  __shared__ __align__(16) float xcoef[NG][kThreads];

  // XCD-aware tile order: workgroups go to the 8 XCDs round-robin, so tile
  // (rb, cb) runs as workgroup b with b % 8 == rb % 8.  All column blocks of
  // a row block then share one XCD's L2, which serves the scale lines, ids
  // and h of those rows once instead of once per column block.
  const int xcd = blockIdx.x % kXcds;
  const int w = blockIdx.x / kXcds;
  const int rb = xcd + kXcds * (w / a.col_blocks);
  const int cb = w % a.col_blocks;
  if (rb >= a.row_blocks) return;  // padding tile (row blocks rounded up to 8)
  const int l = threadIdx.x % LPR;
  const int slot = threadIdx.x / LPR;
  const int cc0 = cb * LPR + l;  // my chunk within a row
  const size_t row_bytes = (size_t)(a.out_features >> 1);
  const int ngroups = a.out_features >> 7;

  // lane l: id and h of the slot's row l (position clamped; past k -> kPadRow)
  const int jl = rb * kRowsPerBlock + slot + l * kSlots;
  const int jc = min(jl, a.k - 1);
  const uint32_t rid_c = down_row<SRC>(a, jc);
  const uint32_t rid_l = jl < a.k ? rid_c : kPadRow;
  const int hix = !a.h_by_row ? jc : (rid_c < (uint32_t)a.rows_a ? (int)rid_c : 0);
  const uint32_t h_l = a.h[hix];

  // lane l: the scales of row l for the slot's NG column groups
  const int g0 = cb * LPR / kChunksPerGroup;
  uint32_t s_l[NG];
  load_down_scales<SRC, NG, SL>(a, rid_l, g0, ngroups, s_l);

  // the slot's LPR row ids (the exchange stays inside one wave, so a wave
  // barrier, which only orders the wave's own LDS accesses, suffices)
  const uint32_t r_off = rid_l >= kPadRow ? 0u : rid_l;  // bad and padding rows read row 0
  xid[threadIdx.x] = OFF32 ? r_off * (uint32_t)row_bytes : rid_l;
  __builtin_amdgcn_wave_barrier();
  uint32_t ids[LPR];
  {
    const uint4* src = reinterpret_cast<const uint4*>(xid + slot * LPR);
#pragma unroll
    for (int v = 0; v < LPR / 4; ++v) {
      const uint4 q = src[v];
      ids[4 * v] = q.x;
      ids[4 * v + 1] = q.y;
      ids[4 * v + 2] = q.z;
      ids[4 * v + 3] = q.w;
    }
  }
  DownRow ring[LPR];
#pragma unroll
  for (int d = 0; d < LPR; ++d) {
    if constexpr (OFF32)
      ring[d].w = ldg_nt(reinterpret_cast<const uint4*>(a.qw_a + (size_t)(ids[d] + 16u * (uint32_t)cc0)));
    else
      load_down_row<SRC>(a, ids[d], cc0, row_bytes, ring[d]);
  }

  // h by position (the API's h_out), stored once the rows are in flight:
  // before them it would hold up the first column block's tiles by a round
  // trip for h
  if (a.h_out && cb == 0 && jl < a.k) a.h_out[jl] = (uint16_t)h_l;

  // each row's coefficient for my column group
  float f_l[NG];
  down_coef<NG>(rid_l, h_l, s_l, f_l);
#pragma unroll
  for (int g = 0; g < NG; ++g) xcoef[g][threadIdx.x] = f_l[g];
  __builtin_amdgcn_wave_barrier();
  float f[LPR];
  {
    const float4* src = reinterpret_cast<const float4*>(&xcoef[l / kChunksPerGroup][slot * LPR]);
#pragma unroll
    for (int v = 0; v < LPR / 4; ++v) {
      const float4 q = src[v];
      f[4 * v] = q.x;
      f[4 * v + 1] = q.y;
      f[4 * v + 2] = q.z;
      f[4 * v + 3] = q.w;
    }
  }
  float acc[kDownAcc];
#pragma unroll
  for (int m = 0; m < kDownAcc; ++m) acc[m] = 0.f;
  down_accumulate<LPR>(ring, f, acc);
  down_block_partial<LPR>(acc, red, a.partial + (size_t)rb * a.out_features + (size_t)cb * kCols);
}

// The decode step's form of down_kernel<8, kGather, kScGm, true> (h by
// channel, group-major scales, one matrix under 4 GiB), with a compact
// argument block: the same tiles, loads, exchange and arithmetic, so y and
// h_out are bit for bit the general kernel's; measured 12.4 against
// 12.9-13.3 us per launch (partials + reduce) on the Qwen3-32B layer.
struct DownGmArgs {
  const int8_t* qw;
  const uint16_t* sc_gm;  // [groups][rows]
  const uint16_t* h;      // by channel
  const int32_t* sel;
  float* partial;
  uint16_t* h_out;
  uint32_t* counters;  // XCD-local reduce: one arrival counter per column block
  uint16_t* y;         // XCD-local reduce: the output
  int rows, k, out_features, col_blocks, row_blocks;
};

// The XCD-local reduce at the end of a tile of down_gm_kernel<true>.  Every
// tile of column block cb runs on the same XCD (workgroups b with the same
// b % 8 share an XCD), so the partial stores and the arrival counter of cb
// meet in that XCD's L2: each thread waits until its partial store is
// acknowledged by the L2, the block synchronises, one L2 atomic counts the
// arrival, and the tile that arrives last (it sees row_blocks - 1) resets
// the counter for the next launch and sums the column block's partials,
// which it reads back from the same L2, in the order of down_reduce_kernel.
DIP_DEV void down_xcd_tail(const DownGmArgs& a, int cb, float* red, uint32_t* last) {
  constexpr int kCols = 8 * kDownAcc, kWaves = kThreads / 64;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t* ctr = a.counters + (size_t)cb * (kDownCounterStride / sizeof(uint32_t));
    const uint32_t old =
        __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    const bool is_last = old == (uint32_t)(a.row_blocks - 1);
    if (is_last) *ctr = 0u;
    *last = is_last;
  }
  __syncthreads();
  if (!*last) return;
  // wave w sums row blocks w, w + 4, ... in ascending order (4 columns per
  // lane, 8 row blocks per round trip), then the waves' sums meet in LDS
  const int w = threadIdx.x >> 6, ln = threadIdx.x & 63;
  const float4* base = reinterpret_cast<const float4*>(a.partial + (size_t)cb * kCols) + ln;
  const size_t stride = (size_t)a.out_features / 4;
  float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int b0 = w; b0 < a.row_blocks; b0 += kWaves * 8) {
    float4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      v[u] = base[(size_t)min(b0 + kWaves * u, a.row_blocks - 1) * stride];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (b0 + kWaves * u < a.row_blocks) {
        sum.x += v[u].x;
        sum.y += v[u].y;
        sum.z += v[u].z;
        sum.w += v[u].w;
      }
    }
  }
  *reinterpret_cast<float4*>(red + w * kCols + 4 * ln) = sum;
  __syncthreads();
  float t = red[threadIdx.x];
#pragma unroll
  for (int q = 1; q < kWaves; ++q) t += red[q * kCols + threadIdx.x];
  a.y[(size_t)cb * kCols + threadIdx.x] = (uint16_t)f32_to_bf16(t);
}

// XCD_REDUCE: the tiles of column block cb run as workgroups b with b % 8 ==
// cb / (col_blocks / 8) (col_blocks a multiple of 8), and the last tile of
// each column block writes its y (down_xcd_tail); otherwise tile (rb, cb)
// runs with b % 8 == rb % 8 and a reduce kernel follows.  IDENT: position j
// is row j (no id list: the every-row down of a dense layer), so the row
// loads do not wait for an id load.
template <bool XCD_REDUCE, bool IDENT>
__global__ __launch_bounds__(kThreads) void down_gm_kernel(DownGmArgs a) {
  DIP_STAMP_START(g_stamps_down);
  constexpr int LPR = 8, kSlots = kThreads / LPR, kCols = LPR * kDownAcc, kWaves = kThreads / 64;
  __shared__ __align__(16) float red[down_red_floats<LPR>()];
  __shared__ __align__(16) uint32_t xoff[kWaves][64];
  __shared__ __align__(16) float xcoef[kWaves][2][64];
  __shared__ uint32_t last;
  const int xcd = blockIdx.x % kXcds, w = blockIdx.x / kXcds;
  const int cpx = a.col_blocks / kXcds;
  const int rb = XCD_REDUCE ? w / cpx : xcd + kXcds * (w / a.col_blocks);
  const int cb = XCD_REDUCE ? xcd * cpx + w % cpx : w % a.col_blocks;
  if (rb >= a.row_blocks) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l = tid % LPR, slot = tid / LPR, sw = lane / LPR;
  const int cc0 = cb * LPR + l;
  const int g0 = cb * 2;
  const uint32_t row_bytes = (uint32_t)(a.out_features >> 1);
  const uint32_t lane_off = (uint32_t)cc0 * 16u;
  const int jl = rb * kRowsPerBlock + slot + l * kSlots;
  const bool live = jl < a.k;
  const uint32_t raw = IDENT ? (uint32_t)jl : (uint32_t)a.sel[min(jl, a.k - 1)];
  const uint32_t rid = !live ? kPadRow : (raw < (uint32_t)a.rows ? raw : kBadRow);
  const uint32_t r = rid >= kPadRow ? 0u : rid;  // bad and padding rows read row 0
  const uint32_t hb = a.h[r];
  uint32_t sv[2];
  sv[0] = a.sc_gm[(size_t)g0 * a.rows + r];
  sv[1] = a.sc_gm[(size_t)(g0 + 1) * a.rows + r];
  // the slot's row offsets through the per-wave exchange
  xoff[wave][lane] = r * row_bytes;
  __builtin_amdgcn_wave_barrier();
  const uint4 o0 = *reinterpret_cast<const uint4*>(&xoff[wave][sw * LPR]);
  const uint4 o1 = *reinterpret_cast<const uint4*>(&xoff[wave][sw * LPR + 4]);
  const uint32_t off[LPR] = {o0.x, o0.y, o0.z, o0.w, o1.x, o1.y, o1.z, o1.w};
  DownRow ring[LPR];
#pragma unroll
  for (int d = 0; d < LPR; ++d)
    ring[d].w = ldg_nt(reinterpret_cast<const uint4*>(a.qw + (size_t)(off[d] + lane_off)));
  if (a.h_out && cb == 0 && live) a.h_out[jl] = (uint16_t)hb;
  float f2[2];
  down_coef<2>(rid, hb, sv, f2);
  xcoef[wave][0][lane] = f2[0];
  xcoef[wave][1][lane] = f2[1];
  __builtin_amdgcn_wave_barrier();
  const int myg = l / kChunksPerGroup;
  const float4 c0 = *reinterpret_cast<const float4*>(&xcoef[wave][myg][sw * LPR]);
  const float4 c1 = *reinterpret_cast<const float4*>(&xcoef[wave][myg][sw * LPR + 4]);
  const float f[LPR] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
  float acc[kDownAcc];
#pragma unroll
  for (int m = 0; m < kDownAcc; ++m) acc[m] = 0.f;
  down_accumulate<LPR>(ring, f, acc);
  down_block_partial<LPR>(acc, red, a.partial + (size_t)rb * a.out_features + (size_t)cb * kCols);
  if constexpr (XCD_REDUCE) down_xcd_tail(a, cb, red, &last);
  DIP_STAMP_END(g_stamps_down);
}

// y[o] = bf16(sum over row blocks rb of partial[rb][o]), rb ascending in
// kRedSplit interleaved splits (split p sums rb = p, p+kRedSplit, ...), the
// splits then added in order.  A thread issues all its loads at once (NB per
// split; row blocks past row_blocks read a clamped address and are skipped).
template <int NB>
__global__ __launch_bounds__(kRedOut * kRedSplit) void down_reduce_kernel(
    const float* __restrict__ partial, int row_blocks, int out_features, uint16_t* __restrict__ y) {
  __shared__ float part[kRedSplit][kRedOut];
  DIP_STAMP_START(g_stamps_reduce);
  const int oo = threadIdx.x % kRedOut;
  const int p = threadIdx.x / kRedOut;
  const int o = min(blockIdx.x * kRedOut + oo, out_features - 1);
  float s = 0.f;
  for (int r0 = p; r0 < row_blocks; r0 += NB * kRedSplit) {
    float v[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int rb = min(r0 + u * kRedSplit, row_blocks - 1);
      v[u] = partial[(size_t)rb * out_features + o];
    }
#pragma unroll
    for (int u = 0; u < NB; ++u) s = r0 + u * kRedSplit < row_blocks ? s + v[u] : s;
  }
  part[p][oo] = s;
  __syncthreads();
  if (p == 0 && blockIdx.x * kRedOut + oo < out_features) {
    float t = part[0][oo];
#pragma unroll
    for (int q = 1; q < kRedSplit; ++q) t += part[q][oo];
    y[blockIdx.x * kRedOut + oo] = (uint16_t)f32_to_bf16(t);
  }
  DIP_STAMP_END(g_stamps_reduce);
}

// k == 0: y = bf16(0).
__global__ void down_zero_kernel(int out_features, uint16_t* __restrict__ y) {
  const int o = blockIdx.x * blockDim.x + threadIdx.x;
  if (o < out_features) y[o] = 0;
}

namespace {

uint64_t row_bytes_of(int64_t out_features) { return (uint64_t)(out_features / 2); }

// Lanes per row segment: 8 (128 B per row, 256 outputs per column block)
// wherever the width allows, else 4.
int down_lpr(int64_t out_features) {
  const int64_t chunks = out_features / kChunkCols;
  if (chunks % 8 == 0) return 8;
  if (chunks % 4 == 0) return 4;
  return 0;
}

void launch_reduce(const float* partial, int row_blocks, int out_features, uint16_t* y,
                   hipStream_t stream) {
  const unsigned blocks = (unsigned)((out_features + kRedOut - 1) / kRedOut);
  const dim3 threads(kRedOut * kRedSplit);
  const int per = (row_blocks + kRedSplit - 1) / kRedSplit;  // row blocks per split
  if (per <= 8)
    hipLaunchKernelGGL((down_reduce_kernel<8>), dim3(blocks), threads, 0, stream, partial,
                       row_blocks, out_features, y);
  else
    hipLaunchKernelGGL((down_reduce_kernel<16>), dim3(blocks), threads, 0, stream, partial,
                       row_blocks, out_features, y);
}

template <int LPR, int SL>
void launch_down(int src, bool off32, const DownArgs& a, int blocks, hipStream_t stream) {
  const dim3 grid(blocks), block(kThreads);
  if (src == kContig && off32)
    hipLaunchKernelGGL((down_kernel<LPR, kContig, SL, true>), grid, block, 0, stream, a);
  else if (src == kContig)
    hipLaunchKernelGGL((down_kernel<LPR, kContig, SL, false>), grid, block, 0, stream, a);
  else if (src == kGather && off32)
    hipLaunchKernelGGL((down_kernel<LPR, kGather, SL, true>), grid, block, 0, stream, a);
  else if (src == kGather)
    hipLaunchKernelGGL((down_kernel<LPR, kGather, SL, false>), grid, block, 0, stream, a);
  else if constexpr (SL != kScGm)
    hipLaunchKernelGGL((down_kernel<LPR, kDual, SL, false>), grid, block, 0, stream, a);
}

}  // namespace

int launch_down_reduce(const float* partial, int row_blocks, int out_features, uint16_t* y,
                       hipStream_t stream) {
  launch_reduce(partial, row_blocks, out_features, y, stream);
  return hip_status(hipGetLastError());
}

size_t down_workspace_bytes(int64_t k, int64_t out_features) {
  // the XCD-local reduce's arrival counters (kept zero between calls), then
  // one fp32 partial row of out_features per block of 256 selected positions
  if (out_features <= 0) return kDownCounterBytes + 256;
  const int64_t blocks = k > 0 ? (k + kRowsPerBlock - 1) / kRowsPerBlock : 1;
  return kDownCounterBytes + (size_t)blocks * (size_t)out_features * sizeof(float);
}

// The XCD-local reduce needs every tile of a column block on one XCD: a
// full 256-CU gfx950 (MI350X / MI355X: 8 XCDs of 32 CUs), whose dispatcher
// hands workgroup b to XCD (b + c) mod 8 for one c per launch.  Cached per
// device.
bool xcd_reduce_device() {
  static int cache[64] = {0};  // 0 unknown, 1 no, 2 yes
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
  if (!cache[dev]) {
    hipDeviceProp_t p{};
    const bool ok = hipGetDeviceProperties(&p, dev) == hipSuccess &&
                    strncmp(p.gcnArchName, "gfx950", 6) == 0 && p.multiProcessorCount == 256;
    cache[dev] = ok ? 2 : 1;
  }
  return cache[dev] == 2;
}

int64_t down_max_k() { return (int64_t)kMaxRowBlocks * kRowsPerBlock; }

int run_down(int src, const int8_t* qw_a, const uint16_t* sc_a, int64_t rows_a,
             const int8_t* qw_b, const uint16_t* sc_b, int64_t rows_b, const uint16_t* h,
             const int32_t* sel, const int32_t* sel2, int64_t k, int64_t out_features,
             uint16_t* y, void* workspace, size_t ws_bytes, hipStream_t stream, int h_by_row,
             uint16_t* h_out, const uint16_t* sc_gm) {
  if (!qw_a || !sc_a || !y) return DIP_ERR_NULL;
  if (out_features <= 0 || out_features % kGroupSize != 0 || out_features > (1 << 20))
    return DIP_ERR_SHAPE;
  // row ids stay below 2^31 - 2 so that B-tagged ids never reach kPadRow
  if (k < 0 || k > down_max_k() || rows_a < 0 || rows_a >= INT32_MAX - 1 ||
      rows_b >= INT32_MAX - 1)
    return DIP_ERR_SHAPE;
  if (!aligned16(qw_a) || (qw_b && !aligned16(qw_b))) return DIP_ERR_ALIGN;
  if (sc_gm && src == kDual) return DIP_ERR_ARG;
  if (k > 0 && !h) return DIP_ERR_NULL;
  if (k == 0) {
    hipLaunchKernelGGL(down_zero_kernel, dim3((unsigned)((out_features + 255) / 256)), dim3(256),
                       0, stream, (int)out_features, y);
    return hip_status(hipGetLastError());
  }
  if (rows_a == 0 && (src != kDual || rows_b <= 0)) return DIP_ERR_SHAPE;
  const int lpr = down_lpr(out_features);
  if (!lpr) return DIP_ERR_UNSUPPORTED;
  if (!workspace || ws_bytes < down_workspace_bytes(k, out_features)) return DIP_ERR_WORKSPACE;
  if (!aligned16(workspace)) return DIP_ERR_ALIGN;
  DownArgs a{};
  a.qw_a = qw_a;
  a.sc_a = sc_a;
  a.qw_b = qw_b;
  a.sc_b = sc_b;
  a.sc_gm = sc_gm;
  a.qw_safe = rows_a > 0 ? qw_a : qw_b;
  a.sc_safe = rows_a > 0 ? sc_a : sc_b;
  a.h = h;
  a.sel = sel;
  a.sel2 = sel2;
  a.partial = reinterpret_cast<float*>(static_cast<char*>(workspace) + kDownCounterBytes);
  a.h_out = h_out;
  a.h_by_row = h_by_row;
  a.rows_a = (int)rows_a;
  a.rows_b = (int)rows_b;
  a.k = (int)k;
  a.out_features = (int)out_features;
  a.col_blocks = (int)(out_features / (kChunkCols * lpr));
  a.row_blocks = (int)((k + kRowsPerBlock - 1) / kRowsPerBlock);
  const int blocks = (a.row_blocks + kXcds - 1) / kXcds * kXcds * a.col_blocks;
  // the scale pair of a slot is one 32-bit load when every scale matrix is
  // 4-byte aligned (rows of an even number of groups, pairs at even groups)
  const bool a4 = lpr == 8 && ((reinterpret_cast<uintptr_t>(sc_a) |
                                reinterpret_cast<uintptr_t>(sc_b)) & 3u) == 0;
  // one matrix whose every row offset fits 32 bits
  const bool off32 = src != kDual && (uint64_t)rows_a * row_bytes_of(out_features) <= 0xFFFFFFFFull;
  if (sc_gm && (src == kGather || src == kContig) && h_by_row && lpr == 8 && off32) {
    const bool ident = src == kContig;
    DownGmArgs g{};
    g.qw = qw_a;
    g.sc_gm = sc_gm;
    g.h = h;
    g.sel = sel;
    g.partial = a.partial;
    g.h_out = h_out;
    g.rows = a.rows_a;
    g.k = a.k;
    g.out_features = a.out_features;
    g.col_blocks = a.col_blocks;
    g.row_blocks = a.row_blocks;
    if (a.col_blocks % kXcds == 0 && a.col_blocks <= kMaxXcdColBlocks && xcd_reduce_device()) {
      g.counters = static_cast<uint32_t*>(workspace);
      g.y = y;
      const int xblocks = kXcds * (a.col_blocks / kXcds) * a.row_blocks;
      if (ident)
        hipLaunchKernelGGL((down_gm_kernel<true, true>), dim3(xblocks), dim3(kThreads), 0, stream, g);
      else
        hipLaunchKernelGGL((down_gm_kernel<true, false>), dim3(xblocks), dim3(kThreads), 0, stream, g);
      return hip_status(hipGetLastError());
    }
    if (ident)
      hipLaunchKernelGGL((down_gm_kernel<false, true>), dim3(blocks), dim3(kThreads), 0, stream, g);
    else
      hipLaunchKernelGGL((down_gm_kernel<false, false>), dim3(blocks), dim3(kThreads), 0, stream, g);
  } else if (sc_gm) {
    if (lpr == 8) launch_down<8, kScGm>(src, off32, a, blocks, stream);
    else launch_down<4, kScGm>(src, off32, a, blocks, stream);
  } else if (lpr == 8 && a4) {
    launch_down<8, kScRow4>(src, off32, a, blocks, stream);
  } else if (lpr == 8) {
    launch_down<8, kScRow>(src, off32, a, blocks, stream);
  } else {
    launch_down<4, kScRow>(src, off32, a, blocks, stream);
  }
  int st = hip_status(hipGetLastError());
  if (st) return st;
  launch_reduce(a.partial, a.row_blocks, (int)out_features, y, stream);
  return hip_status(hipGetLastError());
}

}  // namespace dip

using namespace dip;

extern "C" size_t dip_gather_down_workspace_size(int64_t k, int64_t out_features) {
  return down_workspace_bytes(k, out_features);
}

extern "C" int dip_int4_gather_down(const int8_t* down_t, const uint16_t* scales,
                                    const uint16_t* h, const int32_t* indices, uint16_t* y,
                                    int64_t rows, int64_t out_features, int64_t k,
                                    void* workspace, size_t ws_bytes, void* stream) {
  if (!indices && k > rows) return DIP_ERR_SHAPE;
  return run_down(indices ? kGather : kContig, down_t, scales, rows, nullptr, nullptr, 0, h,
                  indices, nullptr, k, out_features, y, workspace, ws_bytes,
                  (hipStream_t)stream);
}

extern "C" int dip_int4_gather_down_by_channel(const int8_t* down_t, const uint16_t* scales,
                                               const uint16_t* scales_gm,
                                               const uint16_t* h_full, const int32_t* indices,
                                               uint16_t* y, uint16_t* h_out, int64_t rows,
                                               int64_t out_features, int64_t k, void* workspace,
                                               size_t ws_bytes, void* stream) {
  if (!indices && k > rows) return DIP_ERR_SHAPE;
  return run_down(indices ? kGather : kContig, down_t, scales, rows, nullptr, nullptr, 0, h_full,
                  indices, nullptr,
                  k, out_features, y, workspace, ws_bytes, (hipStream_t)stream, 1, h_out,
                  scales_gm);
}

extern "C" int dip_ca_down(const int8_t* res_qw, const uint16_t* res_sc, const int8_t* str_qw,
                           const uint16_t* str_sc, const uint16_t* h, const int32_t* src,
                           const int32_t* row, uint16_t* y, int64_t res_rows, int64_t str_rows,
                           int64_t out_features, int64_t k, void* workspace, size_t ws_bytes,
                           void* stream) {
  if (!str_qw || !str_sc) return DIP_ERR_NULL;
  if (k > 0 && (!src || !row)) return DIP_ERR_NULL;
  return run_down(kDual, res_qw, res_sc, res_rows, str_qw, str_sc, str_rows, h, src, row, k,
                  out_features, y, workspace, ws_bytes, (hipStream_t)stream);
}
