// dip_misc.hip — cache-aware hit/miss assembly, row dequantisation, the
// host-side miss gather, the one-call resident MLP decode step and the
// library's status helpers.
#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstring>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

#include "dip_common.h"
#include "dip_host_pool.h"
#include "dip_internal.h"

namespace dip {

// ---------------------------------------------------------------------------
// Cache-aware assembly (dip_ca.py:137-171).  One workgroup: each thread owns a
// contiguous segment of idx, counts its hits, a block scan gives every
// element its place in [hits in idx order, misses in idx order].
// ---------------------------------------------------------------------------
namespace {
constexpr int kAsmThreads = 1024;
constexpr int kAsmWaves = kAsmThreads / 64;

DIP_DEV uint32_t wave_prefix32(uint32_t v, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    uint32_t t = __shfl_up(v, d, 64);
    if (lane >= d) v += t;
  }
  return v;
}
}  // namespace

__global__ __launch_bounds__(kAsmThreads) void ca_assemble_kernel(
    const int64_t* __restrict__ id2slot, const int32_t* __restrict__ idx, int inter, int k,
    int32_t* __restrict__ combined, int32_t* __restrict__ src, int32_t* __restrict__ row,
    int32_t* __restrict__ miss_ids, int32_t* __restrict__ counts) {
  __shared__ uint32_t wave_excl[kAsmWaves];
  __shared__ uint32_t total_hits;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int per = (k + kAsmThreads - 1) / kAsmThreads;
  const int beg = min(k, tid * per);
  const int end = min(k, beg + per);

  uint32_t hits = 0;
  for (int j = beg; j < end; ++j) {
    const int c = idx[j];
    const int64_t s = ((unsigned)c < (unsigned)inter) ? id2slot[c] : -1;
    hits += s >= 0 ? 1u : 0u;
  }
  const uint32_t incl = wave_prefix32(hits, lane);
  if (lane == 63) wave_excl[wave] = incl;
  __syncthreads();
  if (wave == 0) {
    const uint32_t v = lane < kAsmWaves ? wave_excl[lane] : 0u;
    const uint32_t p = wave_prefix32(v, lane);
    if (lane < kAsmWaves) wave_excl[lane] = p - v;
    const uint32_t tot = __shfl(p, kAsmWaves - 1, 64);
    if (lane == 0) total_hits = tot;
  }
  __syncthreads();
  const uint32_t n_hit = total_hits;
  uint32_t hit_pos = wave_excl[wave] + incl - hits;  // hits before this segment
  for (int j = beg; j < end; ++j) {
    const int c = idx[j];
    const int64_t s = ((unsigned)c < (unsigned)inter) ? id2slot[c] : -1;
    if (s >= 0) {
      combined[hit_pos] = c;
      src[hit_pos] = 0;
      row[hit_pos] = (int32_t)s;
      ++hit_pos;
    } else {
      const uint32_t miss_rank = (uint32_t)j - hit_pos;  // misses before j
      const uint32_t pos = n_hit + miss_rank;
      combined[pos] = c;
      src[pos] = 1;
      row[pos] = (int32_t)miss_rank;
      miss_ids[miss_rank] = c;
    }
  }
  if (tid == 0) {
    counts[0] = (int32_t)n_hit;
    counts[1] = k - (int32_t)n_hit;
  }
}

// ---------------------------------------------------------------------------
// Row dequantisation (bit-exact dequant check).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void dequant_rows_kernel(
    const int8_t* __restrict__ qw, const uint16_t* __restrict__ sc,
    const int32_t* __restrict__ indices, void* __restrict__ out, int n_out_rows, int rows,
    int cols, int mode) {
  const int half = cols >> 1;
  const int ngroups = cols >> 7;
  const size_t total = (size_t)n_out_rows * half;
  for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < total;
       e += (size_t)gridDim.x * 256) {
    const int i = (int)(e / half);
    const int b = (int)(e % half);
    const int r = indices ? indices[i] : i;
    float v0, v1;
    if ((unsigned)r < (unsigned)rows) {
      const uint32_t byte = (uint8_t)qw[(size_t)r * half + b];
      const int q0 = (int)(byte & 0xFu) - (int)((byte & 0x8u) << 1);
      const int q1 = (int)(byte >> 4) - (int)((byte & 0x80u) >> 3);
      const float s = bf16_to_f32(sc[(size_t)r * ngroups + (2 * b) / kGroupSize]);
      v0 = (float)q0 * s;
      v1 = (float)q1 * s;
    } else {
      v0 = v1 = __builtin_nanf("");
    }
    const size_t o = (size_t)i * cols + 2 * (size_t)b;
    if (mode == 0) {
      reinterpret_cast<float*>(out)[o] = v0;
      reinterpret_cast<float*>(out)[o + 1] = v1;
    } else {
      reinterpret_cast<uint16_t*>(out)[o] = (uint16_t)f32_to_bf16(v0);
      reinterpret_cast<uint16_t*>(out)[o + 1] = (uint16_t)f32_to_bf16(v1);
    }
  }
}

}  // namespace dip

using namespace dip;

extern "C" const char* dip_status_string(int status) {
  switch (status) {
    case DIP_OK: return "ok";
    case DIP_ERR_NULL: return "a required pointer is NULL";
    case DIP_ERR_SHAPE: return "invalid or unsupported size";
    case DIP_ERR_ALIGN: return "pointer is not 16-byte aligned";
    case DIP_ERR_UNSUPPORTED: return "no kernel instantiation for this shape";
    case DIP_ERR_WORKSPACE: return "workspace missing or too small";
    case DIP_ERR_ARG: return "invalid argument";
    case DIP_ERR_SCRATCH: return "the shape needs more workspace than the no-alloc scratch holds";
    default: break;
  }
  if (status > 0) return hipGetErrorString((hipError_t)status);
  return "unknown status";
}

extern "C" int dip_version(void) { return DIP_VERSION; }

extern "C" int dip_timeline_read(int kernel, dip_wg_stamps* dst) {
  if (!dst) return DIP_ERR_NULL;
  if (kernel < DIP_STAMP_GATE || kernel > DIP_STAMP_REDUCE) return DIP_ERR_ARG;
#ifdef DIP_WG_STAMPS
  if (hipDeviceSynchronize() != hipSuccess) return hip_status(hipGetLastError());
#endif
  switch (kernel) {
    case DIP_STAMP_GATE: return timeline_read_rowdot(dst);
    case DIP_STAMP_TOPK: return timeline_read_topk(dst);
    case DIP_STAMP_DOWN: return timeline_read_down(0, dst);
    default: return timeline_read_down(1, dst);
  }
}

// ---------------------------------------------------------------------------
// Tuning table and device facts.
// ---------------------------------------------------------------------------
namespace {
int g_tune[DIP_TUNE_COUNT] = {0, 0, 8, 0, 1};  // [3]: not a knob
}  // namespace

int dip::tuning(int knob) { return g_tune[knob]; }

int dip::device_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cache[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

extern "C" int dip_set_tuning(int knob, int value) {
  switch (knob) {
    case DIP_TUNE_ROWDOT_WGS_PER_CU:
      if (value < 0 || value > 16) return DIP_ERR_ARG;
      break;
    case DIP_TUNE_TOPK_STAMPS:
      if (value != 0 && value != 1) return DIP_ERR_ARG;
      break;
    case DIP_TUNE_SPEC_MARGIN:
      if (value < 0 || value > 1024) return DIP_ERR_ARG;
      break;
    case DIP_TUNE_ROW_TIERS:
      if (value != 0 && value != 1) return DIP_ERR_ARG;
      break;
    default:
      return DIP_ERR_ARG;
  }
  g_tune[knob] = value;
  return DIP_OK;
}

extern "C" int dip_get_tuning(int knob) {
  if (knob < 0 || knob >= DIP_TUNE_COUNT || knob == 3) return DIP_ERR_ARG;
  return g_tune[knob];
}

extern "C" int dip_ca_assemble(const int64_t* id2slot, const int32_t* idx, int32_t* combined,
                               int32_t* src, int32_t* row, int32_t* miss_ids, int32_t* counts,
                               int64_t inter, int64_t k, void* stream) {
  if (inter < 0 || k < 0 || inter > INT32_MAX || k > INT32_MAX) return DIP_ERR_SHAPE;
  if (!counts || !id2slot) return DIP_ERR_NULL;
  if (k > 0 && (!idx || !combined || !src || !row || !miss_ids)) return DIP_ERR_NULL;
  hipLaunchKernelGGL(ca_assemble_kernel, dim3(1), dim3(kAsmThreads), 0, (hipStream_t)stream,
                     id2slot, idx, (int)inter, (int)k, combined, src, row, miss_ids, counts);
  return hip_status(hipGetLastError());
}

extern "C" int dip_dequant_rows(const int8_t* qweight, const uint16_t* scales,
                                const int32_t* indices, void* out, int64_t n_out_rows,
                                int64_t rows, int64_t cols, int mode, void* stream) {
  if (!qweight || !scales || !out) return DIP_ERR_NULL;
  if (cols <= 0 || cols % kGroupSize != 0 || rows < 0 || n_out_rows < 0 ||
      rows > INT32_MAX || n_out_rows > INT32_MAX)
    return DIP_ERR_SHAPE;
  if (!indices && n_out_rows > rows) return DIP_ERR_SHAPE;
  if (mode != 0 && mode != 1) return DIP_ERR_ARG;
  if (n_out_rows == 0) return DIP_OK;
  const size_t total = (size_t)n_out_rows * (size_t)(cols / 2);
  const unsigned blocks = (unsigned)std::min<size_t>((total + 255) / 256, 4096);
  hipLaunchKernelGGL(dequant_rows_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                     qweight, scales, indices, out, (int)n_out_rows, (int)rows, (int)cols, mode);
  return hip_status(hipGetLastError());
}

// ---------------------------------------------------------------------------
// Host-side miss gather (the pinned index_select of dip_ca.py:148-153) on the
// persistent host thread pool of dip_host_pool.h.
// ---------------------------------------------------------------------------
namespace {

int check_pieces(int npieces, const void* const* src, void* const* dst, const int64_t* row_bytes,
                 const int32_t* ids, int64_t n, int64_t src_rows) {
  if (n < 0 || src_rows < 0 || npieces < 0 || npieces > 64) return DIP_ERR_SHAPE;
  if (n == 0 || npieces == 0) return DIP_OK;
  if (!ids || !src || !dst || !row_bytes) return DIP_ERR_NULL;
  for (int p = 0; p < npieces; ++p) {
    if (row_bytes[p] < 0) return DIP_ERR_SHAPE;
    if (row_bytes[p] > 0 && (!src[p] || !dst[p])) return DIP_ERR_NULL;
  }
  for (int64_t i = 0; i < n; ++i)
    if (ids[i] < 0 || ids[i] >= src_rows) return DIP_ERR_SHAPE;
  return DIP_OK;
}

// dst_p[i] = src_p[ids[i]] for every piece p and i in [b, e).
void copy_rows(int npieces, const void* const* src, void* const* dst, const int64_t* row_bytes,
               const int32_t* ids, int64_t b, int64_t e) {
  for (int p = 0; p < npieces; ++p) {
    const int64_t rb = row_bytes[p];
    const char* s = static_cast<const char*>(src[p]);
    char* d = static_cast<char*>(dst[p]);
    for (int64_t i = b; i < e; ++i) std::memcpy(d + i * rb, s + (int64_t)ids[i] * rb, (size_t)rb);
  }
}

int pool_threads(int threads, int64_t n) {
  int nt = std::max(1, std::min(threads, 64));
  return (int)std::min<int64_t>(nt, n);
}

int gather_rows(int npieces, const void* const* src, void* const* dst, const int64_t* row_bytes,
                const int32_t* ids, int64_t n, int64_t src_rows, int threads) {
  const int st = check_pieces(npieces, src, dst, row_bytes, ids, n, src_rows);
  if (st || n == 0 || npieces == 0) return st;
  const int nt = pool_threads(threads, n);
  const int64_t per = (n + nt - 1) / nt;
  auto work = [&](int t) {
    copy_rows(npieces, src, dst, row_bytes, ids, std::min(n, t * per), std::min(n, (t + 1) * per));
  };
  if (nt == 1)
    work(0);
  else
    HostPool::get().run(nt, work);
  return DIP_OK;
}

}  // namespace

extern "C" int dip_host_gather_rows(const void* src, const int32_t* ids, void* dst, int64_t n,
                                    int64_t row_bytes, int64_t src_rows, int threads) {
  return gather_rows(1, &src, &dst, &row_bytes, ids, n, src_rows, threads);
}

extern "C" int dip_host_gather_rows_multi(const void* const* src, void* const* dst,
                                          const int64_t* row_bytes, int64_t npieces,
                                          const int32_t* ids, int64_t n, int64_t src_rows,
                                          int threads) {
  if (npieces < 0 || npieces > 64) return DIP_ERR_SHAPE;
  return gather_rows((int)npieces, src, dst, row_bytes, ids, n, src_rows, threads);
}

namespace {

// The miss stream's second copy stream on the current device and the events
// that fork it from and join it to the caller's stream (created on first
// use, kept for the life of the process; default priority).
struct SideStream {
  hipStream_t stream = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};

int side_stream(SideStream** out) {
  static SideStream table[64];
  static std::mutex mu;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= 64) return DIP_ERR_ARG;
  std::lock_guard<std::mutex> lock(mu);
  SideStream& t = table[dev];
  if (!t.stream) {
    e = hipStreamCreateWithFlags(&t.stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&t.fork, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&t.join, hipEventDisableTiming);
    if (e != hipSuccess) {
      if (t.fork) (void)hipEventDestroy(t.fork);
      if (t.stream) (void)hipStreamDestroy(t.stream);
      t = SideStream{};
      return (int)e;
    }
  }
  *out = &t;
  return DIP_OK;
}

}  // namespace

extern "C" int dip_host_stream_rows(const void* const* src, void* const* pinned,
                                    void* const* dst, const int64_t* row_bytes, int64_t npieces,
                                    const int32_t* ids, int64_t n, int64_t src_rows,
                                    int64_t chunk_rows, int threads, void* stream,
                                    float* copy_ms) {
  if (copy_ms) *copy_ms = 0.f;
  if (chunk_rows <= 0) return DIP_ERR_ARG;
  int st = check_pieces((int)npieces, src, pinned, row_bytes, ids, n, src_rows);
  if (st) return st;
  st = check_pieces((int)npieces, pinned, dst, row_bytes, ids, n, src_rows);
  if (st || n == 0 || npieces == 0) return st;
  const int np = (int)npieces;
  // Chunk c covers rows [cut[c], cut[c + 1]).  The first chunks ramp up from
  // chunk_rows / 8, doubling, so the first copy starts after a short gather
  // instead of a whole chunk's; the rest are chunk_rows.
  std::vector<int64_t> cut{0};
  for (int64_t c = std::max<int64_t>(chunk_rows / 8, 1); cut.back() < n;
       c = std::min(chunk_rows, 2 * c))
    cut.push_back(std::min(n, cut.back() + c));
  const int64_t nchunks = (int64_t)cut.size() - 1;
  const int nt = std::min(pool_threads(threads, chunk_rows), HostPool::max_async_jobs());
  hipStream_t s = (hipStream_t)stream;
  // Pieces [0, np/2) are copied on the caller's stream, the rest on a side
  // stream, so two DMA engines share each chunk; the caller's stream waits
  // for the side stream before the call returns.
  // (without it, as without a device, the gather still runs to the end and
  // the call returns the error, as for a failed copy)
  SideStream* side = nullptr;
  const int st_side = side_stream(&side);
  hipStream_t ss = side ? side->stream : nullptr;
  const int np0 = np / 2 > 0 ? np / 2 : np;  // one piece: the caller's stream alone
  std::vector<hipEvent_t> ev;
  if (copy_ms && st_side == DIP_OK) {
    ev.assign(4 * nchunks, nullptr);
    for (auto& e : ev)
      if (hipEventCreate(&e) != hipSuccess) {
        for (auto& e2 : ev)
          if (e2) (void)hipEventDestroy(e2);
        return hip_status(hipGetLastError());
      }
  }
  // The pool's threads only gather (left[c]: their slices of chunk c not yet
  // gathered); this thread queues each chunk's copies as soon as it is
  // complete, so every HIP call stays on the caller's thread.
  std::vector<std::atomic<int>> left(nchunks);
  for (auto& l : left) l.store(nt, std::memory_order_relaxed);
  // a named std::function: the workers call it until pool.finish() returns
  const std::function<void(int)> work = [&](int t) {
    for (int64_t c = 0; c < nchunks; ++c) {
      const int64_t c0 = cut[c], c1 = cut[c + 1];
      const int64_t per = (c1 - c0 + nt - 1) / nt;
      copy_rows(np, src, pinned, row_bytes, ids, std::min(c1, c0 + t * per),
                std::min(c1, c0 + (t + 1) * per));
      left[c].fetch_sub(1, std::memory_order_release);
    }
  };
  const bool copies = st_side == DIP_OK;
  hipError_t e = hipSuccess;
  HostPool& pool = HostPool::get();
  // Callers run one at a time from start() to finish(), so the side stream
  // and its two events serve one call at a time.
  pool.start(nt, &work);
  // the side stream starts after the work already queued on the caller's
  if (copies) {
    e = hipEventRecord(side->fork, s);
    if (e == hipSuccess) e = hipStreamWaitEvent(ss, side->fork, 0);
  }
  for (int64_t c = 0; c < nchunks; ++c) {
    while (left[c].load(std::memory_order_acquire) != 0) std::this_thread::yield();
    // let the gather finish; report the first error
    if (!copies || e != hipSuccess) continue;
    const int64_t c0 = cut[c], c1 = cut[c + 1];
    if (copy_ms) e = hipEventRecord(ev[4 * c], s);
    if (copy_ms && e == hipSuccess) e = hipEventRecord(ev[4 * c + 2], ss);
    for (int p = 0; p < np && e == hipSuccess; ++p) {
      const int64_t rb = row_bytes[p];
      if (rb == 0) continue;
      e = hipMemcpyAsync(static_cast<char*>(dst[p]) + c0 * rb,
                         static_cast<const char*>(pinned[p]) + c0 * rb,
                         (size_t)((c1 - c0) * rb), hipMemcpyHostToDevice, p < np0 ? s : ss);
    }
    if (copy_ms && e == hipSuccess) e = hipEventRecord(ev[4 * c + 1], s);
    if (copy_ms && e == hipSuccess) e = hipEventRecord(ev[4 * c + 3], ss);
  }
  if (copies && e == hipSuccess) e = hipEventRecord(side->join, ss);
  if (copies && e == hipSuccess) e = hipStreamWaitEvent(s, side->join, 0);
  pool.finish();
  st = !copies ? st_side : (e == hipSuccess ? DIP_OK : (int)e);
  if (copy_ms && copies) {
    // a chunk's copy time: the longer of its two streams' spans
    float total = 0.f;
    if (!st) {
      for (int64_t c = 0; c < nchunks && !st; ++c) {
        float ms[2] = {0.f, 0.f};
        for (int k = 0; k < 2 && !st; ++k) {
          hipError_t e2 = hipEventSynchronize(ev[4 * c + 2 * k + 1]);
          if (e2 == hipSuccess) e2 = hipEventElapsedTime(&ms[k], ev[4 * c + 2 * k],
                                                         ev[4 * c + 2 * k + 1]);
          if (e2 != hipSuccess) st = (int)e2;
        }
        total += std::max(ms[0], ms[1]);
      }
    }
    for (auto& ev1 : ev) (void)hipEventDestroy(ev1);
    *copy_ms = total;
  }
  return st;
}

// ---------------------------------------------------------------------------
// One resident DIP MLP decode step.
//   workspace: [0, 512) top-k state | the down workspace (the XCD-local
//   reduce's counters at a fixed offset, then the partials) | h by channel
//   [inter] bf16
// ---------------------------------------------------------------------------
namespace {
constexpr size_t kMlpTopkBytes = 512;
static_assert(kTopkWorkspace <= kMlpTopkBytes, "top-k state");
size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }
}  // namespace

extern "C" size_t dip_mlp_workspace_size(int64_t hidden, int64_t inter, int64_t k) {
  const size_t hfull = inter > 0 ? align256((size_t)inter * sizeof(uint16_t)) : 0;
  return kMlpTopkBytes + align256(down_workspace_bytes(k, hidden)) + hfull;
}

extern "C" int dip_mlp_decode_rmsnorm(const int8_t* gate_qw, const uint16_t* gate_sc,
                                      const int8_t* up_qw, const uint16_t* up_sc,
                                      const int8_t* down_t_qw, const uint16_t* down_t_sc,
                                      const uint16_t* down_t_sc_gm, const uint16_t* h,
                                      const uint16_t* add, const uint16_t* norm_w, float eps, uint16_t* h_res_out,
                                      uint16_t* x_out, uint16_t* y, uint16_t* g_out,
                                      int32_t* idx_out, uint16_t* h_out, int64_t hidden,
                                      int64_t inter, int64_t k, void* workspace, size_t ws_bytes,
                                      void* layer_state, void* stream) {
  if (!gate_qw || !gate_sc || !up_qw || !up_sc || !h || !norm_w || !x_out || !g_out || !y)
    return DIP_ERR_NULL;
  if (k < 0 || k > inter || inter <= 0 || inter > INT32_MAX) return DIP_ERR_SHAPE;
  if (k > 0 && (!idx_out || !h_out)) return DIP_ERR_NULL;
  if (!rowdot_norm_supported(hidden)) return DIP_ERR_UNSUPPORTED;
  if (!(eps >= 0.f)) return DIP_ERR_ARG;
  if (!aligned16(gate_qw) || !aligned16(up_qw) || !aligned16(h) || !aligned16(norm_w) ||
      !aligned16(x_out) || !aligned16(g_out) || (add && !aligned16(add)) ||
      (h_res_out && !aligned16(h_res_out)))
    return DIP_ERR_ALIGN;
  // every workgroup of the gate reads h and add while workgroup 0 writes
  // the residual and x
  if (x_out == h || x_out == add || (h_res_out && (h_res_out == h || h_res_out == add)))
    return DIP_ERR_ARG;
  if (!workspace || ws_bytes < dip_mlp_workspace_size(hidden, inter, k)) return DIP_ERR_WORKSPACE;
  if (!aligned16(workspace)) return DIP_ERR_ALIGN;
  char* ws = static_cast<char*>(workspace);
  char* down_ws = ws + kMlpTopkBytes;
  const size_t down_bytes = align256(down_workspace_bytes(k, hidden));
  uint16_t* h_full = reinterpret_cast<uint16_t*>(down_ws + down_bytes);
  hipStream_t s = (hipStream_t)stream;
  RowdotArgs a{};
  a.qw_a = gate_qw;
  a.sc_a = gate_sc;
  a.qw_safe = gate_qw;
  a.sc_safe = gate_sc;
  a.x = h;
  a.out = g_out;
  a.nrows = (int)inter;
  a.in_features = (int)hidden;
  a.rows_a = (int)inter;
  a.norm_w = norm_w;
  a.norm_add = add;
  a.norm_h_out = h_res_out;
  a.norm_x_out = x_out;
  a.norm_eps = eps;
  const bool spec = layer_state && k > 0 && topk_spec_supported(hidden) && inter <= kTopkMaxN;
  if (spec) {
    if (reinterpret_cast<uintptr_t>(layer_state) & 3u) return DIP_ERR_ALIGN;
    a.rotate = static_cast<uint32_t*>(layer_state);
    int st = launch_rowdot_norm(kSilu, a, s);
    if (st) return st;
    st = launch_spec_after_gate(g_out, inter, hidden, k, idx_out, h_full, up_qw, up_sc, x_out, ws,
                                layer_state, s);
    if (st) return st;
    return dip_int4_gather_down_by_channel(down_t_qw, down_t_sc, down_t_sc_gm, h_full, idx_out,
                                           y, h_out, inter, hidden, k, down_ws, down_bytes,
                                           stream);
  }
  int st = launch_rowdot_norm(kSilu, a, s);
  if (st) return st;
  st = dip_topk_select(g_out, idx_out, inter, k, ws, kMlpTopkBytes, stream);
  if (st) return st;
  if (k > 0) {
    st = dip_up_gather_h(up_qw, up_sc, x_out, idx_out, g_out, h_out, inter, hidden, k, stream);
    if (st) return st;
  }
  return run_down(kGather, down_t_qw, down_t_sc, inter, nullptr, nullptr, 0, h_out, idx_out,
                  nullptr, k, hidden, y, down_ws, down_bytes, (hipStream_t)stream, 0, nullptr,
                  down_t_sc_gm);
}

extern "C" int dip_mlp_decode(const int8_t* gate_qw, const uint16_t* gate_sc,
                              const int8_t* up_qw, const uint16_t* up_sc,
                              const int8_t* down_t_qw, const uint16_t* down_t_sc,
                              const uint16_t* down_t_sc_gm, const uint16_t* x, uint16_t* y,
                              uint16_t* g_out, int32_t* idx_out, uint16_t* h_out, int64_t hidden, int64_t inter, int64_t k,
                              void* workspace, size_t ws_bytes, void* layer_state,
                              void* stream) {
  if (!g_out || !y || !x) return DIP_ERR_NULL;
  if (k < 0 || k > inter) return DIP_ERR_SHAPE;
  if (k > 0 && (!idx_out || !h_out)) return DIP_ERR_NULL;
  if (!workspace || ws_bytes < dip_mlp_workspace_size(hidden, inter, k)) return DIP_ERR_WORKSPACE;
  char* ws = static_cast<char*>(workspace);
  char* down_ws = ws + kMlpTopkBytes;
  const size_t down_bytes = align256(down_workspace_bytes(k, hidden));
  uint16_t* h_full = reinterpret_cast<uint16_t*>(down_ws + down_bytes);
  if (layer_state && k > 0 && topk_spec_supported(hidden) && inter <= kTopkMaxN) {
    int st = dip_gate_silu_topk_spec(gate_qw, gate_sc, up_qw, up_sc, x, g_out, idx_out, h_full,
                                     inter, hidden, k, ws, kMlpTopkBytes, layer_state, stream);
    if (st) return st;
    return dip_int4_gather_down_by_channel(down_t_qw, down_t_sc, down_t_sc_gm, h_full, idx_out,
                                           y, h_out, inter, hidden, k, down_ws, down_bytes,
                                           stream);
  }
  int st = dip_gate_silu_topk(gate_qw, gate_sc, x, g_out, idx_out, inter, hidden, k, ws,
                              kMlpTopkBytes, stream);
  if (st) return st;
  if (k > 0) {
    st = dip_up_gather_h(up_qw, up_sc, x, idx_out, g_out, h_out, inter, hidden, k, stream);
    if (st) return st;
  }
  return run_down(kGather, down_t_qw, down_t_sc, inter, nullptr, nullptr, 0, h_out, idx_out,
                  nullptr, k, hidden, y, down_ws, down_bytes, (hipStream_t)stream, 0, nullptr,
                  down_t_sc_gm);
}
