// dip_probe.hip — libdip_probe.so, the bench's read-ceiling probes (not part
// of libdip_hip.so and not declared in dip_hip.h: nothing on the decode path
// calls them).  They measure the read bandwidth this GPU gives the two access
// patterns of the decode step, with no arithmetic beyond folding the loaded
// words (so the loads are not optimised away):
//   * contiguous: one buffer read front to back, grid-stride, each thread
//     RING 16-byte non-temporal loads in flight (the gate's pattern: whole
//     rows of one matrix);
//   * gathered: k rows picked by a sorted index list (the up/down rows of the
//     selected channels), each row read whole by one 32-lane group (row_bytes
//     / 512 load instructions of 512 bytes, the up rows' layout), RING rows
//     in flight per group; group q of the grid takes list positions q, q +
//     groups, ...
// Both take the grid size and the ring depth as arguments, so a sweep can
// vary the bytes in flight.  A sink word is written only if the folded value
// hits a fixed constant (practically never), which keeps every load live.
//
// C ABI (bench.py --ceiling binds these through ctypes):
//   int dip_probe_read(const void* src, size_t bytes, int wgs, int ring,
//                      uint32_t* sink, void* stream);
//   int dip_probe_gather(const void* rows, int64_t nrows, int64_t row_bytes,
//                        const int32_t* idx, int64_t k, int wgs, int ring,
//                        uint32_t* sink, void* stream);
// ring in {1, 2, 4, 8}; wgs in [1, 65536]; row_bytes a multiple of 512 up to
// 4096; idx entries outside [0, nrows) read row 0.  Returns 0 or a negative
// argument code (-1 null pointer, -2 size, -3 alignment, -6 other argument),
// or a positive hipError_t from the launch.
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace {

constexpr uint32_t kMagic = 0x9E3779B9u;
constexpr int kThreads = 256;
constexpr int kLanes = 32;      // one row per 32-lane group
constexpr int kMaxChunks = 8;   // 16-byte chunks per lane: rows up to 4096 B

__device__ __forceinline__ uint4 ldg_nt(const uint4* p) {
  uint4 v;
  v.x = __builtin_nontemporal_load(&p->x);
  v.y = __builtin_nontemporal_load(&p->y);
  v.z = __builtin_nontemporal_load(&p->z);
  v.w = __builtin_nontemporal_load(&p->w);
  return v;
}

template <int RING>
__global__ __launch_bounds__(kThreads) void read_kernel(const uint4* __restrict__ p, size_t n16,
                                                        uint32_t* sink) {
  const size_t nt = (size_t)gridDim.x * blockDim.x;
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  uint32_t acc = 0;
  for (; i + (RING - 1) * nt < n16; i += RING * nt) {
    uint4 v[RING];
#pragma unroll
    for (int u = 0; u < RING; ++u) v[u] = ldg_nt(p + i + u * nt);
#pragma unroll
    for (int u = 0; u < RING; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; i < n16; i += nt) {
    const uint4 v = ldg_nt(p + i);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == kMagic) sink[0] = acc;
}

// CH chunks of 16 bytes per lane: rows of 512 * CH bytes.
template <int RING, int CH>
__global__ __launch_bounds__(kThreads) void gather_kernel(const uint4* __restrict__ m,
                                                          const int32_t* __restrict__ idx,
                                                          int nrows, int k, uint32_t* sink) {
  const int groups = gridDim.x * (kThreads / kLanes);
  const int grp = blockIdx.x * (kThreads / kLanes) + threadIdx.x / kLanes;
  const int l = threadIdx.x % kLanes;
  if (grp >= k) return;  // no rows: nothing to load (uniform within the group)
  const int n = (k - grp + groups - 1) / groups;  // my rows, >= 1
  auto row_at = [&](int i) {  // my i-th row, clamped to my last one
    const int v = idx[grp + groups * min(i, n - 1)];
    return (unsigned)v < (unsigned)nrows ? v : 0;
  };
  uint32_t acc = 0;
  uint4 ring[RING][CH];
  auto load = [&](int i, int d) {
    const uint4* r = m + (size_t)row_at(i) * (kLanes * CH) + l;
#pragma unroll
    for (int c = 0; c < CH; ++c) ring[d][c] = ldg_nt(r + kLanes * c);
  };
#pragma unroll
  for (int d = 0; d < RING; ++d) load(d, d);
  const int rounds = (n + RING - 1) / RING;
  for (int r = 0; r + 1 < rounds; ++r) {
#pragma unroll
    for (int d = 0; d < RING; ++d) {
#pragma unroll
      for (int c = 0; c < CH; ++c) acc ^= ring[d][c].x ^ ring[d][c].y ^ ring[d][c].z ^ ring[d][c].w;
      load((r + 1) * RING + d, d);
    }
  }
#pragma unroll
  for (int d = 0; d < RING; ++d)
#pragma unroll
    for (int c = 0; c < CH; ++c) acc ^= ring[d][c].x ^ ring[d][c].y ^ ring[d][c].z ^ ring[d][c].w;
  if (acc == kMagic) sink[0] = acc;
}

int status(hipError_t e) { return e == hipSuccess ? 0 : (int)e; }
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <int RING>
void launch_gather(int ch, dim3 grid, hipStream_t s, const uint4* m, const int32_t* idx, int nrows,
                   int k, uint32_t* sink) {
  switch (ch) {
#define DIP_CH(C) \
    case C: hipLaunchKernelGGL((gather_kernel<RING, C>), grid, dim3(kThreads), 0, s, m, idx, nrows, k, sink); break;
    DIP_CH(1) DIP_CH(2) DIP_CH(3) DIP_CH(4) DIP_CH(5) DIP_CH(6) DIP_CH(7) DIP_CH(8)
#undef DIP_CH
    default: break;
  }
}

}  // namespace

extern "C" int dip_probe_read(const void* src, size_t bytes, int wgs, int ring, uint32_t* sink,
                              void* stream) {
  if (!src || !sink) return -1;
  if (bytes == 0 || bytes % 16 != 0) return -2;
  if (!aligned16(src)) return -3;
  if (wgs < 1 || wgs > 65536) return -6;
  const dim3 grid((unsigned)wgs);
  hipStream_t s = (hipStream_t)stream;
  const uint4* p = static_cast<const uint4*>(src);
  switch (ring) {
    case 1: hipLaunchKernelGGL(read_kernel<1>, grid, dim3(kThreads), 0, s, p, bytes / 16, sink); break;
    case 2: hipLaunchKernelGGL(read_kernel<2>, grid, dim3(kThreads), 0, s, p, bytes / 16, sink); break;
    case 4: hipLaunchKernelGGL(read_kernel<4>, grid, dim3(kThreads), 0, s, p, bytes / 16, sink); break;
    case 8: hipLaunchKernelGGL(read_kernel<8>, grid, dim3(kThreads), 0, s, p, bytes / 16, sink); break;
    default: return -6;
  }
  return status(hipGetLastError());
}

extern "C" int dip_probe_gather(const void* rows, int64_t nrows, int64_t row_bytes,
                                const int32_t* idx, int64_t k, int wgs, int ring, uint32_t* sink,
                                void* stream) {
  if (!rows || !idx || !sink) return -1;
  if (nrows <= 0 || k <= 0 || k > INT32_MAX || nrows > INT32_MAX) return -2;
  if (row_bytes <= 0 || row_bytes % (16 * kLanes) != 0 || row_bytes > 16 * kLanes * kMaxChunks)
    return -2;
  if (!aligned16(rows)) return -3;
  if (wgs < 1 || wgs > 65536) return -6;
  const int ch = (int)(row_bytes / (16 * kLanes));
  const dim3 grid((unsigned)wgs);
  hipStream_t s = (hipStream_t)stream;
  const uint4* m = static_cast<const uint4*>(rows);
  switch (ring) {
    case 1: launch_gather<1>(ch, grid, s, m, idx, (int)nrows, (int)k, sink); break;
    case 2: launch_gather<2>(ch, grid, s, m, idx, (int)nrows, (int)k, sink); break;
    case 4: launch_gather<4>(ch, grid, s, m, idx, (int)nrows, (int)k, sink); break;
    case 8: launch_gather<8>(ch, grid, s, m, idx, (int)nrows, (int)k, sink); break;
    default: return -6;
  }
  return status(hipGetLastError());
}
