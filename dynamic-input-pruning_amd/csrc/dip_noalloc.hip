// dip_noalloc.hip — the resident DIP MLP decode step for callers that cannot
// allocate device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc).  It runs dip_mlp_decode's kernels with
// the step's workspace in a file-scope device array instead of a caller
// buffer.
//
// The array ("scratch") is one per GPU the library runs on and lives until
// the process ends.  In host code its name is only a host-side stand-in, so
// its device address is looked up once per device with hipGetSymbolAddress
// (the device current at the first call on it) and that pointer is what the
// kernels receive.  Every call on a GPU shares that GPU's array: calls that
// overlap on one GPU (different streams or threads) race on it.  Nothing in
// the workspace is read before the same call writes it (top-k state, h by
// channel, down partials), so no clearing is needed between calls.
#include <atomic>
#include <mutex>

#include "dip_internal.h"

namespace {

constexpr size_t kScratchBytes = DIP_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

// The device address of this device's scratch array (looked up on the first
// call with the device current).
int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return DIP_ERR_ARG;
  void* p = g_scratch[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (!p) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return (int)e;
      if (!p) return DIP_ERR_NULL;
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return DIP_OK;
}

}  // namespace

extern "C" int dip_mlp_decode_noalloc(const int8_t* gate_qw, const uint16_t* gate_sc,
                                      const int8_t* up_qw, const uint16_t* up_sc,
                                      const int8_t* down_t_qw, const uint16_t* down_t_sc,
                                      const uint16_t* down_t_sc_gm, const uint16_t* x,
                                      uint16_t* y, uint16_t* g_out, int32_t* idx_out, uint16_t* h_out, int64_t hidden,
                                      int64_t inter, int64_t k, void* layer_state,
                                      void* stream) {
  if (hidden < 0 || inter < 0 || k < 0) return DIP_ERR_SHAPE;
  if (dip_mlp_workspace_size(hidden, inter, k) > kScratchBytes) return DIP_ERR_SCRATCH;
  void* ws = nullptr;
  const int st = scratch_address(&ws);
  if (st) return st;
  return dip_mlp_decode(gate_qw, gate_sc, up_qw, up_sc, down_t_qw, down_t_sc, down_t_sc_gm, x, y,
                        g_out, idx_out, h_out, hidden, inter, k, ws, kScratchBytes, layer_state,
                        stream);
}
