// Allocation-free variant of the cached decode step (include/dilution_hip.h:
// dil_decode_step_noalloc).  It runs the kernels of dil_decode_step with their
// scratch (the per-key affinities and the per-chunk partials) in a file-scope
// device array instead of a caller-provided workspace, for callers that cannot
// allocate device memory: code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc.
//
//   * Every GPU the library runs on holds its own copy of `scratch`
//     (kNoAllocScratchBytes) until the process ends.
//   * The array's device address is looked up once per device, on the entry
//     point's first call with that device current (hipGetSymbolAddress), and
//     only that address is handed to the kernels: in host code the symbol
//     itself is a host-side stand-in, not a device address.  The address is
//     kept for the process; hipDeviceReset() reloads the module and
//     invalidates it, so the entry point is not for use on a device after a
//     reset.
//   * The decode kernels overwrite every scratch word they later read (the
//     affinities of keys [0, length), the statistics and partials of every
//     chunk), so nothing is cleared between calls and a call never sees the
//     previous call's contents.
//   * All calls on one GPU share that GPU's array: calls that overlap on one
//     GPU (on different streams, or from different host threads) race.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/dilution_hip.h"
#include "dil_internal.hpp"

namespace {

constexpr int64_t kNoAllocScratchBytes = DIL_NOALLOC_SCRATCH_BYTES;
static_assert(kNoAllocScratchBytes % 256 == 0, "scratch size must keep 256-byte alignment");

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up on the first
// call per device and kept).  Returns 0 or a status.
int scratch_on_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  if (dev < 0 || dev >= kMaxDevices) return static_cast<int>(hipErrorInvalidDevice);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return static_cast<int>(e);
    if (p == nullptr) return static_cast<int>(hipErrorInvalidSymbol);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

}  // namespace

extern "C" int dil_decode_step_noalloc(const void* q1, const void* k_cache, const void* v_cache,
                                       float* committed, void* out, int64_t n, int64_t capacity,
                                       int64_t length, int head_dim, int dtype, int q_dtype,
                                       void* stream) {
  if (!(head_dim == 16 || head_dim == 32 || head_dim == 64 || head_dim == 128 || head_dim == 256))
    return dil::kErrHeadDim;
  if (dtype < 0 || dtype > 2 || q_dtype < 0 || q_dtype > 2) return dil::kErrDtype;
  if (n < 1 || length < 1 || length > capacity) return dil::kErrShape;
  if (q1 == nullptr || k_cache == nullptr || v_cache == nullptr || committed == nullptr ||
      out == nullptr)
    return dil::kErrShape;
  const int64_t need = dil::decode_workspace_bytes(n, length, head_dim);
  if (need > kNoAllocScratchBytes) return dil::kErrScratch;
  void* ws = nullptr;
  if (const int st = scratch_on_current_device(&ws)) return st;
  dil::DecodeArgs a{};
  a.q1 = q1;
  a.q_sn = head_dim;
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.kv_sn = capacity * head_dim;
  a.committed = committed;
  a.c_sn = capacity;
  a.out = out;
  a.o_sn = head_dim;
  a.workspace = ws;
  a.workspace_bytes = kNoAllocScratchBytes;
  a.n = n;
  a.length = length;
  a.head_dim = head_dim;
  a.dtype = dtype;
  a.q_dtype = q_dtype;
  a.var = dil::Variant{};
  a.stream = stream;
  return dil::decode_step(a);
}
