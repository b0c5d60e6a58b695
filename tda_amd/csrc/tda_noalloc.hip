// tda_noalloc.hip -- tda_fwd_noalloc: the forward pass with its workspace taken from a fixed
// device array of this library instead of a caller buffer, for callers that cannot allocate
// device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc).  No counterpart in the reference.
//
// The array `scratch` (TDA_NOALLOC_SCRATCH_BYTES) is a file-scope __device__ variable: every GPU
// the library runs on holds its own copy, at its own address, until the process ends.  Its
// name is a host-side stand-in in host code; the device address comes from
// hipGetSymbolAddress, looked up once per device (with that device current) on the first call
// there, and is the only thing passed to the kernels.  Every call on a GPU shares that GPU's
// array, so calls that overlap on one GPU (different streams, different host threads without
// ordering) race.  The kernels initialise every workspace word they read (the bitmask and
// candidate words, the decode partials, the tile-pass queue count), so nothing is cleared
// between calls.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "../../include/tda.h"
#include "tda_params.hpp"

namespace {

constexpr size_t kScratchBytes = TDA_NOALLOC_SCRATCH_BYTES;
static_assert(kScratchBytes % 256 == 0, "scratch size must keep 256-byte granularity");

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_lock;
void* g_scratch[kMaxDevices];  // device address of `scratch` per device (null: not looked up)

// Device address of the current device's `scratch`, looked up on the first call on that device.
int32_t current_scratch(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    tda::record_hip_error((int)e);
    return TDA_ERR_HIP;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    tda::record_hip_error((int)hipErrorInvalidDevice);
    return TDA_ERR_HIP;
  }
  std::lock_guard<std::mutex> guard(g_lock);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      tda::record_hip_error(e != hipSuccess ? (int)e : (int)hipErrorInvalidSymbol);
      return TDA_ERR_HIP;
    }
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return TDA_OK;
}

}  // namespace

extern "C" int32_t tda_fwd_noalloc(const tda_fwd_args* a, void* stream) {
  if (!a) return TDA_ERR_NULL_POINTER;
  tda_fwd_args b = *a;
  const size_t need = tda_fwd_workspace_bytes_for(a);
  // every other argument is checked first, against a stand-in workspace that is never touched
  b.workspace = reinterpret_cast<void*>(uintptr_t(256));
  b.workspace_bytes = need;
  int32_t rc = tda_validate_fwd(&b);
  if (rc) return rc;
  if (need > kScratchBytes) return TDA_ERR_SCRATCH;
  void* ptr = nullptr;
  if ((rc = current_scratch(&ptr))) return rc;
  b.workspace = ptr;
  b.workspace_bytes = kScratchBytes;
  return tda_fwd(&b, stream);
}
