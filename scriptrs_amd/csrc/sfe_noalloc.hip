// Static device scratch for sfe_extract_chunks_noalloc, the entry point for
// callers that cannot allocate device memory.
//
// `scratch` is a file-scope device array: each GPU the library runs on holds
// its own copy, at its own address, from module load until the process ends.
// Its name in host code is only a host-side stand-in, so the device address
// is looked up once per device with hipGetSymbolAddress (with that device
// current) and only that address is passed to kernels and copies.
//
// Layout: [item table: kNoAllocItemBytes][raw log-mel: kNoAllocRawBytes].
// Every call on one GPU shares the array; the next call overwrites it, so
// calls that overlap on one GPU race (see the header).
#include <hip/hip_runtime.h>

#include <mutex>

#include "sfe_internal.hpp"

namespace sfe {

static_assert(kNoAllocItemBytes % 256 == 0, "raw region stays 256-byte aligned");
static __device__ __align__(256) unsigned char scratch[kNoAllocItemBytes + kNoAllocRawBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};

}  // namespace

hipError_t noalloc_scratch(int device, void** out) {
  *out = nullptr;
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_ptr[device]) {
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return e;
    if (cur != device && (e = hipSetDevice(device)) != hipSuccess) return e;
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != device) (void)hipSetDevice(cur);
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_ptr[device] = p;
  }
  *out = g_ptr[device];
  return hipSuccess;
}

}  // namespace sfe
