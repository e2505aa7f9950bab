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
// Every call on one GPU shares the array: calls are serialised on the host
// by a per-device lock and ordered on the device by a per-device event, so
// calls from several contexts, threads or streams of one process do not
// race (calls from several processes on one GPU each have their own copy).
#include <hip/hip_runtime.h>

#include <mutex>

#include "sfe_internal.hpp"

namespace sfe {

static_assert(kNoAllocItemBytes % 256 == 0, "raw region stays 256-byte aligned");
static __device__ __align__(256) unsigned char scratch[kNoAllocItemBytes + kNoAllocRawBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;                    // guards the tables below
void* g_ptr[kMaxDevices] = {};
// Per device: the lock held through each call, and the end of the last call
// (an event recorded on its stream; created with the address lookup).
std::mutex g_call_mu[kMaxDevices];
hipEvent_t g_ev[kMaxDevices] = {};
bool g_has_last[kMaxDevices] = {};
hipStream_t g_last_stream[kMaxDevices] = {};

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
    hipEvent_t ev = nullptr;
    if (e == hipSuccess && p) e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (cur != device) (void)hipSetDevice(cur);
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_ptr[device] = p;
    g_ev[device] = ev;
  }
  *out = g_ptr[device];
  return hipSuccess;
}

hipError_t noalloc_lock(int device, std::unique_lock<std::mutex>* lock) {
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  *lock = std::unique_lock<std::mutex>(g_call_mu[device]);
  return hipSuccess;
}

hipError_t noalloc_order(int device, hipStream_t stream) {
  if (!g_has_last[device] || g_last_stream[device] == stream) return hipSuccess;
  return hipStreamWaitEvent(stream, g_ev[device], 0);
}

hipError_t noalloc_mark(int device, hipStream_t stream) {
  g_has_last[device] = false;
  if (!g_ev[device]) return hipErrorInvalidResourceHandle;
  hipError_t e = hipEventRecord(g_ev[device], stream);
  if (e != hipSuccess) return e;
  g_has_last[device] = true;
  g_last_stream[device] = stream;
  return hipSuccess;
}

}  // namespace sfe
