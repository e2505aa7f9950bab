// Silero VAD model-input framing on the GPU.
//
// The reference's VAD loop (src/long_form/vad.rs:62-99) walks the recording
// in 512-sample windows (VAD_WINDOW_SAMPLES, src/constants.rs) and feeds the
// model [64 context | 512 window] = 576 samples per window.  The context is
// zero for the first window and the last 64 samples of the previous window
// otherwise; a short last window is padded with its own last sample.  Every
// window but the last is full, so the previous window's tail is plain
// recording, and the whole sequence of model inputs is one gather:
//
//   out[w][p] = x(512 w - 64 + p),  p in [0, 576),
//   x(i) = 0 for i < 0, recording[min(i, len - 1)] otherwise.
//
// The kernel writes that [n_windows][576] f32 array (the model's input
// tensors back to back), decoding integer PCM on the fly.  It moves
// 4 B/sample in (f32; 2 for 16-bit PCM) and 4.5 B/sample out, and is bound
// by HBM bandwidth: no arithmetic beyond the decode.  The 64-sample context
// re-read hits L2 (the neighbouring window is read by the same workgroup).

#include <hip/hip_runtime.h>

#include <cstdint>

#include "sfe_internal.hpp"
#include "sfe_pcm.hpp"

namespace sfe {
namespace {

constexpr int kVadRowVec = kVadRow / 4;   // 144 float4 per model input
constexpr int kVadThreads = 256;
constexpr int kVadRowsPerBlock = 16;
constexpr int kVadVecPerThread = kVadRowsPerBlock * kVadRowVec / kVadThreads;  // 9
static_assert(kVadRowsPerBlock * kVadRowVec % kVadThreads == 0, "whole float4s per thread");
static_assert(kVadCtx % 4 == 0 && kVadWin % 4 == 0, "rows start on float4 boundaries of the recording");


template <typename S>
__device__ __forceinline__ float vad_sample(const S* x, int64_t len, int64_t i, const Decode& d) {
  if (i < 0) return 0.0f;
  return Pcm<S>::dec(x[i < len ? i : len - 1], d);
}

// One workgroup writes kVadRowsPerBlock model inputs; thread t handles the
// float4s t, t + 256, ... of the block's rows, so a wave's loads and stores
// are contiguous except across a row boundary.  All loads are issued before
// the first store.
template <typename S>
__global__ __launch_bounds__(kVadThreads) void sfe_vad_frames_kernel(const S* __restrict__ x, int64_t len,
                                                                     int64_t n_windows, Decode dc,
                                                                     float* __restrict__ out) {
  const int64_t row0 = (int64_t)blockIdx.x * kVadRowsPerBlock;
  float4 v[kVadVecPerThread];
  int64_t dst[kVadVecPerThread];
#pragma unroll
  for (int k = 0; k < kVadVecPerThread; ++k) {
    const int e = (int)threadIdx.x + kVadThreads * k;  // float4 index in the block
    const int r = e / kVadRowVec;
    const int p = 4 * (e - r * kVadRowVec);
    const int64_t w = row0 + r;
    const int64_t i = w * kVadWin - kVadCtx + p;
    dst[k] = w < n_windows ? w * kVadRow + p : -1;
    if (i >= 0 && i + 4 <= len) {
      v[k] = Pcm<S>::dec4(Pcm<S>::load4(x + i), dc);
    } else {
      v[k] = make_float4(vad_sample(x, len, i, dc), vad_sample(x, len, i + 1, dc), vad_sample(x, len, i + 2, dc),
                         vad_sample(x, len, i + 3, dc));
    }
  }
  // Nontemporal stores: the output is not read again by this kernel, and
  // streaming it past the caches measured 73 us against 96 us for plain
  // stores on the 1 h recording.
  typedef float F4 __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int k = 0; k < kVadVecPerThread; ++k)
    if (dst[k] >= 0) {
      const F4 t = {v[k].x, v[k].y, v[k].z, v[k].w};
      __builtin_nontemporal_store(t, reinterpret_cast<F4*>(out + dst[k]));
    }
}

}  // namespace

int64_t vad_num_windows(int64_t len) { return len <= 0 ? 0 : (len + kVadWin - 1) / kVadWin; }

hipError_t launch_vad_frames(const void* samples, int pcm, float pcm_scale, int64_t len, float* out,
                             hipStream_t stream) {
  const int64_t n = vad_num_windows(len);
  if (n == 0) return hipSuccess;
  const dim3 g((unsigned)((n + kVadRowsPerBlock - 1) / kVadRowsPerBlock)), b(kVadThreads);
  const Decode dc{pcm_scale, 1.0f / pcm_scale, 1.0 / (double)pcm_scale};
  if (pcm == kPcmI16)
    sfe_vad_frames_kernel<int16_t><<<g, b, 0, stream>>>(static_cast<const int16_t*>(samples), len, n, dc, out);
  else if (pcm == kPcmI32)
    sfe_vad_frames_kernel<int32_t><<<g, b, 0, stream>>>(static_cast<const int32_t*>(samples), len, n, dc, out);
  else
    sfe_vad_frames_kernel<float><<<g, b, 0, stream>>>(static_cast<const float*>(samples), len, n, dc, out);
  return hipGetLastError();
}

}  // namespace sfe
