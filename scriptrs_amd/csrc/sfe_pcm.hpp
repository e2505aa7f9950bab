// Integer PCM decode shared by the featurization and VAD framing kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sfe {

// Input samples: f32, or integer PCM decoded as the reference's WAV reader
// does (examples/transcribe_wav.rs:342-348): value as f32 / scale with
// scale = ((1 << (bits - 1)) - 1) as f32.  The division is correctly rounded
// by one residual step from r = RN(1 / scale): q = RN(v r) is within an ulp
// of v / scale, and q + r fma(-scale, q, v) rounds to RN(v / scale)
// (Markstein; checked exhaustively for 16-bit PCM by the tests).
struct Decode {
  float scale, recip;
};

__device__ __forceinline__ float pcm_div(float v, const Decode& d) {
#pragma clang fp contract(off)  // q is the rounded product
  const float q = v * d.recip;
  return __fmaf_rn(__fmaf_rn(-d.scale, q, v), d.recip, q);
}

template <typename S>
struct Pcm;
template <>
struct Pcm<float> {
  using V4 = float4;  // 4 raw samples
  static __device__ __forceinline__ V4 load4(const float* p) { return *reinterpret_cast<const float4*>(p); }
  static __device__ __forceinline__ float dec(float v, const Decode&) { return v; }
  static __device__ __forceinline__ float4 dec4(const V4& v, const Decode&) { return v; }
};
template <>
struct Pcm<int16_t> {
  typedef short V4 __attribute__((ext_vector_type(4), aligned(2)));
  static __device__ __forceinline__ V4 load4(const int16_t* p) { return *reinterpret_cast<const V4*>(p); }
  static __device__ __forceinline__ float dec(int16_t v, const Decode& d) { return pcm_div((float)v, d); }
  static __device__ __forceinline__ float4 dec4(const V4& v, const Decode& d) {
    return make_float4(pcm_div((float)v.x, d), pcm_div((float)v.y, d), pcm_div((float)v.z, d), pcm_div((float)v.w, d));
  }
};
template <>
struct Pcm<int32_t> {
  typedef int V4 __attribute__((ext_vector_type(4), aligned(4)));
  static __device__ __forceinline__ V4 load4(const int32_t* p) { return *reinterpret_cast<const V4*>(p); }
  static __device__ __forceinline__ float dec(int32_t v, const Decode& d) { return pcm_div((float)v, d); }
  static __device__ __forceinline__ float4 dec4(const V4& v, const Decode& d) {
    return make_float4(pcm_div((float)v.x, d), pcm_div((float)v.y, d), pcm_div((float)v.z, d), pcm_div((float)v.w, d));
  }
};

}  // namespace sfe
