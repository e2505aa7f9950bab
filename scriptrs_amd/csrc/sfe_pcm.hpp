// Integer PCM decode shared by the featurization and VAD framing kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sfe {

// Input samples: f32, or integer PCM decoded as the reference's WAV reader
// does (examples/transcribe_wav.rs:342-348): value as f32 / scale with
// scale = ((1 << (bits - 1)) - 1) as f32, correctly rounded.
//  * int32 containers: one residual step from r = RN(1 / scale): q = RN(v r)
//    is within an ulp of v / scale, and q + r fma(-scale, q, v) rounds to
//    RN(v / scale) (Markstein).
//  * int16 containers: RN_f32(RN_f64(v * RN_f64(1 / scale))).  For 15-bit
//    integers the f64 product is far closer to v / scale than the distance
//    from v / scale to any f32 rounding boundary, so the final rounding is
//    that of the exact quotient.  Three operations instead of five; the
//    tests check it against correctly rounded division for every int16
//    value at every width 2..16.
struct Decode {
  float scale, recip;
  double recip64;
};

__device__ __forceinline__ float pcm_div(float v, const Decode& d) {
#pragma clang fp contract(off)  // q is the rounded product
  const float q = v * d.recip;
  return __fmaf_rn(__fmaf_rn(-d.scale, q, v), d.recip, q);
}

template <typename S>
struct Pcm;
// V4: 4 raw samples.  Recordings and item starts are only sample-aligned
// (ragged batches start items anywhere), so the vector types carry the
// sample's own alignment; gfx950 takes such addresses in one vector load.
template <>
struct Pcm<float> {
  typedef float V4 __attribute__((ext_vector_type(4), aligned(4)));
  static __device__ __forceinline__ V4 load4(const float* p) { return *reinterpret_cast<const V4*>(p); }
  static __device__ __forceinline__ float dec(float v, const Decode&) { return v; }
  static __device__ __forceinline__ float4 dec4(const V4& v, const Decode&) { return make_float4(v.x, v.y, v.z, v.w); }
};
template <>
struct Pcm<int16_t> {
  typedef short V4 __attribute__((ext_vector_type(4), aligned(2)));
  static __device__ __forceinline__ V4 load4(const int16_t* p) { return *reinterpret_cast<const V4*>(p); }
  static __device__ __forceinline__ float dec(int16_t v, const Decode& d) { return (float)((double)v * d.recip64); }
  static __device__ __forceinline__ float4 dec4(const V4& v, const Decode& d) {
    return make_float4(dec(v.x, d), dec(v.y, d), dec(v.z, d), dec(v.w, d));
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
