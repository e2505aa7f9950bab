// Register-level pieces of the log-mel kernel's 512-point real FFT, written
// for both the device and the host so that the host test
// (tests/fft_host_driver.cpp) runs the same arithmetic against a float64
// DFT.
//
// The 256-point complex FFT is 16 x 16: each of 16 lanes runs a 16-point
// DFT over its registers, the inter-stage twiddles are applied, the 16 x 16
// block is transposed (through LDS in the kernel) and a second 16-point DFT
// finishes it (the inter-stage twiddles in tangent form, their cosines
// fused into the second DFT's inner layer).  A 16-point DFT is an inner
// radix-4 layer, the internal
// twiddles e^{-2 pi i p c / 16} and an outer radix-4 layer.  Its instruction
// count is what the kernel's time goes to, so the constant multiplications
// are folded into fused multiply-adds:
//  * the window product of the first DFT's inputs goes into the inner
//    layer's first additions (fma(v, w, .));
//  * an internal twiddle e^{-i theta} is written as cos(theta) (1 - i
//    tan(theta)) (theta = pi/8, 3pi/8 through 1/tan) or sqrt(1/2) (1 - i):
//    the bracket costs two fmas or two additions, and the common factor
//    (cos(pi/8) or sqrt(1/2)) multiplies the outer layer's additions as fmas.
// Every arithmetic instruction is then an fma or an addition, except the
// window products that cannot be fused (values used four times).
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>

namespace sfe {

struct __align__(8) cf {
  float x, y;
};

__host__ __device__ __forceinline__ cf cadd(cf a, cf b) { return {a.x + b.x, a.y + b.y}; }
__host__ __device__ __forceinline__ cf csub(cf a, cf b) { return {a.x - b.x, a.y - b.y}; }
__host__ __device__ __forceinline__ cf cmul(cf a, cf w) { return {a.x * w.x - a.y * w.y, a.x * w.y + a.y * w.x}; }
// c + s v and c - s v for a real s
__host__ __device__ __forceinline__ cf cfma(float s, cf v, cf c) { return {fmaf(s, v.x, c.x), fmaf(s, v.y, c.y)}; }

namespace fftc {
constexpr float kR = 0.70710678118654752f;   // sqrt(1/2) = cos(pi/4)
constexpr float kC1 = 0.92387953251128674f;  // cos(pi/8)
constexpr float kT1 = 0.41421356237309505f;  // tan(pi/8)
}  // namespace fftc

// 4-point forward DFT in place on (a0, a1, a2, a3); when Z3 the caller
// guarantees a3 == 0 and it is never read.
template <bool Z3>
__host__ __device__ __forceinline__ void dft4(cf& a0, cf& a1, cf& a2, cf& a3) {
  cf t0 = cadd(a0, a2), t1 = csub(a0, a2);
  cf t2 = Z3 ? a1 : cadd(a1, a3);
  cf t3 = Z3 ? a1 : csub(a1, a3);
  a0 = cadd(t0, t2);
  a2 = csub(t0, t2);
  a1 = {t1.x + t3.y, t1.y - t3.x};  // t1 - i t3
  a3 = {t1.x - t3.y, t1.y + t3.x};  // t1 + i t3
}

// The outputs of a radix-4 butterfly from t0 = v0 + v2, t1 = v0 - v2 and
// t2 = k s, t3 = k d (k real, applied here as fmas):
//   y0 = t0 + t2, y2 = t0 - t2, y1 = t1 - i t3, y3 = t1 + i t3.
__host__ __device__ __forceinline__ void bfly_out(cf t0, cf t1, float k, cf s, cf d, cf& y0, cf& y1, cf& y2,
                                                  cf& y3) {
  y0 = cfma(k, s, t0);
  y2 = cfma(-k, s, t0);
  y1 = {fmaf(k, d.y, t1.x), fmaf(-k, d.x, t1.y)};
  y3 = {fmaf(-k, d.y, t1.x), fmaf(k, d.x, t1.y)};
}

// u e^{-i pi/8} = cos(pi/8) g1(u), g1(u) = (x + y t, y - x t), t = tan(pi/8)
__host__ __device__ __forceinline__ cf g1(cf u) { return {fmaf(u.y, fftc::kT1, u.x), fmaf(-u.x, fftc::kT1, u.y)}; }
// u e^{-3 i pi/8} = cos(pi/8) g3(u), g3(u) = (x t + y, y t - x)
__host__ __device__ __forceinline__ cf g3(cf u) { return {fmaf(u.x, fftc::kT1, u.y), fmaf(u.y, fftc::kT1, -u.x)}; }

// Outer layer of a 16-point DFT: a[p + 4c] holds the inner layer's U[p][c]
// (inner DFT over q of the inputs m = p + 4q, output index c).  Applies the
// twiddles e^{-2 pi i p c / 16} and the 4-point DFTs over p, and leaves
// X[k] at a[k] (natural order).
__host__ __device__ __forceinline__ void dft16_outer(cf (&a)[16]) {
  using namespace fftc;
  cf y[16];
  // c = 0: no twiddles
  {
    cf v0 = a[0], v1 = a[1], v2 = a[2], v3 = a[3];
    dft4<false>(v0, v1, v2, v3);
    y[0] = v0, y[4] = v1, y[8] = v2, y[12] = v3;
  }
  // c = 1: v1 = U e^{-i pi/8}, v2 = U e^{-i pi/4}, v3 = U e^{-3 i pi/8}
  {
    const cf u2 = {a[6].x + a[6].y, a[6].y - a[6].x};  // v2 = kR u2
    const cf t0 = cfma(kR, u2, a[4]), t1 = cfma(-kR, u2, a[4]);
    const cf h1 = g1(a[5]), h3 = g3(a[7]);               // v1 = kC1 h1, v3 = kC1 h3
    bfly_out(t0, t1, kC1, cadd(h1, h3), csub(h1, h3), y[1], y[5], y[9], y[13]);
  }
  // c = 2: v1 = U e^{-i pi/4}, v2 = U e^{-i pi/2} = -i U, v3 = U e^{-3 i pi/4}
  {
    const cf t0 = {a[8].x + a[10].y, a[8].y - a[10].x};
    const cf t1 = {a[8].x - a[10].y, a[8].y + a[10].x};
    const cf u1 = {a[9].x + a[9].y, a[9].y - a[9].x};       // v1 = kR u1
    const float w = a[11].x + a[11].y;
    const cf u3 = {a[11].y - a[11].x, -w};                 // v3 = kR u3
    bfly_out(t0, t1, kR, cadd(u1, u3), csub(u1, u3), y[2], y[6], y[10], y[14]);
  }
  // c = 3: v1 = U e^{-3 i pi/8}, v2 = U e^{-3 i pi/4}, v3 = U e^{-9 i pi/8} = -U e^{-i pi/8}
  {
    const cf u2 = {a[14].y - a[14].x, -(a[14].x + a[14].y)};  // v2 = kR u2
    const cf t0 = cfma(kR, u2, a[12]), t1 = cfma(-kR, u2, a[12]);
    const cf h1 = g3(a[13]), h3 = g1(a[15]);                 // v1 = kC1 h1, v3 = -kC1 h3
    bfly_out(t0, t1, kC1, csub(h1, h3), cadd(h1, h3), y[3], y[7], y[11], y[15]);
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) a[i] = y[i];
}

// Inter-stage twiddle in tangent form: a e^{-i theta} = cos(theta) g with
// g = (x + y tan(theta), y - x tan(theta)), two fmas; the cosine is applied
// by the next stage (dft16_scaled).  Where cos(theta) is 0 the table holds
// cos = 2^-100, tan = 2^100 (products exact in range: |x| < 2^27).
__host__ __device__ __forceinline__ cf tan_twiddle(cf a, float t) {
  return {fmaf(a.y, t, a.x), fmaf(-a.x, t, a.y)};
}

// 16-point forward DFT of the inputs c[m] a[m] (real scale factors, c[0] =
// 1 and not read), into a[k], natural order.  The scales are fused into the
// inner layer: per inner DFT (inputs p, p + 4, p + 8, p + 12) the first
// input of each pair is scaled by a multiplication and the second by the
// fmas of the pair's sum and difference.
__host__ __device__ __forceinline__ void dft16_scaled(cf (&a)[16], const float (&c)[16]) {
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const cf x0 = p == 0 ? a[0] : cf{c[p] * a[p].x, c[p] * a[p].y};
    const cf x1 = {c[p + 4] * a[p + 4].x, c[p + 4] * a[p + 4].y};
    const float c2 = c[p + 8], c3 = c[p + 12];
    const cf t0 = cfma(c2, a[p + 8], x0), t1 = cfma(-c2, a[p + 8], x0);
    const cf t2 = cfma(c3, a[p + 12], x1), t3 = cfma(-c3, a[p + 12], x1);
    a[p] = cadd(t0, t2);
    a[p + 8] = csub(t0, t2);
    a[p + 4] = {t1.x + t3.y, t1.y - t3.x};   // t1 - i t3
    a[p + 12] = {t1.x - t3.y, t1.y + t3.x};  // t1 + i t3
  }
  dft16_outer(a);
}

// 16-point forward DFT in registers: a[m] -> a[k], natural order.
__host__ __device__ __forceinline__ void dft16(cf (&a)[16]) {
  dft4<false>(a[0], a[4], a[8], a[12]);
  dft4<false>(a[1], a[5], a[9], a[13]);
  dft4<false>(a[2], a[6], a[10], a[14]);
  dft4<false>(a[3], a[7], a[11], a[15]);
  dft16_outer(a);
}

// 16-point forward DFT of the windowed inputs a[m] = (v[m].x w[m].x,
// v[m].y w[m].y) for m < 13 (inputs 13..15 are zero), into a[k].  The
// window products are fused into the inner layer: per inner DFT (inputs p,
// p + 4, p + 8, p + 12), the first input's product goes into both of its
// additions, and in the pruned ones (p > 0, input p + 12 zero) the second
// input's product into the four output additions it feeds.
__host__ __device__ __forceinline__ void dft16_windowed(const cf (&v)[13], const cf (&w)[13], cf (&a)[16]) {
  // p = 0: all four inputs
  {
    const cf A2 = {v[8].x * w[8].x, v[8].y * w[8].y}, A3 = {v[12].x * w[12].x, v[12].y * w[12].y};
    const cf t0 = {fmaf(v[0].x, w[0].x, A2.x), fmaf(v[0].y, w[0].y, A2.y)};
    const cf t1 = {fmaf(v[0].x, w[0].x, -A2.x), fmaf(v[0].y, w[0].y, -A2.y)};
    const cf t2 = {fmaf(v[4].x, w[4].x, A3.x), fmaf(v[4].y, w[4].y, A3.y)};
    const cf t3 = {fmaf(v[4].x, w[4].x, -A3.x), fmaf(v[4].y, w[4].y, -A3.y)};
    a[0] = cadd(t0, t2);
    a[8] = csub(t0, t2);
    a[4] = {t1.x + t3.y, t1.y - t3.x};
    a[12] = {t1.x - t3.y, t1.y + t3.x};
  }
#pragma unroll
  for (int p = 1; p < 4; ++p) {
    const cf A2 = {v[p + 8].x * w[p + 8].x, v[p + 8].y * w[p + 8].y};
    const cf t0 = {fmaf(v[p].x, w[p].x, A2.x), fmaf(v[p].y, w[p].y, A2.y)};
    const cf t1 = {fmaf(v[p].x, w[p].x, -A2.x), fmaf(v[p].y, w[p].y, -A2.y)};
    // t2 = t3 = A1 = (v[p+4].x w[p+4].x, v[p+4].y w[p+4].y)
    const float bx = v[p + 4].x, by = v[p + 4].y, wx = w[p + 4].x, wy = w[p + 4].y;
    a[p] = {fmaf(bx, wx, t0.x), fmaf(by, wy, t0.y)};           // t0 + A1
    a[p + 8] = {fmaf(-bx, wx, t0.x), fmaf(-by, wy, t0.y)};     // t0 - A1
    a[p + 4] = {fmaf(by, wy, t1.x), fmaf(-bx, wx, t1.y)};      // t1 - i A1
    a[p + 12] = {fmaf(-by, wy, t1.x), fmaf(bx, wx, t1.y)};     // t1 + i A1
  }
  dft16_outer(a);
}

// Split twiddle of bin k: od e^{-2 pi i k / 512} = s g, with (s, r) from the
// table: k < 64 (angle below pi/4): s = cos, r = tan, g = (x + y r, y - x r);
// k >= 64: s = sin, r = cot (= cos / sin), g = (x r + y, y r - x).
template <bool COT>
__host__ __device__ __forceinline__ cf split_g(cf od, float r) {
  if constexpr (COT) return {fmaf(od.x, r, od.y), fmaf(od.y, r, -od.x)};
  else return {fmaf(od.y, r, od.x), fmaf(-od.x, r, od.y)};
}

// 4|X[k]|^2 and 4|X[256-k]|^2 from A = Z[k], B = Z[256-k] (256-point FFT of
// z[m] = r[2m] + i r[2m+1]): 2E = A + conj B, 2O = (A - conj B) / i, X[k] =
// E + W O, X[256-k] = conj(E - W O), W = e^{-2 pi i k/512} = s (g / od).
template <bool COT>
__host__ __device__ __forceinline__ void split_power(cf A, cf B, float s, float r, float& pp, float& pm) {
  const cf e = {A.x + B.x, A.y - B.y};
  const cf od = {A.y + B.y, B.x - A.x};
  const cf g = split_g<COT>(od, r);
  const cf xp = cfma(s, g, e), xm = cfma(-s, g, e);
  pp = fmaf(xp.y, xp.y, xp.x * xp.x);
  pm = fmaf(xm.y, xm.y, xm.x * xm.x);
}

}  // namespace sfe
