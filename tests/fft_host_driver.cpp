// Host run of the log-mel kernel's FFT arithmetic (scriptrs_amd/csrc/sfe_fft.hpp)
// against float64 DFTs: the 16-point DFTs on their own, then the whole
// 512-point real power spectrum of a frame as the kernel computes it (16
// lanes x 16 registers, inter-stage twiddles from the device tables in
// tangent form, the transpose, the second DFT applying their cosines, the
// even/odd split with the table's split twiddles, bin 128 from Z[128]).
// No GPU is used.
//
// Prints one line per check and "bad N" at the end (N checks failed).
#include <math.h>
#include <stdio.h>
#include <stdlib.h>

#include <complex>
#include <random>
#include <vector>

#include "sfe_fft.hpp"
#include "sfe_internal.hpp"

using sfe::cf;
typedef std::complex<double> C;

static int bad = 0;

static void check(const char* what, double err, double bound) {
  const bool ok = err <= bound;
  printf("%s: %.3e (bound %.1e) %s\n", what, err, bound, ok ? "ok" : "FAIL");
  if (!ok) ++bad;
}

static std::vector<C> dft(const std::vector<C>& x) {
  const size_t n = x.size();
  std::vector<C> y(n);
  for (size_t k = 0; k < n; ++k) {
    C s = 0;
    for (size_t m = 0; m < n; ++m) s += x[m] * std::polar(1.0, -2.0 * M_PI * (double)((k * m) % n) / (double)n);
    y[k] = s;
  }
  return y;
}

int main() {
  std::mt19937 rng(1234);
  std::normal_distribution<float> nd(0.0f, 1.0f);
  const double u = ldexp(1.0, -24);

  // 16-point DFTs: error relative to the input norm
  double e16 = 0, e16w = 0;
  for (int trial = 0; trial < 2000; ++trial) {
    cf a[16];
    std::vector<C> x(16);
    double nrm = 0;
    for (int m = 0; m < 16; ++m) {
      a[m] = {nd(rng), nd(rng)};
      x[m] = C(a[m].x, a[m].y);
      nrm += std::norm(x[m]);
    }
    sfe::dft16(a);
    std::vector<C> y = dft(x);
    for (int k = 0; k < 16; ++k) e16 = fmax(e16, std::abs(C(a[k].x, a[k].y) - y[k]) / sqrt(nrm) / u);
    // windowed, inputs 13..15 zero
    cf v[13], w[13], b[16];
    std::vector<C> xw(16, 0.0);
    double nw = 0;
    for (int m = 0; m < 13; ++m) {
      v[m] = {nd(rng), nd(rng)};
      w[m] = {fabsf(nd(rng)), fabsf(nd(rng))};
      xw[m] = C((double)v[m].x * w[m].x, (double)v[m].y * w[m].y);
      nw += std::norm(xw[m]);
    }
    sfe::dft16_windowed(v, w, b);
    std::vector<C> yw = dft(xw);
    for (int k = 0; k < 16; ++k) e16w = fmax(e16w, std::abs(C(b[k].x, b[k].y) - yw[k]) / sqrt(nw) / u);
  }
  // Twiddled inputs in tangent form, the cosines applied by dft16_scaled:
  // the DFT of a[m] e^{-i theta_m}, including theta = pi/2 and 3 pi/2 (the
  // tables' 2^-100 / 2^100 pair).
  double e16s = 0;
  std::uniform_real_distribution<double> ud(0.0, 2.0 * M_PI);
  for (int trial = 0; trial < 2000; ++trial) {
    cf a[16];
    float c[16];
    std::vector<C> x(16);
    double nrm = 0;
    for (int m = 0; m < 16; ++m) {
      const cf v = {nd(rng), nd(rng)};
      double th = m == 0 ? 0.0 : ud(rng);
      if (trial % 7 == 0 && m == 5) th = M_PI / 2;
      if (trial % 7 == 1 && m == 9) th = 3 * M_PI / 2;
      double cc = cos(th), tn;
      if (fabs(th - M_PI / 2) < 1e-12 || fabs(th - 3 * M_PI / 2) < 1e-12) {
        cc = ldexp(1.0, -100);
        tn = (th < M_PI ? 1.0 : -1.0) * ldexp(1.0, 100);
      } else {
        tn = sin(th) / cc;
      }
      a[m] = m == 0 ? v : sfe::tan_twiddle(v, (float)tn);
      c[m] = m == 0 ? 1.0f : (float)cc;
      x[m] = C(v.x, v.y) * std::polar(1.0, -th);
      nrm += std::norm(x[m]);
    }
    sfe::dft16_scaled(a, c);
    std::vector<C> y = dft(x);
    for (int k = 0; k < 16; ++k) e16s = fmax(e16s, std::abs(C(a[k].x, a[k].y) - y[k]) / sqrt(nrm) / u);
  }
  // A radix-4 x 4 DFT in f32: a few ulps of the input norm per output.
  check("dft16, max |err| / (|x| u)", e16, 16.0);
  check("tan_twiddle + dft16_scaled, max |err| / (|x| u)", e16s, 24.0);
  check("dft16_windowed, max |err| / (|x w| u)", e16w, 16.0);

  // Whole frames: 4|X_k|^2 of the windowed 512-point frame
  sfe::DevTables tb;
  if (!sfe::build_dev_tables(16000, &tb)) {
    printf("tables failed\nbad 1\n");
    return 1;
  }
  double emag = 0, ep128 = 0, esilent = 0;
  for (int trial = 0; trial < 200; ++trial) {
    std::vector<float> y(512, 0.0f);
    const float amp = trial % 4 == 0 ? 1e-3f : 1.0f;
    for (int n = 0; n < 400; ++n) y[n] = amp * nd(rng);
    if (trial % 5 == 1)  // a loud low tone over near silence: low-energy bins next to a strong one
      for (int n = 0; n < 400; ++n) y[n] = 0.5f * sinf(0.05f * n) + 1e-5f * nd(rng);
    // lane l: z[l + 16 m2] = (y[2(l + 16 m2)], y[2(l + 16 m2) + 1]), taps past 400 zero
    cf X[16][16];
    for (int l = 0; l < 16; ++l) {
      cf v[13], w[13], a[16];
      for (int m2 = 0; m2 < 13; ++m2) {
        const int n = 2 * l + 32 * m2;
        v[m2] = (m2 < 12 || l < 8) ? cf{y[n], y[n + 1]} : cf{0.0f, 0.0f};
        w[m2] = {tb.window[n], tb.window[n + 1]};
      }
      sfe::dft16_windowed(v, w, a);
      for (int k1 = 1; k1 < 16; ++k1) a[k1] = sfe::tan_twiddle(a[k1], tb.tan256[l * 16 + k1]);
      for (int k1 = 0; k1 < 16; ++k1) X[k1][l] = a[k1];
    }
    cf Z[256];
    for (int l = 0; l < 16; ++l) {
      cf a[16];
      float c[16];
      for (int m1 = 0; m1 < 16; ++m1) {
        a[m1] = X[l][m1];
        c[m1] = tb.cos256[l * 16 + m1];
      }
      sfe::dft16_scaled(a, c);
      for (int k2 = 0; k2 < 16; ++k2) Z[l + 16 * k2] = a[k2];
    }
    float P[257];
    for (int l = 0; l < 16; ++l)
      for (int k2 = 0; k2 < 8; ++k2) {
        const int k = l + 16 * k2;
        const cf A = Z[k], B = Z[(256 - k) & 255];
        const float s = tb.split[k].x, r = tb.split[k].y;
        float pp, pm;
        if (k2 < 4) sfe::split_power<false>(A, B, s, r, pp, pm);
        else sfe::split_power<true>(A, B, s, r, pp, pm);
        P[k] = pp;
        P[256 - k] = pm;
      }
    P[128] = 4.0f * fmaf(Z[128].y, Z[128].y, Z[128].x * Z[128].x);
    // float64 reference
    std::vector<C> xr(512, 0.0);
    double nrm = 0;
    for (int n = 0; n < 400; ++n) {
      xr[n] = (double)y[n] * (double)tb.window[n];
      nrm += std::norm(xr[n]);
    }
    std::vector<C> Xr(257);
    for (int k = 0; k <= 256; ++k) {
      C s = 0;
      for (int n = 0; n < 400; ++n) s += xr[n] * std::polar(1.0, -2.0 * M_PI * (double)((k * n) % 512) / 512.0);
      Xr[k] = s;
    }
    // |X_k| to within a small multiple of u log2(N) |x| (the error any f32
    // FFT carries, independent of the bin)
    const double scale = u * 9.0 * sqrt(nrm) * sqrt(512.0);
    for (int k = 0; k <= 256; ++k) {
      const double m = sqrt((double)P[k]) / 2.0;
      const double e = fabs(m - std::abs(Xr[k])) / scale;
      emag = fmax(emag, e);
      if (k == 128) ep128 = fmax(ep128, e);
      if (trial % 5 == 1 && std::abs(Xr[k]) < 1e-3) esilent = fmax(esilent, e);
    }
  }
  check("frame |X_k|, max err / (u log2(512) |x| sqrt(512))", emag, 1.0);
  check("bin 128, same scale", ep128, 1.0);
  check("low-energy bins of a loud tone, same scale", esilent, 1.0);
  printf("bad %d\n", bad);
  return bad != 0;
}
