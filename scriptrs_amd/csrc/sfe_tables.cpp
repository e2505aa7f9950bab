// Host-side construction of the constant tables the kernels read.
//
// hann_window and mel_filterbank follow src/frontend.rs:161-223 with the
// reference's operation order and precision (f32 for the window, f64 for
// the mel points and triangle weights with an f32 cast, then an f32
// multiply by the f32-cast Slaney norm).  This file is built with
// -ffp-contract=off so each operation rounds as in the reference.
#include <math.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "sfe_internal.hpp"

namespace sfe {

void hann_window(int win, float* out) {
  const float pi = 3.14159265358979323846f;  // std::f32::consts::PI
  for (int n = 0; n < win; ++n) {
    float num = (2.0f * pi) * (float)n;
    float den = (float)win - 1.0f;
    out[n] = 0.5f - 0.5f * cosf(num / den);
  }
}

namespace {
const double kFsp = 200.0 / 3.0;            // F_SP, src/frontend.rs:167
const double kMinLogHz = 1000.0;            // MIN_LOG_HZ
const double kLogStep = 0.06875177742094912;  // LOG_STEP = ln(6.4)/27

double hz_to_mel(double hz) {
  const double min_log_mel = kMinLogHz / kFsp;
  return hz < kMinLogHz ? hz / kFsp : min_log_mel + log(hz / kMinLogHz) / kLogStep;
}

double mel_to_hz(double mel) {
  const double min_log_mel = kMinLogHz / kFsp;
  return mel < min_log_mel ? mel * kFsp : kMinLogHz * exp((mel - min_log_mel) * kLogStep);
}
}  // namespace

void mel_filterbank(int n_fft, int n_mels, int sample_rate, float* out) {
  const int bins = n_fft / 2 + 1;
  const double mel_min = hz_to_mel(0.0);
  const double mel_max = hz_to_mel((double)sample_rate / 2.0);
  std::vector<double> pts(n_mels + 2), freqs(bins), diffs(n_mels + 1);
  for (int i = 0; i <= n_mels + 1; ++i)
    pts[i] = mel_to_hz(mel_min + (mel_max - mel_min) * (double)i / (double)(n_mels + 1));
  for (int k = 0; k < bins; ++k) freqs[k] = (double)k * (double)sample_rate / (double)n_fft;
  for (int i = 0; i <= n_mels; ++i) diffs[i] = pts[i + 1] - pts[i];
  for (int m = 0; m < n_mels; ++m)
    for (int k = 0; k < bins; ++k) {
      double lower = (freqs[k] - pts[m]) / diffs[m];
      double upper = (pts[m + 2] - freqs[k]) / diffs[m + 1];
      double v = lower < upper ? lower : upper;
      out[(size_t)m * bins + k] = (float)(v > 0.0 ? v : 0.0);
    }
  for (int m = 0; m < n_mels; ++m) {
    float enorm = (float)(2.0 / (pts[m + 2] - pts[m]));
    for (int k = 0; k < bins; ++k) out[(size_t)m * bins + k] *= enorm;
  }
}

bool build_dev_tables(int sample_rate, DevTables* t) {
  memset(t, 0, sizeof(*t));
  hann_window(kWin, t->window);
  for (int l = 0; l < 16; ++l)
    for (int k1 = 0; k1 < 16; ++k1) {
      // e^{-i theta} = cos(theta) (1 - i tan(theta)), theta = 2 pi l k1 / 256;
      // laid out per lane so the kernel indexes it affinely
      const int m = (l * k1) % 256;
      double c, tn;
      if (m == 64 || m == 192) {
        // cos = 0: a tiny cosine and a huge tangent with an exact product
        // (sin = +-1 there)
        c = ldexp(1.0, -100);
        tn = (m == 64 ? 1.0 : -1.0) * ldexp(1.0, 100);
      } else {
        const double th = 2.0 * M_PI * (double)m / 256.0;
        c = cos(th);
        tn = sin(th) / c;
      }
      t->tan256[l * 16 + k1] = (float)tn;
      t->cos256[k1 * 16 + l] = (float)c;
    }
  for (int k = 0; k < 128; ++k) {
    const double b = 2.0 * M_PI * (double)k / 512.0, c = cos(b), s = sin(b);
    t->split[k] = k < 64 ? make_float2((float)c, (float)(s / c)) : make_float2((float)s, (float)(c / s));
  }
  std::vector<float> fb((size_t)kMel * kBins);
  mel_filterbank(kNfft, kMel, sample_rate, fb.data());
  // 4-filter blocks: the first bin (a multiple of 4) is chosen here; the
  // block's nonzero bins must fit its chain's step count, and every bin
  // read must lie within the bins the FFT stage writes (kBinsWritten).  The
  // first schedule every block fits is used.
  auto fill = [&](int sch) -> bool {
    for (int c = 0; c < kChains; ++c) {
      const int S = kChainSteps[sch][c];
      for (int j = 0; j < 16; ++j) {
        const int f0 = 64 * c + 4 * j;
        int lo = -1, hi = -1;
        for (int m = f0; m < f0 + 4; ++m)
          for (int k = 0; k < kBins; ++k)
            if (fb[(size_t)m * kBins + k] != 0.0f) {
              if (lo < 0 || k < lo) lo = k;
              if (k > hi) hi = k;
            }
        if (lo < 0) lo = hi = 0;
        int k0 = lo / 4 * 4;
        if (k0 + S > kBinsWritten[sch]) k0 = (kBinsWritten[sch] - S) / 4 * 4;
        if (lo < k0 || hi >= k0 + S) return false;  // filters too wide for this schedule
        t->k0[c][j] = k0;
        for (int s = 0; s < S; ++s)
          for (int m = 0; m < 4; ++m) {
            const int v = (c == 0 ? 0 : kChainSteps[sch][0] / 4) + s / 4;
            float* a = reinterpret_cast<float*>(&t->mel_a[v][4 * j + m]);
            a[s % 4] = fb[(size_t)(f0 + m) * kBins + k0 + s] * 0.25f;
          }
      }
    }
    t->schedule = sch;
    return true;
  };
  bool ok = false;
  for (int sch = 0; sch < kSchedules && !ok; ++sch) {
    memset(t->mel_a, 0, sizeof(t->mel_a));
    memset(t->k0, 0, sizeof(t->k0));
    ok = fill(sch);
  }
  if (!ok) return false;
  return true;
}

}  // namespace sfe
