/*
 * sfe_oracle.c -- CPU restatement of scriptrs' Parakeet log-mel front end.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * product path and the CPU baseline that bench.py times beside it.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it; the product library never links or calls it.
 *
 * Every function follows the reference op for op, in f32 where the
 * reference computes in f32 and in f64 where it computes in f64, with no
 * floating-point contraction (built with -ffp-contract=off), so that the
 * table builders are bit-exact with the reference and the per-frame path
 * differs only where the reference calls third-party code whose rounding is
 * not restated here:
 *   - realfft 3.5.0 / rustfft 6.4.1 (the 512-point real FFT,
 *     src/frontend.rs:82,89-90): restated as the same two-step algorithm
 *     realfft publishes (an N/2 complex FFT of the even/odd packed input
 *     followed by the split post-pass), with a radix-2 complex FFT;
 *     butterfly rounding differs from rustfft's planned kernels.
 *   - ndarray 0.17.2 / matrixmultiply 0.3.10 (the 128x257 dot,
 *     src/frontend.rs:110): restated as a plain f32 dot in bin order;
 *     matrixmultiply's blocked summation order is not restated.
 * Those two boundaries are "parity unpinned" element-wise; tests pin them
 * with the reference's own invariants (peak bin, shape, mean ~ 0), closed
 * forms and an independent float64 numpy restatement.
 *
 * Citations are to files under the reference repository root.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
  int32_t sample_rate;   /* src/config.rs:33 (SAMPLE_RATE = 16000)          */
  int32_t feature_size;  /* src/config.rs:34 (128)                           */
  int32_t n_fft;         /* src/config.rs:35 (512)                           */
  int32_t win_length;    /* src/config.rs:36 (400)                           */
  int32_t hop_length;    /* src/config.rs:37 (MEL_HOP_SAMPLES = 160)         */
  float preemphasis;     /* src/config.rs:38 (0.97)                          */
} sfo_config;

void sfo_config_default(sfo_config* c) {
  c->sample_rate = 16000;
  c->feature_size = 128;
  c->n_fft = 512;
  c->win_length = 400;
  c->hop_length = 160;
  c->preemphasis = 0.97f;
}

/* Frame count: src/frontend.rs:124-127 with padded.len() = L + n_fft,
 * i.e. (L + n_fft - n_fft) / hop + 1 = L / hop + 1. */
int64_t sfo_num_frames(int64_t len, int32_t hop) { return len / hop + 1; }

/* src/frontend.rs:161-165: w[n] = 0.5 - 0.5*cos((2*PI*n) / (N - 1)), all f32.
 * Rust evaluates `2.0 * PI * index as f32` left to right. */
void sfo_hann_window(int32_t win, float* out) {
  const float pi = 3.14159265358979323846f; /* std::f32::consts::PI */
  for (int32_t n = 0; n < win; ++n) {
    float num = (2.0f * pi) * (float)n;
    float den = (float)win - 1.0f;
    out[n] = 0.5f - 0.5f * cosf(num / den);
  }
}

/* src/frontend.rs:167-186: Slaney mel scale in f64. */
static const double F_SP = 200.0 / 3.0;
static const double MIN_LOG_HZ = 1000.0;
static const double LOG_STEP = 0.06875177742094912;

static double hz_to_mel_slaney(double hz) {
  const double min_log_mel = MIN_LOG_HZ / F_SP;
  if (hz < MIN_LOG_HZ) return hz / F_SP;
  return min_log_mel + log(hz / MIN_LOG_HZ) / LOG_STEP;
}

static double mel_to_hz_slaney(double mel) {
  const double min_log_mel = MIN_LOG_HZ / F_SP;
  if (mel < min_log_mel) return mel * F_SP;
  return MIN_LOG_HZ * exp((mel - min_log_mel) * LOG_STEP);
}

/* src/frontend.rs:188-223.  out is [n_mels][n_fft/2+1] row-major.
 * Triangle weights are formed in f64 and cast to f32; the Slaney area
 * normalisation is cast to f32 and applied as an f32 multiply. */
void sfo_mel_filterbank(int32_t n_fft, int32_t n_mels, int32_t sample_rate, float* out) {
  const int32_t bins = n_fft / 2 + 1;
  const double fmax = (double)sample_rate / 2.0;
  const double mel_min = hz_to_mel_slaney(0.0);
  const double mel_max = hz_to_mel_slaney(fmax);
  double* pts = (double*)malloc(sizeof(double) * (size_t)(n_mels + 2));
  double* freqs = (double*)malloc(sizeof(double) * (size_t)bins);
  double* diffs = (double*)malloc(sizeof(double) * (size_t)(n_mels + 1));
  for (int32_t i = 0; i <= n_mels + 1; ++i)
    pts[i] = mel_to_hz_slaney(mel_min + (mel_max - mel_min) * (double)i / (double)(n_mels + 1));
  for (int32_t k = 0; k < bins; ++k) freqs[k] = (double)k * (double)sample_rate / (double)n_fft;
  for (int32_t i = 0; i < n_mels + 1; ++i) diffs[i] = pts[i + 1] - pts[i];
  for (int32_t m = 0; m < n_mels; ++m) {
    for (int32_t k = 0; k < bins; ++k) {
      double lower = (freqs[k] - pts[m]) / diffs[m];
      double upper = (pts[m + 2] - freqs[k]) / diffs[m + 1];
      double v = lower < upper ? lower : upper;
      out[(size_t)m * bins + k] = (float)(v > 0.0 ? v : 0.0);
    }
  }
  for (int32_t m = 0; m < n_mels; ++m) {
    float enorm = (float)(2.0 / (pts[m + 2] - pts[m]));
    for (int32_t k = 0; k < bins; ++k) out[(size_t)m * bins + k] *= enorm;
  }
  free(pts);
  free(freqs);
  free(diffs);
}

/* ---- 512-point real FFT restated as realfft's algorithm ---------------- */
/* In-place iterative radix-2 complex FFT (forward, e^{-2 pi i nk/N}), f32. */
static void cfft_f32(float* re, float* im, int32_t n) {
  for (int32_t i = 1, j = 0; i < n; ++i) {
    int32_t bit = n >> 1;
    for (; j & bit; bit >>= 1) j ^= bit;
    j ^= bit;
    if (i < j) {
      float t = re[i]; re[i] = re[j]; re[j] = t;
      t = im[i]; im[i] = im[j]; im[j] = t;
    }
  }
  for (int32_t len = 2; len <= n; len <<= 1) {
    int32_t half = len >> 1;
    for (int32_t k = 0; k < half; ++k) {
      double ang = -2.0 * M_PI * (double)k / (double)len;
      float wr = (float)cos(ang), wi = (float)sin(ang);
      for (int32_t s = 0; s < n; s += len) {
        int32_t a = s + k, b = s + k + half;
        float tr = re[b] * wr - im[b] * wi;
        float ti = re[b] * wi + im[b] * wr;
        re[b] = re[a] - tr; im[b] = im[a] - ti;
        re[a] = re[a] + tr; im[a] = im[a] + ti;
      }
    }
  }
}

/* Real forward FFT of x[n_fft] -> power |X[k]|^2, k = 0..n_fft/2.
 * Step 1: z[m] = x[2m] + i x[2m+1], Z = FFT_{N/2}(z).
 * Step 2: E[k] = (Z[k] + conj Z[N/2-k]) / 2, O[k] = (Z[k] - conj Z[N/2-k]) / 2i,
 *         X[k] = E[k] + e^{-2 pi i k/N} O[k].
 * Power as Complex::norm_sqr: re*re + im*im (src/frontend.rs:141-143). */
static void rfft_power_f32(const float* x, int32_t n_fft, float* zr, float* zi, float* power) {
  const int32_t h = n_fft / 2;
  for (int32_t m = 0; m < h; ++m) { zr[m] = x[2 * m]; zi[m] = x[2 * m + 1]; }
  cfft_f32(zr, zi, h);
  for (int32_t k = 0; k <= h; ++k) {
    int32_t a = k % h, b = (h - k) % h;
    float er = 0.5f * (zr[a] + zr[b]);
    float ei = 0.5f * (zi[a] - zi[b]);
    /* (Z[k] - conj Z[h-k]) / 2i = ((zi[a] + zi[b]) - i (zr[a] - zr[b])) / 2 */
    float orr = 0.5f * (zi[a] + zi[b]);
    float oi = -0.5f * (zr[a] - zr[b]);
    double ang = -2.0 * M_PI * (double)k / (double)n_fft;
    float wr = (float)cos(ang), wi = (float)sin(ang);
    float xr = er + (wr * orr - wi * oi);
    float xi = ei + (wr * oi + wi * orr);
    power[k] = xr * xr + xi * xi;
  }
}

/* ---- the extractor --------------------------------------------------- */
typedef struct {
  sfo_config cfg;
  float* window;      /* [win_length]              */
  float* filterbank;  /* [feature_size][n_fft/2+1] */
} sfo_tables;

static void tables_init(sfo_tables* t, const sfo_config* c) {
  t->cfg = *c;
  t->window = (float*)malloc(sizeof(float) * (size_t)c->win_length);
  t->filterbank = (float*)malloc(sizeof(float) * (size_t)c->feature_size * (size_t)(c->n_fft / 2 + 1));
  sfo_hann_window(c->win_length, t->window);
  sfo_mel_filterbank(c->n_fft, c->feature_size, c->sample_rate, t->filterbank);
}

static void tables_free(sfo_tables* t) {
  free(t->window);
  free(t->filterbank);
}

/* src/frontend.rs:120-147 (stft) with apply_preemphasis_into (:150-159) and
 * prepare_padded_audio (:59-65).  power is [n_fft/2+1][T] row-major. */
static void stft_power(const sfo_tables* t, const float* audio, int64_t len, float* power) {
  const sfo_config* c = &t->cfg;
  const int64_t pad = c->n_fft / 2;
  const int64_t plen = len + 2 * pad;
  const int64_t frames = (plen - c->n_fft) / c->hop_length + 1;
  const int32_t bins = c->n_fft / 2 + 1;
  float* padded = (float*)calloc((size_t)plen, sizeof(float));
  float* frame = (float*)malloc(sizeof(float) * (size_t)c->n_fft);
  float* zr = (float*)malloc(sizeof(float) * (size_t)c->n_fft);
  float* zi = (float*)malloc(sizeof(float) * (size_t)c->n_fft);
  float* pw = (float*)malloc(sizeof(float) * (size_t)bins);
  /* preemphasis: y0 = x0, y[i] = x[i] - coef * x[i-1]  (f32, not fused) */
  padded[pad] = audio[0];
  for (int64_t i = 1; i < len; ++i) {
    float prod = c->preemphasis * audio[i - 1];
    padded[pad + i] = audio[i] - prod;
  }
  for (int64_t f = 0; f < frames; ++f) {
    int64_t start = f * c->hop_length;
    int64_t avail = plen - start;
    if (avail < 0) avail = 0;
    if (avail > c->win_length) avail = c->win_length;
    memset(frame, 0, sizeof(float) * (size_t)c->n_fft);
    for (int64_t n = 0; n < avail; ++n) frame[n] = padded[start + n] * t->window[n];
    rfft_power_f32(frame, c->n_fft, zr, zi, pw);
    for (int32_t k = 0; k < bins; ++k) power[(size_t)k * (size_t)frames + (size_t)f] = pw[k];
  }
  free(padded);
  free(frame);
  free(zr);
  free(zi);
  free(pw);
}

/* src/frontend.rs:225-241 on one feature row x[0..T) (contiguous, because the
 * reference's [T,128] array is stored feature-major): sequential f32 sums. */
static void normalize_row(float* x, int64_t T) {
  float sum = 0.0f;
  for (int64_t i = 0; i < T; ++i) sum += x[i];
  float mean = sum / (float)T;
  float acc = 0.0f;
  for (int64_t i = 0; i < T; ++i) {
    float d = x[i] - mean;
    acc += d * d;
  }
  float var = acc / ((float)T - 1.0f);
  float sd = sqrtf(var) + 1e-5f;
  for (int64_t i = 0; i < T; ++i) x[i] = (x[i] - mean) / sd;
}

/* src/frontend.rs:104-118.  out is feature-major [feature_size][T] (the
 * memory order of the reference's `.t().to_owned()` [T,128] array).
 * Returns 0, or 1 for EmptyAudio (src/frontend.rs:105-107). */
static int extract_with(const sfo_tables* t, const float* audio, int64_t len, float* out) {
  if (len <= 0) return 1;
  const sfo_config* c = &t->cfg;
  const int32_t bins = c->n_fft / 2 + 1;
  const int64_t T = sfo_num_frames(len, c->hop_length);
  float* power = (float*)malloc(sizeof(float) * (size_t)bins * (size_t)T);
  stft_power(t, audio, len, power);
  const float guard = 5.9604644775390625e-08f; /* 2^-24, src/frontend.rs:111 */
  float* col = (float*)malloc(sizeof(float) * (size_t)bins);
  for (int64_t f = 0; f < T; ++f) {
    for (int32_t k = 0; k < bins; ++k) col[k] = power[(size_t)k * (size_t)T + (size_t)f];
    for (int32_t m = 0; m < c->feature_size; ++m) {
      const float* w = t->filterbank + (size_t)m * bins;
      float acc = 0.0f;
      for (int32_t k = 0; k < bins; ++k) acc += w[k] * col[k];
      out[(size_t)m * (size_t)T + (size_t)f] = logf(acc + guard);
    }
  }
  for (int32_t m = 0; m < c->feature_size; ++m) normalize_row(out + (size_t)m * (size_t)T, T);
  free(col);
  free(power);
  return 0;
}

int sfo_extract_cfg(const sfo_config* c, const float* audio, int64_t len, float* out) {
  sfo_tables t;
  tables_init(&t, c);
  int rc = extract_with(&t, audio, len, out);
  tables_free(&t);
  return rc;
}

int sfo_extract(const float* audio, int64_t len, float* out) {
  sfo_config c;
  sfo_config_default(&c);
  return sfo_extract_cfg(&c, audio, len, out);
}

/* The reference's stft() output, [n_fft/2+1][T] power (used by its own
 * peak-bin test, src/frontend.rs:258-281). */
int sfo_stft_power(const float* audio, int64_t len, float* power) {
  if (len <= 0) return 1;
  sfo_config c;
  sfo_config_default(&c);
  sfo_tables t;
  tables_init(&t, &c);
  stft_power(&t, audio, len, power);
  tables_free(&t);
  return 0;
}

/* ---- batched spans with a worker pool (src/long_form.rs:266-314) ------- */
typedef struct {
  const sfo_tables* t;
  const float* samples;
  const int64_t* starts;
  const int64_t* lens;
  const int64_t* frame_offsets;
  float* out;
  int32_t n;
  int32_t next; /* shared task counter (atomic fetch-add, as the reference) */
  int32_t status;
} span_job;

static void* span_worker(void* arg) {
  span_job* j = (span_job*)arg;
  for (;;) {
    int32_t i = __atomic_fetch_add(&j->next, 1, __ATOMIC_RELAXED);
    if (i >= j->n) break;
    float* dst = j->out + (size_t)j->t->cfg.feature_size * (size_t)j->frame_offsets[i];
    if (extract_with(j->t, j->samples + j->starts[i], j->lens[i], dst) != 0)
      __atomic_store_n(&j->status, 1, __ATOMIC_RELAXED);
  }
  return NULL;
}

/* Featurize n spans [starts[i], starts[i]+lens[i]) of one sample buffer,
 * each independently (preemphasis restarts per span, as every chunk goes
 * through its own extract call, src/long_form.rs:584-592).  Writes
 * frame_offsets[0..n] (prefix sums of T_i) and out (item i at
 * out + feature_size * frame_offsets[i], [feature_size][T_i]). */
int sfo_extract_spans(const float* samples, const int64_t* starts, const int64_t* lens, int32_t n,
                      float* out, int64_t* frame_offsets, int32_t nthreads) {
  sfo_config c;
  sfo_config_default(&c);
  frame_offsets[0] = 0;
  for (int32_t i = 0; i < n; ++i) {
    if (lens[i] <= 0) return 1;
    frame_offsets[i + 1] = frame_offsets[i] + sfo_num_frames(lens[i], c.hop_length);
  }
  sfo_tables t;
  tables_init(&t, &c);
  span_job job = {&t, samples, starts, lens, frame_offsets, out, n, 0, 0};
  if (nthreads < 1) nthreads = 1;
  if (nthreads > n) nthreads = n;
  pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)nthreads);
  for (int32_t i = 1; i < nthreads; ++i) pthread_create(&th[i], NULL, span_worker, &job);
  span_worker(&job);
  for (int32_t i = 1; i < nthreads; ++i) pthread_join(th[i], NULL);
  free(th);
  tables_free(&t);
  return job.status;
}

/* Silero VAD model inputs, restated as the reference's loop
 * (process_coreml_vad, src/long_form/vad.rs:62-99; window 512, context 64,
 * src/constants.rs:6-11): per window, copy the chunk, pad a short one with
 * its last sample, emit [context | chunk], then keep the chunk's last 64
 * samples as the next context.  out: ceil(len/512) rows of 576 floats.
 * Returns the number of rows. */
int64_t sfo_vad_frames(const float* audio, int64_t len, float* out) {
  enum { WIN = 512, CTX = 64 };
  float context[CTX];
  float chunk[WIN];
  memset(context, 0, sizeof(context));
  memset(chunk, 0, sizeof(chunk));
  int64_t rows = 0;
  for (int64_t start = 0; start < len; start += WIN) {
    const int64_t end = start + WIN < len ? start + WIN : len;
    const int64_t n = end - start;
    memcpy(chunk, audio + start, (size_t)n * sizeof(float));
    if (n < WIN) {
      const float last = chunk[n > 0 ? n - 1 : 0];
      for (int64_t k = n; k < WIN; ++k) chunk[k] = last;
    }
    float* row = out + rows * (WIN + CTX);
    memcpy(row, context, sizeof(context));
    memcpy(row + CTX, chunk, sizeof(chunk));
    memcpy(context, chunk + (WIN - CTX), sizeof(context));
    ++rows;
  }
  return rows;
}
