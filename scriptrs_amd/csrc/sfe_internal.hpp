// Internal declarations shared by the kernels and the C-ABI layer.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sfe {

// Shape the kernels are specialised to: TranscriptionConfig::default()
// (src/config.rs:30-44).
constexpr int kNfft = 512;
constexpr int kWin = 400;
constexpr int kHop = 160;
constexpr int kMel = 128;
constexpr int kBins = kNfft / 2 + 1;  // 257
constexpr int kPad = kNfft / 2;       // 256 zeros each side (src/frontend.rs:124-125)
constexpr int kMelW = 12;             // max contiguous nonzeros per filter row

// One featurized item: a clip or a long-form chunk task.  samples[start,
// start+len) is featurized into out[out_off + m*T + t].
struct Item {
  int64_t start;
  int64_t len;
  int64_t out_off;   // element offset = feature_size * frame_offset
  int32_t T;         // len / hop + 1
  int32_t tile_off;  // first frame tile of this item, relative to the launch
};

// Constant tables, uploaded once per context.
struct DevTables {
  float window[kNfft];       // hann_window(400), zero past 400
  float2 tw256[256];         // [l * 16 + k1] = e^{-2 pi i l k1 / 256}, l, k1 < 16
  float2 tw512[256];         // e^{-2 pi i k / 512}, k < 256
  int32_t mel_lo[kMel];      // first nonzero bin of filter m
  int32_t mel_cnt[kMel];     // contiguous bins from mel_lo
  float mel_w[kMel * kMelW]; // weights * 0.25 (the FFT stage yields 4*|X|^2)
};

// Host table builders (sfe_tables.cpp).
void hann_window(int win, float* out);
void mel_filterbank(int n_fft, int n_mels, int sample_rate, float* out);
// Returns false if some filter row has more than kMelW contiguous bins.
bool build_dev_tables(int sample_rate, DevTables* t);

// Kernel launchers (sfe_kernels.hip).  All asynchronous on `stream`.
constexpr int kTile = 32;  // frames per workgroup of the log-mel kernel
int64_t tiles_for(int64_t T);
hipError_t launch_logmel(const float* samples, const Item* items, int n_items, int total_tiles,
                         const DevTables* tables, float preemph, float* raw_out, hipStream_t stream);
// Normalises raw (f32, layout as above) per (item, feature) row and writes
// to out (f32, may alias raw) or bf16 (uint16_t*) when out_bf16 is set.
hipError_t launch_norm(const float* raw, const Item* items, int n_items, void* out, bool out_bf16,
                       hipStream_t stream);

}  // namespace sfe
