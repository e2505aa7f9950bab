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

// Mel contraction schedule for v_mfma_f32_16x16x4_f32.  The 128 filters form
// 8 blocks of 16; block b is contracted over kBlockSteps[b] steps of 4 bins
// starting at a bin taken from the device table (so other sample rates work
// when their filters fit the same step counts).  The step counts are those
// of the 16 kHz Slaney filterbank.  Blocks are assigned to the 4 waves of a
// workgroup at compile time so each wave's MFMA chains have static control
// flow; the busiest wave runs 22 steps.
constexpr int kWaves = 4;
constexpr int kBlocks = kMel / 16;
constexpr int kBlockSteps[kBlocks] = {4, 4, 4, 5, 8, 11, 15, 22};
constexpr int kWaveBlocks[kWaves][3] = {{7, -1, -1}, {6, -1, -1}, {5, 3, 0}, {4, 2, 1}};
constexpr int wave_steps(int w) {
  int n = 0;
  for (int i = 0; i < 3; ++i)
    if (kWaveBlocks[w][i] >= 0) n += kBlockSteps[kWaveBlocks[w][i]];
  return n;
}
constexpr int kMaxSteps = 22;  // per wave
static_assert(wave_steps(0) <= kMaxSteps && wave_steps(1) <= kMaxSteps && wave_steps(2) <= kMaxSteps &&
                  wave_steps(3) <= kMaxSteps,
              "schedule exceeds the per-wave step budget");

// One featurized item: a clip or a long-form chunk task.  samples[start,
// start+len) is featurized into out[dst_off + m*S + t] (S = T, or the
// padded row length of the encoder-input layout).  The raw log-mel (log2;
// times ln 2 is the log-mel) goes to scratch in tiles of 16 frames: tile
// t / 16 of the item at raw[out_off + 2048 * (t / 16)], holding 8 slabs of
// 16 features, each [16 frames][16 features] (the slab order inside the tile
// is the log-mel kernel's kSlabPos).
struct Item {
  int64_t start;
  int64_t len;
  int64_t out_off;   // raw (scratch) element offset: kRawTile * (tiles of the items before it)
  int64_t dst_off;   // output element offset: out_off when packed, i * feature_size * pad_to when padded
  int32_t T;         // len / hop + 1
  int32_t tile_off;  // first 16-frame unit of this item, relative to the launch
};

// Constant tables, uploaded once per context.
struct DevTables {
  float window[kNfft];       // hann_window(400), zero past 400
  float2 tw256[256];         // [l * 16 + k1] = e^{-2 pi i l k1 / 256}, l, k1 < 16
  float2 tw512[256];         // e^{-2 pi i k / 512}, k < 256
  int32_t block_k0[kBlocks];               // first bin of each block (multiple of 4)
  // A operand of each step of wave w, in the wave's block order, in lane
  // order: lane L holds W[16 b + L % 16][k0_b + 4 s + L / 16] * 0.25 (the FFT
  // stage yields 4|X|^2)
  float a[kWaves][kMaxSteps][64];
};

// Host table builders (sfe_tables.cpp).
void hann_window(int win, float* out);
void mel_filterbank(int n_fft, int n_mels, int sample_rate, float* out);
// Returns false if the filterbank does not fit the MFMA schedule.
bool build_dev_tables(int sample_rate, DevTables* t);

// Kernel launchers (sfe_kernels.hip).  All asynchronous on `stream`.
constexpr int kTile = 16;  // frames per unit of work (one pass) of the log-mel kernel
constexpr int kRawTile = kTile * 128;  // raw scratch floats per tile of 16 frames
int64_t tiles_for(int64_t T);
// grid_cap: workgroups resident on the device at once (the kernel loops
// over tiles, so launching more than that only adds scheduling overhead).
// Input sample formats: f32, or integer PCM (16-bit or 32-bit containers)
// decoded as value / pcm_scale in the kernel.
constexpr int kPcmF32 = 0;
constexpr int kPcmI16 = 1;
constexpr int kPcmI32 = 2;
// Units [unit0, unit0 + n_units) in the numbering of items[].tile_off.
hipError_t launch_logmel(const void* samples, int pcm, float pcm_scale, const Item* items, int n_items, int unit0,
                         int n_units, const DevTables* tables, float preemph, float* raw_out, int grid_cap,
                         hipStream_t stream);
constexpr int kLogmelWavesPerSimd = 2;
constexpr int kLogmelBlocksPerCU = kLogmelWavesPerSimd;  // 4-wave workgroups: one wave per SIMD each
// Normalises raw (f32 log2 values in 16-frame tiles, see Item) per (item, feature)
// and writes feature-major [128][T] per item to out (f32, must not alias
// raw) or bf16 (uint16_t*) when out_bf16 is set.  max_T: the longest item's
// frame count (sizes the kernel's register budget).  pad_to > 0: rows of
// pad_to frames, zero past T (the encoder input layout).
hipError_t launch_norm(const float* raw, const Item* items, int n_items, int max_T, int pad_to, void* out,
                       bool out_bf16, hipStream_t stream);

// Static scratch of the allocation-free entry point (sfe_noalloc.hip): an
// item table of up to kNoAllocMaxItems items, then kNoAllocRawBytes of raw
// log-mel (kNoAllocRawBytes / (kRawTile * 4) 16-frame tiles).
constexpr int kNoAllocMaxItems = 4096;
constexpr size_t kNoAllocItemBytes = ((size_t)kNoAllocMaxItems * sizeof(Item) + 255) / 256 * 256;
constexpr size_t kNoAllocRawBytes = (size_t)64 << 20;
// Device address of this device's static scratch (looked up once per device).
hipError_t noalloc_scratch(int device, void** out);

// Silero VAD model inputs (sfe_vad.hip): [64 context | 512 window] f32 per
// 512-sample window (src/long_form/vad.rs:62-99, src/constants.rs).
constexpr int kVadWin = 512;
constexpr int kVadCtx = 64;
constexpr int kVadRow = kVadWin + kVadCtx;
int64_t vad_num_windows(int64_t len);  // ceil(len / 512); 0 for len <= 0
// Writes vad_num_windows(len) rows of kVadRow floats to out (16-byte aligned).
hipError_t launch_vad_frames(const void* samples, int pcm, float pcm_scale, int64_t len, float* out,
                             hipStream_t stream);

}  // namespace sfe
