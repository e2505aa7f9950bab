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

// Mel contraction schedule for v_mfma_f32_4x4x1_16b_f32.  One wave
// contracts the power spectra of its own 4 frames: an MFMA is 16 blocks of
// [4 filters x 1 bin] . [1 bin x 4 frames].  Chain 0 holds the blocks of
// filters 0..63 (block j: filters 4j..4j+3), chain 1 those of filters
// 64..127.  Block j of chain c runs kChainSteps[c] consecutive bins from its
// own first bin (a multiple of 4, from the device table), so the dense
// 128x257 product is never formed.  The step counts fit the 16 kHz Slaney
// filterbank (widest block of chain 0: 7 bins, of chain 1: 32).
constexpr int kChains = 2;
constexpr int kChainSteps[kChains] = {8, 32};
constexpr int kMelSteps = 40;       // both chains
constexpr int kMelVec = kMelSteps / 4;  // float4 A operands per lane
static_assert(kChainSteps[0] + kChainSteps[1] == kMelSteps && kChainSteps[0] % 4 == 0 && kChainSteps[1] % 4 == 0,
              "chains are whole float4 steps");

// One featurized item: a clip or a long-form chunk task.  samples[start,
// start+len) is featurized into out[dst_off + m*S + t] (S = T, or the
// padded row length of the encoder-input layout).  The raw log-mel (log2;
// times ln 2 is the log-mel) goes to scratch in tiles of 16 frames: tile
// t / 16 of the item at raw[out_off + 2048 * (t / 16)], holding 8 slabs of
// 16 features, each [16 frames][16 features], slab s holding features
// 16s..16s+15.
struct Item {
  int64_t start;
  int64_t len;
  int64_t out_off;   // raw (scratch) element offset: kRawTile * (tiles of the items before it)
  int64_t dst_off;   // output element offset: out_off when packed, i * feature_size * pad_to when padded
  int32_t T;         // len / hop + 1
  int32_t unit_off;  // first unit (4-frame quad) of this item, relative to the launch
};

// Constant tables, uploaded once per context.
struct DevTables {
  float window[kNfft];       // hann_window(400), zero past 400
  float2 tw256[256];         // [l * 16 + k1] = e^{-2 pi i l k1 / 256}, l, k1 < 16
  float2 tw512[256];         // e^{-2 pi i k / 512}, k < 256
  // A operands of the mel MFMAs: [v][lane] holds steps 4v..4v+3 (v < 2:
  // chain 0, else chain 1, steps 4(v-2)..) of lane L = 4j + m: filter
  // 64c + 4j + m at bin k0[c][j] + step, times 0.25 (the FFT stage yields
  // 4|X|^2).
  float4 mel_a[kMelVec][64];
  int32_t k0[kChains][16];  // first bin of each block (multiple of 4)
};

// Host table builders (sfe_tables.cpp).
void hann_window(int win, float* out);
void mel_filterbank(int n_fft, int n_mels, int sample_rate, float* out);
// Returns false if the filterbank does not fit the MFMA schedule.
bool build_dev_tables(int sample_rate, DevTables* t);

// Kernel launchers (sfe_kernels.hip).  All asynchronous on `stream`.
constexpr int kTile = 16;  // frames per raw tile
constexpr int kRawTile = kTile * 128;  // raw scratch floats per tile of 16 frames
constexpr int kQuad = 4;   // frames per unit of work (one wave pass) of the log-mel kernel
int64_t tiles_for(int64_t T);
int64_t units_for(int64_t T);  // quads of an item: ceil(T / 4)
// grid_cap: workgroups resident on the device at once (the kernel loops
// over tiles, so launching more than that only adds scheduling overhead).
// Input sample formats: f32, or integer PCM (16-bit or 32-bit containers)
// decoded as value / pcm_scale in the kernel.
constexpr int kPcmF32 = 0;
constexpr int kPcmI16 = 1;
constexpr int kPcmI32 = 2;
// Units [unit0, unit0 + n_units) in the numbering of items[].unit_off.
hipError_t launch_logmel(const void* samples, int pcm, float pcm_scale, const Item* items, int n_items, int unit0,
                         int n_units, const DevTables* tables, float preemph, float* raw_out, int grid_cap,
                         hipStream_t stream);
constexpr int kLogmelWavesPerSimd = 3;
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
