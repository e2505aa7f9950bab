// Internal declarations shared by the kernels and the C-ABI layer.
#pragma once
#include <hip/hip_runtime.h>

#include <mutex>
#include <stdint.h>

#include <vector>

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
// 64..127.  Block j of chain c runs kChainSteps[schedule][c] consecutive
// bins from its own first bin (a multiple of 4, from the device table), so
// the dense 128x257 product is never formed.  Schedule 0 fits the Slaney
// filterbank at 16, 22.05 and 24 kHz (at 16 kHz the widest block of chain 0
// spans 7 bins, of chain 1 32); schedule 1, with 50% more steps, fits the
// other sample rates from 3.5 to 107 kHz (at 8 kHz chain 0 needs 10 bins,
// at 48 kHz chain 1 needs 41).  The tables take the first that fits.
constexpr int kChains = 2;
constexpr int kSchedules = 2;
constexpr int kChainSteps[kSchedules][kChains] = {{8, 32}, {12, 48}};
constexpr int mel_vec(int schedule) { return (kChainSteps[schedule][0] + kChainSteps[schedule][1]) / 4; }
// Power-spectrum bins each schedule's FFT stage writes per frame: the 257
// bins, and for schedule 1 three zeros after them, so that a block whose
// filters reach bin 256 can start at a multiple of 4 (the float4 operand
// loads) and still run its 48 steps inside the written bins.
constexpr int kBinsWritten[kSchedules] = {kBins, kBins + 3};
constexpr int kMelVecMax = mel_vec(1);  // float4 A operands per lane, either schedule
static_assert(kChainSteps[0][0] % 4 == 0 && kChainSteps[0][1] % 4 == 0 && kChainSteps[1][0] % 4 == 0 &&
                  kChainSteps[1][1] % 4 == 0 && kChainSteps[0][0] <= kChainSteps[0][1] &&
                  kChainSteps[1][0] <= kChainSteps[1][1] && mel_vec(0) <= kMelVecMax,
              "chains are whole float4 steps, chain 1 the longer");

// Raw log-mel (log2; times ln 2 is the log-mel) lives in scratch in tiles
// of 16 frames (kRawTile floats): 8 slabs of 16 features, each [16 frames]
// [16 features], slab s holding features 16s..16s+15.  Frame f of a region
// whose tile 0 holds frames 0..15 sits at region + raw_frame(f).
constexpr int kTile = 16;              // frames per raw tile
constexpr int kRawTile = kTile * 128;  // raw scratch floats per tile of 16 frames
constexpr int kQuad = 4;               // frames per unit of work (one wave pass) of the log-mel kernel
__host__ __device__ constexpr int64_t raw_frame(int64_t f) { return kRawTile * (f >> 4) + 16 * (f & 15); }

// One entry of either kernel's table.
//
// Log-mel entries: frames 4 q0 .. 4 (q0 + n_units) - 1 of samples[start,
// start + len) (preemphasis restarting at `start`, zero padding outside),
// frame f written to raw[out_off + raw_frame(f)]; its units (4-frame quads)
// are numbered from unit_off.  Entries are whole items, or parts of them
// (first or last quads), or spans that several overlapping items share.
//
// Normalisation entries, one per featurized item (a clip or a long-form
// chunk task) of T frames, written to out[dst_off + m*S + t] (S = T, or the
// padded row length of the encoder-input layout).  Frame f of its raw
// log-mel is read from raw[grid_off + raw_frame(f + gshift)] for f in
// [f_lo, f_hi], raw[tail_off + raw_frame(f)] past f_hi and raw[out_off +
// raw_frame(f)] below f_lo.  An item with its own region has f_lo = 0,
// f_hi = T - 1, grid_off = out_off and gshift = 0.
struct Item {
  int64_t start;
  int64_t len;
  int64_t out_off;
  int64_t dst_off;
  int64_t grid_off;
  int64_t tail_off;
  int32_t T;         // len / hop + 1
  int32_t unit_off;  // log-mel: first unit, relative to the launch
  int32_t n_units;   // log-mel: units of the entry
  int32_t q0;        // log-mel: first quad of the entry within its frames
  int32_t f_lo, f_hi, gshift;
  int32_t pad_;
};
static_assert(sizeof(Item) == 80, "item table layout");

// An item with its own raw region at out_off (both kernels' view).
inline Item own_item(int64_t start, int64_t len, int64_t out_off, int64_t dst_off, int32_t unit_off) {
  Item it{};
  it.start = start;
  it.len = len;
  it.out_off = out_off;
  it.dst_off = dst_off;
  it.grid_off = out_off;
  it.tail_off = out_off;
  it.T = (int32_t)(len / kHop + 1);
  it.unit_off = unit_off;
  it.n_units = (int32_t)((it.T + kQuad - 1) / kQuad);
  it.q0 = 0;
  it.f_lo = 0;
  it.f_hi = it.T - 1;
  it.gshift = 0;
  return it;
}

// Shared frames (sfe_share.cpp).  Frames of overlapping items whose samples
// lie at least one sample inside each item and whose starts agree modulo the
// hop are computed once: items' own regions keep only their first quad and
// their last quads, and a shared log-mel entry per run of such items covers
// the union of their interior frames.  Given items with their own regions
// (own_item; out_off ignored), plan_table fills one table, table[0, *n_lm)
// with the log-mel entries and table[*n_lm, *n_lm + n) with the
// normalisation entries in item order, and returns the raw tiles they use.
// With share = false, or where sharing saves no quads, every item keeps its
// own region.  table holds (kPlanEntriesPerItem + 1) n entries; nothing is
// allocated when ws was reserved for at least n items.
constexpr int kPlanEntriesPerItem = 3;  // log-mel entries per item at most
struct PlanWorkspace {
  struct Span {
    int idx;              // item index
    int64_t res, lo, hi;  // start mod hop; interior frames in recording frame indices
  };
  struct Run {
    int64_t res, lo, hi;   // union of interior frames (recording frame indices)
    int64_t vstart, vend;  // samples of the shared entry
    int64_t cv;            // vstart / hop
    int64_t grid;          // out_off of the shared entry once placed, else -1
    int k0, k1;            // members: sp[k0, k1)
  };
  struct Piece {
    int64_t pos;  // recording position of the first frame
    int32_t seq;  // creation order
    Item e;
  };
  std::vector<Span> sp;
  std::vector<int> run_of;
  std::vector<Run> runs;
  std::vector<Piece> pieces;
  void reserve(size_t n);
};
int64_t plan_table(const Item* items, int n, bool share, PlanWorkspace* ws, Item* table, size_t* n_lm);
// Normalisation entries reordered longest first (in 256-frame classes, call
// order within one); allocates nothing.
void order_norm(Item* norm, int n);
// Frames of one run's shared entry at most (512 MB of raw log-mel), and
// members of one run at most (each with at most 3 tiles of its own, 384 MB
// in all): an item's first and last tiles follow its run's shared region,
// and every frame of the item lies within kNormBufRange bytes of the
// region's start (the normalisation kernel's 32-bit buffer offsets).
constexpr int64_t kMaxShareFrames = (int64_t)1 << 20;
constexpr int kMaxShareMembers = 1 << 14;
constexpr int kNormBufRange = 0x7ffffff0;
static_assert(kMaxShareFrames * kRawTile / kTile * 4 + (int64_t)kMaxShareMembers * 3 * kRawTile * 4 +
                      (int64_t)2 * kRawTile * 4 <
                  kNormBufRange,
              "a run's regions fit the normalisation kernel's offsets");

// Constant tables, uploaded once per context.
struct DevTables {
  float window[kNfft];       // hann_window(400), zero past 400
  // Inter-stage twiddles e^{-2 pi i l k1 / 256} (l, k1 < 16) in tangent
  // form (sfe_fft.hpp tan_twiddle): tan256[l * 16 + k1] = tan, read by lane
  // l of the first stage; cos256[k1 * 16 + l] = cos, read by lane k1 of the
  // second stage (dft16_scaled).  At cos = 0 (l k1 = 64): 2^-100 and 2^100.
  float tan256[256];
  float cos256[256];
  // Split twiddles e^{-2 pi i k / 512}, k < 128, as (s, r): k < 64: (cos,
  // tan); k >= 64: (sin, cos / sin) (sfe_fft.hpp split_g).
  float2 split[128];
  // A operands of the mel MFMAs: [v][lane] holds steps 4v..4v+3 (v < S0 /
  // 4: chain 0, else chain 1, steps 4(v - S0 / 4)..; S0 = chain 0's steps)
  // of lane L = 4j + m: filter 64c + 4j + m at bin k0[c][j] + step, times
  // 0.25 (the FFT stage yields 4|X|^2).  The first mel_vec(schedule) rows
  // are used.
  float4 mel_a[kMelVecMax][64];
  int32_t k0[kChains][16];  // first bin of each block (multiple of 4)
  int32_t schedule;         // index into kChainSteps
};

// Host table builders (sfe_tables.cpp).
void hann_window(int win, float* out);
void mel_filterbank(int n_fft, int n_mels, int sample_rate, float* out);
// Returns false if the filterbank does not fit the MFMA schedule.
bool build_dev_tables(int sample_rate, DevTables* t);

// Kernel launchers (sfe_kernels.hip).  All asynchronous on `stream`.
int64_t tiles_for(int64_t T);
int64_t units_for(int64_t T);  // quads of an item: ceil(T / 4)
// cus: the device's compute units (the log-mel grid is persistent: at most
// the workgroups resident at once).  Input sample formats: f32, or integer PCM (16-bit or 32-bit containers)
// decoded as value / pcm_scale in the kernel.
constexpr int kPcmF32 = 0;
constexpr int kPcmI16 = 1;
constexpr int kPcmI32 = 2;
// Units [unit0, unit0 + n_units) in the numbering of items[].unit_off.
// Timestamp buffer of measurement builds (-DSFE_TIMESTAMPS, sfe_kernels.hip);
// stamps_built() is false and set_stamp_buffer fails in the product build.
bool stamps_built();
hipError_t set_stamp_buffer(void* buf, int64_t words);
constexpr int kLogmelWavesPerSimd = 3;
// Log-mel launch shape: launches with at least 4 units per wave on every
// CU's 12 waves take one 12-wave workgroup per CU; smaller ones 4-wave
// workgroups, up to 3 per CU, each wave taking at least one unit.
constexpr int kLogmelWavesSmall = 4;
constexpr int kLogmelWavesBig = 12;
struct LogmelGrid {
  int waves;   // per workgroup
  int blocks;  // workgroups
};
inline LogmelGrid logmel_grid(int n_units, int cus) {
  if ((int64_t)n_units >= (int64_t)4 * kLogmelWavesBig * cus) {
    const int want = (n_units + kLogmelWavesBig - 1) / kLogmelWavesBig;
    return {kLogmelWavesBig, want < cus ? want : cus};
  }
  const int want = (n_units + kLogmelWavesSmall - 1) / kLogmelWavesSmall;
  const int cap = kLogmelWavesPerSimd * cus;
  return {kLogmelWavesSmall, want < cap ? want : cap};
}
// Units [*wb, *we) of workgroup b of G workgroups of NW waves, over units
// [unit0, unit0 + n_units).  4-wave grids run 3 workgroups per CU, dispatched
// a CU slot at a time, and a SIMD issues its oldest wave first, so the later
// slots run slower: their shares are weighted 11 : 10 : 9 by slot (blocks in
// thirds of the grid) when every wave has at least 8 units.  The log-mel
// kernel and the host's first-item table (logmel_wave_items) both use this.
__host__ __device__ inline void logmel_share(int64_t G, int64_t b, int NW, int unit0, int n_units, int* wb, int* we) {
  const int64_t B1 = G / 3, B2 = 2 * G / 3;
  const bool weighted = NW == kLogmelWavesSmall && G >= 3 && (int64_t)n_units >= (int64_t)8 * NW * G;
  auto cum = [=](int64_t c) -> int64_t {  // share of the blocks before block c
    if (!weighted) return c;
    const int64_t c1 = c < B1 ? c : B1, c2 = c < B1 ? 0 : (c < B2 ? c - B1 : B2 - B1), c3 = c > B2 ? c - B2 : 0;
    return 11 * c1 + 10 * c2 + 9 * c3;
  };
  const int64_t tot = cum(G);
  *wb = unit0 + (int)((int64_t)n_units * cum(b) / tot);
  *we = unit0 + (int)((int64_t)n_units * cum(b + 1) / tot);
}
// Item of each wave's first unit, for a launch of grid g over units
// [unit0, unit0 + n_units) of items[0, n_items) (sorted by unit_off):
// out[b * g.waves + w] = the last item whose unit_off <= wb + w (0 for a wave
// with no unit).  The kernel then skips its item search, a chain of
// dependent loads at the start of every wave.  At most kMaxLogmelWaves
// entries; larger grids go without (the kernel searches).
constexpr int kMaxLogmelWaves = 4096;
void logmel_wave_items(const Item* items, int n_items, int unit0, int n_units, LogmelGrid g, int32_t* out);
// wave_item: the table above on the device for this launch, or null.
// schedule: the tables' mel schedule (DevTables::schedule).
hipError_t launch_logmel(const void* samples, int pcm, float pcm_scale, const Item* items, int n_items, int unit0,
                         int n_units, const DevTables* tables, int schedule, float preemph, float* raw_out, int cus,
                         const int32_t* wave_item, hipStream_t stream);
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
// (a plan has at most kPlanEntriesPerItem log-mel entries and one
// normalisation entry per item)
constexpr size_t kNoAllocItemBytes =
    ((size_t)(kPlanEntriesPerItem + 1) * kNoAllocMaxItems * sizeof(Item) + kMaxLogmelWaves * sizeof(int32_t) +
     255) / 256 * 256;
constexpr size_t kNoAllocRawBytes = (size_t)64 << 20;
// Device address of this device's static scratch (looked up once per device).
hipError_t noalloc_scratch(int device, void** out);
// Host lock of a device's static scratch (held for a whole call), and the
// device-side order of calls on it: noalloc_order makes `stream` wait for
// the previous call's end when that call ran on another stream, noalloc_mark
// records this call's end on `stream`.  Both need the lock held.
hipError_t noalloc_lock(int device, std::unique_lock<std::mutex>* lock);
hipError_t noalloc_order(int device, hipStream_t stream);
hipError_t noalloc_mark(int device, hipStream_t stream);

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
