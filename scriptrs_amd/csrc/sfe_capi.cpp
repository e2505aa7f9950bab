// C-ABI of the MI355X log-mel front end (declared in include/scriptrs_fe.h).
//
// Host responsibilities: argument validation with the reference's error
// semantics, per-call item tables (one H2D copy from a pinned staging
// buffer), device buffer management, host->device streaming and stream
// ordering.  All compute runs in the HIP kernels of sfe_kernels.hip and
// sfe_vad.hip; there is no CPU compute path.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <exception>
#include <memory>
#include <mutex>
#include <new>
#include <string>
#include <thread>
#include <vector>

#include "../../include/scriptrs_fe.h"
#include "sfe_internal.hpp"

using sfe::Item;

namespace {

// Where the samples come from: f32, or integer PCM decoded in the kernel.
struct Source {
  const void* ptr;
  int pcm;      // sfe::kPcm*
  float scale;  // PCM decode divisor
  size_t esize;
};

// Streamed extraction normalises after every this many windows.
constexpr size_t kStreamNormWindows = 32;
// Streamed windows are featurized in batches of consecutive windows.  A
// batch covers one contiguous range of the recording, which goes to the
// device in one copy into one half of a two-batch device buffer: one H2D
// copy, one log-mel launch and one pair of cross-stream waits per batch,
// while the next batch's copy lands in the other half.  A batch holds as many
// windows as fit kStreamBatchBytes (at least one, at most
// kStreamMaxBatchWindows).  Measured on the 8 h recording in 60 s windows:
// 39 GB/s with one copy per window, 44 GB/s with 4 windows per copy, 55 GB/s
// with 16 (the link's peak for large copies is about 57 GB/s).
constexpr size_t kStreamBatchBytes = 64u << 20;
constexpr size_t kStreamMaxBatchWindows = 64;

// Copies from pageable host memory into pinned staging run on this many
// threads: one thread's memcpy bounds the pageable stream at about 27 GB/s,
// half the PCIe rate.
constexpr unsigned kStageThreads = 8;
constexpr size_t kStageMinBytes = 1u << 20;  // per thread

void parallel_memcpy(void* dst, const void* src, size_t bytes) {
  unsigned nt = (unsigned)std::min<size_t>(kStageThreads, bytes / kStageMinBytes);
  const unsigned hw = std::thread::hardware_concurrency();
  if (hw > 0) nt = std::min(nt, hw);
  if (nt <= 1) {
    memcpy(dst, src, bytes);
    return;
  }
  const size_t part = (bytes / nt + 63) / 64 * 64;
  std::vector<std::thread> th;
  th.reserve(nt - 1);
  for (unsigned i = 1; i < nt; ++i) {
    const size_t lo = std::min(bytes, part * i), hi = std::min(bytes, part * (i + 1));
    if (lo < hi) th.emplace_back([=] { memcpy(static_cast<char*>(dst) + lo, static_cast<const char*>(src) + lo, hi - lo); });
  }
  memcpy(dst, src, std::min(bytes, part));
  for (std::thread& t : th) t.join();
}

thread_local std::string g_last_error;

// Device and pinned host allocations made by the library (every hipMalloc
// and hipHostMalloc below counts one), read by sfe_debug_allocation_count.
std::atomic<int64_t> g_allocations{0};

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(SFE_HIP_ERROR, std::string(what) + ": " + hipGetErrorString(e));
}

#define SFE_HIP(call)                             \
  do {                                            \
    hipError_t e_ = (call);                       \
    if (e_ != hipSuccess) return hip_fail(e_, #call); \
  } while (0)

// Device buffer that grows on demand.  Growth synchronises the device
// first, so no queued kernel still reads the old allocation.
struct DevBuf {
  void* ptr = nullptr;
  size_t cap = 0;
  hipError_t reserve(size_t bytes) {
    if (bytes <= cap) return hipSuccess;
    hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) return e;
    size_t want = std::max(bytes, cap * 3 / 2);
    if (ptr) (void)hipFree(ptr);
    ptr = nullptr;
    cap = 0;
    e = hipMalloc(&ptr, want);
    g_allocations.fetch_add(1);
    if (e != hipSuccess && want > bytes) {  // the headroom does not fit: exactly what is asked
      (void)hipGetLastError();
      want = bytes;
      e = hipMalloc(&ptr, want);
      g_allocations.fetch_add(1);
    }
    if (e == hipSuccess) cap = want;
    return e;
  }
  void release() {
    if (ptr) (void)hipFree(ptr);
    ptr = nullptr;
    cap = 0;
  }
};

// Pinned host buffer that grows on demand; `ev` marks the last copy out of it.
struct PinBuf {
  void* ptr = nullptr;
  size_t cap = 0;
  hipEvent_t ev = nullptr;
  bool pending = false;
  hipError_t wait() {
    if (!pending) return hipSuccess;
    pending = false;
    return hipEventSynchronize(ev);
  }
  hipError_t reserve(size_t bytes) {
    hipError_t e = wait();
    if (e != hipSuccess) return e;
    if (!ev) {
      e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
      if (e != hipSuccess) return e;
    }
    if (bytes <= cap) return hipSuccess;
    if (ptr) (void)hipHostFree(ptr);
    ptr = nullptr;
    cap = 0;
    size_t want = std::max(bytes, (size_t)4096);
    e = hipHostMalloc(&ptr, want, hipHostMallocDefault);
    g_allocations.fetch_add(1);
    if (e == hipSuccess) cap = want;
    return e;
  }
  void release() {
    if (ptr) (void)hipHostFree(ptr);
    if (ev) (void)hipEventDestroy(ev);
    ptr = nullptr;
    ev = nullptr;
    cap = 0;
  }
};

bool shape_supported(const sfe_config* c, std::string* why) {
  if (c->n_fft != sfe::kNfft || c->win_length != sfe::kWin || c->hop_length != sfe::kHop ||
      c->feature_size != sfe::kMel) {
    *why = "unsupported frontend shape: the kernels are specialised to n_fft=512, win_length=400, "
           "hop_length=160, feature_size=128";
    return false;
  }
  if (c->sample_rate <= 0) {
    *why = "sample_rate must be positive";
    return false;
  }
  return true;
}

}  // namespace

struct sfe_ctx {
  sfe_config cfg;
  int device = 0;
  int cus = 256;  // compute units of the device
  std::mutex mu;
  sfe::DevTables* d_tables = nullptr;
  int schedule = 0;  // the tables' mel schedule (sfe::DevTables::schedule)
  // Internal streams (default priority) of the host-buffer entry points,
  // created on first use (internal_streams).
  hipStream_t s_compute = nullptr;
  hipStream_t s_copy = nullptr;
  DevBuf meta;      // Item tables
  std::vector<Item> meta_items;  // host copy of what meta holds (empty: unknown)
  // Orders calls on one context across streams (they share the item table
  // and the raw scratch): see order_after_last.
  hipEvent_t ev_last = nullptr;
  bool has_last = false;
  bool last_marked = false;   // ev_last marks the end of the previous call
  bool multi_stream = false;  // calls have come on more than one stream
  hipStream_t last_stream = nullptr;  // the stream the previous call's device work ran on
  PinBuf h_meta;
  DevBuf scratch;   // raw log-mel in 16-frame tiles, f32 (the normalisation kernel's input)
  DevBuf io_in;     // sfe_extract staging (audio)
  DevBuf io_out;    // sfe_extract staging (features)
  PinBuf h_io_in;   // sfe_extract pinned host staging: copies of pageable
  PinBuf h_io_out;  // memory run as plain memcpy + DMA instead of HIP's own staging
  DevBuf win;       // streamed windows: two halves of one batch each
  PinBuf h_win[2];
  hipEvent_t ev_copied[2] = {nullptr, nullptr};
  hipEvent_t ev_done[2] = {nullptr, nullptr};
  // Frames that overlapping chunk tasks share are computed once
  // (sfe_set_frame_sharing).
  bool share = true;
  // The last plan (run_items): its input items and sharing flag, and the
  // table it produced (log-mel entries, then normalisation entries).  A call
  // with the same items reuses it.
  std::vector<Item> plan_in;
  bool plan_share = false;
  std::vector<Item> plan_table;
  size_t plan_n_lm = 0;
  int64_t plan_tiles = 0;
  // kernel timing (sfe_set_timing): events around each launch, summed on read
  bool timing = false;
  std::vector<hipEvent_t> tev;  // pairs: start, end; kind alternates logmel, norm
  size_t tev_used = 0;
  // This device's static scratch (sfe_extract_chunks_noalloc): item table,
  // then raw log-mel.  Looked up by the entry point's first call on the
  // context; h_meta is reserved for its largest item table at creation.
  unsigned char* noalloc = nullptr;
  // Host staging of its planner, also reserved at creation for
  // kNoAllocMaxItems items: the chunks' own items and the planner's lists.
  std::vector<Item> na_in;
  sfe::PlanWorkspace na_ws;
};

namespace {

// Orders this call's work on `stream` after the context's previous call (the
// calls share the item table and the raw scratch).  Nothing is ever enqueued
// on an earlier call's stream, which its owner may have destroyed since.
// * Same stream: stream order is enough.
// * Another stream, previous call marked by ev_last: wait for that event.
// * Another stream, previous call unmarked: a context whose calls have all
//   been on one stream records no event (a marker after every call costs
//   launch-bound calls about 3 us: one 10 s clip 0.0156 -> 0.0189 ms), so the
//   first switch waits on the host for the device to drain (work on a
//   destroyed stream included), and from then on every call records ev_last.
hipError_t order_after_last(sfe_ctx* ctx, hipStream_t stream) {
  if (!ctx->has_last || stream == ctx->last_stream) return hipSuccess;
  if (ctx->last_marked) return hipStreamWaitEvent(stream, ctx->ev_last, 0);
  ctx->multi_stream = true;
  return hipDeviceSynchronize();
}

// The call just enqueued ran on `stream`; a context that has used more than
// one stream marks its end there with ev_last.
hipError_t mark_last(sfe_ctx* ctx, hipStream_t stream) {
  ctx->has_last = false;
  ctx->last_marked = false;
  if (ctx->multi_stream) {
    hipError_t e = hipEventRecord(ctx->ev_last, stream);
    if (e != hipSuccess) return e;
    ctx->last_marked = true;
  }
  ctx->has_last = true;
  ctx->last_stream = stream;
  return hipSuccess;
}

// Builds the item table for n spans and returns total tiles.
int build_items(const int64_t* starts, const int64_t* lens, int32_t n, std::vector<Item>* items,
                int64_t* frame_offsets, int64_t* total_tiles) {
  items->resize(n);
  int64_t fo = 0, tiles = 0, units = 0;
  if (frame_offsets) frame_offsets[0] = 0;
  for (int32_t i = 0; i < n; ++i) {
    if (lens[i] <= 0) return fail(SFE_EMPTY_AUDIO, "audio input was empty (item " + std::to_string(i) + ")");
    const int64_t T = lens[i] / sfe::kHop + 1;
    if (T > INT32_MAX / 2) return fail(SFE_INVALID_ARG, "item too long");
    (*items)[i] = sfe::own_item(starts[i], lens[i], (int64_t)sfe::kRawTile * tiles, (int64_t)sfe::kMel * fo,
                                (int32_t)units);
    fo += T;
    tiles += sfe::tiles_for(T);
    units += sfe::units_for(T);
    if (frame_offsets) frame_offsets[i + 1] = fo;
    if (units > INT32_MAX) return fail(SFE_INVALID_ARG, "batch too large for one launch");
  }
  *total_tiles = tiles;
  return SFE_OK;
}

hipEvent_t timing_event(sfe_ctx* ctx) {
  if (ctx->tev_used == ctx->tev.size()) {
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    ctx->tev.push_back(e);
  }
  return ctx->tev[ctx->tev_used++];
}

// Log-mel then normalisation over host items[0, n) (device copy d_items,
// unit_off relative to the launch), asynchronously on `stream`.  With timing
// on, every kernel is bracketed by events (read by sfe_get_timing).  stages
// selects the kernels: kLogmel, kNorm or both.
//
// (Splitting a call into batches, with the log-mel of batch b + 1 overlapping
// a low-footprint normalisation of batch b on a second stream, measured
// slower: 0.453 ms against 0.368 ms for the 1 h workload.  Log-mel is
// VALU-bound, and the co-resident normalisation took VALU issue and memory
// bandwidth from it.)
enum Stages { kLogmel = 1, kNorm = 2, kBoth = 3 };

int launch_pair(sfe_ctx* ctx, const Source& src, const Item* lm, const Item* d_lm, int n_lm, const Item* norm,
                const Item* d_norm, int n_norm, float* raw, void* out, int32_t out_dtype, int pad_to,
                hipStream_t stream, int stages = kBoth, bool allow_timing = true,
                const int32_t* d_wave_item = nullptr) {
  if (n_lm <= 0 && n_norm <= 0) return SFE_OK;
  const int u0 = n_lm > 0 ? lm[0].unit_off : 0;
  const int u1 = n_lm > 0 ? lm[n_lm - 1].unit_off + lm[n_lm - 1].n_units : 0;
  int max_T = 0;
  for (int i = 0; i < n_norm; ++i) max_T = std::max(max_T, (int)norm[i].T);
  hipEvent_t e[4] = {nullptr, nullptr, nullptr, nullptr};
  if (ctx->timing && allow_timing)
    for (int i = 0; i < 4; ++i)
      if (!(e[i] = timing_event(ctx))) return fail(SFE_HIP_ERROR, "hipEventCreate failed");
  if (e[0]) SFE_HIP(hipEventRecord(e[0], stream));
  if (stages & kLogmel)
    SFE_HIP(sfe::launch_logmel(src.ptr, src.pcm, src.scale, d_lm, n_lm, u0, u1 - u0, ctx->d_tables, ctx->schedule,
                               ctx->cfg.preemphasis, raw, ctx->cus, d_wave_item, stream));
  if (e[1]) SFE_HIP(hipEventRecord(e[1], stream));
  if (e[2]) SFE_HIP(hipEventRecord(e[2], stream));
  if (stages & kNorm)
    SFE_HIP(sfe::launch_norm(raw, d_norm, n_norm, max_T, pad_to, out, out_dtype == SFE_BF16, stream));
  if (e[3]) SFE_HIP(hipEventRecord(e[3], stream));
  return SFE_OK;
}

// The log-mel launch over table[0, n_lm): its grid, and whether its
// first-item table (sfe::logmel_wave_items) fits kMaxLogmelWaves entries.
struct WaveTable {
  sfe::LogmelGrid grid{0, 0};
  int u0 = 0, n_units = 0;
  size_t entries = 0;  // 0: the kernel searches instead
};
WaveTable wave_table(const Item* lm, size_t n_lm, int cus) {
  WaveTable t;
  if (n_lm == 0) return t;
  t.u0 = lm[0].unit_off;
  t.n_units = lm[n_lm - 1].unit_off + lm[n_lm - 1].n_units - t.u0;
  t.grid = sfe::logmel_grid(t.n_units, cus);
  const size_t n = (size_t)t.grid.waves * t.grid.blocks;
  if (t.n_units > 0 && n <= (size_t)sfe::kMaxLogmelWaves) t.entries = n;
  return t;
}

// Uploads items through the pinned staging buffer on `stream`, then runs
// the log-mel and normalisation kernels.
int run_items(sfe_ctx* ctx, const Source& src, const std::vector<Item>& items, int32_t out_dtype, void* out,
              hipStream_t stream, int pad_to = 0) {
  SFE_HIP(order_after_last(ctx, stream));
  // one table: the log-mel entries, then the normalisation entries
  if (!(ctx->plan_share == ctx->share && ctx->plan_in.size() == items.size() &&
        memcmp(ctx->plan_in.data(), items.data(), items.size() * sizeof(Item)) == 0)) {
    const int n = (int)items.size();
    sfe::PlanWorkspace ws;
    ws.reserve(items.size());
    std::vector<Item> table((size_t)(sfe::kPlanEntriesPerItem + 1) * items.size());
    size_t n_lm = 0;
    ctx->plan_tiles = sfe::plan_table(items.data(), n, ctx->share, &ws, table.data(), &n_lm);
    sfe::order_norm(table.data() + n_lm, n);
    table.resize(n_lm + items.size());
    ctx->plan_n_lm = n_lm;
    ctx->plan_table.swap(table);
    ctx->plan_in = items;
    ctx->plan_share = ctx->share;
  }
  const std::vector<Item>& table = ctx->plan_table;
  const size_t n_lm = ctx->plan_n_lm;
  const int64_t total_tiles = ctx->plan_tiles;
  // The upload: the table, then the log-mel launch's first-item table.
  const size_t tbytes = table.size() * sizeof(Item);
  const WaveTable wt = wave_table(table.data(), n_lm, ctx->cus);
  const size_t mbytes = tbytes + wt.entries * sizeof(int32_t);
  // A call with the same table as the previous upload (repeated plans,
  // equal-sized windows) reuses the device copy (the first-item table
  // follows from the table).  The table is only read by the kernels, so
  // earlier work still in flight is unaffected.
  const bool same = ctx->meta.ptr && ctx->meta_items.size() == table.size() &&
                    memcmp(ctx->meta_items.data(), table.data(), tbytes) == 0;
  if (!same) {
    ctx->meta_items.clear();
    SFE_HIP(ctx->h_meta.reserve(mbytes));
    SFE_HIP(ctx->meta.reserve(mbytes));
    memcpy(ctx->h_meta.ptr, table.data(), tbytes);
    if (wt.entries)
      sfe::logmel_wave_items(table.data(), (int)n_lm, wt.u0, wt.n_units, wt.grid,
                             reinterpret_cast<int32_t*>(static_cast<char*>(ctx->h_meta.ptr) + tbytes));
    SFE_HIP(hipMemcpyAsync(ctx->meta.ptr, ctx->h_meta.ptr, mbytes, hipMemcpyHostToDevice, stream));
    SFE_HIP(hipEventRecord(ctx->h_meta.ev, stream));
    ctx->h_meta.pending = true;
    ctx->meta_items = table;
  }
  const Item* d_table = static_cast<const Item*>(ctx->meta.ptr);
  const int32_t* d_wave =
      wt.entries ? reinterpret_cast<const int32_t*>(static_cast<const char*>(ctx->meta.ptr) + tbytes) : nullptr;
  SFE_HIP(ctx->scratch.reserve((size_t)total_tiles * sfe::kRawTile * sizeof(float)));
  float* raw = static_cast<float*>(ctx->scratch.ptr);
  const int rc = launch_pair(ctx, src, table.data(), d_table, (int)n_lm, table.data() + n_lm, d_table + n_lm,
                             (int)items.size(), raw, out, out_dtype, pad_to, stream, kBoth, true, d_wave);
  if (rc) return rc;
  SFE_HIP(mark_last(ctx, stream));
  return SFE_OK;
}

// Runs an entry point's body and turns a C++ exception (host allocation
// failure, thread creation failure) into a status: no exception crosses the
// C ABI.
template <class F>
int guarded(F&& body) {
  try {
    return body();
  } catch (const std::bad_alloc&) {
    g_last_error.clear();  // assigning a message could throw again
    return SFE_HIP_ERROR;
  } catch (const std::exception& e) {
    try {
      return fail(SFE_HIP_ERROR, std::string("host error: ") + e.what());
    } catch (...) {
      return SFE_HIP_ERROR;
    }
  } catch (...) {
    return SFE_HIP_ERROR;
  }
}

Source f32_source(const float* p) { return Source{p, sfe::kPcmF32, 1.0f, sizeof(float)}; }

// The reference's WAV decode divisor: ((1 << (bits - 1)) - 1) as f32
// (examples/transcribe_wav.rs:342-343).  Widths below 2 bits (a zero
// divisor) are rejected.
int pcm_source(const void* p, int32_t pcm, int32_t bits, Source* out) {
  if (pcm == SFE_PCM_F32) {
    *out = f32_source(static_cast<const float*>(p));
    return SFE_OK;
  }
  const int maxbits = pcm == SFE_PCM_I16 ? 16 : (pcm == SFE_PCM_I32 ? 32 : 0);
  if (!maxbits) return fail(SFE_INVALID_ARG, "pcm_format must be SFE_PCM_F32, SFE_PCM_I16 or SFE_PCM_I32");
  if (bits < 2 || bits > maxbits)
    return fail(SFE_INVALID_ARG, "bits_per_sample must be in [2, " + std::to_string(maxbits) + "] for this pcm_format");
  const float scale = (float)((((int64_t)1) << (bits - 1)) - 1);
  *out = Source{p, pcm == SFE_PCM_I16 ? sfe::kPcmI16 : sfe::kPcmI32, scale, pcm == SFE_PCM_I16 ? 2u : 4u};
  return SFE_OK;
}

// Creates the context's internal streams on their first use (each takes
// milliseconds to create: most of what sfe_create took when it made them).
// The caller holds ctx->mu.
hipError_t internal_streams(sfe_ctx* ctx) {
  hipError_t e = hipSuccess;
  if (!ctx->s_compute && (e = hipStreamCreateWithFlags(&ctx->s_compute, hipStreamNonBlocking)) != hipSuccess) {
    ctx->s_compute = nullptr;
    return e;
  }
  if (!ctx->s_copy && (e = hipStreamCreateWithFlags(&ctx->s_copy, hipStreamNonBlocking)) != hipSuccess) {
    ctx->s_copy = nullptr;
    return e;
  }
  return hipSuccess;
}

int check_ctx(sfe_ctx* ctx) {
  if (!ctx) return fail(SFE_INVALID_ARG, "null context");
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
  return SFE_OK;
}

int check_dtype(int32_t d) {
  if (d != SFE_F32 && d != SFE_BF16) return fail(SFE_INVALID_ARG, "out_dtype must be SFE_F32 or SFE_BF16");
  return SFE_OK;
}

}  // namespace

extern "C" {

void sfe_config_default(sfe_config* c) {
  c->sample_rate = 16000;
  c->feature_size = 128;
  c->n_fft = 512;
  c->win_length = 400;
  c->hop_length = 160;
  c->preemphasis = 0.97f;
  c->max_audio_samples = 240000;
  c->samples_per_encoder_frame = 1280;
}

void sfe_overlap_config_default(sfe_overlap_config* c) {
  c->overlap_seconds = 2.0;
  c->context_samples = 1280;
  c->max_model_samples = 240000;
}

int64_t sfe_num_frames(const sfe_config* cfg, int64_t len) {
  const int64_t hop = cfg && cfg->hop_length > 0 ? cfg->hop_length : sfe::kHop;
  return len < 0 ? 0 : len / hop + 1;
}

int64_t sfe_max_feature_frames(const sfe_config* cfg) {
  sfe_config def;
  sfe_config_default(&def);
  const sfe_config* c = cfg ? cfg : &def;
  const int64_t hop = c->hop_length > 0 ? c->hop_length : sfe::kHop;
  return c->max_audio_samples < 0 ? 0 : c->max_audio_samples / hop + 1;
}

int sfe_plan_fast(const sfe_overlap_config* cfg, int64_t audio_len, sfe_chunk* tasks, int32_t cap,
                  int32_t* n_out) {
  return guarded([&]() -> int {
    if (!cfg || !n_out) return fail(SFE_INVALID_ARG, "null argument");
    if (audio_len < 0) return fail(SFE_INVALID_ARG, "negative audio length");
    const int64_t spf = 1280;  // SAMPLES_PER_ENCODER_FRAME, src/constants.rs:4-5
    const int64_t hop = 160;   // MEL_HOP_SAMPLES
    auto sat = [](int64_t a, int64_t b) { return a > b ? a - b : (int64_t)0; };
    // chunk_samples / overlap_samples / stride_samples: src/long_form/planner.rs:105-122
    int64_t raw = std::max(sat(sat(cfg->max_model_samples, cfg->context_samples), hop), spf);
    const int64_t chunk = raw / spf * spf;
    double req_d = cfg->overlap_seconds * 16000.0;
    int64_t req = req_d != req_d || req_d <= 0.0 ? 0 : (req_d >= 9.2e18 ? INT64_MAX : (int64_t)req_d);
    const int64_t overlap = std::min(req, chunk / 2) / spf * spf;
    const int64_t stride = std::max(sat(chunk, overlap), spf) / spf * spf;
    // plan (planner.rs:124-137) + push_overlap_task (long_form.rs:566-582)
    int64_t count = 0;
    int64_t start = 0;
    while (start < audio_len) {
      int64_t end = std::min(start + chunk, audio_len);
      if (tasks && count < cap) {
        int64_t ctx_start = sat(start, cfg->context_samples);
        tasks[count] = {ctx_start, end, start, start - ctx_start};
      }
      ++count;
      if (end == audio_len) break;
      start += stride;
    }
    if (count > INT32_MAX) return fail(SFE_INVALID_ARG, "too many tasks");
    *n_out = (int32_t)count;
    if (count > cap || (!tasks && count > 0)) return fail(SFE_INVALID_ARG, "task buffer too small");
    return SFE_OK;
  });
}

int sfe_build_tables(const sfe_config* cfg, float* window, float* filterbank) {
  return guarded([&]() -> int {
    if (!cfg || cfg->win_length <= 1 || cfg->n_fft <= 0 || cfg->feature_size <= 0 || cfg->sample_rate <= 0)
      return fail(SFE_INVALID_ARG, "invalid config");
    if (window) sfe::hann_window(cfg->win_length, window);
    if (filterbank) sfe::mel_filterbank(cfg->n_fft, cfg->feature_size, cfg->sample_rate, filterbank);
    return SFE_OK;
  });
}

const char* sfe_last_error(void) { return g_last_error.c_str(); }

int sfe_create(const sfe_config* cfg, int32_t device, sfe_ctx** out) {
  return guarded([&]() -> int {
    if (!cfg || !out) return fail(SFE_INVALID_ARG, "null argument");
    *out = nullptr;
    std::string why;
    if (!shape_supported(cfg, &why)) return fail(SFE_INVALID_ARG, why);
    sfe::DevTables host;
    if (!sfe::build_dev_tables(cfg->sample_rate, &host))
      return fail(SFE_INVALID_ARG, "mel filter wider than the kernel's band table");
    int ndev = 0;
    hipError_t e = hipGetDeviceCount(&ndev);
    if (e != hipSuccess || ndev == 0) return fail(SFE_HIP_ERROR, "no HIP device available");
    if (device < 0 || device >= ndev) return fail(SFE_INVALID_ARG, "device index out of range");
    SFE_HIP(hipSetDevice(device));
    sfe_ctx* ctx = new sfe_ctx();
    ctx->cfg = *cfg;
    ctx->device = device;
    ctx->schedule = host.schedule;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && cus > 0)
      ctx->cus = cus;
    auto cleanup = [&](int rc) {
      sfe_destroy(ctx);
      return rc;
    };
    g_allocations.fetch_add(1);
    if ((e = hipMalloc(&ctx->d_tables, sizeof(sfe::DevTables))) != hipSuccess) return cleanup(hip_fail(e, "hipMalloc"));
    if ((e = hipMemcpy(ctx->d_tables, &host, sizeof(host), hipMemcpyHostToDevice)) != hipSuccess)
      return cleanup(hip_fail(e, "hipMemcpy"));
    if ((e = hipEventCreateWithFlags(&ctx->ev_last, hipEventDisableTiming)) != hipSuccess)
      return cleanup(hip_fail(e, "hipEventCreate"));
    if ((e = ctx->h_meta.reserve(sfe::kNoAllocItemBytes)) != hipSuccess) return cleanup(hip_fail(e, "hipHostMalloc"));
    ctx->na_in.reserve(sfe::kNoAllocMaxItems);
    ctx->na_ws.reserve(sfe::kNoAllocMaxItems);
    for (int i = 0; i < 2; ++i) {
      if ((e = hipEventCreateWithFlags(&ctx->ev_copied[i], hipEventDisableTiming)) != hipSuccess)
        return cleanup(hip_fail(e, "hipEventCreate"));
      if ((e = hipEventCreateWithFlags(&ctx->ev_done[i], hipEventDisableTiming)) != hipSuccess)
        return cleanup(hip_fail(e, "hipEventCreate"));
    }
    *out = ctx;
    return SFE_OK;
  });
}

void sfe_destroy(sfe_ctx* ctx) {
  if (!ctx) return;
  (void)hipSetDevice(ctx->device);
  (void)hipDeviceSynchronize();
  if (ctx->d_tables) (void)hipFree(ctx->d_tables);
  ctx->meta.release();
  ctx->h_meta.release();
  ctx->scratch.release();
  ctx->io_in.release();
  ctx->io_out.release();
  ctx->h_io_in.release();
  ctx->h_io_out.release();
  ctx->win.release();
  for (int i = 0; i < 2; ++i) {
    ctx->h_win[i].release();
    if (ctx->ev_copied[i]) (void)hipEventDestroy(ctx->ev_copied[i]);
    if (ctx->ev_done[i]) (void)hipEventDestroy(ctx->ev_done[i]);
  }
  for (hipEvent_t e : ctx->tev) (void)hipEventDestroy(e);
  if (ctx->ev_last) (void)hipEventDestroy(ctx->ev_last);
  if (ctx->s_compute) (void)hipStreamDestroy(ctx->s_compute);
  if (ctx->s_copy) (void)hipStreamDestroy(ctx->s_copy);
  delete ctx;
}

int sfe_extract(sfe_ctx* ctx, const float* audio, int64_t len, float* out, int64_t out_capacity) {
  return guarded([&]() -> int {
    if (len <= 0) return fail(SFE_EMPTY_AUDIO, "audio input was empty");
    if (!audio || !out) return fail(SFE_INVALID_ARG, "null buffer");
    int rc = check_ctx(ctx);
    if (rc) return rc;
    std::lock_guard<std::mutex> lock(ctx->mu);
    const int64_t T = len / sfe::kHop + 1;
    const int64_t nout = T * sfe::kMel;
    if (out_capacity < nout) return fail(SFE_INVALID_ARG, "output buffer too small");
    const size_t in_bytes = (size_t)len * sizeof(float), out_bytes = (size_t)nout * sizeof(float);
    SFE_HIP(ctx->io_in.reserve(in_bytes));
    SFE_HIP(ctx->io_out.reserve(out_bytes));
    SFE_HIP(ctx->h_io_in.reserve(in_bytes));
    SFE_HIP(ctx->h_io_out.reserve(out_bytes));
    SFE_HIP(internal_streams(ctx));
    hipStream_t s = ctx->s_compute;
    parallel_memcpy(ctx->h_io_in.ptr, audio, in_bytes);
    SFE_HIP(hipMemcpyAsync(ctx->io_in.ptr, ctx->h_io_in.ptr, in_bytes, hipMemcpyHostToDevice, s));
    std::vector<Item> items;
    int64_t start = 0, tiles = 0, fo[2];
    if ((rc = build_items(&start, &len, 1, &items, fo, &tiles))) return rc;
    if ((rc = run_items(ctx, f32_source(static_cast<float*>(ctx->io_in.ptr)), items, SFE_F32, ctx->io_out.ptr, s)))
      return rc;
    SFE_HIP(hipMemcpyAsync(ctx->h_io_out.ptr, ctx->io_out.ptr, out_bytes, hipMemcpyDeviceToHost, s));
    SFE_HIP(hipStreamSynchronize(s));
    parallel_memcpy(out, ctx->h_io_out.ptr, out_bytes);
    return SFE_OK;
  });
}

int sfe_prepare_chunk(sfe_ctx* ctx, const float* audio, int64_t len, float* out, int64_t out_capacity,
                      int64_t* feature_frames) {
  return guarded([&]() -> int {
    if (len <= 0) return fail(SFE_EMPTY_AUDIO, "audio input was empty");
    if (!ctx) return fail(SFE_INVALID_ARG, "null context");
    if (len > ctx->cfg.max_audio_samples) {
      char buf[160];
      snprintf(buf, sizeof buf, "audio exceeds the single-chunk limit: actual=%.2fs max=%.2fs",
               (double)len / ctx->cfg.sample_rate, (double)ctx->cfg.max_audio_samples / ctx->cfg.sample_rate);
      return fail(SFE_AUDIO_TOO_LONG, buf);
    }
    int rc = sfe_extract(ctx, audio, len, out, out_capacity);
    if (rc == SFE_OK && feature_frames) *feature_frames = len / sfe::kHop + 1;
    return rc;
  });
}

int sfe_extract_batch(sfe_ctx* ctx, const float* samples, const int64_t* offsets, int32_t n, int32_t out_dtype,
                      void* out, int64_t* frame_offsets, void* stream) {
  return guarded([&]() -> int {
    if (n <= 0 || !offsets || !samples || !out || !frame_offsets) return fail(SFE_INVALID_ARG, "invalid batch arguments");
    int rc = check_dtype(out_dtype);
    if (rc) return rc;
    std::vector<int64_t> starts(n), lens(n);
    for (int32_t i = 0; i < n; ++i) {
      if (offsets[i + 1] < offsets[i] || offsets[i] < 0)
        return fail(SFE_INVALID_ARG, "offsets must be non-negative and non-decreasing");
      starts[i] = offsets[i];
      lens[i] = offsets[i + 1] - offsets[i];
    }
    if ((rc = check_ctx(ctx))) return rc;
    std::lock_guard<std::mutex> lock(ctx->mu);
    std::vector<Item> items;
    int64_t tiles = 0;
    if ((rc = build_items(starts.data(), lens.data(), n, &items, frame_offsets, &tiles))) return rc;
    return run_items(ctx, f32_source(samples), items, out_dtype, out,
                     static_cast<hipStream_t>(stream));
  });
}

int sfe_extract_chunks(sfe_ctx* ctx, const float* recording, int64_t len, const sfe_chunk* tasks, int32_t n,
                       int32_t out_dtype, void* out, int64_t* frame_offsets, void* stream) {
  return sfe_extract_chunks_pcm(ctx, recording, SFE_PCM_F32, 32, len, tasks, n, out_dtype, out, frame_offsets, stream);
}

int sfe_extract_chunks_pcm(sfe_ctx* ctx, const void* recording, int32_t pcm_format, int32_t bits_per_sample,
                           int64_t len, const sfe_chunk* tasks, int32_t n, int32_t out_dtype, void* out,
                           int64_t* frame_offsets, void* stream) {
  return guarded([&]() -> int {
    if (n <= 0 || !tasks || !recording || !out || !frame_offsets) return fail(SFE_INVALID_ARG, "invalid chunk arguments");
    int rc = check_dtype(out_dtype);
    if (rc) return rc;
    Source src;
    if ((rc = pcm_source(recording, pcm_format, bits_per_sample, &src))) return rc;
    std::vector<int64_t> starts(n), lens(n);
    for (int32_t i = 0; i < n; ++i) {
      const sfe_chunk& t = tasks[i];
      if (t.audio_start < 0 || t.audio_end > len || t.audio_end < t.audio_start)
        return fail(SFE_INVALID_ARG, "task " + std::to_string(i) + " lies outside the recording");
      starts[i] = t.audio_start;
      lens[i] = t.audio_end - t.audio_start;
    }
    if ((rc = check_ctx(ctx))) return rc;
    std::lock_guard<std::mutex> lock(ctx->mu);
    std::vector<Item> items;
    int64_t tiles = 0;
    if ((rc = build_items(starts.data(), lens.data(), n, &items, frame_offsets, &tiles))) return rc;
    return run_items(ctx, src, items, out_dtype, out, static_cast<hipStream_t>(stream));
  });
}

int sfe_extract_chunks_padded(sfe_ctx* ctx, const float* recording, int64_t len, const sfe_chunk* tasks, int32_t n,
                              int32_t target_frames, int32_t out_dtype, void* out, int64_t* feature_frames,
                              void* stream) {
  return guarded([&]() -> int {
    if (n <= 0 || !tasks || !recording || !out || !feature_frames || target_frames <= 0)
      return fail(SFE_INVALID_ARG, "invalid chunk arguments");
    int rc = check_dtype(out_dtype);
    if (rc) return rc;
    std::vector<int64_t> starts(n), lens(n), fo(n + 1);
    for (int32_t i = 0; i < n; ++i) {
      const sfe_chunk& t = tasks[i];
      if (t.audio_start < 0 || t.audio_end > len || t.audio_end < t.audio_start)
        return fail(SFE_INVALID_ARG, "task " + std::to_string(i) + " lies outside the recording");
      starts[i] = t.audio_start;
      lens[i] = t.audio_end - t.audio_start;
    }
    if ((rc = check_ctx(ctx))) return rc;
    std::lock_guard<std::mutex> lock(ctx->mu);
    std::vector<Item> items;
    int64_t tiles = 0;
    if ((rc = build_items(starts.data(), lens.data(), n, &items, fo.data(), &tiles))) return rc;
    for (int32_t i = 0; i < n; ++i) {
      // EncoderInputBuffer::copy_from_features rejects more frames than the
      // encoder input holds (src/model.rs:259-264)
      if (items[i].T > target_frames)
        return fail(SFE_INVALID_ARG, "feature frame count " + std::to_string(items[i].T) + " exceeded encoder target " +
                                         std::to_string(target_frames));
      items[i].dst_off = (int64_t)i * sfe::kMel * target_frames;
      feature_frames[i] = items[i].T;
    }
    return run_items(ctx, f32_source(recording), items, out_dtype, out, static_cast<hipStream_t>(stream),
                     target_frames);
  });
}

int sfe_extract_chunks_noalloc(sfe_ctx* ctx, const float* recording, int64_t len, const sfe_chunk* tasks,
                               int32_t n, int32_t out_dtype, void* out, int64_t* frame_offsets, void* stream) {
  // sfe_extract_chunks with the item table and the raw log-mel in this
  // device's static scratch: no device or host allocation on any path that
  // succeeds.  The plan (frames shared as in sfe_extract_chunks) is built in
  // host buffers that sfe_create reserved for kNoAllocMaxItems items: the
  // planner's lists stay within that capacity and std::sort allocates
  // nothing.
  return guarded([&]() -> int {
    if (n <= 0 || !tasks || !recording || !out || !frame_offsets) return fail(SFE_INVALID_ARG, "invalid chunk arguments");
    if (n > sfe::kNoAllocMaxItems)
      return fail(SFE_INVALID_ARG, "sfe_extract_chunks_noalloc takes at most " + std::to_string(sfe::kNoAllocMaxItems) +
                                       " tasks");
    int rc = check_dtype(out_dtype);
    if (rc) return rc;
    int64_t tiles = 0;
    for (int32_t i = 0; i < n; ++i) {
      const sfe_chunk& t = tasks[i];
      if (t.audio_start < 0 || t.audio_end > len || t.audio_end < t.audio_start)
        return fail(SFE_INVALID_ARG, "task " + std::to_string(i) + " lies outside the recording");
      const int64_t L = t.audio_end - t.audio_start;
      if (L == 0) return fail(SFE_EMPTY_AUDIO, "audio input was empty (item " + std::to_string(i) + ")");
      tiles += sfe::tiles_for(L / sfe::kHop + 1);
    }
    // The limit is on the tasks' own regions: a plan with shared frames that
    // would need more tiles than that (tile rounding of the items' first and
    // last quads) is replaced by the plan without sharing.
    const size_t raw_bytes = (size_t)tiles * sfe::kRawTile * sizeof(float);
    if (raw_bytes > sfe::kNoAllocRawBytes)
      return fail(SFE_INVALID_ARG, "sfe_extract_chunks_noalloc: the tasks need " + std::to_string(raw_bytes) +
                                       " bytes of scratch, more than its " + std::to_string(sfe::kNoAllocRawBytes));
    if ((rc = check_ctx(ctx))) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    // Not under stream capture: the pinned item table a captured copy would
    // read is rewritten by every later call on the context, so a replay
    // would upload another call's table.
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    SFE_HIP(hipStreamIsCapturing(s, &cap));
    if (cap != hipStreamCaptureStatusNone)
      return fail(SFE_INVALID_ARG, "sfe_extract_chunks_noalloc cannot be captured into a graph");
    // Calls on one device share its static scratch: the device lock orders
    // them on the host, and its event orders them on the device, whatever
    // context or stream they come from.
    std::unique_lock<std::mutex> dev_lock;
    SFE_HIP(sfe::noalloc_lock(ctx->device, &dev_lock));
    std::lock_guard<std::mutex> lock(ctx->mu);
    const size_t entries = (size_t)(sfe::kPlanEntriesPerItem + 1) * n;
    if (!ctx->noalloc) {
      // The first call on this context looks up the device's static array
      // (the first lookup in the process loads the code object that holds
      // it, about 25 ms; kept out of sfe_create for callers that never use
      // this entry point).  It allocates nothing: the array exists from the
      // library's load.
      void* na = nullptr;
      SFE_HIP(sfe::noalloc_scratch(ctx->device, &na));
      ctx->noalloc = static_cast<unsigned char*>(na);
    }
    if (ctx->h_meta.cap < entries * sizeof(Item) + sfe::kMaxLogmelWaves * sizeof(int32_t) ||
        ctx->na_in.capacity() < (size_t)n)
      return fail(SFE_HIP_ERROR, "context has no reserved planner buffers");
    int64_t fo = 0, own_tiles = 0;
    frame_offsets[0] = 0;
    ctx->na_in.clear();
    for (int32_t i = 0; i < n; ++i) {
      const Item it = sfe::own_item(tasks[i].audio_start, tasks[i].audio_end - tasks[i].audio_start, 0,
                                    (int64_t)sfe::kMel * fo, 0);
      ctx->na_in.push_back(it);
      fo += it.T;
      own_tiles += sfe::tiles_for(it.T);
      frame_offsets[i + 1] = fo;
    }
    // The pinned table is free once its previous upload has finished.
    SFE_HIP(ctx->h_meta.wait());
    Item* table = static_cast<Item*>(ctx->h_meta.ptr);
    size_t n_lm = 0;
    bool share = ctx->share;
    tiles = sfe::plan_table(ctx->na_in.data(), n, share, &ctx->na_ws, table, &n_lm);
    if (share && tiles > own_tiles) tiles = sfe::plan_table(ctx->na_in.data(), n, false, &ctx->na_ws, table, &n_lm);
    sfe::order_norm(table + n_lm, n);
    SFE_HIP(order_after_last(ctx, s));
    SFE_HIP(sfe::noalloc_order(ctx->device, s));
    Item* d_table = reinterpret_cast<Item*>(ctx->noalloc);
    float* raw = reinterpret_cast<float*>(ctx->noalloc + sfe::kNoAllocItemBytes);
    // the table, then the log-mel launch's first-item table, in one copy
    // (the item region holds kMaxLogmelWaves entries past the largest table)
    const size_t tbytes = (n_lm + n) * sizeof(Item);
    const WaveTable wt = wave_table(table, n_lm, ctx->cus);
    if (wt.entries)
      sfe::logmel_wave_items(table, (int)n_lm, wt.u0, wt.n_units, wt.grid,
                             reinterpret_cast<int32_t*>(reinterpret_cast<char*>(table) + tbytes));
    const int32_t* d_wave =
        wt.entries ? reinterpret_cast<const int32_t*>(ctx->noalloc + tbytes) : nullptr;
    SFE_HIP(hipMemcpyAsync(d_table, table, tbytes + wt.entries * sizeof(int32_t), hipMemcpyHostToDevice, s));
    SFE_HIP(hipEventRecord(ctx->h_meta.ev, s));
    ctx->h_meta.pending = true;
    rc = launch_pair(ctx, f32_source(recording), table, d_table, (int)n_lm, table + n_lm, d_table + n_lm, n, raw, out,
                     out_dtype, 0, s, kBoth, false, d_wave);
    if (rc) return rc;
    SFE_HIP(mark_last(ctx, s));
    SFE_HIP(sfe::noalloc_mark(ctx->device, s));
    return SFE_OK;
  });
}

int64_t sfe_vad_num_windows(int64_t len) { return sfe::vad_num_windows(len); }

int sfe_vad_frames(sfe_ctx* ctx, const void* recording, int32_t pcm_format, int32_t bits_per_sample, int64_t len,
                   float* out, int64_t out_windows, void* stream) {
  return guarded([&]() -> int {
    if (len < 0) return fail(SFE_INVALID_ARG, "negative recording length");
    Source src;
    int rc = pcm_source(recording, pcm_format, bits_per_sample, &src);
    if (rc) return rc;
    const int64_t n = sfe::vad_num_windows(len);
    if (n == 0) return SFE_OK;  // empty audio: no windows (src/long_form/vad.rs:67-69)
    if (!recording || !out) return fail(SFE_INVALID_ARG, "null recording or output");
    if (out_windows < n)
      return fail(SFE_INVALID_ARG, "output holds " + std::to_string(out_windows) + " windows, " + std::to_string(n) +
                                       " needed");
    if (reinterpret_cast<uintptr_t>(out) % 16 != 0) return fail(SFE_INVALID_ARG, "output must be 16-byte aligned");
    if (reinterpret_cast<uintptr_t>(recording) % src.esize != 0)
      return fail(SFE_INVALID_ARG, "recording is not aligned to its sample size");
    if ((rc = check_ctx(ctx))) return rc;
    std::lock_guard<std::mutex> lock(ctx->mu);
    hipStream_t s = static_cast<hipStream_t>(stream);
    SFE_HIP(order_after_last(ctx, s));
    SFE_HIP(sfe::launch_vad_frames(src.ptr, src.pcm, src.scale, len, out, s));
    SFE_HIP(mark_last(ctx, s));
    return SFE_OK;
  });
}

int sfe_extract_chunks_streamed(sfe_ctx* ctx, const float* host, int64_t len, const sfe_chunk* tasks, int32_t n,
                                int32_t out_dtype, void* out, int64_t* frame_offsets, int64_t window_samples) {
  return sfe_extract_chunks_streamed_pcm(ctx, host, SFE_PCM_F32, 32, len, tasks, n, out_dtype, out, frame_offsets,
                                         window_samples);
}

int sfe_extract_chunks_streamed_pcm(sfe_ctx* ctx, const void* host_recording, int32_t pcm_format,
                                    int32_t bits_per_sample, int64_t len, const sfe_chunk* tasks, int32_t n,
                                    int32_t out_dtype, void* out, int64_t* frame_offsets, int64_t window_samples) {
  return guarded([&]() -> int {
    const char* host = static_cast<const char*>(host_recording);
    if (n <= 0 || !tasks || !host || !out || !frame_offsets) return fail(SFE_INVALID_ARG, "invalid chunk arguments");
    int rc = check_dtype(out_dtype);
    if (rc) return rc;
    Source src;
    if ((rc = pcm_source(host_recording, pcm_format, bits_per_sample, &src))) return rc;
    const size_t es = src.esize;
    std::vector<int64_t> starts(n), lens(n);
    for (int32_t i = 0; i < n; ++i) {
      const sfe_chunk& t = tasks[i];
      if (t.audio_start < 0 || t.audio_end > len || t.audio_end < t.audio_start)
        return fail(SFE_INVALID_ARG, "task " + std::to_string(i) + " lies outside the recording");
      if (t.audio_end - t.audio_start > window_samples)
        return fail(SFE_INVALID_ARG, "window_samples is shorter than task " + std::to_string(i));
      if (i > 0 && t.audio_start < tasks[i - 1].audio_start)
        return fail(SFE_INVALID_ARG, "tasks must be ordered by audio_start");
      starts[i] = t.audio_start;
      lens[i] = t.audio_end - t.audio_start;
    }
    // A window longer than the recording holds no more than the recording:
    // clamping keeps the device ring and the batch sizes (window_samples
    // times the sample size and the batch count) from overflowing.
    window_samples = std::min(window_samples, std::max<int64_t>(len, 1));
    if ((rc = check_ctx(ctx))) return rc;
    std::lock_guard<std::mutex> lock(ctx->mu);
    std::vector<Item> items;
    int64_t tiles = 0;
    if ((rc = build_items(starts.data(), lens.data(), n, &items, frame_offsets, &tiles))) return rc;

    // Group tasks into windows [wstart, wend) no longer than window_samples.
    struct Group {
      int32_t first, count;
      int64_t wstart, wend;
    };
    std::vector<Group> groups;
    for (int32_t i = 0; i < n;) {
      Group g{i, 0, items[i].start, items[i].start};
      while (i < n && items[i].start + items[i].len - g.wstart <= window_samples) {
        g.wend = std::max(g.wend, items[i].start + items[i].len);
        ++i;
        ++g.count;
      }
      groups.push_back(g);
    }
    // Batches of up to batch_windows consecutive windows.  A batch is copied
    // as one recording range [start, end) into half (bi & 1) of the device
    // buffer, so a window joins a batch only while that range stays within
    // batch_windows * window_samples samples and the gaps between
    // the batch's windows (copied but unused) add up to at most one window.
    // Items are re-based to their half.
    struct Batch {
      size_t g0, g1;
      int64_t start, end;
    };
    const size_t batch_windows =
        std::min(kStreamMaxBatchWindows, std::max<size_t>(1, kStreamBatchBytes / ((size_t)window_samples * es)));
    const int64_t half = (int64_t)batch_windows * window_samples;
    std::vector<Batch> batches;
    for (size_t gi = 0; gi < groups.size();) {
      Batch bt{gi, gi + 1, groups[gi].wstart, groups[gi].wend};
      int64_t covered = groups[gi].wend - groups[gi].wstart;
      for (++gi; gi < groups.size() && bt.g1 - bt.g0 < batch_windows; ++gi) {
        const int64_t end = std::max(bt.end, groups[gi].wend);
        const int64_t cov = covered + (groups[gi].wend - groups[gi].wstart);
        if (end - bt.start > half || (end - bt.start) - std::min(cov, end - bt.start) > window_samples) break;
        bt.end = end;
        covered = cov;
        bt.g1 = gi + 1;
      }
      batches.push_back(bt);
    }
    for (size_t bi = 0; bi < batches.size(); ++bi) {
      const int64_t base = (int64_t)(bi & 1) * half - batches[bi].start;
      for (size_t gi = batches[bi].g0; gi < batches[bi].g1; ++gi)
        for (int32_t i = groups[gi].first; i < groups[gi].first + groups[gi].count; ++i) items[i].start += base;
    }
    // A recording already in pinned (page-locked) host memory is copied to
    // the device directly; pageable memory goes through two pinned staging
    // windows.
    bool pinned = false;
    {
      hipPointerAttribute_t attr;
      if (hipPointerGetAttributes(&attr, host_recording) == hipSuccess) pinned = attr.type == hipMemoryTypeHost;
      (void)hipGetLastError();  // a pageable pointer leaves an error code behind
    }
    SFE_HIP(ctx->win.reserve(2 * (size_t)half * es));
    if (!pinned)
      for (int b = 0; b < 2; ++b) SFE_HIP(ctx->h_win[b].reserve((size_t)half * es));
    SFE_HIP(internal_streams(ctx));
    hipStream_t sc = ctx->s_compute, sx = ctx->s_copy;
    SFE_HIP(order_after_last(ctx, sc));
    SFE_HIP(order_after_last(ctx, sx));
    char* ring = static_cast<char*>(ctx->win.ptr);
    // Batch bi's samples into half (bi & 1) of the ring, on the copy stream.
    auto issue_copy = [&](size_t bi) -> int {
      const Batch& bt = batches[bi];
      const int e = (int)(bi & 1);
      // This half was last read by the log-mel launch of batch bi - 2.
      if (bi >= 2) SFE_HIP(hipStreamWaitEvent(sx, ctx->ev_done[e], 0));
      const size_t bytes = (size_t)(bt.end - bt.start) * es;
      const void* hsrc = host + (size_t)bt.start * es;
      if (!pinned) {
        // the pinned staging buffer is free once its previous H2D copy has finished
        PinBuf& hb = ctx->h_win[e];
        SFE_HIP(hb.wait());
        parallel_memcpy(hb.ptr, hsrc, bytes);
        hsrc = hb.ptr;
      }
      SFE_HIP(hipMemcpyAsync(ring + (size_t)e * (size_t)half * es, hsrc, bytes, hipMemcpyHostToDevice, sx));
      if (!pinned) {
        SFE_HIP(hipEventRecord(ctx->h_win[e].ev, sx));
        ctx->h_win[e].pending = true;
      }
      SFE_HIP(hipEventRecord(ctx->ev_copied[e], sx));
      return SFE_OK;
    };
    // The first batch's copy goes out before the host plans the tables.
    if ((rc = issue_copy(0))) return rc;

    // Per batch, the plan with shared frames (plan_table) over the batch's
    // re-based items: frames that overlapping tasks of one batch share are
    // computed once (tasks of different batches keep their own).  The
    // batches' raw regions follow one another in the scratch; the table is
    // every batch's log-mel entries, then every batch's normalisation
    // entries (item order).
    std::vector<Item> lm_tab, nm_tab;
    std::vector<size_t> lm_at(batches.size() + 1, 0);
    lm_tab.reserve(items.size());
    nm_tab.reserve(items.size());
    {
      sfe::PlanWorkspace ws;
      std::vector<Item> tbl;
      int64_t raw_tiles = 0;
      for (size_t bi = 0; bi < batches.size(); ++bi) {
        const int32_t first = groups[batches[bi].g0].first;
        const int32_t end = groups[batches[bi].g1 - 1].first + groups[batches[bi].g1 - 1].count;
        const int nb = end - first;
        ws.reserve((size_t)nb);
        tbl.resize((size_t)(sfe::kPlanEntriesPerItem + 1) * (size_t)nb);
        size_t n_lm = 0;
        const int64_t bt_tiles = sfe::plan_table(items.data() + first, nb, ctx->share, &ws, tbl.data(), &n_lm);
        const int64_t shift = (int64_t)sfe::kRawTile * raw_tiles;
        for (size_t k = 0; k < n_lm + (size_t)nb; ++k) {
          Item& e = tbl[k];
          e.out_off += shift;
          e.grid_off += shift;
          e.tail_off += shift;
          (k < n_lm ? lm_tab : nm_tab).push_back(e);
        }
        lm_at[bi + 1] = lm_tab.size();
        raw_tiles += bt_tiles;
      }
      tiles = raw_tiles;
    }
    const size_t n_lm_all = lm_tab.size();
    lm_tab.insert(lm_tab.end(), nm_tab.begin(), nm_tab.end());
    const std::vector<Item>& table = lm_tab;  // log-mel entries, then normalisation entries
    const size_t mbytes = table.size() * sizeof(Item);
    ctx->meta_items.clear();  // the table uploaded below is re-based per window group
    SFE_HIP(ctx->h_meta.reserve(mbytes));
    SFE_HIP(ctx->meta.reserve(mbytes));
    SFE_HIP(ctx->scratch.reserve((size_t)tiles * sfe::kRawTile * sizeof(float)));
    float* raw = static_cast<float*>(ctx->scratch.ptr);
    memcpy(ctx->h_meta.ptr, table.data(), mbytes);
    SFE_HIP(hipMemcpyAsync(ctx->meta.ptr, ctx->h_meta.ptr, mbytes, hipMemcpyHostToDevice, sc));
    SFE_HIP(hipEventRecord(ctx->h_meta.ev, sc));
    ctx->h_meta.pending = true;
    const Item* d_items = static_cast<const Item*>(ctx->meta.ptr);
    Source rsrc = src;
    rsrc.ptr = ring;
    int32_t norm_first = 0;
    size_t norm_windows = 0;  // windows featurized since the last normalisation
    for (size_t bi = 0; bi < batches.size(); ++bi) {
      const Batch& bt = batches[bi];
      const int e = (int)(bi & 1);
      if (bi > 0 && (rc = issue_copy(bi))) return rc;
      SFE_HIP(hipStreamWaitEvent(sc, ctx->ev_copied[e], 0));
      const int32_t end = groups[bt.g1 - 1].first + groups[bt.g1 - 1].count;
      const Item* lm = table.data() + lm_at[bi];
      const int n_lm = (int)(lm_at[bi + 1] - lm_at[bi]);
      rc = launch_pair(ctx, rsrc, lm, d_items + lm_at[bi], n_lm, nullptr, nullptr, 0, raw, out, out_dtype, 0, sc,
                       kLogmel);
      if (rc) return rc;
      SFE_HIP(hipEventRecord(ctx->ev_done[e], sc));
      // Normalisation reads only the raw log-mel (all of it stays in HBM), so
      // it runs once per kStreamNormWindows windows or more instead of per
      // batch: one launch over many items instead of many launches over a few.
      norm_windows += bt.g1 - bt.g0;
      if (bi + 1 == batches.size() || norm_windows >= kStreamNormWindows) {
        const size_t nf = n_lm_all + (size_t)norm_first;
        rc = launch_pair(ctx, rsrc, nullptr, nullptr, 0, table.data() + nf, d_items + nf, end - norm_first, raw, out,
                         out_dtype, 0, sc, kNorm);
        if (rc) return rc;
        norm_first = end;
        norm_windows = 0;
      }
    }
    SFE_HIP(hipStreamSynchronize(sc));
    SFE_HIP(hipStreamSynchronize(sx));
    ctx->has_last = false;  // everything has completed
    return SFE_OK;
  });
}

int sfe_set_frame_sharing(sfe_ctx* ctx, int32_t enable) {
  if (!ctx) return fail(SFE_INVALID_ARG, "null context");
  std::lock_guard<std::mutex> lock(ctx->mu);
  ctx->share = enable != 0;
  return SFE_OK;
}

int64_t sfe_debug_allocation_count(void) { return g_allocations.load(); }

int sfe_debug_mel_schedule(const sfe_config* cfg) {
  const int rc = guarded([&]() -> int {
    if (!cfg) return fail(SFE_INVALID_ARG, "null argument");
    std::string why;
    if (!shape_supported(cfg, &why)) return fail(SFE_INVALID_ARG, why);
    std::unique_ptr<sfe::DevTables> t(new sfe::DevTables);
    if (!sfe::build_dev_tables(cfg->sample_rate, t.get()))
      return fail(SFE_INVALID_ARG, "mel filter wider than the kernel's band table");
    return -1 - t->schedule;  // (kept apart from the error codes)
  });
  return rc < 0 ? -1 - rc : -1;
}

int sfe_debug_stamps(void* device_buf, int64_t words) {
  if (!sfe::stamps_built()) return fail(SFE_INVALID_ARG, "this library was built without SFE_TIMESTAMPS");
  if (words < 0 || (!device_buf && words != 0)) return fail(SFE_INVALID_ARG, "invalid stamp buffer");
  hipError_t e = sfe::set_stamp_buffer(device_buf, words);
  if (e != hipSuccess) return hip_fail(e, "set_stamp_buffer");
  return SFE_OK;
}

int sfe_set_timing(sfe_ctx* ctx, int32_t enable) {
  if (!ctx) return fail(SFE_INVALID_ARG, "null context");
  std::lock_guard<std::mutex> lock(ctx->mu);
  ctx->timing = enable != 0;
  ctx->tev_used = 0;
  return SFE_OK;
}

int sfe_get_timing(sfe_ctx* ctx, double* logmel_ms, double* norm_ms, int32_t* launches) {
  return guarded([&]() -> int {
    if (!ctx || !logmel_ms || !norm_ms) return fail(SFE_INVALID_ARG, "null argument");
    std::lock_guard<std::mutex> lock(ctx->mu);
    double a = 0.0, b = 0.0;
    for (size_t i = 0; i + 3 < ctx->tev_used; i += 4) {
      float t0 = 0.f, t1 = 0.f;
      SFE_HIP(hipEventSynchronize(ctx->tev[i + 3]));
      SFE_HIP(hipEventElapsedTime(&t0, ctx->tev[i], ctx->tev[i + 1]));
      SFE_HIP(hipEventElapsedTime(&t1, ctx->tev[i + 2], ctx->tev[i + 3]));
      a += t0;
      b += t1;
    }
    *logmel_ms = a;
    *norm_ms = b;
    if (launches) *launches = (int32_t)(ctx->tev_used / 4);
    ctx->tev_used = 0;
    return SFE_OK;
  });
}

}  // extern "C"
