/*
 * scriptrs_fe.h -- C ABI of the MI355X log-mel front end.
 *
 * This library replaces scriptrs' Parakeet feature extractor
 * (src/frontend.rs:11-241) and the feature-extraction step of its
 * long-form chunk workers (src/long_form.rs:266-314, :584-592).
 * The API is plain C: status codes, plain pointers and sizes.
 * No Rust, torch or HIP types cross it; a `stream` argument is an opaque
 * hipStream_t (NULL = the null stream).
 *
 * Layout convention (matches the reference's memory order).  The
 * reference's `extract` returns an Array2<f32> of logical shape [T, 128]
 * built by `.t().to_owned()` of a [128, T] array (src/frontend.rs:112-115),
 * whose storage is feature-major.  Every output here is therefore
 * [feature_size][T] per item.  Item i starts at element
 * feature_size * frame_offsets[i].
 *
 * Threading: one sfe_ctx per host thread.  The reference extractor is
 * !Sync for the same reason (RefCell workspace, src/frontend.rs:16); calls
 * on one ctx are serialised by an internal mutex.
 * Errors: every entry point returns an sfe_status.  sfe_last_error()
 * returns the calling thread's message for the last failure.  No C++
 * exception crosses this interface: a host allocation or thread failure
 * inside the library returns SFE_HIP_ERROR.
 */
#ifndef SCRIPTRS_FE_H
#define SCRIPTRS_FE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  They map onto the reference's TranscriptionError
 * (src/error.rs:5-40) as follows:
 *   SFE_EMPTY_AUDIO     -> EmptyAudio                  (src/frontend.rs:105-107)
 *   SFE_AUDIO_TOO_LONG  -> AudioTooLong{..}            (src/pipeline.rs:153-158, :205-210)
 *   SFE_INVALID_ARG     -> InvalidModelOutput(message)
 *   SFE_HIP_ERROR       -> InvalidModelOutput(message) (the slot the reference uses
 *                                                      for "fft failed", src/frontend.rs:82-83) */
typedef enum sfe_status {
  SFE_OK = 0,
  SFE_EMPTY_AUDIO = 1,
  SFE_INVALID_ARG = 2,
  SFE_HIP_ERROR = 3,
  SFE_AUDIO_TOO_LONG = 4
} sfe_status;

typedef enum sfe_dtype { SFE_F32 = 0, SFE_BF16 = 1 } sfe_dtype;

/* Input sample formats.  Integer PCM is decoded in the kernel exactly as the
 * reference's WAV reader does (examples/transcribe_wav.rs:342-348,
 * dev-tools/src/bin/compare_parakeet_rs.rs:540-546): value as f32 divided by
 * ((1 << (bits_per_sample - 1)) - 1) as f32, correctly rounded.  SFE_PCM_I16
 * holds samples of 2..16 bits in int16, SFE_PCM_I32 2..32 bits in int32. */
typedef enum sfe_pcm { SFE_PCM_F32 = 0, SFE_PCM_I16 = 1, SFE_PCM_I32 = 2 } sfe_pcm;

/* Mirrors TranscriptionConfig (src/config.rs:11-28, defaults :30-44). */
typedef struct sfe_config {
  int32_t sample_rate;               /* 16000 */
  int32_t feature_size;              /* 128   */
  int32_t n_fft;                     /* 512   */
  int32_t win_length;                /* 400   */
  int32_t hop_length;                /* 160   */
  float preemphasis;                 /* 0.97  */
  int64_t max_audio_samples;         /* 240000 */
  int32_t samples_per_encoder_frame; /* 1280  */
} sfe_config;

/* Mirrors OverlapChunkConfig (src/long_form/planner.rs:85-102). */
typedef struct sfe_overlap_config {
  double overlap_seconds;    /* 2.0    */
  int64_t context_samples;   /* 1280   */
  int64_t max_model_samples; /* 240000 */
} sfe_overlap_config;

/* Mirrors ChunkTask for an overlap window (src/long_form.rs:566-582):
 * the chunk featurized is recording[audio_start, audio_end). */
typedef struct sfe_chunk {
  int64_t audio_start;
  int64_t audio_end;
  int64_t global_sample_offset;
  int64_t context_samples;
} sfe_chunk;

typedef struct sfe_ctx sfe_ctx;

/* ---- host-only helpers (no GPU needed) -------------------------------- */

/* TranscriptionConfig::default() (src/config.rs:30-44). */
void sfe_config_default(sfe_config* cfg);

/* OverlapChunkConfig::default() (src/long_form/planner.rs:94-102). */
void sfe_overlap_config_default(sfe_overlap_config* cfg);

/* Frame count of one item: len / hop + 1 (src/frontend.rs:124-127). */
int64_t sfe_num_frames(const sfe_config* cfg, int64_t len);

/* TranscriptionConfig::max_feature_frames (src/config.rs:50-52). */
int64_t sfe_max_feature_frames(const sfe_config* cfg);

/* Fast-mode long-form plan: OverlapChunkConfig::plan over [0, audio_len)
 * (src/long_form/planner.rs:124-137) mapped through push_overlap_task
 * (src/long_form.rs:566-582), as build_fast_execution_plan does
 * (src/long_form.rs:439-459).  Writes at most `cap` tasks and sets *n_out
 * to the full count.  Returns SFE_INVALID_ARG if cap is too small.  The
 * query pattern (tasks = NULL, cap = 0) also returns SFE_INVALID_ARG
 * and still sets *n_out. */
int sfe_plan_fast(const sfe_overlap_config* cfg, int64_t audio_len, sfe_chunk* tasks, int32_t cap,
                  int32_t* n_out);

/* The host tables the device path uploads.  window[win_length] is
 * hann_window (src/frontend.rs:161-165).  filterbank is
 * [feature_size][n_fft/2+1] (src/frontend.rs:188-223).  Both are built
 * with the reference's f32/f64 operation order.  Either pointer may be
 * NULL. */
int sfe_build_tables(const sfe_config* cfg, float* window, float* filterbank);

/* Message of the calling thread's last failed call ("" if none). */
const char* sfe_last_error(void);

/* ---- device context ---------------------------------------------------- */

/* ParakeetFeatureExtractor::new (src/frontend.rs:88-102).  Builds the
 * tables and uploads them to `device`.  The kernels are specialised to
 * n_fft 512, win 400, hop 160, 128 features; any other shape returns
 * SFE_INVALID_ARG.  preemphasis is free; sample_rate sets the mel band
 * edges, and every rate from 3.5 to 107 kHz fits one of the kernel's two
 * mel schedules (outside it, a rate whose filters do not fit returns
 * SFE_INVALID_ARG: sfe_debug_mel_schedule). */
int sfe_create(const sfe_config* cfg, int32_t device, sfe_ctx** out);
void sfe_destroy(sfe_ctx* ctx);

/* ParakeetFeatureExtractor::extract (src/frontend.rs:104-118).  Takes
 * host audio[len] and writes host out[feature_size * T] (feature-major,
 * T = len/hop + 1).  Fails with SFE_INVALID_ARG if out_capacity (in floats)
 * is smaller.  Synchronous.  len == 0 -> SFE_EMPTY_AUDIO.  As in the
 * reference there is no upper length limit here; that check belongs to
 * sfe_prepare_chunk. */
int sfe_extract(sfe_ctx* ctx, const float* audio, int64_t len, float* out, int64_t out_capacity);

/* ChunkPreparer::prepare / TranscriptionPipeline::prepare_chunk
 * (src/pipeline.rs:201-216, :145-164).  Checks order: empty ->
 * SFE_EMPTY_AUDIO; len > cfg.max_audio_samples -> SFE_AUDIO_TOO_LONG; then
 * sfe_extract.  *feature_frames receives T.  The caller pads to
 * sfe_max_feature_frames() (PreparedChunk::target_frames). */
int sfe_prepare_chunk(sfe_ctx* ctx, const float* audio, int64_t len, float* out, int64_t out_capacity,
                      int64_t* feature_frames);

/* Batched extraction of n independent clips from one device buffer.
 * Clip i is samples[offsets[i], offsets[i+1]).  Dense batches use
 * offsets[i] = i * L; ragged batches use any non-decreasing offsets.
 * Each clip is featurized exactly as one extract() call.  samples and out
 * are device pointers; offsets is host memory with n+1 entries.
 * frame_offsets (host, n+1 entries) receives the prefix sums of T_i.
 * out receives sum(T_i) * feature_size elements of out_dtype.
 * Asynchronous on `stream`.  A clip of length 0 -> SFE_EMPTY_AUDIO. */
int sfe_extract_batch(sfe_ctx* ctx, const float* samples, const int64_t* offsets, int32_t n, int32_t out_dtype,
                      void* out, int64_t* frame_offsets, void* stream);

/* Long-form batched extraction: featurizes n overlapping chunk tasks that
 * all index into one device recording[len], without copying the overlaps.
 * This replaces the per-task ChunkPreparer::prepare calls of the
 * long-form workers (src/long_form.rs:584-592).  Preemphasis restarts at
 * every task's audio_start, as in the reference.  tasks and frame_offsets
 * are host memory.  Asynchronous on `stream`. */
int sfe_extract_chunks(sfe_ctx* ctx, const float* recording, int64_t len, const sfe_chunk* tasks, int32_t n,
                       int32_t out_dtype, void* out, int64_t* frame_offsets, void* stream);

/* sfe_extract_chunks over a device recording in PCM format `pcm_format`
 * (sfe_pcm; bits_per_sample is ignored for SFE_PCM_F32).  The decode to f32
 * (the WAV reader's int -> f32 scaling, examples/transcribe_wav.rs:342-348)
 * is fused into the log-mel kernel's sample loads, so 16-bit input moves half
 * the bytes of f32.  Results equal sfe_extract_chunks on the decoded
 * samples. */
int sfe_extract_chunks_pcm(sfe_ctx* ctx, const void* recording, int32_t pcm_format, int32_t bits_per_sample,
                           int64_t len, const sfe_chunk* tasks, int32_t n, int32_t out_dtype, void* out,
                           int64_t* frame_offsets, void* stream);

/* Encoder-ready long-form extraction: as sfe_extract_chunks, but chunk i is
 * written in the encoder input layout that EncoderInputBuffer::
 * copy_from_features builds on the host (src/model.rs:241-278):
 * out[i * feature_size * target_frames + m * target_frames + t], zero for
 * t >= T_i.  target_frames is PreparedChunk::target_frames
 * (sfe_max_feature_frames(), src/pipeline.rs:160-163).  feature_frames (host,
 * n entries) receives T_i.  A chunk with T_i > target_frames fails with
 * SFE_INVALID_ARG ("feature frame count ... exceeded encoder target ...",
 * src/model.rs:259-264).  Asynchronous on `stream`. */
int sfe_extract_chunks_padded(sfe_ctx* ctx, const float* recording, int64_t len, const sfe_chunk* tasks, int32_t n,
                              int32_t target_frames, int32_t out_dtype, void* out, int64_t* feature_frames,
                              void* stream);

/* Allocation-free variant of sfe_extract_chunks.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (tight
 * serving loops, harnesses that forbid hipMalloc).  It runs the same kernels
 * as sfe_extract_chunks, with the same results (frames that tasks share
 * computed once, as there), but keeps its item table and raw log-mel in a
 * static device array of the library (one per GPU, held until the process
 * ends) instead of the context's growable buffers, and calls no hipMalloc,
 * hipFree or other allocating routine (sfe_create reserves the host
 * buffers its planner uses, about 1.3 MB of pinned memory per context).
 * Its first call on a device looks the array up (hipGetSymbolAddress;
 * about 25 ms once per process while the code object holding the array
 * loads).
 * Limits: at most 4096 tasks, and at most 64 MiB of raw log-mel, which is
 * 8192 tiles of 16 frames per task rounded up (131,072 frames, about 22
 * minutes of audio in 15 s chunks); larger calls return SFE_INVALID_ARG.
 * Every call on one GPU shares that array, from every context: the library
 * serialises such calls on the host and orders them on the device (an event
 * per GPU), so calls from several threads, contexts or streams do not race;
 * they do not overlap on the device either.  It cannot be captured into a
 * HIP graph (its item-table upload reads a pinned buffer that the next call
 * rewrites): on a capturing stream it returns SFE_INVALID_ARG.  Arguments,
 * outputs and errors otherwise as sfe_extract_chunks. */
int sfe_extract_chunks_noalloc(sfe_ctx* ctx, const float* recording, int64_t len, const sfe_chunk* tasks, int32_t n,
                               int32_t out_dtype, void* out, int64_t* frame_offsets, void* stream);

/* Silero VAD model inputs.  Replaces the framing half of the reference's
 * VAD loop (process_coreml_vad, src/long_form/vad.rs:62-99; window 512 and
 * context 64 samples, src/constants.rs:6-11): for each 512-sample window w
 * of the recording, the 576 floats the model is fed, [64 context | 512
 * window].  The first context is zeros; later contexts are the previous
 * window's last 64 samples; a short last window repeats its last sample
 * (vad.rs:81-84).  sfe_vad_num_windows(len) = ceil(len / 512) rows. */
int64_t sfe_vad_num_windows(int64_t len);

/* Writes sfe_vad_num_windows(len) rows of 576 f32 to out (device memory,
 * 16-byte aligned, room for out_windows rows), row-major [n][576].  The
 * recording is a device buffer in PCM format `pcm_format` (sfe_pcm), decoded
 * as in sfe_extract_chunks_pcm.  len == 0 writes nothing and returns SFE_OK
 * (the reference returns an empty probability list for empty audio,
 * vad.rs:67-69).  Asynchronous on `stream`; ordered after the context's
 * earlier calls. */
int sfe_vad_frames(sfe_ctx* ctx, const void* recording, int32_t pcm_format, int32_t bits_per_sample, int64_t len,
                   float* out, int64_t out_windows, void* stream);

/* Streaming long-form extraction from HOST memory.  Tasks are grouped
 * into windows of at most window_samples samples; each window carries every
 * task that ends inside it, plus its left halo.  Consecutive windows form
 * batches of about 64 MB (1 to 64 windows), each copied host->device as one
 * contiguous range and featurized by one launch, double-buffered on two
 * streams: the copy of batch b+1 overlaps the compute of batch b.  Frames
 * that overlapping tasks of one batch share are computed once
 * (sfe_set_frame_sharing), with the same output.  Device
 * memory for the copies: two batches.  `out` is a device buffer sized as for
 * sfe_extract_chunks.  A pinned (page-locked) `host` buffer is copied
 * directly; a pageable one is staged through pinned buffers.  Synchronous:
 * returns after all work completes.  window_samples must be at least the
 * longest task, and tasks must be ordered by audio_start. */
int sfe_extract_chunks_streamed(sfe_ctx* ctx, const float* host_recording, int64_t len, const sfe_chunk* tasks,
                                int32_t n, int32_t out_dtype, void* out, int64_t* frame_offsets,
                                int64_t window_samples);

/* sfe_extract_chunks_streamed over a host recording in PCM format
 * `pcm_format` (see sfe_extract_chunks_pcm): integer PCM crosses PCIe at its
 * own width (2 bytes per sample for 16-bit audio) and is decoded on the
 * GPU. */
int sfe_extract_chunks_streamed_pcm(sfe_ctx* ctx, const void* host_recording, int32_t pcm_format,
                                    int32_t bits_per_sample, int64_t len, const sfe_chunk* tasks, int32_t n,
                                    int32_t out_dtype, void* out, int64_t* frame_offsets, int64_t window_samples);

/* ---- tuning and instrumentation (no reference counterpart) ----------- */

/* Shared frames: on by default.  Overlapping chunk tasks of one call
 * (sfe_extract_chunks, _pcm, _padded, sfe_extract_batch; in the streamed
 * entry points, the tasks of one batch of windows) whose starts agree
 * modulo the hop have identical log-mel for a frame whose 512 padded
 * samples lie, in every task that holds it, after the task's first sample
 * and before its end; such frames are computed once and each task keeps
 * its first and last 4-frame groups.  The output is bitwise the same either
 * way; turning it off makes every task compute all of its frames.
 * sfe_extract_chunks_noalloc and the streamed entry points follow the
 * setting too.  Returns
 * SFE_INVALID_ARG for a null ctx. */
int sfe_set_frame_sharing(sfe_ctx* ctx, int32_t enable);

/* Test hook, no counterpart in the reference: the number of device and
 * pinned host allocations (hipMalloc, hipHostMalloc) the library has made in
 * this process, over all contexts.  It lets a test check that a call
 * allocated nothing. */
int64_t sfe_debug_allocation_count(void);

/* Test hook, no counterpart in the reference: the mel contraction schedule
 * sfe_create would use for cfg (0: the default, which fits 16, 22.05 and
 * 24 kHz; 1: the wider one, 50% more matrix steps), or -1 with SFE_INVALID_ARG's
 * message in sfe_last_error when no schedule fits the filterbank (or the
 * shape is unsupported).  No GPU is used. */
int sfe_debug_mel_schedule(const sfe_config* cfg);

/* Measurement hook, no counterpart in the reference.  In a library built
 * with -DSFE_TIMESTAMPS (python -m scriptrs_amd.build --timestamps, which
 * writes libscriptrs_fe_ts.so; never the product library), the kernels of
 * later launches on the current device write s_memrealtime stamps (100 MHz)
 * into device_buf (words 64-bit words; NULL and 0 turn them off):
 *   log-mel, per wave w = block * waves + wave, words 8w .. 8w + 5: start,
 *   loop entry, end, units processed, (unused), item descriptors loaded;
 *   normalisation, per workgroup b (item * 8 + 16-feature slab), words
 *   524288 + 4b .. + 3: start, first statistics reduced (its loads have
 *   landed), statistics published, end.
 * Stamps past `words` are dropped.  The product library returns
 * SFE_INVALID_ARG. */
int sfe_debug_stamps(void* device_buf, int64_t words);

/* Turn per-kernel timing on or off for ctx.  When on, every launch of the
 * log-mel and normalisation kernels is bracketed by HIP events on the stream
 * it runs on.  Turning it on or off clears the recorded launches. */
int sfe_set_timing(sfe_ctx* ctx, int32_t enable);

/* Waits for the recorded launches and returns the summed durations (ms) of
 * the log-mel and normalisation kernels since the last read.  Clears the
 * record.  *launches (may be NULL) receives the number of launch pairs. */
int sfe_get_timing(sfe_ctx* ctx, double* logmel_ms, double* norm_ms, int32_t* launches);

#ifdef __cplusplus
}
#endif

#endif /* SCRIPTRS_FE_H */
