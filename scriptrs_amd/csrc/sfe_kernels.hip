// CDNA4 (gfx950) kernels of the log-mel front end.
//
// sfe_logmel_kernel fuses, per quad of 4 frames of one item, everything
// ParakeetFeatureExtractor::extract does before normalisation
// (src/frontend.rs:104-147, :150-159):
//   preemphasis restarted at the item start -> 256-zero padding ->
//   400-tap left-aligned Hann window -> 512-point real FFT -> |X|^2 ->
//   128x257 Slaney mel contraction -> ln(x + 2^-24)
// and writes the raw log-mel to scratch in tiles of 16 frames (8 slabs of 16
// features, frame-major inside each slab), in base 2 (the normalisation
// kernel multiplies by ln 2 as it loads).
// sfe_norm_kernel then applies normalize_columns (src/frontend.rs:225-241)
// per (item, feature) and writes the reference's feature-major layout
// ([128][T] per item).
//
// FFT mapping: the 512-point real FFT is a 256-point complex FFT of
// z[m] = r[2m] + i r[2m+1] followed by the even/odd split.  The 256-point
// FFT is 16 x 16: 16 lanes own one frame, each lane holds 16 complex values
// in VGPRs, runs a 16-point DFT, applies the inter-stage twiddles, the 16x16
// transpose goes through LDS (row stride 17 complex, conflict-free), and a
// second 16-point DFT finishes the transform.  A 64-wide wavefront therefore
// transforms 4 frames at once, and every lane of the wave is busy.
// The split partner Z[256-k] is fetched with one cross-lane shuffle per
// value.
#include <hip/hip_runtime.h>

#include "sfe_fft.hpp"
#include "sfe_internal.hpp"
#include "sfe_pcm.hpp"

namespace sfe {

// Measurement builds (compiled with -DSFE_TIMESTAMPS, never the product
// library): the kernels write s_memrealtime stamps (a 100 MHz clock shared
// by all CUs) into a device buffer the host registers with
// sfe_debug_stamps.  Log-mel: per wave (blockIdx * waves + wave) 8 words at
// kStampLogmel: start, loop entry (end of the prologue), end, units
// processed, (unused), item descriptors loaded (after their first use).
// (A stamp after the workgroup barrier of the mel table made the compiler
// spill 42 registers in the main loop, so there is none.)  Normalisation: per workgroup 4 words at kStampNorm: start,
// first statistics reduced (its loads have landed), statistics published,
// end.  Every launch overwrites its region.
#ifdef SFE_TIMESTAMPS
constexpr int64_t kStampLogmel = 0;
constexpr int64_t kStampNorm = 8 * 65536;
__device__ unsigned long long* g_stamps;
__device__ long long g_stamp_words;
__device__ __forceinline__ void stamp(int64_t word, unsigned long long v) {
  if (g_stamps && word < g_stamp_words) g_stamps[word] = v;
}
__device__ __forceinline__ unsigned long long stamp_now() { return __builtin_amdgcn_s_memrealtime(); }
#define SFE_STAMP(word, value) stamp((word), (value))
#else
#define SFE_STAMP(word, value) ((void)0)
#endif

namespace {

// Log-mel workgroups hold independent waves: 4 (three workgroups per CU)
// for launches that do not fill the machine, 12 (one per CU, all of its
// waves sharing one work counter) for those that do.
constexpr int kWavesSmall = kLogmelWavesSmall;
constexpr int kWavesBig = kLogmelWavesBig;
constexpr int kXStride = 17;                         // transpose row stride (complex)
constexpr int kSlot = 16 * kXStride;                 // complex per frame slot
constexpr float kGuard = 5.9604644775390625e-08f;    // 2^-24, src/frontend.rs:111
constexpr float kLn2 = 0.69314718055994531f;

// Orders LDS traffic among the lanes of one wavefront: earlier LDS writes of
// all lanes are visible to later reads, and the compiler keeps LDS accesses
// on their side of it.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Work of one wave: units taken one at a time from its workgroup's range; a
// unit (a quad) is 4 consecutive frames of one item.  Waves are independent
// but for that counter: each owns an LDS
// region in which its quad's samples, FFT transpose and power spectra live
// in turn, and contracts its own 4 frames with all 128 filters on the matrix
// cores (v_mfma_f32_4x4x1_16b_f32).  The only workgroup barrier is the one
// after the A operands of those MFMAs are staged in LDS at kernel start.
constexpr int kSpan = 3 * kHop + kWin;  // samples under 4 consecutive frames (880)
constexpr int kWaveBuf = 4 * kSlot * 2; // floats: 4 transpose slots; also holds the span and the power spectra
constexpr int kPStride = 276;           // floats per power-spectrum row (frame)
static_assert(kSpan <= kWaveBuf, "span must fit the wave buffer");
static_assert(4 * kPStride <= kWaveBuf && kPStride >= kBins && kPStride % 4 == 0, "power rows fit the wave buffer");
constexpr int kSpanVec = (kSpan + 255) / 256;  // 16-byte loads per lane (4)
static_assert(kSpan % 4 == 0, "span is whole float4s");

// The 880 samples under one wave's quad: span sample j is item sample
// s0 + j, valid for j in [jlo, jhi).
template <typename S>
struct Span {
  const S* xb;
  int64_t s0;
  int jlo, jhi;
  bool interior;  // the whole span lies inside the item, after its first sample
};

template <typename S>
__device__ __forceinline__ Span<S> make_span(const Item& it, const S* samples, int u) {
  const int fw = (u - it.unit_off + it.q0) * kQuad;
  Span<S> sp;
  sp.s0 = (int64_t)fw * kHop - kPad;
  sp.jlo = sp.s0 < 0 ? (int)(-sp.s0) : 0;
  sp.jhi = (int)(it.len - sp.s0 < (int64_t)kSpan ? (it.len - sp.s0 > 0 ? it.len - sp.s0 : 0) : (int64_t)kSpan);
  sp.xb = samples + it.start + sp.s0;
  sp.interior = sp.jlo == 0 && sp.jhi == kSpan && sp.s0 > 0;
  return sp;
}

// Issues the loads of an interior span (lane L: samples 4L + 256 h + 0..3)
// and, per lane, the sample before its first vector (4L - 1), which is that
// vector's preemphasis neighbour.  The per-lane address keeps it a vector
// load: a scalar load would share lgkmcnt with LDS, and every later LDS wait
// would also wait for it.  Other spans are read when processed.  Samples
// stay raw (undecoded) in registers until used.
template <typename S>
__device__ __forceinline__ void prefetch_span(const Span<S>& sp, int lane, typename Pcm<S>::V4 (&v)[kSpanVec], S& xm1) {
  if (!sp.interior) return;
#pragma unroll
  for (int h = 0; h < kSpanVec; ++h) {
    const int j = 4 * lane + 256 * h;
    v[h] = Pcm<S>::load4(sp.xb + (j < kSpan ? j : 0));
  }
  xm1 = sp.xb[4 * lane - 1];
}

// Guarded log (src/frontend.rs:111-113) in base 2: log2(v + 2^-24), where
// the guard 2^-24 is already in v (the mel accumulators start at it).  The
// log-mel value is this times ln 2, rounded to f32, which the normalisation
// kernel applies as it loads the raw values (ln2_scale), so the VALU-bound
// log-mel kernel does one operation less per value.  A mel value that adds
// nothing to the guard gives log2(2^-24) = -24 exactly, and -24 * f32(ln 2)
// rounds to f32(ln 2^-24), the reference's value for digital silence.
// Raw value loaded by the normalisation kernel: RN(log2 * ln 2).
__device__ __forceinline__ float4 ln2_scale(float4 v) {
#pragma clang fp contract(off)  // rounded on its own, never fused into a later add
  return make_float4(v.x * kLn2, v.y * kLn2, v.z * kLn2, v.w * kLn2);
}

// Raw log-mel is written in tiles of 16 frames: 8 slabs of 16 features, each
// slab [16 frames][16 features] (1 KB), slab s holding features 16s..16s+15.
// After a quad's MFMAs, lane 4j + n holds filters 4j..4j+3 (chain 0) and
// 64 + 4j..+3 (chain 1) of frame n: two aligned 16-byte stores per lane, and
// one store instruction writes 4 slabs x 256 contiguous bytes.  The
// normalisation kernel, which works per (item, slab), reads 1 KB contiguous
// per load instruction.
__device__ __forceinline__ float4 log4(const f32x4& v) {
  return make_float4(__log2f(v[0]), __log2f(v[1]), __log2f(v[2]), __log2f(v[3]));
}

// Keeps a float4 of MFMA A operands and one of B operands allocated up to
// this point (an empty asm that reads them), placed after their MFMAs with a
// scheduling barrier between.  Otherwise the register allocator may give an
// MFMA a destination overlapping one of its own operands (their last use).
// Whether v_mfma_f32_4x4x1_16b_f32 reads every block's operands before its
// destination is written is not documented, so this kernel never relies on
// it: the build rejects any MFMA whose destination overlaps its A or B
// operand in the generated assembly.
__device__ __forceinline__ void mfma_keep(const float4& a, const float4& b) {
  asm volatile("" ::"v"(a.x), "v"(a.y), "v"(a.z), "v"(a.w), "v"(b.x), "v"(b.y), "v"(b.z), "v"(b.w));
}

template <typename S, int NW, int SCH>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(kLogmelWavesPerSimd, kLogmelWavesPerSimd)))
void sfe_logmel_kernel(const S* __restrict__ samples, const Item* __restrict__ items, int n_items, int unit0,
                       int n_units, const DevTables* __restrict__ tb, float coef, Decode dc, float* __restrict__ out,
                       const int32_t* __restrict__ wave_item) {
  constexpr int kWaves = NW;
  constexpr int kThreads = 64 * NW;
  constexpr int kS0 = kChainSteps[SCH][0], kS1 = kChainSteps[SCH][1];  // mel chain steps
  constexpr int kMelVec = mel_vec(SCH);
  __shared__ __align__(16) float wbuf[kWaves][kWaveBuf];
  __shared__ __align__(16) float4 mel_a[kMelVec][64];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4;  // frame of this lane within the wave's 4
#ifdef SFE_TIMESTAMPS
  // (the word index is recomputed where used: kept live it cost a register)
#define SFE_LOGMEL_WORD (kStampLogmel + 8 * ((int64_t)blockIdx.x * NW + w))
  if (lane == 0) SFE_STAMP(SFE_LOGMEL_WORD, stamp_now());
  int n_done = 0;
#endif
  const int l = lane & 15;
  const int partner = (16 - l) & 15;

  // Work: workgroup b owns units [wb, we) of this launch's [unit0, unit0 +
  // n_units) (items[].unit_off counts in the same numbering; logmel_share,
  // which weights 4-wave grids' slots), and its waves take them one at a
  // time through an LDS counter, so a wave that gets less issue on its SIMD
  // takes fewer units.
  __shared__ int wg_next;
  int wb, we;
  logmel_share(gridDim.x, blockIdx.x, NW, unit0, n_units, &wb, &we);
  if (tid == 0) wg_next = wb + kWaves;  // each wave's first unit is wb + w

  // A operands of the mel MFMAs, shared by the workgroup's waves.
#pragma unroll
  for (int i0 = 0; i0 < kMelVec * 64; i0 += kThreads)  // (a wave-uniform loop)
    if (i0 + tid < kMelVec * 64) mel_a[(i0 + tid) / 64][(i0 + tid) % 64] = tb->mel_a[(i0 + tid) / 64][(i0 + tid) % 64];
  __syncthreads();

  // Per-lane constants: window taps of this lane's FFT inputs, inter-stage
  // twiddles e^{-2 pi i l k1/256}, split twiddles e^{-2 pi i k/512}.
  cf wv[13];
#pragma unroll
  for (int m2 = 0; m2 < 13; ++m2) {
    int n = 2 * l + 32 * m2;  // < 512, taps past 400 are zero
    wv[m2] = {tb->window[n], tb->window[n + 1]};
  }
  // Inter-stage twiddles: tangents for this lane as a first-stage lane,
  // cosines for it as a second-stage lane.  Per-lane table rows, indexed
  // affinely: hipcc 7.2 (LLVM 22) miscompiled an equivalent
  // tw[(l * k1) & 255] gather, loading .y of k1 = 1 from element 2l.
  float tt[16], ct[16];
#pragma unroll
  for (int k1 = 0; k1 < 16; ++k1) {
    tt[k1] = tb->tan256[l * 16 + k1];
    ct[k1] = tb->cos256[l * 16 + k1];
  }
  // split twiddles of bins l + 16 k2, k2 < 8, as (scale, tan or cot)
  float2 spt[8];
#pragma unroll
  for (int k2 = 0; k2 < 8; ++k2) spt[k2] = tb->split[l + 16 * k2];

  float* sb = wbuf[w];
  cf* X = reinterpret_cast<cf*>(sb) + g * kSlot;
  // MFMA B operands: lane 4j + n reads frame n's power from the first bin of
  // block j of each chain.
  const int mj = lane >> 2, mn = lane & 3;
  const float* pb0 = sb + mn * kPStride + tb->k0[0][mj];
  const float* pb1 = sb + mn * kPStride + tb->k0[1][mj];
  // Store offset of this lane's filters within a raw tile: frame row mn,
  // slab mj / 4 (chain 0; chain 1 is 4 slabs on), 4 features at 4 (mj % 4).
  const int so = 16 * mn + 256 * (mj >> 2) + 4 * (mj & 3);

  const int u_first = wb + w;
  if (u_first >= we) {
#ifdef SFE_TIMESTAMPS
    if (lane == 0) {
      const unsigned long long t = stamp_now();
      SFE_STAMP(SFE_LOGMEL_WORD + 1, t);
      SFE_STAMP(SFE_LOGMEL_WORD + 2, t);
      SFE_STAMP(SFE_LOGMEL_WORD + 3, 0ull);
    }
#endif
    return;
  }
  // The unit after the one being prefetched is taken one iteration ahead
  // (lane 0's LDS add), so its result is in by the time it is needed.
  int grab = 0;
  if (lane == 0) grab = atomicAdd(&wg_next, 1);
  // Item descriptors stay in scalar registers: it_c is the item of the unit
  // being prefetched, it_n the item after it, loaded one item ahead so an
  // item boundary never waits on memory.  Every item spans at least one unit.
  int li = 0;
  if (wave_item) {
    li = wave_item[(int64_t)blockIdx.x * NW + w];  // from the host (logmel_wave_items)
  } else {
    int hi = n_items - 1;
    while (li < hi) {
      int mid = (li + hi + 1) >> 1;
      if (items[mid].unit_off <= u_first) li = mid;
      else hi = mid - 1;
    }
  }
  Item it_c = items[li];
  Item it_n = items[li + 1 < n_items ? li + 1 : li];
  // The samples of unit u + 1 are loaded into registers while unit u is
  // transformed, so the global-load latency hides behind the FFT.
  Span<S> sp_n = make_span(it_c, samples, u_first);
#ifdef SFE_TIMESTAMPS
  // (after the first use of the item descriptor, which waits for it)
  if (lane == 0) SFE_STAMP(SFE_LOGMEL_WORD + 5, stamp_now());
#endif
  typename Pcm<S>::V4 nv[kSpanVec] = {};
  S nxm1 = 0;
  prefetch_span(sp_n, lane, nv, nxm1);

  f32x4 acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = acc0;
  // Raw offset (uniform) of the quad whose log-mel is held in acc0/acc1, or -1.
  int64_t pend = -1;

  for (int u = u_first, un; u < we; u = un) {
#ifdef SFE_TIMESTAMPS
    // (stamped here rather than before the loop: there it cost a register)
    if (n_done == 0 && lane == 0) SFE_STAMP(SFE_LOGMEL_WORD + 1, stamp_now());
    n_done = __builtin_amdgcn_readfirstlane(n_done) + 1;
#endif
    const Item it = it_c;
    const Span<S> sp = sp_n;
    // (for a span that is not interior nv holds stale values, decoded and
    // never used)
    float4 cv[kSpanVec];
#pragma unroll
    for (int h = 0; h < kSpanVec; ++h) cv[h] = Pcm<S>::dec4(nv[h], dc);
    const float cxm1 = Pcm<S>::dec(nxm1, dc);

    // From here to the FFT's input reads the wave runs at priority 1: the
    // span's LDS writes, the previous quad's stores and the next quad's
    // loads are a round trip the wave waits on before any arithmetic, and
    // issuing it ahead of the SIMD's other waves (in their FFT arithmetic)
    // shortens that wait (log-mel -1.6% on the 1 h workload, -3% on the
    // 64-clip batch; priority 2 here was less good).
    __builtin_amdgcn_s_setprio(1);
    // ---- 1. preemphasised, zero-padded samples of this wave's 4 frames
    // y[0] = x[0], y[s] = x[s] - coef * x[s-1] (separately rounded, as
    // src/frontend.rs:157 computes it), zero outside [0, L).  The previous
    // quad's MFMA reads of this buffer were issued earlier, and LDS
    // operations of a wave complete in order.
    if (sp.interior) {
#pragma clang fp contract(off)
#pragma unroll
      for (int h = 0; h < kSpanVec; ++h) {
        const int j = 4 * lane + 256 * h;
        // x[j - 1]: for h = 0 the lane's own prefetched neighbour; else lane
        // L - 1's last sample, lane 0 taking the previous vector's lane 63.
        float p0 = cxm1;
        if (h > 0) {
          const float edge = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cv[h - 1].w), 63));
          p0 = __int_as_float(
              __builtin_amdgcn_update_dpp(__float_as_int(edge), __float_as_int(cv[h].w), 0x138, 0xf, 0xf, false));
        }
        float4 y;
        y.x = cv[h].x - coef * p0;
        y.y = cv[h].y - coef * cv[h].x;
        y.z = cv[h].z - coef * cv[h].y;
        y.w = cv[h].w - coef * cv[h].z;
        if (j < kSpan) *reinterpret_cast<float4*>(sb + j) = y;
      }
    } else {
      // span crossing the item's start or end: per-sample bounds
#pragma unroll
      for (int h = 0; h < kSpanVec; ++h) {
        const int j = 4 * lane + 256 * h;
        if (j < kSpan) {
          float y[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
#pragma clang fp contract(off)
            const int je = j + e;
            float v = 0.0f;
            if (je >= sp.jlo && je < sp.jhi) {
              const float cur = Pcm<S>::dec(sp.xb[je], dc);
              // item sample 0 (je == jlo with the span starting before the item)
              v = (je == sp.jlo && sp.s0 <= 0) ? cur : cur - coef * Pcm<S>::dec(sp.xb[je - 1], dc);
            }
            y[e] = v;
          }
          *reinterpret_cast<float4*>(sb + j) = make_float4(y[0], y[1], y[2], y[3]);
        }
      }
    }
    // The previous quad's log-mel goes out while the span's LDS writes land.
    if (pend >= 0) {
      float* o = out + pend;
      *reinterpret_cast<float4*>(o + so) = log4(acc0);
      *reinterpret_cast<float4*>(o + so + 4 * 256) = log4(acc1);
    }
    // Then the next unit's samples are requested.  Vector memory operations
    // complete in issue order, so loading after the stores means the wait
    // for these samples, a quad from now, never waits on fresh stores.
    un = __builtin_amdgcn_readfirstlane(grab);
    if (un < we) {
      if (lane == 0) grab = atomicAdd(&wg_next, 1);
      // (units only increase: the items are walked forward)
      while (li + 1 < n_items && un >= it_n.unit_off) {
        ++li;
        it_c = it_n;
        it_n = items[li + 1 < n_items ? li + 1 : li];
      }
      sp_n = make_span(it_c, samples, un);
      prefetch_span(sp_n, lane, nv, nxm1);
    }
    wave_lds_sync();

    // ---- 2. 512-point real FFT of frame g: lane l owns z[l + 16 m2]
    const float* fin = sb + g * kHop + 2 * l;
    cf zv[13];
#pragma unroll
    for (int m2 = 0; m2 < 12; ++m2) {
      float2 v = *reinterpret_cast<const float2*>(fin + 32 * m2);
      zv[m2] = {v.x, v.y};
    }
    {
      float2 v = make_float2(0.0f, 0.0f);
      if (l < 8) v = *reinterpret_cast<const float2*>(fin + 384);
      zv[12] = {v.x, v.y};
    }
    wave_lds_sync();  // the transpose below reuses the span's LDS
    __builtin_amdgcn_s_setprio(0);
    cf a[16];
    dft16_windowed(zv, wv, a);  // window taps past 400 are zero
#pragma unroll
    for (int k1 = 1; k1 < 16; ++k1) a[k1] = tan_twiddle(a[k1], tt[k1]);
#pragma unroll
    for (int k1 = 0; k1 < 16; ++k1) X[k1 * kXStride + l] = a[k1];
    wave_lds_sync();
    // From the transposed reads to the MFMAs the wave runs at raised priority:
    // it is then on a chain of LDS round trips (transpose, split shuffles,
    // power rows, MFMA operands), and letting it issue ahead of the SIMD's
    // other waves, which are in their FFT arithmetic, shortens that chain
    // (3% on the 1 h workload; raising it for the whole FFT was slower).
    __builtin_amdgcn_s_setprio(2);
#pragma unroll
    for (int m1 = 0; m1 < 16; ++m1) a[m1] = X[l * kXStride + m1];
    dft16_scaled(a, ct);  // a[k2] = Z[l + 16 k2] (the twiddles' cosines applied here)

    // Split partner Z[256 - k] for k = l + 16 k2 lives in lane 16 - l,
    // register 15 - k2 (lane 0 pairs with itself, register (16 - k2) & 15).
    // P holds 4|X|^2 (the 0.25 is folded into the filter weights).  Bins
    // k2 < 8 pair k with 256 - k; bin 128 (lane 0, k2 = 8) is conj Z[128],
    // so P[128] = 4|Z[128]|^2.  All 16 shuffles are issued before the
    // arithmetic that consumes them.
    cf sh[8];
#pragma unroll
    for (int k2 = 0; k2 < 8; ++k2) {
      const cf src = a[15 - k2];
      sh[k2] = {__shfl(src.x, partner, 16), __shfl(src.y, partner, 16)};
    }
    // The power rows overwrite the transpose slots: every lane's reads of
    // them above were issued first.
    float* P = sb + g * kPStride;
#pragma unroll
    for (int k2 = 0; k2 < 8; ++k2) {
      const cf A = a[k2];
      const cf B = (l == 0) ? a[(16 - k2) & 15] : sh[k2];
      float pp, pm;
      if (k2 < 4) split_power<false>(A, B, spt[k2].x, spt[k2].y, pp, pm);
      else split_power<true>(A, B, spt[k2].x, spt[k2].y, pp, pm);
      const int k = l + 16 * k2;
      P[k] = pp;
      P[256 - k] = pm;
    }
    if (l == 0) P[128] = 4.0f * fmaf(a[8].y, a[8].y, a[8].x * a[8].x);
    if constexpr (kBinsWritten[SCH] > kBins) {
      static_assert(kBinsWritten[SCH] - kBins <= 15 && kBinsWritten[SCH] <= kPStride, "zero bins fit the row");
      if (l >= 1 && l <= kBinsWritten[SCH] - kBins) P[256 + l] = 0.0f;  // the zero bins after bin 256
    }
    wave_lds_sync();

    // ---- 3. mel on the matrix cores: block j of chain c accumulates
    // W[64c + 4j + m][k0 + s] . P[frame n][k0 + s] over its steps s, 4 steps
    // (one float4 of A and of B operands) per group; the next group's
    // operands are loaded while this group's MFMAs issue.  Chain 1 alternates
    // between two accumulators so consecutive MFMAs do not wait on each
    // other.
    // The guard 2^-24 of the log (src/frontend.rs:111) is added first
    // instead of last: the accumulators start at it (chain 1's second
    // accumulator at zero).  Digital silence still sums to exactly 2^-24.
    f32x4 c0 = {kGuard, kGuard, kGuard, kGuard}, c1 = c0, c2 = {0.0f, 0.0f, 0.0f, 0.0f};
    float4 a1n = mel_a[kS0 / 4][lane], b1n = *reinterpret_cast<const float4*>(pb1);
    float4 a0n = mel_a[0][lane], b0n = *reinterpret_cast<const float4*>(pb0);
#pragma unroll
    for (int v = 0; v < kS1 / 4; ++v) {
      const float4 a1 = a1n, b1 = b1n, a0 = a0n, b0 = b0n;
      if (v + 1 < kS1 / 4) {
        a1n = mel_a[kS0 / 4 + v + 1][lane];
        b1n = *reinterpret_cast<const float4*>(pb1 + 4 * (v + 1));
      }
      if (v + 1 < kS0 / 4) {
        a0n = mel_a[v + 1][lane];
        b0n = *reinterpret_cast<const float4*>(pb0 + 4 * (v + 1));
      }
      c1 = __builtin_amdgcn_mfma_f32_4x4x1f32(a1.x, b1.x, c1, 0, 0, 0);
      if (v < kS0 / 4) c0 = __builtin_amdgcn_mfma_f32_4x4x1f32(a0.x, b0.x, c0, 0, 0, 0);
      c2 = __builtin_amdgcn_mfma_f32_4x4x1f32(a1.y, b1.y, c2, 0, 0, 0);
      if (v < kS0 / 4) c0 = __builtin_amdgcn_mfma_f32_4x4x1f32(a0.y, b0.y, c0, 0, 0, 0);
      c1 = __builtin_amdgcn_mfma_f32_4x4x1f32(a1.z, b1.z, c1, 0, 0, 0);
      if (v < kS0 / 4) c0 = __builtin_amdgcn_mfma_f32_4x4x1f32(a0.z, b0.z, c0, 0, 0, 0);
      c2 = __builtin_amdgcn_mfma_f32_4x4x1f32(a1.w, b1.w, c2, 0, 0, 0);
      if (v < kS0 / 4) c0 = __builtin_amdgcn_mfma_f32_4x4x1f32(a0.w, b0.w, c0, 0, 0, 0);
      // The group's operands stay allocated past its MFMAs (see mfma_keep).
      __builtin_amdgcn_sched_barrier(0);
      mfma_keep(a1, b1);
      if (v < kS0 / 4) mfma_keep(a0, b0);
    }
    __builtin_amdgcn_s_setprio(0);
    acc0 = c0;
    acc1 = c1 + c2;
    // Every frame of the quad is stored: frames past the item's end land in
    // its last tile's padding, which nothing reads.
    pend = it.out_off + raw_frame((int64_t)(u - it.unit_off + it.q0) * kQuad);
  }
  if (pend >= 0) {
    // the store offset computed afresh from the lane id: kept from the
    // prologue it would stay allocated through the loop (or spill)
    int ln;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
    const int soe = 16 * (ln & 3) + 256 * (ln >> 4) + 4 * ((ln >> 2) & 3);
    float* o = out + pend;
    *reinterpret_cast<float4*>(o + soe) = log4(acc0);
    *reinterpret_cast<float4*>(o + soe + 4 * 256) = log4(acc1);
  }
#ifdef SFE_TIMESTAMPS
  if (lane == 0) {
    SFE_STAMP(SFE_LOGMEL_WORD + 2, stamp_now());
    SFE_STAMP(SFE_LOGMEL_WORD + 3, (unsigned long long)__builtin_amdgcn_readfirstlane(n_done));
  }
#endif
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);                                            // round to nearest even
  return (uint16_t)(u >> 16);
}

// Statistics of a row whose values are all bitwise equal to x0.  This is
// where the reference's sequential f32 sums decide the result: their
// rounding leaves x - mean != 0 (about +-0.93 for digital silence), so the
// sums are replayed on one lane in the reference's order
// (src/frontend.rs:230-236).
__device__ __forceinline__ void constant_row_stats(float x0, int T, float* mean_out, float* sd_out) {
#pragma clang fp contract(off)  // every f32 operation rounded, as the reference's
  float sum = 0.0f;
  for (int t = 0; t < T; ++t) sum = sum + x0;
  const float mean = __fdiv_rn(sum, (float)T);
  const float d = x0 - mean;
  float acc = 0.0f;
  for (int t = 0; t < T; ++t) acc = acc + d * d;
  const float var = __fdiv_rn(acc, (float)T - 1.0f);
  *mean_out = mean;
  *sd_out = __fsqrt_rn(var) + 1e-5f;
}

// normalize_columns (src/frontend.rs:225-241).  Input: raw log-mel in
// 16-frame tiles of 8 slabs (as the log-mel kernel writes it).
// Output: feature-major ([128][T] per item, the reference's memory order).
//
// One workgroup of W waves per (item, slab of F features).  Loads: in round
// j, lane i of wave v holds frame j R + v (256 / F) + i / (F / 4) (R frames
// per round), features 4 (i % (F / 4)) .. + 3 of the slab, as one float4.
// Items of up to R N frames are read from HBM once and held in registers (N
// float4s per lane); longer ones are streamed three times.  Stores: chunks
// of 4 rounds are transposed through LDS and each lane writes 4 consecutive
// frames of one feature row, so a store instruction covers F / W rows of
// contiguous bytes (rows are only 4-byte aligned when T is odd; gfx950 takes
// unaligned 16-byte stores).
//
// Statistics: per-lane sums of (x - x0) (x0 the feature's first value) in
// f32 over at most kNormFlush values, accumulated in f64, then reduced
// across lanes by shuffles and across waves through LDS, always in the same
// order, so results are deterministic; the sum of squared deviations from
// the f32 mean likewise.  Then out = (x - mean) / (sqrt(var) + 1e-5) in
// f32, var over T - 1 (T == 1 gives NaN, as the reference).  A feature whose
// values are all equal replays the reference's sequential f32 sums
// (constant_row_stats).
constexpr int kNormBatch = 8;                  // rounds of loads in flight on the streaming path
// Fourth word of a raw buffer resource (no format conversion, no swizzle).
constexpr int kBufWord3 = 0x00020000;
constexpr int kNormFlush = 8;                  // f32 partial sums span at most this many values

// Shape of a normalisation workgroup: W waves, a slab of F features.
template <int W, int F>
struct NormShape {
  static_assert(F == 16, "slabs of 16 features (half a 128-byte frame line)");
  static constexpr int kThreads = 64 * W;
  static constexpr int kLanesPerFrame = F / 4;            // float4 per lane
  static constexpr int kGroup = 64 / kLanesPerFrame;      // frames per load instruction
  static constexpr int kSpan = kGroup * W;                // frames per round
  static constexpr int kChunk = 4 * kSpan;                // frames per LDS transpose
  static constexpr int kTStride = kChunk + 4;             // LDS row stride (floats), rows 16-byte aligned
  static constexpr int kRowsPerWave = F / W;
  static constexpr int kLanesPerRow = 64 / kRowsPerWave;  // each writes 4 frames per store
  static constexpr int kSlabs = kMel / F;
  static_assert(4 * kLanesPerRow == kSpan, "a store instruction covers one round of a row");
};

__device__ __forceinline__ float comp(const float4& v, int c) {
  return c == 0 ? v.x : (c == 1 ? v.y : (c == 2 ? v.z : v.w));
}

// Sum over the lanes that hold the same features (lane % L equal).
template <int L>
__device__ __forceinline__ double group_sum(double v) {
#pragma unroll
  for (int off = L; off < 64; off <<= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Workgroup reduction of 4 per-lane partials (features 4 q .. 4 q + 3,
// q = lane % (F / 4)) into the totals over the item; every lane gets the
// totals of its own 4 features.  red holds W x F doubles.
template <int W, int F>
__device__ __forceinline__ void slab_sum(double (&v)[4], double* red, int lane, int w) {
  constexpr int L = F / 4;
#pragma unroll
  for (int c = 0; c < 4; ++c) v[c] = group_sum<L>(v[c]);
  if (lane < L) {
#pragma unroll
    for (int c = 0; c < 4; ++c) red[w * F + 4 * lane + c] = v[c];
  }
  __syncthreads();
  const int q = lane % L;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    double t = 0.0;
#pragma unroll
    for (int u = 0; u < W; ++u) t += red[u * F + 4 * q + c];
    v[c] = t;
  }
  __syncthreads();  // red is reused by the next reduction
}

// slab_sum of s together with the workgroup AND of the flags f (one LDS
// round for both).
template <int W, int F>
__device__ __forceinline__ void slab_sum_all(double (&v)[4], bool (&f)[4], double* red, int* redi, int lane, int w) {
  constexpr int L = F / 4;
  unsigned m = 0;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    v[c] = group_sum<L>(v[c]);
    m |= (f[c] ? 1u : 0u) << c;
  }
#pragma unroll
  for (int off = L; off < 64; off <<= 1) m &= __shfl_xor(m, off, 64);
  if (lane < L) {
#pragma unroll
    for (int c = 0; c < 4; ++c) red[w * F + 4 * lane + c] = v[c];
    redi[w * L + lane] = (int)m;
  }
  __syncthreads();
  const int q = lane % L;
  unsigned t = 0xfu;
#pragma unroll
  for (int u = 0; u < W; ++u) t &= (unsigned)redi[u * L + q];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    double a = 0.0;
#pragma unroll
    for (int u = 0; u < W; ++u) a += red[u * F + 4 * q + c];
    v[c] = a;
    f[c] = (t >> c) & 1u;
  }
  __syncthreads();  // red is reused by the next reduction
}

// (x - mean) / sd, correctly rounded, from r = RN(1 / sd): q = RN(d r) is
// within one ulp of d / sd, and one residual step q + r fma(-sd, q, d)
// rounds to RN(d / sd) (Markstein's theorem; d and sd are far from overflow
// and underflow here).  Three VALU operations instead of a full division.
__device__ __forceinline__ float norm_div(float x, float mean, float sd, float r) {
  const float d = __fsub_rn(x, mean);
  const float q = __fmul_rn(d, r);
  return __fmaf_rn(__fmaf_rn(-sd, q, d), r, q);
}

// s holds sums of (x - x0) (x0 the feature's first value), q sums of
// squared deviations from the f32 mean, both reduced over the item.
// Per-feature (mean, sd, 1/sd) of the slab, published in LDS for the store
// phase by wave 0's lanes 0 .. F - 1, one feature each (lane i: feature
// 4 (i % (F / 4)) + i / (F / 4), whose totals it holds).
template <int F>
__device__ __forceinline__ void publish_stats(const double (&s)[4], const double (&q)[4], const bool (&cst)[4],
                                              const float4& x0, int T, int lane, int w, float* st) {
  constexpr int L = F / 4;
  if (w == 0 && lane < F) {
    const int c = lane / L;
    const int f = 4 * (lane % L) + c;
    const double S = c == 0 ? s[0] : (c == 1 ? s[1] : (c == 2 ? s[2] : s[3]));
    const double Q = c == 0 ? q[0] : (c == 1 ? q[1] : (c == 2 ? q[2] : q[3]));
    const bool k = c == 0 ? cst[0] : (c == 1 ? cst[1] : (c == 2 ? cst[2] : cst[3]));
    const float xf = comp(x0, c);
    float mean, sd;
    if (k) {
      constant_row_stats(xf, T, &mean, &sd);
    } else {
      mean = (float)((double)xf + S / (double)T);
      sd = __fadd_rn(__fsqrt_rn((float)(Q / (double)(T - 1))), 1e-5f);
    }
    st[3 * f] = mean;
    st[3 * f + 1] = sd;
    st[3 * f + 2] = __fdiv_rn(1.0f, sd);
  }
  __syncthreads();
}

__device__ __forceinline__ void put4(float* o, float4 y) {
  typedef float f4u __attribute__((ext_vector_type(4), aligned(4)));
  *reinterpret_cast<f4u*>(o) = f4u{y.x, y.y, y.z, y.w};
}
__device__ __forceinline__ void put4(uint16_t* o, float4 y) {
  typedef uint16_t u4u __attribute__((ext_vector_type(4), aligned(2)));
  *reinterpret_cast<u4u*>(o) = u4u{f32_to_bf16(y.x), f32_to_bf16(y.y), f32_to_bf16(y.z), f32_to_bf16(y.w)};
}
__device__ __forceinline__ void put1(float* o, float y) { *o = y; }
__device__ __forceinline__ void put1(uint16_t* o, float y) { *o = f32_to_bf16(y); }

// Store phase of one chunk: its frames are in tb[F][kTStride]
// (feature-major); wave v writes rows R v .. R v + R - 1 (R = F / W).
template <int W, int F, typename O>
__device__ __forceinline__ void store_chunk(const float* tb, const float* st, int t0, int T, int rs, int lane, int w,
                                            O* __restrict__ ob) {
  using S = NormShape<W, F>;
  const int r = S::kRowsPerWave * w + lane / S::kLanesPerRow;
  const float mean = st[3 * r], sd = st[3 * r + 1], rc = st[3 * r + 2];
  O* orow = ob + (size_t)r * rs;
#pragma unroll
  for (int s = 0; s < S::kChunk / S::kSpan; ++s) {
    const int k = 4 * (lane % S::kLanesPerRow) + S::kSpan * s;
    const float4 x = *reinterpret_cast<const float4*>(tb + r * S::kTStride + k);
    const float4 y = make_float4(norm_div(x.x, mean, sd, rc), norm_div(x.y, mean, sd, rc),
                                 norm_div(x.z, mean, sd, rc), norm_div(x.w, mean, sd, rc));
    const int t = t0 + k;
    if (t + 3 < T) {
      put4(orow + t, y);
    } else {
      if (t < T) put1(orow + t, y.x);
      if (t + 1 < T) put1(orow + t + 1, y.y);
      if (t + 2 < T) put1(orow + t + 2, y.z);
    }
  }
}

// Zeroes frames [T, rs) of the slab's F rows (the encoder-input padding,
// src/model.rs:266-271).
template <int W, int F, typename O>
__device__ __forceinline__ void zero_tail(O* __restrict__ ob, int T, int rs, int lane, int w) {
  const int tail = rs - T;
  for (int e = w * 64 + lane; e < F * tail; e += W * 64) put1(ob + (size_t)(e / tail) * rs + T + e % tail, 0.0f);
}

// Stage one round's float4 (4 features of one frame) of the lane into the
// transpose buffer at column col.
template <int W, int F>
__device__ __forceinline__ void stage(float* tb, int q, int col, const float4& v) {
  constexpr int ts = NormShape<W, F>::kTStride;
  tb[(4 * q + 0) * ts + col] = v.x;
  tb[(4 * q + 1) * ts + col] = v.y;
  tb[(4 * q + 2) * ts + col] = v.z;
  tb[(4 * q + 3) * ts + col] = v.w;
}

// W waves, slab of F features, N float4 registers per lane: items of up to
// kSpan * N frames are held in registers and read once; the X rounds after
// those (a multiple of 8) are read again for the variance and the stores
// (mostly cache hits), and longer items take the streaming path (three
// passes).  Every path sums the same rounds in the same groups of
// kNormFlush, so the class does not change the result.  `work` is the
// (item, slab) index.
template <int W, int F, int N, int X, typename O>
__device__ __forceinline__ void norm_body(const float* __restrict__ raw, const Item* __restrict__ items,
                                          int n_items, int work, int pad_to, O* __restrict__ out) {
  static_assert(N % 4 == 0, "whole chunks");
  using S = NormShape<W, F>;
  constexpr int kSpan = S::kSpan;
  constexpr int kChunk = S::kChunk;
  __shared__ double red[W * F];
  __shared__ int redi[W * (F / 4)];
  __shared__ float st[3 * F];
  // Two transpose buffers in the 4-wave form (chunk ch stages into tb[ch %
  // 2]: the next chunk's staging does not wait for this chunk's stores, one
  // barrier per chunk); one in the 8-wave form, whose buffer is twice as
  // large.
  constexpr int kTBufs = W == 4 ? 2 : 1;
  __shared__ __align__(16) float tb[kTBufs][F * S::kTStride];
  const int item = work / S::kSlabs;
  if (item >= n_items) return;
#ifdef SFE_TIMESTAMPS
  const int64_t sn = kStampNorm + 4 * (int64_t)work;
  if (threadIdx.x == 0) SFE_STAMP(sn, stamp_now());
#endif
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int q = lane % S::kLanesPerFrame;
  const int fr = w * S::kGroup + lane / S::kLanesPerFrame;  // frame of this lane in each round
  const int slab = (work % S::kSlabs) * F;
  const Item it = items[item];
  const int T = it.T;
  // Frame f of the item, features 4 q .. 4 q + 3 of this slab: from the
  // shared region for f in [f_lo, f_hi], else from the item's own first or
  // last tiles (raw_frame: 16-frame tiles, the slab 1 KB frame-major inside).
  static_assert(F == 16 && S::kGroup == 16, "one wave's load covers one tile of one slab");
  // Loads address a uniform base (the start of the item's shared frames,
  // this slab) plus a 32-bit per-lane byte offset: an item's own first and
  // last tiles come after its shared region (at most kMaxShareFrames
  // frames, then at most 3 tiles for each of at most kMaxShareMembers
  // members), and an item with its own region has all three at out_off.  The region is chosen by adding differences under
  // conditions (a choice among several values compiles to a table in
  // private memory).  The own first tile holds frames below f_lo <= 16, so
  // only round 0 can reach it.
  const int f_lo = it.f_lo, f_hi = it.f_hi;
  const char* bg = reinterpret_cast<const char*>(raw + it.grid_off + 256 * (slab / 16));
  // Frame 0 is always at out_off: below f_lo for an item that shares
  // frames, and an item with its own region has grid_off = out_off.
  const float4* p0 = reinterpret_cast<const float4*>(raw + it.out_off + 256 * (slab / 16) + 4 * q);
  // This lane's frame in round j is fr + kSpan j, kSpan / 16 tiles on from
  // round 0 in whichever region holds it.
  static_assert(kSpan % 16 == 0 && kSpan > 16, "rounds are whole tiles, past the own first tile");
  constexpr uint32_t kRound = 4u * kRawTile * (kSpan / 16);  // bytes
  const uint32_t og = 4u * (uint32_t)(raw_frame(fr + it.gshift) + 4 * q);
  const uint32_t dlo = 4u * (uint32_t)(it.out_off - it.grid_off + raw_frame(fr) - raw_frame(fr + it.gshift));
  const uint32_t dhi = 4u * (uint32_t)(it.tail_off - it.grid_off + raw_frame(fr) - raw_frame(fr + it.gshift));
  const int flo = f_lo - fr, fhi = f_hi - fr;  // round j holds frame fr + kSpan j
  auto roff = [og, dlo, dhi, flo, fhi](int j) -> uint32_t {
    const int d = kSpan * j;
    uint32_t o = og + kRound * (uint32_t)j + (d > fhi ? dhi : 0u);
    if (j == 0) o += flo > 0 ? dlo : 0u;
    return o;
  };
  auto round = [roff, bg](int j) -> const float4* { return reinterpret_cast<const float4*>(bg + roff(j)); };
  const int rs = pad_to > 0 ? pad_to : T;  // output row length
  O* ob = out + it.dst_off + (size_t)slab * rs;
  if (pad_to > 0) zero_tail<W, F>(ob, T, rs, lane, w);
  const int nr = fr < T ? (T - 1 - fr) / kSpan + 1 : 0;  // rounds holding a frame of this lane
  const float4 x0 = ln2_scale(*p0);

  double s[4] = {0.0, 0.0, 0.0, 0.0}, sq[4] = {0.0, 0.0, 0.0, 0.0};
  bool eq[4] = {true, true, true, true};
  if constexpr (N > 0) {
    if (T <= kSpan * (N + X)) {
      float4 v[N];
      // Raw buffer loads from the uniform base, all issued before any is
      // used (a load under a per-lane branch would wait for itself).  Rounds
      // past the lane's frames take an offset past the buffer's range: the
      // hardware returns zeros for them without a memory access, and the
      // select below replaces them.
      const __amdgpu_buffer_rsrc_t rsrc =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(bg), 0, kNormBufRange, kBufWord3);
#pragma unroll
      for (int j = 0; j < N; ++j)
        v[j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                              rsrc, (int)(j < nr ? roff(j) : kNormBufRange), 0, 0));
#pragma unroll
      for (int j = 0; j < N; ++j) v[j] = j < nr ? ln2_scale(v[j]) : x0;  // x0 padding keeps the constancy test exact
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        float a = 0.0f;
#pragma unroll
        for (int j = 0; j < N; ++j) {
          a += comp(v[j], c) - comp(x0, c);  // exactly 0 for the x0 padding past nr
          eq[c] = eq[c] && (comp(v[j], c) == comp(x0, c));
          if ((j + 1) % kNormFlush == 0 || j + 1 == N) {
            s[c] += (double)a;
            a = 0.0f;
          }
        }
      }
      // Round j >= N, loaded again in each pass.  The round index passes
      // through an empty asm so that the offset and the lane test are
      // computed afresh in each pass: shared between passes, they stay live
      // over the whole kernel (one VGPR and one lane mask per round).
      auto reload = [&](int j) -> float4 {
        asm volatile("" : "+s"(j));
        const int o = (int)(j < nr ? roff(j) : kNormBufRange);
        const float4 e = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, o, 0, 0));
        return j < nr ? ln2_scale(e) : x0;
      };
      if constexpr (X > 0) {
        static_assert(N % kNormFlush == 0 && X % kNormFlush == 0, "whole flush groups");
        float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 1
        for (int g = 0; g < X / 4; ++g) {
          float4 e[4];
#pragma unroll
          for (int jr = 0; jr < 4; ++jr) e[jr] = reload(N + 4 * g + jr);
#pragma unroll
          for (int c = 0; c < 4; ++c) {
#pragma unroll
            for (int jr = 0; jr < 4; ++jr) {
              a[c] += comp(e[jr], c) - comp(x0, c);  // exactly 0 past nr (x0)
              eq[c] = eq[c] && (comp(e[jr], c) == comp(x0, c));
            }
            if ((4 * g + 4) % kNormFlush == 0) {
              s[c] += (double)a[c];
              a[c] = 0.0f;
            }
          }
        }
      }
      slab_sum_all<W, F>(s, eq, red, redi, lane, w);
#ifdef SFE_TIMESTAMPS
      if (threadIdx.x == 0) SFE_STAMP(sn + 1, stamp_now());
#endif
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float m = (float)((double)comp(x0, c) + s[c] / (double)T);
        float a = 0.0f;
#pragma unroll
        for (int j = 0; j < N; ++j) {
          const float d = comp(v[j], c) - m;
          if (j < nr) a += d * d;
          if ((j + 1) % kNormFlush == 0 || j + 1 == N) {
            sq[c] += (double)a;
            a = 0.0f;
          }
        }
      }
      if constexpr (X > 0) {
        float m[4], a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < 4; ++c) m[c] = (float)((double)comp(x0, c) + s[c] / (double)T);
#pragma unroll 1
        for (int g = 0; g < X / 4; ++g) {
          float4 e[4];
#pragma unroll
          for (int jr = 0; jr < 4; ++jr) e[jr] = reload(N + 4 * g + jr);
#pragma unroll
          for (int c = 0; c < 4; ++c) {
#pragma unroll
            for (int jr = 0; jr < 4; ++jr) {
              const float d = comp(e[jr], c) - m[c];
              if (N + 4 * g + jr < nr) a[c] += d * d;
            }
            if ((4 * g + 4) % kNormFlush == 0) {
              sq[c] += (double)a[c];
              a[c] = 0.0f;
            }
          }
        }
      }
      slab_sum<W, F>(sq, red, lane, w);
      publish_stats<F>(s, sq, eq, x0, T, lane, w, st);
#ifdef SFE_TIMESTAMPS
      if (threadIdx.x == 0) SFE_STAMP(sn + 2, stamp_now());
#endif
      const int chunks = (T + kChunk - 1) / kChunk;
#pragma unroll
      for (int ch = 0; ch < (N + X) / 4; ++ch) {
        if (ch < chunks) {
          float* t = tb[ch % kTBufs];
          if (ch < N / 4) {
#pragma unroll
            for (int jr = 0; jr < 4; ++jr) stage<W, F>(t, q, kSpan * jr + fr, v[4 * ch + jr]);
          } else {
#pragma unroll
            for (int jr = 0; jr < 4; ++jr) stage<W, F>(t, q, kSpan * jr + fr, reload(4 * ch + jr));
          }
          __syncthreads();
          store_chunk<W, F>(t, st, kChunk * ch, T, rs, lane, w, ob);
          if (kTBufs == 1) __syncthreads();
        }
      }
#ifdef SFE_TIMESTAMPS
      if (threadIdx.x == 0) SFE_STAMP(sn + 3, stamp_now());
#endif
      return;
    }
  }

  // Streaming: three passes over the item, kNormBatch rounds of loads in
  // flight per lane (the second and third passes mostly hit the caches).
  constexpr int G = kNormBatch;
  for (int j0 = 0; j0 < nr; j0 += G) {
    float4 e[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int j = j0 + g < nr ? j0 + g : j0;  // in bounds; unused when past the item
      e[g] = ln2_scale(*round(j));
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float a = 0.0f;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        if (j0 + g < nr) {
          a += comp(e[g], c) - comp(x0, c);
          eq[c] = eq[c] && (comp(e[g], c) == comp(x0, c));
        }
      }
      s[c] += (double)a;
    }
  }
  slab_sum_all<W, F>(s, eq, red, redi, lane, w);
#ifdef SFE_TIMESTAMPS
  if (threadIdx.x == 0) SFE_STAMP(sn + 1, stamp_now());
#endif
  float m[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) m[c] = (float)((double)comp(x0, c) + s[c] / (double)T);
  for (int j0 = 0; j0 < nr; j0 += G) {
    float4 e[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int j = j0 + g < nr ? j0 + g : j0;  // in bounds; unused when past the item
      e[g] = ln2_scale(*round(j));
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float a = 0.0f;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float d = comp(e[g], c) - m[c];
        if (j0 + g < nr) a += d * d;
      }
      sq[c] += (double)a;
    }
  }
  slab_sum<W, F>(sq, red, lane, w);
  publish_stats<F>(s, sq, eq, x0, T, lane, w, st);
#ifdef SFE_TIMESTAMPS
  if (threadIdx.x == 0) SFE_STAMP(sn + 2, stamp_now());
#endif
  const int chunks = (T + kChunk - 1) / kChunk;
  for (int ch = 0; ch < chunks; ++ch) {
    float4 e[4];
#pragma unroll
    for (int jr = 0; jr < 4; ++jr) {
      // past the item: the item's first frame (always in bounds), unused
      const int j = 4 * ch + jr;
      e[jr] = ln2_scale(*(j < nr ? round(j) : p0));
    }
    float* t = tb[ch % kTBufs];
#pragma unroll
    for (int jr = 0; jr < 4; ++jr)
      if (4 * ch + jr < nr) stage<W, F>(t, q, kSpan * jr + fr, e[jr]);
    __syncthreads();
    store_chunk<W, F>(t, st, kChunk * ch, T, rs, lane, w, ob);
    if (kTBufs == 1) __syncthreads();
  }
#ifdef SFE_TIMESTAMPS
  if (threadIdx.x == 0) SFE_STAMP(sn + 3, stamp_now());
#endif
}

// Workgroups of kNormMainWaves waves over 16-feature slabs, three per CU;
// workgroup b normalises slab b % 8 of item b / 8.
constexpr int kNormMainWaves = 4;
constexpr int kNormMainSlab = 16;

template <int N, int X, typename O>
__global__ __launch_bounds__(64 * kNormMainWaves) void sfe_norm_kernel(const float* __restrict__ raw,
                                                                       const Item* __restrict__ items, int n_items,
                                                                       int pad_to, O* __restrict__ out) {
  norm_body<kNormMainWaves, kNormMainSlab, N, X>(raw, items, n_items, blockIdx.x, pad_to, out);
}

// Calls of few items (a clip, a small batch) leave most CUs idle with 4-wave
// workgroups, and each workgroup's loads, reductions and stores run one
// after another: 8-wave workgroups (128 frames per round, 33 KB of LDS for
// the 512-frame transpose chunks) put twice the waves on each slab.
constexpr int kNormWideWaves = 8;
constexpr int kNormWideMaxItems = 16;

template <int N, typename O>
__global__ __launch_bounds__(64 * kNormWideWaves) void sfe_norm_wide_kernel(const float* __restrict__ raw,
                                                                            const Item* __restrict__ items,
                                                                            int n_items, int pad_to,
                                                                            O* __restrict__ out) {
  norm_body<kNormWideWaves, kNormMainSlab, N, 0>(raw, items, n_items, blockIdx.x, pad_to, out);
}

}  // namespace

bool stamps_built() {
#ifdef SFE_TIMESTAMPS
  return true;
#else
  return false;
#endif
}

hipError_t set_stamp_buffer(void* buf, int64_t words) {
#ifdef SFE_TIMESTAMPS
  unsigned long long* p = static_cast<unsigned long long*>(buf);
  long long n = words;
  hipError_t e = hipMemcpyToSymbol(HIP_SYMBOL(g_stamps), &p, sizeof(p));
  if (e == hipSuccess) e = hipMemcpyToSymbol(HIP_SYMBOL(g_stamp_words), &n, sizeof(n));
  return e;
#else
  (void)buf;
  (void)words;
  return hipErrorNotSupported;
#endif
}

int64_t tiles_for(int64_t T) { return (T + kTile - 1) / kTile; }
int64_t units_for(int64_t T) { return (T + kQuad - 1) / kQuad; }

template <int NW, int SCH>
hipError_t launch_logmel_t(const void* samples, int pcm, const Decode& dc, const Item* items, int n_items, int unit0,
                           int n_units, const DevTables* tables, float preemph, float* raw_out, int grid,
                           const int32_t* wave_item, hipStream_t stream) {
  const dim3 g(grid), b(64 * NW);
  if (pcm == kPcmI16)
    sfe_logmel_kernel<int16_t, NW, SCH><<<g, b, 0, stream>>>(static_cast<const int16_t*>(samples), items, n_items,
                                                             unit0, n_units, tables, preemph, dc, raw_out, wave_item);
  else if (pcm == kPcmI32)
    sfe_logmel_kernel<int32_t, NW, SCH><<<g, b, 0, stream>>>(static_cast<const int32_t*>(samples), items, n_items,
                                                             unit0, n_units, tables, preemph, dc, raw_out, wave_item);
  else
    sfe_logmel_kernel<float, NW, SCH><<<g, b, 0, stream>>>(static_cast<const float*>(samples), items, n_items, unit0,
                                                           n_units, tables, preemph, dc, raw_out, wave_item);
  return hipGetLastError();
}

template <int NW>
hipError_t launch_logmel_s(int schedule, const void* samples, int pcm, const Decode& dc, const Item* items,
                           int n_items, int unit0, int n_units, const DevTables* tables, float preemph, float* raw_out,
                           int grid, const int32_t* wave_item, hipStream_t stream) {
  if (schedule == 1)
    return launch_logmel_t<NW, 1>(samples, pcm, dc, items, n_items, unit0, n_units, tables, preemph, raw_out, grid,
                                  wave_item, stream);
  return launch_logmel_t<NW, 0>(samples, pcm, dc, items, n_items, unit0, n_units, tables, preemph, raw_out, grid,
                                wave_item, stream);
}

void logmel_wave_items(const Item* items, int n_items, int unit0, int n_units, LogmelGrid g, int32_t* out) {
  for (int b = 0; b < g.blocks; ++b) {
    int wb, we;
    logmel_share(g.blocks, b, g.waves, unit0, n_units, &wb, &we);
    for (int w = 0; w < g.waves; ++w) {
      const int u = wb + w;
      int li = 0;
      if (u < we) {
        int hi = n_items - 1;
        while (li < hi) {  // the last item whose unit_off <= u
          const int mid = (li + hi + 1) >> 1;
          if (items[mid].unit_off <= u) li = mid;
          else hi = mid - 1;
        }
      }
      out[(size_t)b * g.waves + w] = li;
    }
  }
}

hipError_t launch_logmel(const void* samples, int pcm, float pcm_scale, const Item* items, int n_items, int unit0,
                         int n_units, const DevTables* tables, int schedule, float preemph, float* raw_out, int cus,
                         const int32_t* wave_item, hipStream_t stream) {
  if (n_units <= 0) return hipSuccess;
  Decode dc{pcm_scale, 1.0f / pcm_scale, 1.0 / (double)pcm_scale};  // the host's divisions are correctly rounded
  const LogmelGrid g = logmel_grid(n_units, cus);
  if (g.waves == kWavesBig)
    return launch_logmel_s<kWavesBig>(schedule, samples, pcm, dc, items, n_items, unit0, n_units, tables, preemph,
                                      raw_out, g.blocks, wave_item, stream);
  return launch_logmel_s<kWavesSmall>(schedule, samples, pcm, dc, items, n_items, unit0, n_units, tables, preemph,
                                      raw_out, g.blocks, wave_item, stream);
}

template <typename O>
hipError_t launch_norm_t(const float* raw, const Item* items, int n_items, int max_T, int pad_to, O* out,
                         hipStream_t stream) {
  using S = NormShape<kNormMainWaves, kNormMainSlab>;
  const unsigned blocks = (unsigned)((int64_t)n_items * S::kSlabs);
  using SW = NormShape<kNormWideWaves, kNormMainSlab>;
  if (n_items <= kNormWideMaxItems && max_T <= SW::kSpan * 16) {
    const dim3 grid(blocks), block(SW::kThreads);
    if (max_T <= SW::kSpan * 8) sfe_norm_wide_kernel<8, O><<<grid, block, 0, stream>>>(raw, items, n_items, pad_to, out);
    else sfe_norm_wide_kernel<16, O><<<grid, block, 0, stream>>>(raw, items, n_items, pad_to, out);
    return hipGetLastError();
  }
  const dim3 grid(blocks), block(S::kThreads);
  // Registers per lane sized to the longest item (N float4s hold kSpan N
  // frames); items of up to 2048 frames keep 1536 in registers (32 rounds
  // in registers need 184 VGPRs, 2 workgroups per CU instead of 3), longer
  // ones take the streaming path.
  if (max_T <= S::kSpan * 8) sfe_norm_kernel<8, 0, O><<<grid, block, 0, stream>>>(raw, items, n_items, pad_to, out);
  else if (max_T <= S::kSpan * 16)
    sfe_norm_kernel<16, 0, O><<<grid, block, 0, stream>>>(raw, items, n_items, pad_to, out);
  else if (max_T <= S::kSpan * 24)
    sfe_norm_kernel<24, 0, O><<<grid, block, 0, stream>>>(raw, items, n_items, pad_to, out);
  else sfe_norm_kernel<24, 8, O><<<grid, block, 0, stream>>>(raw, items, n_items, pad_to, out);
  return hipGetLastError();
}

hipError_t launch_norm(const float* raw, const Item* items, int n_items, int max_T, int pad_to, void* out,
                       bool out_bf16, hipStream_t stream) {
  if (n_items <= 0) return hipSuccess;
  if (out_bf16) return launch_norm_t(raw, items, n_items, max_T, pad_to, static_cast<uint16_t*>(out), stream);
  return launch_norm_t(raw, items, n_items, max_T, pad_to, static_cast<float*>(out), stream);
}

}  // namespace sfe
