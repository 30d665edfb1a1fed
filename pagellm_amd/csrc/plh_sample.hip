// gfx950 kernels for the batched sampler (src/pagellm/engine/sampling.py:52-111).
//
// Fast path (V <= 262144, no probability export), two launches:
//   k_sample_chunks  B x C workgroups of 512 threads.  Workgroup (row, c)
//                    reads the c-th 64 KB chunk of the row once, with
//                    16-byte non-temporal loads (32 fp32 or 16 fp64 tokens
//                    per thread), penalises it in float64 registers and
//                    leaves per-chunk partials in a workspace:
//                      greedy       the chunk's argmax;
//                      temperature  per-wave segment softmax partials
//                                   (max, sum of exp);
//                      top-k/top-p  the chunk's largest tokens (a value
//                                   histogram picks the threshold, which
//                                   also bounds the tokens left out);
//                                   top-p-only rows also leave the segment
//                                   partials.
//                    Every chunk costs one 64 KB read whatever its row's
//                    mode, and the hardware dispatcher spreads the B x C
//                    workgroups over the CUs, so mixed batches stay
//                    balanced.
//   k_sample_final   one workgroup per row merges the per-wave partials:
//                    argmax; normaliser and the segment holding the
//                    inverse-CDF point (rescanned with the same
//                    arithmetic); or exact selection over the gathered
//                    candidates (k-th largest, top-p cut, fixed-point draw
//                    in vocabulary order).  A row the candidates cannot
//                    decide exactly is finished by the general pipeline in
//                    the same workgroup.
// General path:
//   k_sample_rows    the general pipeline for every row (and the only kernel
//                    that exports the processed distribution, probs()).
// Others:
//   k_draw           inverse-CDF draw from given distributions (draw()).
//   k_penalize       repetition penalty on a copy (apply_repetition_penalty()).
#include "plh_fast.h"
#include "plh_kernels.h"
#include "plh_pipeline.h"

namespace plh {

// Phase clock stamps of k_sample_final and k_sample_chunks, in a profiling build only
// (-DPLH_PHASE_STAMPS: python -m pagellm_amd.build --phase-stamps): thread
// 0 of row r's workgroup records the shader clock on reaching phase k (and
// the real-time clock at its start and end)
// (0 start, 1 wave parts, 2 normaliser, 3 row buckets, 4 cut-bucket entries
// loaded, 5 cut selected, 6 per-chunk kept sums, 7 draw bins, 8 draw bin
// scattered, 9 end; 10-15 the mass selection: start, a level's pick, rank
// list, ranked, a level's bins counted (thread 0), the level's barrier
// passed).  The default build compiles them out.
#ifdef PLH_PHASE_STAMPS
constexpr int kStampRows = 256, kStampSlots = 16;
__device__ unsigned long long g_phase[kStampRows * kStampSlots];
__device__ unsigned long long g_frt[kStampRows * 2];  // real-time clock at phases 0 and 9
#define PLH_STAMP(row, k)                                                                                   \
  do {                                                                                                      \
    if (threadIdx.x == 0 && (row) < kStampRows) {                                                           \
      g_phase[(row) * kStampSlots + (k)] = __builtin_readcyclecounter();                                    \
      if ((k) == 0 || (k) == 9) g_frt[(row) * 2 + ((k) == 9 ? 1 : 0)] = __builtin_amdgcn_s_memrealtime(); \
    }                                                                                                       \
  } while (0)
#define PLH_STAMP_IF(c, row, k) \
  do {                          \
    if (c) PLH_STAMP(row, k);   \
  } while (0)
// k_sample_chunks, per chunk g < kStampChunks: thread 0 records the shader
// clock on reaching phase k (0 start, 1 register maxima, 2 chunk range, 3
// threshold, 4 counted, 5 placed, 6 buckets written, 7 end), the real-time
// clock (100 MHz, one count for the whole GPU) at its start, and the
// workgroup's hardware id and XCD; lane 0 of each wave records the
// real-time clock at the wave's end.
constexpr int kStampChunks = 4096, kChunkSlots = 8;
__device__ unsigned long long g_cphase[kStampChunks * kChunkSlots];
__device__ unsigned long long g_crt[kStampChunks * (1 + kWaves)];
__device__ unsigned int g_chw[kStampChunks * 2];
#define PLH_CSTAMP(g, k)                                                        \
  do {                                                                          \
    if (threadIdx.x == 0 && (g) < kStampChunks) {                               \
      g_cphase[(g) * kChunkSlots + (k)] = __builtin_readcyclecounter();         \
      if ((k) == 0) {                                                           \
        g_crt[(g) * (1 + kWaves)] = __builtin_amdgcn_s_memrealtime();           \
        g_chw[(g) * 2] = __builtin_amdgcn_s_getreg((31 << 11) | 4);  /* HW_ID */ \
        g_chw[(g) * 2 + 1] = __builtin_amdgcn_s_getreg((31 << 11) | 20); /* XCC_ID */ \
      }                                                                         \
    }                                                                           \
  } while (0)
#define PLH_CWAVE_END(g)                                                                          \
  do {                                                                                            \
    if (lane() == 0 && (g) < kStampChunks) g_crt[(g) * (1 + kWaves) + 1 + wave()] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
#else
#define PLH_STAMP(row, k) \
  do {                    \
  } while (0)
#define PLH_STAMP_IF(c, row, k) \
  do {                          \
  } while (0)
#define PLH_CSTAMP(g, k) \
  do {                   \
  } while (0)
#define PLH_CWAVE_END(g) \
  do {                   \
  } while (0)
#endif

constexpr int kU = 8;             // 16-byte loads per thread per chunk
constexpr int kHB = 1024;         // histogram bins
constexpr int kCandCap = 8192;    // candidates one row gathers
constexpr int kCapChunk = 1024;   // candidate slots per chunk, at most
constexpr int kMaxChunks = 64;    // chunks per row, at most (V <= 262144)
constexpr int kMaxLevels = 12;    // histogram levels of one selection
constexpr int kHBuf = 3;          // rotating histogram buffers of the merge
constexpr int kDrawSpanMax = 256; // tokens per draw bin, at most (V <= 262144)
constexpr int kSegPerLane = 8;    // segments per lane of one wave (V <= 262144)
constexpr int kHistBatch = 8;     // history ids a thread loads at once
constexpr double kNucTopP = 0.98; // top_p from which a row may take the nucleus path

// Chunk geometry per input type: a wave-wide 16-byte load covers kSpan
// consecutive tokens, a wave owns one contiguous segment of kSeg tokens and
// a workgroup one chunk of kChunk tokens (64 KB).
template <typename TIn>
struct Geo {
  static constexpr int kVW = 16 / (int)sizeof(TIn);
  static constexpr int kEpt = kU * kVW;
  static constexpr int kSpan = kWave * kVW;
  static constexpr int kSeg = kEpt * kWave;
  static constexpr int kChunk = kSeg * kWaves;
};
constexpr int kSegMax = Geo<float>::kSeg;

struct Hist {
  uint32_t cnt[kHB];
  uint64_t mass[kHB];
};

// Candidates of a selection's last level, ranked by every wave.
struct RankList {
  uint64_t key[kWave];
  uint64_t w[kWave];
  int idx[kWave];
  uint32_t rank[kWave];   // entries ahead of each entry ...
  uint64_t ahead[kWave];  // ... and their weight (summed over the waves)
  int n;
};

// LDS of k_sample_final (the candidates themselves stay in registers).
struct FastSmem {
  uint64_t xw[4][3][kWaves];          // cross-wave combines
  double exp_tab[kWaves][64];         // one exp table per wave
  int wcnt[kWaves][kMaxChunks];       // per wave: candidate count of each chunk
  Hist h[kHBuf];
  uint64_t dspan[kDrawSpanMax];       // the draw's crossing bin, by token offset
  uint64_t csum[kMaxChunks];          // the draw's per-chunk kept mass
  uint64_t rowm[kBkt];                // top-p rows: the row's bucket masses
  int cq0[kMaxChunks], cq1[kMaxChunks];  // top-p rows: each chunk's list range of the cut bucket
  RankList rl[2];                     // top-k, top-p
  uint32_t segbits[kSegMax / 32];     // penalty bits of a rescanned segment
};

union SmemAll {
  FastSmem f;
  Smem g;
};


__device__ __forceinline__ RowParams load_row_params(const SampleArgs& a, int row) {
  RowParams rp;
  rp.T = a.temperature[row];
  rp.top_k = a.top_k[row];
  rp.top_p = a.top_p[row];
  rp.pen = a.rep_penalty[row];
  rp.u = a.uniforms != nullptr ? a.uniforms[row] : 0.0;
  rp.h0 = a.hist_off != nullptr ? a.hist_off[a.hist_spans ? 2 * row : row] : 0;
  rp.h1 = a.hist_off != nullptr ? a.hist_off[a.hist_spans ? 2 * row + 1 : row + 1] : 0;
  rp.greedy = rp.T == 0.0;  // SamplingParams.greedy (sampling.py:47-49)
  // sampling.py:56: no penalty when it is 1.0 or the context is empty
  rp.pen_active = rp.pen != 1.0 && rp.h1 > rp.h0 && a.hist_ids != nullptr;
  rp.topk = !rp.greedy && rp.top_k > 0 && rp.top_k < a.V;  // :76
  rp.topp = !rp.greedy && rp.top_p < 1.0;                  // :82
  rp.nucleus = a.nucleus != 0 && rp.topp && !rp.topk && rp.top_p >= kNucTopP;
  return rp;
}

// The same parameters read with vector loads (every lane the same
// address), so that they travel in one round trip with the other loads a
// kernel issues before it knows the row's mode; row_params_of() makes them
// uniform once they are in.
struct RowLoad {
  double T, top_p, pen, u;
  int top_k;
  int64_t h0, h1;
};

__device__ __forceinline__ int lane_zero() {
  int z;
  asm volatile("v_mov_b32 %0, 0" : "=v"(z));  // a zero the compiler cannot see as uniform
  return z;
}

__device__ __forceinline__ void issue_row_params(const SampleArgs& a, int row, RowLoad& rl) {
  const int r = row + lane_zero();
  rl.T = a.temperature[r];
  rl.top_k = a.top_k[r];
  rl.top_p = a.top_p[r];
  rl.pen = a.rep_penalty[r];
  rl.u = a.uniforms != nullptr ? a.uniforms[r] : 0.0;
  rl.h0 = a.hist_off != nullptr ? a.hist_off[a.hist_spans ? 2 * r : r] : 0;
  rl.h1 = a.hist_off != nullptr ? a.hist_off[a.hist_spans ? 2 * r + 1 : r + 1] : 0;
}

__device__ __forceinline__ RowParams row_params_of(const SampleArgs& a, const RowLoad& rl) {
  RowParams rp;
  rp.T = uniform(rl.T);
  rp.top_k = uniform(rl.top_k);
  rp.top_p = uniform(rl.top_p);
  rp.pen = uniform(rl.pen);
  rp.u = uniform(rl.u);
  rp.h0 = (int64_t)uniform((uint64_t)rl.h0);
  rp.h1 = (int64_t)uniform((uint64_t)rl.h1);
  rp.greedy = rp.T == 0.0;
  rp.pen_active = rp.pen != 1.0 && rp.h1 > rp.h0 && a.hist_ids != nullptr;
  rp.topk = !rp.greedy && rp.top_k > 0 && rp.top_k < a.V;
  rp.topp = !rp.greedy && rp.top_p < 1.0;
  rp.nucleus = a.nucleus != 0 && rp.topp && !rp.topk && rp.top_p >= kNucTopP;
  return rp;
}

template <typename TIn, bool VEC>
__device__ __forceinline__ int row_general(const SampleArgs& a, int row, const RowParams& rp, Smem& sm,
                                           double* probs_out, PipeIn in = PipeIn{false, 0.0, false, 0.0, false, 0.0}) {
  const TIn* x = reinterpret_cast<const TIn*>(a.logits) + (int64_t)row * a.ld;
  if (rp.pen_active) build_bitmap(sm.bitmap, 0, a.V, a.hist_ids, rp.h0, rp.h1);
  RowSource<TIn, VEC> src{x, a.V, sm.bitmap, rp.pen_active, rp.pen};
  return row_pipeline(src, rp, a.V, in, sm, probs_out);
}

template <typename TIn, bool VEC>
__global__ __launch_bounds__(kThreads) void k_sample_rows(SampleArgs a) {
  __shared__ Smem sm;
  const int row = blockIdx.x;
  const RowParams rp = load_row_params(a, row);
  double* po = a.out_probs != nullptr ? a.out_probs + (int64_t)row * a.V : nullptr;
  const int id = row_general<TIn, VEC>(a, row, rp, sm, po);
  if (threadIdx.x == 0) a.out_ids[row] = id;
}

// y = z / T as the segment partials compute it: multiplication by 1/T
// (exact for T = 1).
struct YScale {
  double T, invT;
  __device__ __forceinline__ double operator()(double z) const { return z * invT; }
};

// ================================================================ chunks

typedef float f4_t __attribute__((ext_vector_type(4)));
typedef double d2_t __attribute__((ext_vector_type(2)));
typedef float f4u_t __attribute__((ext_vector_type(4))) __attribute__((aligned(4)));
// word 3 of a gfx9 buffer resource for raw 32-bit accesses (DATA_FORMAT 32)
constexpr int kBufDword3 = 0x00020000;
typedef double d2u_t __attribute__((ext_vector_type(2))) __attribute__((aligned(8)));
template <typename TIn>
struct VecOf;
template <>
struct VecOf<float> {
  typedef f4_t T;
  typedef f4u_t U;  // the same vector at element alignment
};
template <>
struct VecOf<double> {
  typedef d2_t T;
  typedef d2u_t U;
};

// Penalised tokens a wave keeps aside (their exact float64 value); a wave
// with more makes its chunk incomplete (the row takes the general
// pipeline).
constexpr int kPenPerWave = 128;
constexpr uint32_t kCodePool = 0x80000000u;  // a staged penalised token: | wave << 8 | its entry in the wave's pool

// Raw input values of staged candidates (float32 or float64 bits).
union StageRaw {
  float f;
  double d;
  __device__ __forceinline__ StageRaw& operator=(float v) { f = v; return *this; }
  __device__ __forceinline__ StageRaw& operator=(double v) { d = v; return *this; }
};

// LDS of k_sample_chunks: about 35 KB.
struct ChunkSmem {
  double redd[2 * kWaves];
  uint64_t redu[kWaves];
  int redi[kWaves];
  int ctl[8];
  uint64_t ctlu[4];
  double exp_tab[kWaves][64];  // one copy per wave
  union {
    struct {
      alignas(16) uint32_t hcnt[kHB];  // value histogram (read 16 bins per lane, 16 bytes at a time)
      uint32_t bitmap[Geo<float>::kChunk / 32];
    };
    // top-p rows: candidate buckets (kBkt of them, bucket 0 the chunk's
    // top), used once the histogram and the penalty bitmap are done with
    struct {
      uint32_t bcnt[kBkt];
      uint64_t bmass[kBkt];
      int boff[kBkt];
      int bcur[kBkt];
    };
  };
  double pz[kWaves][kPenPerWave];
  int pt[kWaves][kPenPerWave];
  // candidates staged on their way to the workspace: the raw value and
  // its token index (kCodePool | wave | pool entry for a penalised token);
  // float inputs keep both in one 8-byte pair, (float bits, index)
  union {
    StageRaw sraw[kCapChunk];
    uint2 spair[kCapChunk];
  };
  uint32_t scode[kCapChunk];
  int cand_n;
};

// Chunk-local offset of the calling lane's register slot e: the lane's
// j-th load (j = e / kVW) covers kVW consecutive tokens at
// wave*kSeg + j*kSpan + lane*kVW, so each load instruction of a wave reads
// 1 KB of contiguous HBM.
template <typename TIn>
__device__ __forceinline__ int slot_q(int e) {
  using G = Geo<TIn>;
  return wave() * G::kSeg + (e / G::kVW) * G::kSpan + lane() * G::kVW + (e % G::kVW);
}

// Maxima and the running top two of the register tokens in their input
// precision.  On float, fmax and fmin make the compiler quiet a possible
// signalling NaN in every loaded value first, one more instruction per
// token and pass; NaN is outside the input domain, so float tokens go to
// v_max3_f32, v_max_f32 and v_med3_f32 directly.
template <typename TIn>
__device__ __forceinline__ TIn in_max3(TIn a, TIn b, TIn c) {
  if constexpr (sizeof(TIn) == 4) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
  } else {
    return fmax(fmax(a, b), c);
  }
}
template <typename TIn>
__device__ __forceinline__ TIn in_min3(TIn a, TIn b, TIn c) {
  if constexpr (sizeof(TIn) == 4) {
    float r;
    asm("v_min3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
  } else {
    return fmin(fmin(a, b), c);
  }
}
// (m1, m2): the largest two values seen (m1 >= m2), then x
template <typename TIn>
__device__ __forceinline__ void in_top2(TIn& m1, TIn& m2, TIn x) {
  if constexpr (sizeof(TIn) == 4) {
    asm("v_med3_f32 %0, %1, %2, %3" : "=v"(m2) : "v"(m1), "v"(m2), "v"(x));
    asm("v_max_f32 %0, %1, %2" : "=v"(m1) : "v"(m1), "v"(x));
  } else {
    m2 = fmax(m2, fmin(m1, x));
    m1 = fmax(m1, x);
  }
}

// float64 min / max of values known not to be NaN, without the quieting
// instruction the compiler adds in front of fmin / fmax
__device__ __forceinline__ double dmin_raw(double a, double b) {
  double r;
  asm("v_min_f64 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ double dmax_raw(double a, double b) {
  double r;
  asm("v_max_f64 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

// acc plus the number of lanes below the calling one whose bit is set in m
__device__ __forceinline__ int mbcnt(uint64_t m, int acc) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, (uint32_t)acc));
}

// Wave minimum / maximum of float64 values that are all floats when fl
// (uniform) holds: then reduced in float, half the DPP moves and compares.
__device__ __forceinline__ double wave_min_fd(double v, bool fl) {
  return fl ? (double)wave_min((float)v) : wave_min(v);
}
__device__ __forceinline__ double wave_max_fd(double v, bool fl) {
  return fl ? (double)wave_max((float)v) : wave_max(v);
}

template <typename TIn, bool VEC>
__device__ __forceinline__ void load_chunk(const TIn* x, int V, int c0, typename VecOf<TIn>::T (&v)[kU]) {
  using G = Geo<TIn>;
  using VT = typename VecOf<TIn>::T;
  using UT = typename VecOf<TIn>::U;
  const int off = c0 + wave() * G::kSeg + lane() * G::kVW;
  const bool full = c0 + G::kChunk <= V;  // uniform: no bounds checks needed
  // 128-bit loads; rows that do not start on 16 bytes load at element
  // alignment (dword-aligned multi-dword loads are legal on gfx9 and cost
  // at most one extra cache line per wave load)
  if (full) {
#pragma unroll
    for (int j = 0; j < kU; ++j) {
      const int p = off + j * G::kSpan;
      if (VEC) v[j] = __builtin_nontemporal_load(reinterpret_cast<const VT*>(x + p));
      else v[j] = __builtin_nontemporal_load(reinterpret_cast<const UT*>(x + p));
    }
    return;
  }
  // the row's last chunk: buffer loads range-checked against the row's
  // length (V elements from x), which return 0 past it and cannot fault,
  // with no branch between them (a branch per slot makes the compiler wait
  // between the loads).  The vector that straddles the row's end (at most
  // one per lane) is loaded again element by element; then the slots past
  // the end take -inf.
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<TIn*>(x), (short)0, V * (int)sizeof(TIn), kBufDword3);
  int ps = -1;  // start of the straddling vector
#pragma unroll
  for (int j = 0; j < kU; ++j) {
    const int p = off + j * G::kSpan;
    v[j] = __builtin_bit_cast(VT, __builtin_amdgcn_raw_buffer_load_b128(rs, p * (int)sizeof(TIn), 0, 0));
    if (p < V && p + G::kVW > V) ps = p;
  }
  TIn tl[G::kVW];
#pragma unroll
  for (int s = 0; s < G::kVW; ++s) {
    const int o = ps >= 0 ? (ps + s) * (int)sizeof(TIn) : INT_MAX;  // INT_MAX: out of range, reads 0
    if constexpr (sizeof(TIn) == 4) tl[s] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, o, 0, 0));
    else tl[s] = __builtin_bit_cast(double, __builtin_amdgcn_raw_buffer_load_b64(rs, o, 0, 0));
  }
#pragma unroll
  for (int j = 0; j < kU; ++j) {
    const int p = off + j * G::kSpan;
#pragma unroll
    for (int s = 0; s < G::kVW; ++s) v[j][s] = p + s < V ? (p == ps ? tl[s] : v[j][s]) : (TIn)(-INFINITY);
  }
}

// One bit per distinct history id inside the chunk (np.unique,
// sampling.py:59), then the calling lane's bits in register-slot order.
template <typename TIn>
__device__ __forceinline__ uint32_t chunk_pbits(const SampleArgs& a, const RowParams& rp, int c0, ChunkSmem& cm) {
  using G = Geo<TIn>;
  constexpr int kWords = G::kChunk / 32;
  for (int w = threadIdx.x; w < kWords; w += kThreads) cm.bitmap[w] = 0u;
  wg_barrier();
  // kHistBatch ids per thread per round, all loaded before any is used
  for (int64_t h0 = rp.h0; h0 < rp.h1; h0 += kHistBatch * kThreads) {
    int id[kHistBatch];
#pragma unroll
    for (int j = 0; j < kHistBatch; ++j) {
      const int64_t h = h0 + j * kThreads + threadIdx.x;
      id[j] = h < rp.h1 ? a.hist_ids[h] : -1;
    }
#pragma unroll
    for (int j = 0; j < kHistBatch; ++j) {
      const int off = id[j] - c0;
      if ((unsigned)off < (unsigned)G::kChunk) lds_or(&cm.bitmap[off >> 5], 1u << (off & 31));
    }
  }
  wg_barrier();
  uint32_t pb = 0;
  const int q0 = wave() * G::kSeg + lane() * G::kVW;
#pragma unroll
  for (int j = 0; j < kU; ++j) {
    const int q = q0 + j * G::kSpan;
    pb |= ((cm.bitmap[q >> 5] >> (q & 31)) & ((1u << G::kVW) - 1u)) << (G::kVW * j);
  }
  return pb;
}

// Workgroup min and max in one barrier round.  red is read after the
// barrier and not released: the caller must not write it again before
// another barrier.
__device__ __forceinline__ void block_minmax(double* lo, double* hi, double* red) {
  double a = wave_min(*lo), b = wave_max(*hi);
  if (lane() == 0) {
    red[wave()] = a;
    red[kWaves + wave()] = b;
  }
  wg_barrier();
  a = red[0];
  b = red[kWaves];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) {
    a = fmin(a, red[w]);
    b = fmax(b, red[kWaves + w]);
  }
  *lo = a;
  *hi = b;
}

// The calling thread's tokens of one chunk: the raw registers (penalised
// slots hold -inf) plus its penalised tokens kept aside in its wave's LDS
// pool, entries [po, po + np), with their exact float64 value.  Every pass
// below visits both.
template <typename TIn>
struct ChunkToks {
  using G = Geo<TIn>;
  typename VecOf<TIn>::T v[kU];
  // the lane's share of its wave's pool: entries lane(), lane() + 64, ...
  // below the wave's count (whichever lane set a token aside), so a pass
  // over the pool takes at most kPenPerWave / 64 steps per lane
  int np = 0;
  __device__ __forceinline__ TIn rv(int e) const { return v[e / G::kVW][e % G::kVW]; }
  __device__ __forceinline__ double raw(int e) const { return (double)rv(e); }
  // Called at the start of each pass: the compiler must then widen the
  // registers again instead of keeping a float64 copy of the chunk alive
  // across passes (64 more VGPRs, which would cost occupancy).
  __device__ __forceinline__ void new_pass() {
#pragma unroll
    for (int j = 0; j < kU; ++j) asm volatile("" : "+v"(v[j]));
  }
  __device__ __forceinline__ double pen_z(const ChunkSmem& cm, int i) const { return cm.pz[wave()][lane() + kWave * i]; }
  __device__ __forceinline__ int pen_tok(const ChunkSmem& cm, int i) const { return cm.pt[wave()][lane() + kWave * i]; }
};

// Moves the calling wave's penalised tokens (bits pb of each lane) out of
// the registers: their penalised float64 value goes to the wave's LDS pool,
// the register slot to -inf.  Every lane then takes its share of the pool
// (ChunkToks::np).  Each token of the chunk is then in exactly one lane's
// set (its registers or its share of the pool), so per-lane maxima stay
// maxima of disjoint sets.  Returns true when the pool overflows (the chunk
// is then incomplete).
template <typename TIn>
__device__ __forceinline__ bool set_aside_penalised(ChunkToks<TIn>& tk, uint32_t pb, double pen, int c0, ChunkSmem& cm) {
  using G = Geo<TIn>;
  const int n = __popc(pb);
  const int incl = wave_scan_incl(n, 0, OpAdd{});
  const int total = lane_value(incl, kWave - 1);
  tk.np = 0;
  if (total > kPenPerWave) return true;
  if (pb != 0u) {
    int k = incl - n;
#pragma unroll
    for (int e = 0; e < G::kEpt; ++e) {
      if ((pb >> e) & 1u) {
        cm.pz[wave()][k] = tk.raw(e);
        cm.pt[wave()][k] = c0 + slot_q<TIn>(e);
        ++k;
        tk.v[e / G::kVW][e % G::kVW] = (TIn)(-INFINITY);
      }
    }
  }
  // the lane's share (a wave's own LDS writes complete in order), penalised
  // with one division each
  tk.np = total > lane() ? (total - lane() + kWave - 1) / kWave : 0;
  for (int i = 0; i < tk.np; ++i) {
    double& z = cm.pz[wave()][lane() + kWave * i];
    z = penalize(z, pen);
  }
  return false;
}

// Histogram bins of the register tokens in their input precision: the
// bounds of a float64 Affine rounded to float (lo rounded down) for float
// inputs.  margin() is how far, in bins, rounding can move a bin edge; the
// threshold taken from a bin backs off by it.
template <typename TIn>
struct InAffine {
  Affine af;
  __device__ __forceinline__ explicit InAffine(const Affine& a) : af(a) {}
  __device__ __forceinline__ int bin(TIn x) const { return af.bin(x); }
  __device__ __forceinline__ double lo() const { return af.lo; }
  __device__ __forceinline__ double scale() const { return af.scale; }
  __device__ __forceinline__ double margin() const { return 0.01; }
};
template <>
struct InAffine<float> {
  float lo_f, scale_f, off_f;
  int nb;
  __device__ __forceinline__ explicit InAffine(const Affine& a) : nb(a.nb) {
    lo_f = __double2float_rd(a.lo);
    scale_f = (float)a.scale;
    if (!(scale_f < INFINITY)) scale_f = 0.0f;
    off_f = -lo_f * scale_f;
  }
  // finite x >= lo_f: x * scale - lo * scale in one fma, clamped to
  // [0, nb - 1] by the median.  The rounded off_f moves every bin edge by
  // up to |off_f| * 2^-24 bins and the fma's own rounding adds up to
  // nb * 2^-24: with logits of ordinary range well inside 0.01 bin, but
  // far from zero (logits near 1e4 over a narrow chunk range) it can reach
  // a tenth of a bin, so margin() grows with |off_f|.
  __device__ __forceinline__ int bin(float x) const {
    return (int)__builtin_amdgcn_fmed3f(fmaf(x, scale_f, off_f), 0.0f, (float)(nb - 1));
  }
  __device__ __forceinline__ double lo() const { return (double)lo_f; }
  __device__ __forceinline__ double scale() const { return (double)scale_f; }
  __device__ __forceinline__ double margin() const { return 0.01 + ((double)fabsf(off_f) + nb) * 0x1p-22; }
};

// The smallest input-precision value >= theta (every finite value when theta
// is -inf): x >= in_threshold(theta) holds exactly when x is finite and
// (double)x >= theta.
template <typename TIn>
__device__ __forceinline__ TIn in_threshold(double theta) {
  if constexpr (sizeof(TIn) == 4) return fmaxf(__double2float_ru(theta), -3.402823466e38f);
  else return fmax(theta, -1.7976931348623157e308);
}

// Every wave walks the kHB bins of a count histogram from the highest down
// on its own (no barrier): the bin where the running count first reaches
// target, -1 when the total stays below it.  Exactly one bin takes the
// running count from below target to target or more.  Two levels: lane l
// sums the 16 bins of group 63 - l (four 16-byte reads) and a wave scan
// finds the group; the 16 lanes of each row then take one bin of that
// group each, highest first, and a row scan finds the bin.
__device__ __forceinline__ int hist_reach_desc(const uint32_t* h, uint32_t target) {
  constexpr int PL = kHB / kWave;
  static_assert(PL == 16, "one 16-lane row per group");
  const int grp = kWave - 1 - lane();
  const uint4* hv = reinterpret_cast<const uint4*>(h + grp * PL);
  uint32_t sum = 0;
#pragma unroll
  for (int i = 0; i < PL / 4; ++i) {
    const uint4 q = hv[i];
    sum += (q.x + q.y) + (q.z + q.w);
  }
  const uint32_t inc = wave_scan_incl(sum, 0u, OpAdd{});
  const uint64_t cross = __ballot(inc - sum < target && inc >= target);
  if (cross == 0ull) return -1;
  const int lc = __builtin_ctzll(cross);
  const uint32_t above = lane_value(inc - sum, lc);
  const int base = (kWave - 1 - lc) * PL + PL - 1;  // the group's highest bin
  const int j = lane() & (PL - 1);
  uint32_t r = h[base - j];
  r += dpp<kDppRowShr1, 0xf>(0u, r);
  r += dpp<kDppRowShr2, 0xf>(0u, r);
  r += dpp<kDppRowShr4, 0xf>(0u, r);
  r += dpp<kDppRowShr8, 0xf>(0u, r);
  const uint64_t hit = __ballot(above + r >= target) & 0xffffull;
  return base - __builtin_ctzll(hit);
}

// A staged candidate: its penalised logit and token id (penalised tokens
// from their entry in the wave's pool).
template <typename TIn>
__device__ __forceinline__ void staged(const ChunkSmem& cm, int i, double* z, int* id) {
  uint32_t code;
  double x;
  if constexpr (sizeof(TIn) == 4) {
    const uint2 pr = cm.spair[i];
    code = pr.y;
    x = (double)__uint_as_float(pr.x);
  } else {
    code = cm.scode[i];
    x = cm.sraw[i].d;
  }
  if (code & kCodePool) {
    const int w = (int)((code >> 8) & 0x7fu), e = (int)(code & 0xffu);
    *z = cm.pz[w][e];
    *id = cm.pt[w][e];
  } else {
    *z = x;
    *id = (int)code;
  }
}

// Top-p rows: the chunk's candidates go to the workspace bucket by bucket
// (buckets of kBktPerY per unit of y = z * (1 / T) on an absolute grid,
// bucket 0 the one holding the chunk's max y, the last one open below), each
// as exp(y - ymax_c) and its token id, with the buckets' counts and masses
// (exp sums in 2^-52 units; at most 1024 candidates keep them below 2^62).
// The merge sums the buckets of a row's chunks, which line up on the
// absolute grid, to find the one holding the top-p cut, and then reads only
// that bucket's candidates, and the candidates of the chunk that holds the
// draw.  Skipped when the chunk's candidates overflowed (the row then takes
// the general pipeline).
template <typename TIn>
__device__ __forceinline__ void write_buckets(const SampleArgs& a, int g, double hi, double invT, ChunkSmem& cm) {
  wg_barrier();  // every wave's candidates are staged
  const int n = cm.cand_n;
  const int capc = a.ws.capc;
  if (n > capc) return;  // uniform; the chunk is incomplete and the row takes the general pipeline
  if (!(hi > -INFINITY)) {  // no finite token: no candidates, an empty bucket set
    if (threadIdx.x < kBkt) {
      a.ws.bmass[(size_t)g * kBkt + threadIdx.x] = 0ull;
      a.ws.bcnt[(size_t)g * kBkt + threadIdx.x] = 0u;
    }
    if (threadIdx.x == 0) {
      a.ws.bymax[g] = -INFINITY;
      a.ws.bhb[g] = INT_MIN;
    }
    return;
  }
  // the buckets share their LDS with the histogram and the penalty bitmap,
  // both done with since the barrier above
  if (threadIdx.x < kBkt) {
    cm.bcnt[threadIdx.x] = 0u;
    cm.bmass[threadIdx.x] = 0ull;
    cm.bcur[threadIdx.x] = 0;
  }
  wg_barrier();
  const double ymaxc = hi * invT;
  const double hbc = __builtin_floor(ymaxc * kBktPerY);
  const double* tab = cm.exp_tab[wave()];
  constexpr int kPer = kCapChunk / kThreads;
  double ev[kPer];
  int idv[kPer], lbv[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int i = (int)threadIdx.x + k * kThreads;
    lbv[k] = -1;
    if (i < n) {
      double z;
      staged<TIn>(cm, i, &z, &idv[k]);
      const double y = z * invT;
      ev[k] = fast_exp_neg(y - ymaxc, tab);
      const double d = hbc - __builtin_floor(y * kBktPerY);
      const int lb = d < (double)(kBkt - 1) ? (int)d : kBkt - 1;
      lbv[k] = lb;
      lds_add(&cm.bcnt[lb], 1u);
      lds_add(&cm.bmass[lb], (uint64_t)__double2ull_rn(ev[k] * 4503599627370496.0));
    }
  }
  wg_barrier();
  if (wave() == 0) {  // the buckets' offsets: exclusive prefix of the counts
    constexpr int kB4 = kBkt / kWave;
    uint32_t c[kB4], t = 0;
#pragma unroll
    for (int j = 0; j < kB4; ++j) {
      c[j] = cm.bcnt[kB4 * lane() + j];
      t += c[j];
    }
    uint32_t o = wave_scan_incl(t, 0u, OpAdd{}) - t;
#pragma unroll
    for (int j = 0; j < kB4; ++j) {
      cm.boff[kB4 * lane() + j] = (int)o;
      o += c[j];
    }
  }
  if (threadIdx.x < kBkt) {
    a.ws.bmass[(size_t)g * kBkt + threadIdx.x] = cm.bmass[threadIdx.x];
    a.ws.bcnt[(size_t)g * kBkt + threadIdx.x] = cm.bcnt[threadIdx.x];
  }
  if (threadIdx.x == 0) {
    a.ws.bymax[g] = ymaxc;
    a.ws.bhb[g] = (int)hbc;
  }
  wg_barrier();
  double* cz = a.ws.cz + (size_t)g * capc;
  int32_t* ci = a.ws.ci + (size_t)g * capc;
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    if (lbv[k] >= 0) {
      const int pos = cm.boff[lbv[k]] + lds_fetch_add(&cm.bcur[lbv[k]], 1);
      cz[pos] = ev[k];
      ci[pos] = idv[k];
    }
  }
}

// Candidates of one chunk: every finite z >= theta, with theta below the
// chunk's target-th largest token (all finite tokens when there are fewer).
//   top-k, k <= 512: the k-th largest of the workgroup's 512 per-thread
//     maxima is itself k tokens deep, so a histogram of those maxima alone
//     bounds the k-th largest token from below;
//   otherwise: a value histogram of the chunk's tokens from L up, where L
//     is the smallest per-thread second-largest register token: each of
//     the n2 threads holding two finite ones has two tokens >= L, so when
//     2 * n2 >= target the target-th largest is >= L and the tokens below
//     L (typically three quarters) take no LDS atomic; else L is the
//     smallest finite token.
// theta is the lower edge of the histogram bin holding the target-th
// largest (cm.hcnt is zeroed at kernel start; every wave finds that bin on
// its own), so every token left out is below theta, which serves as the
// chunk's bound on them.  The passes over the register tokens compare in
// the input precision (exact: a float converts to float64 exactly).  Each
// wave counts its candidates with one ballot per register slot (a scalar
// popcount), reserves a range of the chunk's slots with one LDS atomic and
// places them with mbcnt, so consecutive candidates of a slot take
// consecutive slots; then it writes its part: the chunk's largest z,
// theta, the end of its slots.
//   lmax: the calling thread's largest z; wmax: its wave's (uniform);
//   m2: the thread's second-largest register token (when !by_max);
//   fl: every token of the wave is a float (no float64 pool entries).
template <typename TIn>
__device__ __forceinline__ void chunk_candidates(ChunkToks<TIn>& tk, double lmax, double wmax, TIn m2, bool by_max,
                                                 uint64_t target, bool fl, bool bucket, double invT,
                                                 const SampleArgs& a, int g, int c0, int flags, WavePart* wp,
                                                 ChunkSmem& cm) {
  using G = Geo<TIn>;
  constexpr int kEpt = G::kEpt;
  const int capc = a.ws.capc;
  double lo = INFINITY, hi = wmax;
  if (by_max) {  // the smallest per-thread maximum and the chunk's max: one barrier round
    const double l1 = wave_min_fd(lmax > -INFINITY ? lmax : INFINITY, fl);
    if (lane() == 0) {
      cm.redd[wave()] = l1;
      cm.redd[kWaves + wave()] = hi;
    }
    wg_barrier();
    lo = cm.redd[0];
    hi = cm.redd[kWaves];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) {
      lo = dmin_raw(lo, cm.redd[w]);
      hi = dmax_raw(hi, cm.redd[kWaves + w]);
    }
  } else {
    // one barrier round: min of the finite m2, their count, max of wmax
    const TIn inf = (TIn)INFINITY;
    const double l2 = (double)wave_min(m2 > -inf ? m2 : inf);
    const int n2 = (int)__popcll(__ballot(m2 > -inf));
    if (lane() == 0) {
      cm.redd[wave()] = l2;
      cm.redd[kWaves + wave()] = hi;
      cm.redi[wave()] = n2;
    }
    wg_barrier();
    double l2b = cm.redd[0];
    hi = cm.redd[kWaves];
    int n2b = cm.redi[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) {
      l2b = dmin_raw(l2b, cm.redd[w]);
      hi = dmax_raw(hi, cm.redd[kWaves + w]);
      n2b += cm.redi[w];
    }
    if (2 * (uint64_t)uniform(n2b) >= target) {
      lo = l2b;
    } else {  // few finite tokens: L is the smallest one
      TIn m = inf;
      tk.new_pass();
#pragma unroll
      for (int e = 0; e < kEpt; ++e) {
        const TIn x = tk.rv(e);
        m = fmin(m, x > -inf ? x : inf);
      }
      lo = (double)m;
      for (int i = 0; i < tk.np; ++i) {
        const double z = tk.pen_z(cm, i);
        if (z > -INFINITY) lo = fmin(lo, z);
      }
      double h2 = hi;
      wg_barrier();  // the reads of cm.redd above are done
      block_minmax(&lo, &h2, cm.redd);
    }
  }
  lo = uniform(lo);
  hi = uniform(hi);
  PLH_CSTAMP(g, 2);
  double theta = -INFINITY;
  if (hi > -INFINITY) {
    const Affine af = make_affine(lo, hi, kHB);
    const InAffine<TIn> rf(af);
    double tlo = af.lo, tscale = af.scale, tmargin = 0.01;
    if (by_max) {
      if (lmax > -INFINITY) lds_add(&cm.hcnt[af.bin(lmax)], 1u);
    } else {
      tlo = rf.lo();
      tscale = rf.scale();
      tmargin = rf.margin();
      const Affine pf{tlo, tscale, kHB};  // the same bins in float64, for the penalised tokens
      const TIn lin = in_threshold<TIn>(lo);
      uint32_t one = 1u;  // kept in a register, not rematerialised for every slot
      asm volatile("" : "+v"(one));
      tk.new_pass();
#pragma unroll
      for (int e = 0; e < kEpt; ++e) {
        const TIn x = tk.rv(e);
        if (x >= lin) lds_add(&cm.hcnt[rf.bin(x)], one);
      }
      for (int i = 0; i < tk.np; ++i) {
        const double z = tk.pen_z(cm, i);
        if (z > -INFINITY && z >= lo) lds_add(&cm.hcnt[pf.bin(z)], 1u);
      }
    }
    wg_barrier();
    const int d = hist_reach_desc(cm.hcnt, (uint32_t)target);
    // every z with bin(z) >= d is >= lo + (d - margin) / scale (bin(z) is
    // floor((z - lo) * scale) up to rounding); bin 0 starts at lo
    if (d >= 0) theta = d > 0 ? tlo + ((double)d - tmargin) / tscale : lo;
  }
  theta = uniform(theta);
  PLH_CSTAMP(g, 3);
  const TIn tin = in_threshold<TIn>(theta);
  // lane 0 holds the most pool entries (entry i is on lane i mod 64)
  const int npw = uniform(tk.np);
  int wtot = 0;
  tk.new_pass();
#pragma unroll
  for (int e = 0; e < kEpt; ++e) wtot += (int)__popcll(__ballot(tk.rv(e) >= tin));
  for (int i = 0; i < npw; ++i) {
    const double z = i < tk.np ? tk.pen_z(cm, i) : -INFINITY;
    wtot += (int)__popcll(__ballot(z > -INFINITY && z >= theta));
  }
  // one LDS reservation per wave (cm.cand_n was reset before the barriers above)
  int base = 0;
  if (lane() == 0) base = lds_fetch_add(&cm.cand_n, wtot);
  base = lane_value(base, 0);
  PLH_CSTAMP(g, 4);
  // the wave's candidates go to its slots [base, base + wtot) in LDS first,
  // then to the workspace with consecutive lanes on consecutive slots; a
  // wave whose slots would run past capc makes the chunk incomplete
  int wend = base + wtot;
  if (wend > capc) {
    flags |= kChunkIncomplete;
    wend = base;
  } else {
    // register tokens: the raw value and the token index go to LDS; the
    // penalised ones (few) a reference to their entry in the wave's pool
    const int idx0 = c0 + slot_q<TIn>(0);
    int pos = base;
    tk.new_pass();
#pragma unroll
    for (int e = 0; e < kEpt; ++e) {
      const TIn x = tk.rv(e);
      const bool keep = x >= tin;
      const uint64_t m = __ballot(keep);
      if (keep) {
        const int s = pos + mbcnt(m, 0);
        const uint32_t code = (uint32_t)(idx0 + (e / G::kVW) * G::kSpan + (e % G::kVW));
        if constexpr (sizeof(TIn) == 4) {
          cm.spair[s] = make_uint2(__float_as_uint(x), code);
        } else {
          cm.sraw[s] = x;
          cm.scode[s] = code;
        }
      }
      pos += (int)__popcll(m);
    }
    for (int i = 0; i < npw; ++i) {
      const double z = i < tk.np ? tk.pen_z(cm, i) : -INFINITY;
      const bool keep = z > -INFINITY && z >= theta;
      const uint64_t m = __ballot(keep);
      if (keep) {
        const int s = pos + mbcnt(m, 0);
        const uint32_t code = kCodePool | ((uint32_t)wave() << 8) | (uint32_t)(lane() + kWave * i);
        if constexpr (sizeof(TIn) == 4) cm.spair[s].y = code;
        else cm.scode[s] = code;
      }
      pos += (int)__popcll(m);
    }
    if (!bucket) {
      double* cz = a.ws.cz + (size_t)g * capc;
      int32_t* ci = a.ws.ci + (size_t)g * capc;
      for (int i = base + lane(); i < wend; i += kWave) {
        double z;
        int id;
        staged<TIn>(cm, i, &z, &id);
        cz[i] = z;
        ci[i] = id;
      }
    }
  }
  PLH_CSTAMP(g, 5);
  if (bucket) write_buckets<TIn>(a, g, hi, invT, cm);
  PLH_CSTAMP(g, 6);
  // every token left out is below theta
  if (lane() == 0) {
    wp->zmax = hi;
    wp->umax = theta;
    wp->end = wend;
    wp->flags = flags;
  }
}

// Nucleus bins lie on power-of-two grids: with rz = 2^e bins per unit of z,
// a token's bin is floor(zf * rz) for zf its z rounded to float (zf * rz is
// exact, so the bins are exact half-open intervals of zf, monotone in z).
// A grid of 2^e nests inside every finer one: floor(zf * 2^(e + s)) >> s =
// floor(zf * 2^e).  nuc_fit returns the largest rz (2^-40 .. 2^24) that
// fits [lo, hi] in kNucBins bins with every floor(zf * rz) within +-2^30;
// rz = 0 when there is no finite value, -1 when the values are too large
// to bin (|z| >= 2^70).
__device__ __forceinline__ NucGrid nuc_fit(float lo, float hi) {
  if (!(hi >= lo)) return NucGrid{0.0f, 0};  // no finite value (hi = -inf, lo = +inf)
  const float mag = fmaxf(fabsf(lo), fabsf(hi));
  if (!(mag < 1.1805916e21f)) return NucGrid{-1.0f, 0};  // 2^70
  int e = 24;
  if (hi > lo) {
    const float r = (float)(kNucBins - 2) / (hi - lo);
    e = r >= 16777216.0f ? 24 : (r < 9.094947e-13f ? -40 : min(24, (int)floorf(log2f(r))));  // 2^24, 2^-40
  }
  if (mag > 0.0f) e = min(e, 29 - (int)ceilf(log2f(mag)));
  e = max(e, -40);
  float rz = ldexpf(1.0f, e);
  while (e > -40 && __float2int_rd(hi * rz) - __float2int_rd(lo * rz) > kNucBins - 1) {
    rz *= 0.5f;
    --e;
  }
  return NucGrid{rz, __float2int_rd(lo * rz)};
}

// The exponent of a power-of-two float.
__device__ __forceinline__ int pow2_exp(float rz) { return ((__float_as_int(rz) >> 23) & 0xff) - 127; }

// Chunk index (row * C + chunk) of a block of the B x C chunk grids.  The
// hardware deals block ids to the 8 XCDs round robin (block b to XCD b % 8);
// the blocks of one row all carry the same b % 8, so a row's chunks and its
// merge (block `row` of the per-row grids) share one XCD's L2.  -1: a
// padding block (B not a multiple of 8).
constexpr int kXcds = 8;
__device__ __forceinline__ int chunk_block(int C, int B) {
  const int x = (int)blockIdx.x % kXcds, k = (int)blockIdx.x / kXcds;
  const int row = x + kXcds * (k / C);
  return row < B ? row * C + k % C : -1;
}

// One workgroup per 64 KB chunk (rows of any alignment: 16-byte
// non-temporal loads when the row allows, scalar loads otherwise).  The
// waves work on their own segments and write their own parts, so greedy and
// temperature chunks need no workgroup barrier; candidate chunks need the
// few of one value histogram.  Per row mode: greedy argmax, candidates,
// segment partials of the normaliser.
template <typename TIn, bool VEC, bool NUC>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4))) void k_sample_chunks(SampleArgs a) {
  using G = Geo<TIn>;
  __shared__ ChunkSmem cm;
  const int C = a.ws.C;
  const int g = chunk_block(C, a.B);
  if (g < 0) return;
  PLH_CSTAMP(g, 0);
  const int row = g / C;
  const int c0 = (g - row * C) * G::kChunk;
  // the row's parameters as vector loads, in flight with the chunk's (a
  // scalar load of them would hold the chunk's loads behind its return)
  RowLoad rload;
  issue_row_params(a, row, rload);
  const TIn* x = reinterpret_cast<const TIn*>(a.logits) + (int64_t)row * a.ld;
  ChunkToks<TIn> tk;
  load_chunk<TIn, VEC>(x, a.V, c0, tk.v);
  const RowParams rp = row_params_of(a, rload);
  const bool cands = rp.topk || (rp.topp && !(NUC && rp.nucleus));
  if (cands) {  // ordered before use by the first barrier of chunk_candidates
    for (int b = threadIdx.x; b < kHB; b += kThreads) cm.hcnt[b] = 0u;
    if (threadIdx.x == 0) cm.cand_n = 0;
  }
  int flags = 0;
  if (rp.pen_active) {
    const uint32_t pb = chunk_pbits<TIn>(a, rp, c0, cm);
    if (set_aside_penalised<TIn>(tk, pb, rp.pen, c0, cm)) flags = kChunkIncomplete;
    if (NUC && rp.nucleus) {  // the nucleus kernels read the chunk's bitmap from here
      uint32_t* out = a.ws.npen + (size_t)g * kNucPenWords;
      for (int w = threadIdx.x; w < G::kChunk / 32; w += kThreads) out[w] = cm.bitmap[w];
    }
  }
  WavePart* wp = a.ws.part + (size_t)g * kWaves + wave();
  if (rp.greedy) {
    // the register tokens compare exactly in the input precision: their
    // max, then the lowest slot holding it
    TIn m = (TIn)(-INFINITY);
#pragma unroll
    for (int e = 0; e < G::kEpt; e += 2) m = in_max3(m, tk.rv(e), tk.rv(e + 1));
    int first = G::kEpt;  // the lowest register slot holding m
#pragma unroll
    for (int e = G::kEpt - 1; e >= 0; --e) first = tk.rv(e) == m ? e : first;
    ArgMax best{-INFINITY, INT_MAX};
    if (first < G::kEpt) best = ArgMax{(double)m, c0 + slot_q<TIn>(first)};
    for (int i = 0; i < tk.np; ++i) best = argmax_merge(best, ArgMax{tk.pen_z(cm, i), tk.pen_tok(cm, i)});
    best = wave_argmax(best);
    PLH_CSTAMP(g, 1);
    if (lane() == 0) {
      wp->best_z = best.v;
      wp->best_idx = best.i;
      wp->flags = flags;
    }
    PLH_CSTAMP(g, 7);
    PLH_CWAVE_END(g);
    return;
  }
  const double* tab = cm.exp_tab[wave()];
  if (!rp.topk) init_exp_table_wave(cm.exp_tab[wave()]);
  // top-p rows keep as many candidates as the slots allow, less a margin
  // for the histogram bin that straddles the threshold
  const int capc = a.ws.capc;
  const uint64_t keep = (uint64_t)(capc - capc / 16);
  const uint64_t target = rp.topk ? min((uint64_t)rp.top_k, keep) : keep;
  const bool by_max = rp.topk && target <= (uint64_t)kThreads;
  // the thread's largest register token, and its second largest when the
  // chunk's threshold needs a lower edge, in one pass
  TIn m1 = (TIn)(-INFINITY), m2 = (TIn)(-INFINITY);
  tk.new_pass();
  if (cands && !by_max) {
#pragma unroll
    for (int e = 0; e < G::kEpt; ++e) in_top2(m1, m2, tk.rv(e));
  } else {
#pragma unroll
    for (int e = 0; e < G::kEpt; e += 2) m1 = in_max3(m1, tk.rv(e), tk.rv(e + 1));
  }
  double lmax = (double)m1;
  PLH_CSTAMP(g, 1);
  for (int i = 0; i < tk.np; ++i) lmax = fmax(lmax, tk.pen_z(cm, i));
  // lane 0 holds the most pool entries: none there means the wave's
  // tokens are all in the registers, in the input precision
  const bool fl = sizeof(TIn) == 4 && uniform(tk.np) == 0;
  const double wmax = uniform(wave_max_fd(lmax, fl));
  if (cands) chunk_candidates<TIn>(tk, lmax, wmax, m2, by_max, target, fl, !rp.topk && C <= kWaves, 1.0 / rp.T, a, g, c0,
                                     flags, wp, cm);
  else if (lane() == 0) wp->flags = flags;
  if (NUC && rp.nucleus) {  // the row's range, and this chunk's count histogram
    // the smallest finite register token (-inf slots count as +inf)
    const TIn inf = (TIn)INFINITY;
    TIn lmn = inf;
    tk.new_pass();
#pragma unroll
    for (int e = 0; e < G::kEpt; e += 2) {
      const TIn v0 = tk.rv(e), v1 = tk.rv(e + 1);
      lmn = in_min3(lmn, v0 > -inf ? v0 : inf, v1 > -inf ? v1 : inf);
    }
    double zmn = (double)lmn;
    for (int i = 0; i < tk.np; ++i) {
      const double z = tk.pen_z(cm, i);
      if (z > -INFINITY) zmn = fmin(zmn, z);
    }
    zmn = wave_min(zmn);
    if (lane() == 0) {
      wp->umax = zmn;  // the nucleus kernels' lower range edge
      wp->zmax = wmax;
    }
    // the chunk's tokens counted on its own power-of-two grid, in the
    // candidate staging area (nucleus rows stage no candidates); k_nuc_window
    // merges the chunks' histograms on the row's grid
    uint32_t* nh = reinterpret_cast<uint32_t*>(cm.sraw);
    static_assert(sizeof(cm.sraw) >= kNucBins * sizeof(uint32_t), "the staging area holds the histogram");
    for (int b = threadIdx.x; b < kNucBins; b += kThreads) nh[b] = 0u;
    if (lane() == 0) {
      cm.redd[wave()] = zmn;
      cm.redd[kWaves + wave()] = wmax;
    }
    wg_barrier();
    double clo = cm.redd[0], chi = cm.redd[kWaves];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) {
      clo = fmin(clo, cm.redd[w]);
      chi = fmax(chi, cm.redd[kWaves + w]);
    }
    const NucGrid grid = nuc_fit((float)clo, (float)chi);
    if (grid.rz > 0.0f) {
      uint32_t one = 1u;  // kept in a register, not rematerialised for every slot
      asm volatile("" : "+v"(one));
      tk.new_pass();
#pragma unroll
      for (int e = 0; e < G::kEpt; ++e) {
        const TIn v = tk.rv(e);
        if (v > (TIn)(-INFINITY)) lds_add(&nh[__float2int_rd((float)v * grid.rz) - grid.q0], one);
      }
      for (int i = 0; i < tk.np; ++i) {
        const double z = tk.pen_z(cm, i);
        if (z > -INFINITY) lds_add(&nh[__float2int_rd((float)z * grid.rz) - grid.q0], 1u);
      }
    }
    wg_barrier();
    // two 16-bit counts a word (a chunk holds at most 16384 tokens)
    uint32_t* out = a.ws.nhist + (size_t)g * (kNucBins / 2);
    for (int w = threadIdx.x; w < kNucBins / 2; w += kThreads) out[w] = nh[2 * w] | (nh[2 * w + 1] << 16);
    if (threadIdx.x == 0) a.ws.ngrid[g] = grid;
  }
  if (!rp.topk) {  // the full-vocabulary normaliser (sampling.py:79-81)
    // y = z / T is monotone in z, so the segment's max y is y(max z)
    const YScale ys{rp.T, 1.0 / rp.T};
    const double m = uniform(ys(wmax));
    double s = 0.0;
    if (m > -INFINITY) {
      tk.new_pass();
#pragma unroll
      for (int e = 0; e < G::kEpt; ++e) s += exp_neg_term(fma(tk.raw(e), ys.invT, -m), tab);
      for (int i = 0; i < tk.np; ++i) s += exp_neg_term(fma(tk.pen_z(cm, i), ys.invT, -m), tab);
    }
    s = wave_sum(s);
    if (lane() == 0) {
      a.ws.seg_m[(size_t)g * kWaves + wave()] = m;
      a.ws.seg_s[(size_t)g * kWaves + wave()] = s;
    }
  }
  PLH_CSTAMP(g, 7);
  PLH_CWAVE_END(g);
}

// ================================================================ finish

// ================================================================ finalize
// k_sample_final runs one workgroup per row.  Facts every wave needs (the
// chunk partials, the normaliser, the crossing bin of a histogram, the
// winner of a rank list) are computed by each wave on its own from the same
// data in the same order, so the waves agree without a barrier.  Barriers
// remain only where the waves' candidates meet in one LDS structure: a
// cross-wave combine, a histogram level, a rank list, the draw's bins.

// Cross-wave combine with rotating LDS slots: combine i posts one word per
// wave and value to slot i % 4 and reads the table after one barrier.
// Combine i + 4 writes that slot again only after the barriers of combines
// i+1 .. i+3, which no wave passes before finishing its reads of combine i.
struct XWave {
  uint64_t (*slot)[3][kWaves];
  int n;
  __device__ __forceinline__ const uint64_t (*post(uint64_t x, uint64_t y, uint64_t z))[kWaves] {
    uint64_t (*s)[kWaves] = slot[n & 3];
    ++n;
    if (lane() == 0) {
      s[0][wave()] = x;
      s[1][wave()] = y;
      s[2][wave()] = z;
    }
    wg_barrier();
    return s;
  }
};

__device__ __forceinline__ uint64_t bits_of(double d) { return __builtin_bit_cast(uint64_t, d); }
__device__ __forceinline__ double dbl_of(uint64_t u) { return __builtin_bit_cast(double, u); }

// Workgroup sum of doubles (waves left to right).
__device__ __forceinline__ double xw_sum(XWave& xw, double v) {
  const auto s = xw.post(bits_of(wave_sum(v)), 0, 0);
  double r = 0.0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) r += dbl_of(s[0][w]);
  return r;
}

// Workgroup inclusive scan of one double per thread in thread order; *excl
// and *total receive the exclusive value and the total.
__device__ __forceinline__ double xw_scan(XWave& xw, double v, double* excl, double* total) {
  const double x = wave_scan_incl(v, 0.0, OpAdd{});
  const double xe = wave_shift_up1(x, 0.0);
  const auto s = xw.post(bits_of(lane_value(x, kWave - 1)), 0, 0);
  double pre = 0.0, tot = 0.0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const double t = dbl_of(s[0][w]);
    if (w < wave()) pre += t;
    tot += t;
  }
  *excl = pre + xe;
  *total = tot;
  return pre + x;
}

__device__ __forceinline__ int xw_min(XWave& xw, int v) {
  const auto s = xw.post((uint64_t)(uint32_t)wave_min(v), 0, 0);
  int r = INT_MAX;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) r = min(r, (int)(uint32_t)s[0][w]);
  return r;
}

__device__ __forceinline__ int xw_max(XWave& xw, int v) {
  const auto s = xw.post((uint64_t)(uint32_t)wave_max(v), 0, 0);
  int r = INT_MIN;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) r = max(r, (int)(uint32_t)s[0][w]);
  return r;
}

// Candidates of one row, held in registers: thread t owns slots
// q * kThreads + t (q < kPerT) of the row's gathered list; bit q of `valid`
// marks a real candidate.  v[q] holds the penalised logit, then its
// probability; w[q] its fixed-point weight.
constexpr int kPerT = kCandCap / kThreads;
struct RegCands {
  double v[kPerT];
  uint64_t w[kPerT];
  int idx[kPerT];
  uint32_t valid;
};

// The next histogram buffer of the row (zeroed), and zeroing of the one
// after it: buffer g % 3 is last read right after the barrier of use g, and
// zeroed during use g + 2, after the barrier of use g + 1.
__device__ __forceinline__ Hist& next_hist(FastSmem& fs, int& g) {
  Hist& h = fs.h[g % kHBuf];
  Hist& z = fs.h[(g + 1) % kHBuf];
  for (int b = threadIdx.x; b < kHB; b += kThreads) {
    z.cnt[b] = 0u;
    z.mass[b] = 0ull;
  }
  ++g;
  return h;
}

// Shift that maps a key span onto at most kHB bins.
__device__ __forceinline__ int span_shift(uint64_t span) {
  return span < (uint64_t)kHB ? 0 : 64 - __clzll((long long)span) - 10;
}

struct WPick {
  bool found;
  int d;           // the crossing bin
  uint64_t above;  // the running total above it
};

// Per wave: descending walk over the kHB bins of h: the bin where the
// running total from `above` first reaches target.  The running total is
// non-decreasing, so one bin takes it from below target to target or more.
// Lane l sums bins [16(63-l), 16(63-l)+16), reading them in an order rotated
// by l so that the lanes spread over the LDS banks; the lane whose range
// crosses then walks its bins alone.
template <bool MASS>
__device__ __forceinline__ WPick wave_pick_desc(const Hist& h, uint64_t above, uint64_t target) {
  constexpr int kPer = kHB / kWave;
  const int dlo = kPer * (kWave - 1 - lane());
  uint64_t s = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int d = dlo + ((j + lane()) & (kPer - 1));
    s += MASS ? h.mass[d] : (uint64_t)h.cnt[d];
  }
  const uint64_t incl = wave_scan_incl(s, (uint64_t)0, OpAdd{});
  const uint64_t ex = incl - s;
  const uint64_t tot = lane_value(incl, kWave - 1);
  if (above >= target || above + tot < target) return WPick{false, -1, above + tot};
  const int L = __builtin_ctzll(__ballot(above + ex < target && above + incl >= target));
  int d = 0;
  uint64_t ab = 0;
  if (lane() == L) {
    uint64_t run = above + ex;
#pragma unroll
    for (int j = kPer - 1; j >= 0; --j) {
      const uint64_t v = MASS ? h.mass[dlo + j] : (uint64_t)h.cnt[dlo + j];
      if (run < target && run + v >= target) {
        d = dlo + j;
        ab = run;
      }
      run += v;
    }
  }
  return WPick{true, lane_value(d, L), lane_value(ab, L)};
}

// Selection over the register candidates in (key desc, token index asc)
// order, for the slots in act:
//   MASS=false: the target-th entry (its key; the top-k threshold);
//   MASS=true : the first entry whose inclusive weight reaches target (the
//               top-p cut).
// Levels of exact key bins (kHB bins of 2^sh consecutive keys) narrow the
// active set to the crossing bin until at most one wave of candidates is
// left; each wave then ranks them (every lane counts the entries ahead of
// its own).  A run of equal keys is ordered by token index: the level keys
// become V-1-index.  giveup: the levels did not converge (the caller falls
// back to the general pipeline).
struct SelOut {
  bool found;
  bool giveup;
  uint64_t key;
  int idx;
};

// Bounds on the active set known before a selection: every active key lies
// in [lo, hi], and n bounds the active count from above (exact when the
// selection is a top-k one: its n < target test needs the count).
struct KeySpan {
  uint64_t lo, hi, n;
};

// The order key of slot q is keyf(rc.v[q]), non-decreasing in rc.v[q], so
// the key range of the active set comes from the range of the values: one
// cross-wave combine, skipped when the caller passes a KeySpan (known).  The rank
// list reads its entry count from the list itself, so an upper bound n
// only decides whether a histogram level runs first.
template <bool MASS, class KeyF>
__device__ __forceinline__ SelOut select_desc(uint32_t act, const RegCands& rc, const KeyF& keyf, uint64_t target,
                                              int V, RankList& rl, FastSmem& fs, XWave& xw, int& hgen,
                                              bool known = false, KeySpan span = KeySpan{0, 0, 0}) {
  auto key = [&](int q) -> uint64_t { return keyf(rc.v[q]); };
  {
    uint64_t lo, hi, n;
    if (known) {
      // the barrier the combine below would have given: the kernel zeroes
      // the first histogram and the rank lists at its start and orders
      // that before their first use with the row's first barrier, which
      // for a top-p-only row is this one
      wg_barrier();
      lo = span.lo;
      hi = span.hi;
      n = span.n;
    } else {
      double vlo = INFINITY, vhi = -INFINITY;
#pragma unroll
      for (int q = 0; q < kPerT; ++q)
        if ((act >> q) & 1u) {
          vlo = fmin(vlo, rc.v[q]);
          vhi = fmax(vhi, rc.v[q]);
        }
      const auto s = xw.post(bits_of(wave_min(vlo)), bits_of(wave_max(vhi)), (uint64_t)wave_sum((uint32_t)__popc(act)));
      vlo = dbl_of(s[0][0]);
      vhi = dbl_of(s[1][0]);
      n = s[2][0];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) {
        vlo = fmin(vlo, dbl_of(s[0][w]));
        vhi = fmax(vhi, dbl_of(s[1][w]));
        n += s[2][w];
      }
      lo = uniform(keyf(vlo));
      hi = uniform(keyf(vhi));
    }
    if (n == 0 || (!MASS && n < target)) return SelOut{false, false, 0, 0};
    target = uniform(target);
    uint32_t cnt = (uint32_t)uniform(n);
    uint64_t above = 0;
    bool by_idx = false;
    auto lkey = [&](int q) -> uint64_t { return by_idx ? (uint64_t)(V - 1 - rc.idx[q]) : key(q); };
    for (int lev = 0; cnt > (uint32_t)kWave; ++lev) {
      if (lo == hi) {
        if (!MASS) return SelOut{true, false, lo, 0};
        if (by_idx) return SelOut{false, true, 0, 0};
        by_idx = true;
        lo = 0;
        hi = (uint64_t)(V - 1);
      }
      if (lev == kMaxLevels) return SelOut{false, true, 0, 0};
      const int sh = span_shift(hi - lo);
      Hist& h = next_hist(fs, hgen);
#pragma unroll
      for (int q = 0; q < kPerT; ++q)
        if ((act >> q) & 1u) {
          const int b = (int)((lkey(q) - lo) >> sh);
          lds_add(&h.cnt[b], 1u);
          if (MASS) lds_add(&h.mass[b], rc.w[q]);
        }
      wg_barrier();
      const WPick pk = wave_pick_desc<MASS>(h, above, target);
      if (!pk.found) return SelOut{false, false, 0, 0};
      above = uniform(pk.above);
      const int d = uniform(pk.d);
      cnt = (uint32_t)uniform((int)h.cnt[d]);
      const uint64_t nlo = lo + ((uint64_t)d << sh);
      const uint64_t wid = (1ull << sh) - 1;
      const uint64_t nhi = hi - nlo < wid ? hi : nlo + wid;  // no wrap-around
#pragma unroll
      for (int q = 0; q < kPerT; ++q)
        if ((act >> q) & 1u) {
          const uint64_t k = lkey(q);
          if (k < nlo || k > nhi) act &= ~(1u << q);
        }
      lo = nlo;
      hi = nhi;
    }
    // rank list: one LDS reservation per wave
    const int nq = __popc(act);
    const int qi = wave_scan_incl(nq, 0, OpAdd{});
    int rbase = 0;
    if (lane() == kWave - 1 && qi > 0) rbase = lds_fetch_add(&rl.n, qi);
    int slot = lane_value(rbase, kWave - 1) + qi - nq;
#pragma unroll
    for (int q = 0; q < kPerT; ++q)
      if ((act >> q) & 1u) {
        rl.key[slot] = key(q);
        rl.idx[slot] = rc.idx[q];
        rl.w[slot] = MASS ? rc.w[q] : 0ull;
        ++slot;
      }
    wg_barrier();
    // lane i of every wave holds entry i; wave w compares it with entries
    // j in [8w, 8w + 8) (LDS broadcast reads) and adds its counts to the
    // entry's totals
    const int m = uniform(rl.n);
    const int ln = lane();
    uint64_t k = 0ull, w = 0ull;
    int ix = INT_MAX;
    if (ln < m) {
      k = rl.key[ln];
      ix = rl.idx[ln];
      w = rl.w[ln];
    }
    uint32_t rank = 0;
    uint64_t ahead = 0;
    constexpr int kPerWave = kWave / kWaves;
#pragma unroll
    for (int jj = 0; jj < kPerWave; ++jj) {
      const int j = wave() * kPerWave + jj;
      if (j < m) {
        const uint64_t kj = rl.key[j];
        const int ij = rl.idx[j];
        const bool bj = kj > k || (kj == k && ij < ix);
        rank += bj ? 1u : 0u;
        if (MASS) ahead += bj ? rl.w[j] : 0ull;
      }
    }
    if (ln < m) {
      lds_add(&rl.rank[ln], rank);
      if (MASS) lds_add(&rl.ahead[ln], ahead);
    }
    wg_barrier();
    if (ln < m) {
      rank = rl.rank[ln];
      ahead = rl.ahead[ln];
    }
    bool hit;
    if (!MASS) hit = ln < m && (uint64_t)rank == target - above - 1;
    else hit = ln < m && above + ahead < target && above + ahead + w >= target;
    const uint64_t hits = __ballot(hit);
    if (hits == 0) return SelOut{false, !MASS, 0, 0};
    const int L = __builtin_ctzll(hits);
    return SelOut{true, false, lane_value(k, L), lane_value(ix, L)};
  }
}

// Inverse-CDF draw over the kept candidates in vocabulary order
// (sampling.py:94-98): with w[q] the fixed-point probability of kept slots
// (0 otherwise), the first token whose running mass exceeds
// floor(u * total); V-1 when none does.  Index bins of 2^sh consecutive
// tokens locate the crossing bin; its tokens are then laid out by offset
// and scanned.
__device__ __forceinline__ int draw_kept(const RegCands& rc, int V, double u, FastSmem& fs, int& hgen) {
  int sh = 0;
  while (((V - 1) >> sh) >= kHB) ++sh;
  Hist& h = next_hist(fs, hgen);
#pragma unroll
  for (int q = 0; q < kPerT; ++q)
    if (rc.w[q] != 0ull) lds_add(&h.mass[rc.idx[q] >> sh], rc.w[q]);
  wg_barrier();
  // lane l sums bins [16l, 16l+16) (rotated reads, as in wave_pick_desc)
  constexpr int kPer = kHB / kWave;
  const int b0 = kPer * lane();
  uint64_t s = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) s += h.mass[b0 + ((j + lane()) & (kPer - 1))];
  const uint64_t incl = wave_scan_incl(s, (uint64_t)0, OpAdd{});
  const uint64_t tot = lane_value(incl, kWave - 1);
  if (tot == 0) return V - 1;
  const uint64_t t = (uint64_t)__double2ull_rd(u * (double)tot);
  const uint64_t ex = incl - s;
  const uint64_t hits = __ballot(ex <= t && t < incl);
  if (hits == 0) return V - 1;
  const int L = __builtin_ctzll(hits);
  uint64_t bf = 0;
  int bl = 0;
  if (lane() == L) {
    uint64_t run = ex;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const uint64_t v = h.mass[b0 + j];
      if (run <= t && t < run + v) {
        bl = b0 + j;
        bf = run;
      }
      run += v;
    }
  }
  const int b = uniform(lane_value(bl, L));
  const uint64_t before = uniform(lane_value(bf, L));
  // bin b's kept tokens by offset (fs.dspan is zero on entry)
#pragma unroll
  for (int q = 0; q < kPerT; ++q)
    if (rc.w[q] != 0ull && (rc.idx[q] >> sh) == b) fs.dspan[rc.idx[q] - (b << sh)] = rc.w[q];
  wg_barrier();
  constexpr int kPs = kDrawSpanMax / kWave;
  const int o0 = kPs * lane();
  uint64_t ss = 0;
#pragma unroll
  for (int j = 0; j < kPs; ++j) ss += fs.dspan[o0 + ((j + (lane() >> 2)) & (kPs - 1))];
  const uint64_t in2 = wave_scan_incl(ss, (uint64_t)0, OpAdd{});
  const uint64_t e2 = before + in2 - ss;
  const uint64_t h2 = __ballot(e2 <= t && t < before + in2);
  if (h2 == 0) return V - 1;
  const int L2 = __builtin_ctzll(h2);
  int tok = 0;
  if (lane() == L2) {
    uint64_t r2 = e2;
#pragma unroll
    for (int j = 0; j < kPs; ++j) {
      const uint64_t v = fs.dspan[o0 + j];
      if (r2 <= t && t < r2 + v) tok = (b << sh) + o0 + j;
      r2 += v;
    }
  }
  return lane_value(tok, L2);
}

// Per-wave summary of the row's wave partials (every wave reads them all).
struct PartSum {
  int flags;
  double umax, zmax;
  double umin;  // the smallest chunk threshold: every candidate is >= it
  ArgMax best;
};

// The row's first kWave wave parts (all of them for V <= 8 chunks), one per
// lane, read before the row's parameters are known.
struct PartLoad {
  WavePart p;
};

__device__ __forceinline__ void load_parts_first(const SampleArgs& a, int row, PartLoad& pl) {
  // unconditional (lanes past the row's parts read its last one, unused):
  // no branch for the compiler to pull the parts' first uses into
  const int P = a.ws.C * kWaves;
  pl.p = a.ws.part[(size_t)row * P + min(lane(), P - 1)];
}

__device__ __forceinline__ PartSum scan_parts(const SampleArgs& a, int row, bool greedy, bool cands, FastSmem& fs,
                                              const PartLoad& pl) {
  const int P = a.ws.C * kWaves;
  const WavePart* pp = a.ws.part + (size_t)row * P;
  int* wc = fs.wcnt[wave()];
  if (cands) wc[lane()] = 0;
  int fl = 0;
  double um = -INFINITY, zm = -INFINITY, un = INFINITY;
  ArgMax best{-INFINITY, INT_MAX};
  for (int j = lane(); j < P; j += kWave) {
    const WavePart p = j < kWave ? pl.p : pp[j];
    fl |= p.flags;
    if (greedy) best = argmax_merge(best, ArgMax{p.best_z, p.best_idx});
    if (cands) {
      um = fmax(um, p.umax);
      un = fmin(un, p.umax);
      zm = fmax(zm, p.zmax);
      lds_max(&wc[j / kWaves], p.end);  // a chunk's count: the largest end of its waves
    }
  }
  PartSum r;
  r.flags = uniform(wave_max(fl));
  r.umax = uniform(wave_max(um));
  r.umin = cands ? uniform(wave_min(un)) : INFINITY;
  r.zmax = uniform(wave_max(zm));
  r.best = greedy ? wave_argmax(best) : best;
  return r;
}

// Full-distribution normaliser from the per-wave segment partials, by the
// calling wave alone: lane l holds segments 8l .. 8l+7 (loaded by
// load_segs), their masses rescaled to the largest segment max go to ms[],
// and their exclusive prefix (segment order) to *lex.
struct SegNorm {
  double ymax, S;
};

struct SegLoad {
  double mk[kSegPerLane], sk[kSegPerLane];
};

__device__ __forceinline__ void load_segs(const SampleArgs& a, int row, int nseg, SegLoad& sl) {
  const size_t b = (size_t)row * a.ws.C * kWaves;
#pragma unroll
  for (int j = 0; j < kSegPerLane; ++j) {
    const int k = kSegPerLane * lane() + j;
    sl.mk[j] = k < nseg ? a.ws.seg_m[b + k] : -INFINITY;
    sl.sk[j] = k < nseg ? a.ws.seg_s[b + k] : 0.0;
  }
}

__device__ __forceinline__ SegNorm seg_norm(const SegLoad& sl, const double* tab, double (&ms)[kSegPerLane],
                                            double* lex) {
  double ymax = -INFINITY;
#pragma unroll
  for (int j = 0; j < kSegPerLane; ++j) ymax = fmax(ymax, sl.mk[j]);
  ymax = uniform(wave_max(ymax));
  double ls = 0.0;
#pragma unroll
  for (int j = 0; j < kSegPerLane; ++j) {
    ms[j] = sl.mk[j] > -INFINITY ? sl.sk[j] * fast_exp_neg(sl.mk[j] - ymax, tab) : 0.0;
    ls += ms[j];
  }
  const double incl = wave_scan_incl(ls, 0.0, OpAdd{});
  *lex = wave_shift_up1(incl, 0.0);
  return SegNorm{ymax, uniform(lane_value(incl, kWave - 1))};
}

// Temperature only: full-vocabulary softmax and draw (sampling.py:75-81,
// :94-98).  The segment holding the inverse-CDF point is rescanned from HBM
// with the arithmetic of the partials.
template <typename TIn>
__device__ __forceinline__ int finish_temp(const SampleArgs& a, int row, const RowParams& rp, const SegLoad& sg,
                                           FastSmem& fs, XWave& xw) {
  using G = Geo<TIn>;
  const int V = a.V;
  const YScale ys{rp.T, 1.0 / rp.T};
  const double* tab = fs.exp_tab[wave()];
  double ms[kSegPerLane], lex;
  const SegNorm sn = seg_norm(sg, tab, ms, &lex);
  const double t = rp.u * sn.S;
  // the first segment whose running mass exceeds t
  double run = lex, bl = 0.0, ml = 0.0;
  int kl = INT_MAX;
#pragma unroll
  for (int j = 0; j < kSegPerLane; ++j) {
    if (kl == INT_MAX && run + ms[j] > t) {
      kl = kSegPerLane * lane() + j;
      bl = run;
      ml = sg.mk[j];
    }
    run += ms[j];
  }
  const uint64_t hits = __ballot(kl != INT_MAX);
  if (hits == 0) return V - 1;
  const int L = __builtin_ctzll(hits);
  const int kstar = uniform(lane_value(kl, L));
  const double before = uniform(lane_value(bl, L));
  const double mseg = uniform(lane_value(ml, L));
  const int s0 = kstar * G::kSeg;
  if (rp.pen_active) {
    for (int w = threadIdx.x; w < G::kSeg / 32; w += kThreads) fs.segbits[w] = 0u;
    wg_barrier();
    for (int64_t h = rp.h0 + threadIdx.x; h < rp.h1; h += kThreads) {
      const int off = a.hist_ids[h] - s0;
      if ((unsigned)off < (unsigned)G::kSeg) lds_or(&fs.segbits[off >> 5], 1u << (off & 31));
    }
    wg_barrier();
  }
  const double sc = fast_exp_neg(mseg - sn.ymax, tab);
  // thread t holds tokens s0 + kPer*t + q, in vocabulary order
  constexpr int kPer = G::kSeg / kThreads;
  const TIn* x = reinterpret_cast<const TIn*>(a.logits) + (int64_t)row * a.ld;
  const int q0 = kPer * (int)threadIdx.x;
  double e[kPer], es = 0.0;
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    e[q] = 0.0;
    const int pos = s0 + q0 + q;
    if (pos < V) {
      double z = (double)x[pos];
      if (rp.pen_active && ((fs.segbits[(q0 + q) >> 5] >> ((q0 + q) & 31)) & 1u)) z = penalize(z, rp.pen);
      e[q] = z > -INFINITY ? exp_neg_term(fma(z, ys.invT, -mseg), tab) : 0.0;
    }
    es += e[q];
  }
  double pex, ptot;
  xw_scan(xw, es, &pex, &ptot);
  double r = pex;
  int hit = INT_MAX, last = -1;
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    r += e[q];
    if (e[q] > 0.0) last = s0 + q0 + q;
    if (hit == INT_MAX && e[q] > 0.0 && before + r * sc > t) hit = s0 + q0 + q;
  }
  hit = xw_min(xw, hit);
  if (hit == INT_MAX) hit = xw_max(xw, last);  // rounding at the segment end
  return hit < 0 ? V - 1 : hit;
}

struct FastOut {
  int id;
  bool general;  // the candidates cannot decide the row exactly
  double S;      // general: the full normaliser when known (top-p-only rows), else 0
};

// Top-k and/or top-p rows (sampling.py:75-90, :94-98) from the gathered
// chunk candidates.
// Every candidate slot of the row into registers (slot i = q * kThreads + t;
// consecutive lanes read consecutive addresses).
// With wc (a wave's copy of the chunks' candidate counts), only the slots
// that hold a candidate are read.
__device__ __forceinline__ void gather_cands(const SampleArgs& a, int row, RegCands& rc, const int* wc = nullptr) {
  const int slots = a.ws.C * a.ws.capc;
  const int csh = __ffs(a.ws.capc) - 1;  // capc is a power of two
  const size_t base = (size_t)row * slots;
#pragma unroll
  for (int q = 0; q < kPerT; ++q) {
    const int i = q * kThreads + (int)threadIdx.x;
    rc.v[q] = 0.0;
    rc.idx[q] = 0;
    rc.w[q] = 0ull;
    if (i < slots && (wc == nullptr || (i & (a.ws.capc - 1)) < wc[i >> csh])) {
      rc.v[q] = a.ws.cz[base + i];
      rc.idx[q] = a.ws.ci[base + i];
    }
  }
}

template <typename TIn, bool TOPK>
__device__ __forceinline__ FastOut finish_cands(const SampleArgs& a, RegCands& rc, const SegLoad& sg,
                                                const RowParams& rp, const PartSum& ps, FastSmem& fs, XWave& xw,
                                                int& hgen) {
  const int V = a.V;
  const int capc = a.ws.capc;
  const int csh = __ffs(capc) - 1;  // capc is a power of two
  const int slots = a.ws.C * capc;
  const double* tab = fs.exp_tab[wave()];
  // slot i (chunk i / capc) holds a candidate when it lies below its
  // chunk's count
  const int* wc = fs.wcnt[wave()];
  rc.valid = 0;
#pragma unroll
  for (int q = 0; q < kPerT; ++q) {
    const int i = q * kThreads + (int)threadIdx.x;
    if (i < slots && (i & (capc - 1)) < wc[i >> csh]) rc.valid |= 1u << q;
  }
  // the row's candidate count, by every wave from its copy of the counts
  // (computed where needed, to keep it out of the registers in between)
  auto count_cands = [&]() -> uint64_t {
    int nc = 0;
    for (int c = lane(); c < a.ws.C; c += kWave) nc += wc[c];
    return (uint64_t)uniform(wave_sum(nc));
  };
  const double T = rp.T;
  auto yexact = [&](double z) -> double { return T == 1.0 ? z : z / T; };

  // ---- top-k: k-th largest with multiplicity, keep y >= kth_y (:76-78)
  double z_lo = -INFINITY;
  if (TOPK) {
    // every candidate lies in [the smallest chunk threshold, the row max]
    const KeySpan ks{key_of(ps.umin), key_of(ps.zmax), count_cands()};
    const bool known = ps.umin > -INFINITY && ps.umin <= ps.zmax;
    const SelOut r = select_desc<false>(rc.valid, rc, [](double z) { return key_of(z); }, (uint64_t)rp.top_k,
                                        V, fs.rl[0], fs, xw, hgen, known, ks);
    if (!r.found) return FastOut{V - 1, true, 0.0};
    const double kth_z = val_of_key(r.key);
    const double kth_y = yexact(kth_z);
    z_lo = kth_z;
    for (int it = 0; it < 64; ++it) {
      const double zp = dbl_prev(z_lo);
      if (yexact(zp) >= kth_y) z_lo = zp;
      else break;
    }
    if (!(ps.umax < z_lo)) return FastOut{V - 1, true, 0.0};
  }

  // ---- softmax (:79-81): p = exp(y - ymax) / S, once per candidate
  const YScale ys{T, 1.0 / T};
  const double ymax = ys(ps.zmax);
  double s = 0.0;
  uint32_t nkept = 0;
#pragma unroll
  for (int q = 0; q < kPerT; ++q) {
    const double z = rc.v[q];
    const bool kept = ((rc.valid >> q) & 1u) && z >= z_lo;
    const double e = kept ? fast_exp_neg(ys(z) - ymax, tab) : 0.0;
    nkept += kept ? 1u : 0u;
    rc.v[q] = e;
    s += e;
  }
  double S;
  uint64_t nk = 0;  // the top-p selection's active count, bounded above
  if (TOPK) {
    // the normaliser (waves left to right, as xw_sum) and the kept count
    const auto sk = xw.post(bits_of(wave_sum(s)), (uint64_t)wave_sum(nkept), 0);
    S = 0.0;
    nk = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      S += dbl_of(sk[0][w]);
      nk += sk[1][w];
    }
  } else {
    double ms[kSegPerLane], lex;
    S = seg_norm(sg, tab, ms, &lex).S;
    nk = count_cands();
  }
  const double invS = 1.0 / S;
  uint32_t pos = 0;
#pragma unroll
  for (int q = 0; q < kPerT; ++q) {
    rc.v[q] *= invS;
    rc.w[q] = to_fx(rc.v[q]);
    if (rc.v[q] > 0.0) pos |= 1u << q;
  }

  // ---- top-p: first token (p desc, index asc) whose inclusive mass reaches
  // top_p (:82-90)
  if (rp.topp) {
    // every probability lies in [p(smallest chunk threshold), 1 / S] up to
    // rounding: the row max's exp argument ys(z) - ymax may be contracted
    // to an fma and come out a rounding residual above 0, so its e can be
    // 1 + 2^-52, and the exp is monotone only up to an ulp.  Both ends get
    // 2^32 ulps of slack (a relative 2^-20).  The count bounds the active
    // set from above (underflows to 0 drop out).
    constexpr uint64_t kSlack = 1ull << 32;
    const uint64_t plo = pkey_of(fast_exp_neg(ys(ps.umin) - ymax, tab) * invS);
    const KeySpan ps_span{plo > kSlack ? plo - kSlack : 0ull, pkey_of(invS) + kSlack, uniform(nk)};
    const SelOut r = select_desc<true>(pos, rc, [](double p) { return pkey_of(p); }, topp_target(rp.top_p), V,
                                       fs.rl[1], fs, xw, hgen, true, ps_span);
    if (r.giveup) return FastOut{V - 1, true, TOPK ? 0.0 : S};
    if (r.found) {
#pragma unroll
      for (int q = 0; q < kPerT; ++q) {
        const uint64_t k = pkey_of(rc.v[q]);
        if (!(k > r.key || (k == r.key && rc.idx[q] <= r.idx))) rc.w[q] = 0ull;
      }
    }
    if (!TOPK && ps.umax > -INFINITY) {
      // the largest token left out must fall outside the nucleus
      const double pU = fast_exp_neg(ys(ps.umax) - ymax, tab) * invS;
      if (!(r.found && r.key > pkey_of(pU))) return FastOut{V - 1, true, S};
    }
  }

  // ---- draw in vocabulary order (:94-98)
  return FastOut{draw_kept(rc, V, rp.u, fs, hgen), false, 0.0};
}

// ======================================================== candidate merge
// The candidate rows' merge (top-k and/or top-p, sampling.py:75-90 and the
// draw :94-98).  The row's candidate slots are spread so that every chunk
// belongs to one wave: wave w holds chunks w, w + 8, ... (capc slots each),
// lane l's slot j being wave-local slot L = 64 j + l, i.e. chunk
// w + 8 (L / capc), chunk slot L % capc.  Per-chunk sums are then wave
// reductions, and the draw inside the chunk that holds the inverse-CDF
// point is finished by that chunk's wave alone.
constexpr int kMS = kCandCap / kThreads;  // candidate slots per lane

struct MCands {
  double z[kMS];    // penalised logit
  uint64_t w[kMS];  // fixed-point probability while kept, else 0
  int idx[kMS];     // token id
  uint32_t valid;   // bit j: slot j holds a candidate
  uint32_t jm;      // bit j: slot j holds a candidate in some lane of the wave (uniform)
};

// Loops over a lane's slots skip, with a uniform branch, the slots that
// hold no candidate anywhere in the wave (a top-k row's chunk fills one or
// two of its wave's 16).
#define MC_FOR(j, mc) \
  _Pragma("unroll") for (int j = 0; j < kMS; ++j) if (((mc).jm >> j) & 1u)

// Chunk group of slot j (uniform: capc is a power of two >= 64) and its
// chunk slot.
__device__ __forceinline__ int mc_group(int j, int capc) { return (kWave * j) / capc; }
__device__ __forceinline__ int mc_slot(int j, int capc) { return (kWave * j + lane()) & (capc - 1); }

// Loads the slots j whose chunk slot lies in [s0, s1) and below the
// chunk's candidate count (wc, this wave's copy); marks them valid.
__device__ __forceinline__ void mc_load(const SampleArgs& a, int row, MCands& mc, const int* wc, int s0, int s1) {
  const int C = a.ws.C, capc = a.ws.capc;
  const size_t base = (size_t)row * C * capc;
#pragma unroll
  for (int j = 0; j < kMS; ++j) {
    const int c = wave() + kWaves * mc_group(j, capc);
    const int s = mc_slot(j, capc);
    if (c < C && s >= s0 && s < s1 && s < wc[c]) {
      const size_t i = base + (size_t)c * capc + s;
      mc.z[j] = a.ws.cz[i];
      mc.idx[j] = a.ws.ci[i];
      mc.valid |= 1u << j;
    }
  }
}

// The slots below chunk slot smax, loaded before the counts are known
// (top-p rows: every slot, their chunks fill nearly all of them; top-k rows:
// the first 128 of each chunk); validity is set once the counts are in.
__device__ __forceinline__ void mc_load_first(const SampleArgs& a, int row, MCands& mc, int smax) {
  const int C = a.ws.C, capc = a.ws.capc;
  const size_t base = (size_t)row * C * capc;
#pragma unroll
  for (int j = 0; j < kMS; ++j) {
    const int c = wave() + kWaves * mc_group(j, capc);
    mc.z[j] = -INFINITY;
    mc.idx[j] = 0;
    mc.w[j] = 0ull;
    if (c < C && mc_slot(j, capc) < smax) {
      const size_t i = base + (size_t)c * capc + mc_slot(j, capc);
      mc.z[j] = a.ws.cz[i];
      mc.idx[j] = a.ws.ci[i];
    }
  }
}

// The slots with chunk slot in [s0, s1), loaded before the counts are known.
__device__ __forceinline__ void mc_load_range(const SampleArgs& a, int row, MCands& mc, int s0, int s1) {
  const int C = a.ws.C, capc = a.ws.capc;
  const size_t base = (size_t)row * C * capc;
#pragma unroll
  for (int j = 0; j < kMS; ++j) {
    const int c = wave() + kWaves * mc_group(j, capc);
    const int s = mc_slot(j, capc);
    if (c < C && s >= s0 && s < s1) {
      const size_t i = base + (size_t)c * capc + s;
      mc.z[j] = a.ws.cz[i];
      mc.idx[j] = a.ws.ci[i];
    }
  }
}

// Marks the loaded slots that hold candidates, then loads the rest of a
// chunk whose candidates run past smax.
__device__ __forceinline__ void mc_validate(const SampleArgs& a, int row, MCands& mc, const int* wc, int smax) {
  const int C = a.ws.C, capc = a.ws.capc;
  mc.valid = 0;
  bool more = false;
#pragma unroll
  for (int j = 0; j < kMS; ++j) {
    const int c = wave() + kWaves * mc_group(j, capc);
    const int s = mc_slot(j, capc);
    if (c < C && s < wc[c] && s < smax) mc.valid |= 1u << j;
    more |= c < C && s >= smax && s < wc[c];
  }
  if (__ballot(more) != 0ull) mc_load(a, row, mc, wc, smax, capc);
  mc.jm = (uint32_t)__builtin_amdgcn_readlane((int)wave_scan_incl(mc.valid, 0u, OpOr{}), kWave - 1);
}

struct ZSel {
  bool found;
  bool giveup;
  double z;
  int idx;
};

// Every wave on its own: the bin of h where the running total (bins taken
// from the highest down, starting at `above`) first reaches target.  Lane l
// sums the 16 bins of group 63 - l with 16-byte LDS reads and a wave scan
// finds the group; the 16 lanes of each row then read one bin of that group
// each, highest first, and a row scan finds the bin.  The running total is
// non-decreasing, so exactly one bin takes it from below target to target
// or more.
template <bool MASS>
__device__ __forceinline__ WPick wave_pick2(const Hist& h, uint64_t above, uint64_t target) {
  constexpr int PL = kHB / kWave;
  static_assert(PL == 16, "one 16-lane row per group");
  const int grp = kWave - 1 - lane();
  uint64_t s = 0;
  if (MASS) {
    const uint4* hv = reinterpret_cast<const uint4*>(h.mass + grp * PL);
#pragma unroll
    for (int i = 0; i < PL / 2; ++i) {
      const uint4 q = hv[i];
      s += (((uint64_t)q.y << 32) | q.x) + (((uint64_t)q.w << 32) | q.z);
    }
  } else {
    const uint4* hv = reinterpret_cast<const uint4*>(h.cnt + grp * PL);
#pragma unroll
    for (int i = 0; i < PL / 4; ++i) {
      const uint4 q = hv[i];
      s += (uint64_t)((q.x + q.y) + (q.z + q.w));
    }
  }
  const uint64_t incl = wave_scan_incl(s, (uint64_t)0, OpAdd{});
  const uint64_t tot = lane_value(incl, kWave - 1);
  if (above >= target || above + tot < target) return WPick{false, -1, above + tot};
  const uint64_t cross = __ballot(above + incl - s < target && above + incl >= target);
  const int lc = __builtin_ctzll(cross);
  const uint64_t gab = above + lane_value(incl - s, lc);  // the total above the group
  const int top = (kWave - 1 - lc) * PL + PL - 1;         // the group's highest bin
  const int j = lane() & (PL - 1);
  const uint64_t v = MASS ? h.mass[top - j] : (uint64_t)h.cnt[top - j];
  uint64_t r = v;
  r += dpp<kDppRowShr1, 0xf>((uint64_t)0, r);
  r += dpp<kDppRowShr2, 0xf>((uint64_t)0, r);
  r += dpp<kDppRowShr4, 0xf>((uint64_t)0, r);
  r += dpp<kDppRowShr8, 0xf>((uint64_t)0, r);
  const uint64_t hit = __ballot(gab + r >= target) & 0xffffull;
  const int jj = __builtin_ctzll(hit);
  return WPick{true, top - jj, gab + lane_value(r - v, jj)};
}

// Workgroup min and max of the active values (one cross-wave combine).
__device__ __forceinline__ void active_range(uint32_t act, const MCands& mc, bool by_idx, int V, XWave& xw, double* lo,
                                             double* hi) {
  double a = INFINITY, b = -INFINITY;
  MC_FOR(j, mc) {
    if ((act >> j) & 1u) {
      const double v = by_idx ? (double)(V - 1 - mc.idx[j]) : mc.z[j];
      a = fmin(a, v);
      b = fmax(b, v);
    }
  }
  const auto s = xw.post(bits_of(wave_min(a)), bits_of(wave_max(b)), 0);
  a = dbl_of(s[0][0]);
  b = dbl_of(s[1][0]);
#pragma unroll
  for (int w = 1; w < kWaves; ++w) {
    a = fmin(a, dbl_of(s[0][w]));
    b = fmax(b, dbl_of(s[1][w]));
  }
  *lo = uniform(a);
  *hi = uniform(b);
}

// Selection over the active slots in (z descending, token index ascending)
// order, sampling.py:76-77 and :83-86:
//   MASS=false: the target-th entry (its z: the top-k threshold);
//   MASS=true : the first entry whose inclusive weight reaches target (the
//               top-p cut).
// Levels of kHB affine value bins over [lo, hi] (every active z lies there,
// n bounds their count from above) keep the bin where the running count or
// weight crosses the target, until one wave's worth is left; the rank list
// then orders those exactly.  A level that separates nothing narrows the
// range to the values' own; equal values are ordered by token index (levels
// over V - 1 - index).
template <bool MASS>
__device__ __forceinline__ ZSel select_z(uint32_t act, const MCands& mc, double lo, double hi, uint32_t n,
                                         uint64_t target, int V, RankList& rl, FastSmem& fs, XWave& xw, int& hgen,
                                         uint64_t above0 = 0) {
  // the barrier the first level or the rank list relies on: the kernel
  // zeroes the first histogram and the rank lists at its start
  wg_barrier();
  PLH_STAMP_IF(MASS, (int)blockIdx.x, 10);
  if (n == 0 || (!MASS && n < target)) return ZSel{false, false, 0.0, 0};
  target = uniform(target);
  uint32_t cnt = n;
  uint64_t above = uniform(above0);
  bool by_idx = false;
  double vlo = lo, vhi = hi;
  auto val = [&](int j) -> double { return by_idx ? (double)(V - 1 - mc.idx[j]) : mc.z[j]; };
  for (int lev = 0; cnt > (uint32_t)kWave; ++lev) {
    if (lev == kMaxLevels) return ZSel{false, true, 0.0, 0};
    if (!(vhi > vlo)) {
      // every active value is vlo
      if (!MASS) return ZSel{true, false, vlo, 0};
      if (by_idx) return ZSel{false, true, 0.0, 0};
      by_idx = true;
      vlo = 0.0;
      vhi = (double)(V - 1);
    }
    const Affine af = make_affine(vlo, vhi, kHB);
    Hist& h = next_hist(fs, hgen);
    MC_FOR(j, mc) {
      if ((act >> j) & 1u) {
        const int b = af.bin(val(j));
        lds_add(&h.cnt[b], 1u);
        if (MASS) lds_add(&h.mass[b], mc.w[j]);
      }
    }
    PLH_STAMP_IF(MASS, (int)blockIdx.x, 14);
    wg_barrier();
    PLH_STAMP_IF(MASS, (int)blockIdx.x, 15);
    const WPick pk = wave_pick2<MASS>(h, above, target);
    PLH_STAMP_IF(MASS, (int)blockIdx.x, 11);
    if (!pk.found) return ZSel{false, false, 0.0, 0};
    above = uniform(pk.above);
    const int d = uniform(pk.d);
    const uint32_t ncnt = (uint32_t)uniform((int)h.cnt[d]);
    MC_FOR(j, mc) {
      if (((act >> j) & 1u) && af.bin(val(j)) != d) act &= ~(1u << j);
    }
    if (ncnt == cnt) {
      active_range(act, mc, by_idx, V, xw, &vlo, &vhi);  // nothing separated: the values' own range
    } else {
      const double w = 1.0 / af.scale;
      vlo = af.lo + (double)d * w;
      vhi = d == kHB - 1 ? vhi : af.lo + (double)(d + 1) * w;
    }
    cnt = ncnt;
  }
  PLH_STAMP_IF(MASS, (int)blockIdx.x, 12);
  // rank list: one LDS reservation per wave
  int nq = 0;
  MC_FOR(j, mc) { nq += (act >> j) & 1u; }
  const int qi = wave_scan_incl(nq, 0, OpAdd{});
  int rbase = 0;
  if (lane() == kWave - 1 && qi > 0) rbase = lds_fetch_add(&rl.n, qi);
  int slot = lane_value(rbase, kWave - 1) + qi - nq;
  MC_FOR(j, mc) {
    if ((act >> j) & 1u) {
      rl.key[slot] = key_of(mc.z[j]);
      rl.idx[slot] = mc.idx[j];
      rl.w[slot] = MASS ? mc.w[j] : 0ull;
      ++slot;
    }
  }
  wg_barrier();
  // lane i of every wave holds entry i; wave w compares it with entries
  // j in [8w, 8w + 8) (LDS broadcast reads) and adds its counts to the
  // entry's totals
  const int m = uniform(rl.n);
  const int ln = lane();
  uint64_t k = 0ull, wt = 0ull;
  int ix = INT_MAX;
  if (ln < m) {
    k = rl.key[ln];
    ix = rl.idx[ln];
    wt = rl.w[ln];
  }
  uint32_t rank = 0;
  uint64_t ahead = 0;
  constexpr int kPerWave = kWave / kWaves;
#pragma unroll
  for (int jj = 0; jj < kPerWave; ++jj) {
    const int j = wave() * kPerWave + jj;
    if (j < m) {
      const uint64_t kj = rl.key[j];
      const int ij = rl.idx[j];
      const bool bj = kj > k || (kj == k && ij < ix);
      rank += bj ? 1u : 0u;
      if (MASS) ahead += bj ? rl.w[j] : 0ull;
    }
  }
  if (ln < m) {
    lds_add(&rl.rank[ln], rank);
    if (MASS) lds_add(&rl.ahead[ln], ahead);
  }
  PLH_STAMP_IF(MASS, (int)blockIdx.x, 13);
  wg_barrier();
  if (ln < m) {
    rank = rl.rank[ln];
    ahead = rl.ahead[ln];
  }
  bool hit;
  if (!MASS) hit = ln < m && (uint64_t)rank == target - above - 1;
  else hit = ln < m && above + ahead < target && above + ahead + wt >= target;
  const uint64_t hits = __ballot(hit);
  if (hits == 0) return ZSel{false, !MASS, 0.0, 0};
  const int L = __builtin_ctzll(hits);
  return ZSel{true, false, val_of_key(lane_value(k, L)), lane_value(ix, L)};
}

// Inverse-CDF draw over the kept slots in vocabulary order (sampling.py:94-98):
// the first token whose running fixed-point mass exceeds floor(u * total),
// V - 1 when none does.  The chunk holding that point comes from the
// per-chunk kept sums (each chunk's wave sums its own); that chunk's wave
// then locates the token alone, through kDrawBins index bins of the chunk's
// tokens and the crossing bin's tokens laid out by offset.  Returns the id
// in the lanes of the chunk's wave and -1 in the other waves.
constexpr int kDrawBins = 256;
template <typename TIn>
__device__ __forceinline__ int draw_chunks(const SampleArgs& a, const MCands& mc, double u, FastSmem& fs) {
  using G = Geo<TIn>;
  const int C = a.ws.C, capc = a.ws.capc, V = a.V;
  constexpr int kTokPerBin = G::kChunk / kDrawBins;  // 64 (float) or 32 (double) tokens per index bin
  static_assert(kTokPerBin <= kWave && kTokPerBin <= kDrawSpanMax, "one lane per token of a bin");
  // per-chunk kept sums: wave w posts chunks w, w + 8, ...
  const int ng = (C + kWaves - 1) / kWaves;
  for (int g = 0; g < ng; ++g) {
    uint64_t s = 0;
    MC_FOR(j, mc) {
      if (mc_group(j, capc) == g) s += mc.w[j];
    }
    s = wave_sum(s);
    const int c = wave() + kWaves * g;
    if (lane() == 0 && c < C) fs.csum[c] = s;
  }
  wg_barrier();
  // every wave: the total, and the chunk where the running mass crosses t
  const uint64_t cs = lane() < C ? fs.csum[lane()] : 0ull;  // C <= kWave
  const uint64_t incl = wave_scan_incl(cs, (uint64_t)0, OpAdd{});
  const uint64_t tot = lane_value(incl, kWave - 1);
  if (tot == 0) return V - 1;
  const uint64_t t = (uint64_t)__double2ull_rd(u * (double)tot);
  const uint64_t hits = __ballot(incl - cs <= t && t < incl && lane() < C);
  if (hits == 0) return V - 1;
  const int cstar = __builtin_ctzll(hits);
  const uint64_t before = uniform(lane_value(incl - cs, cstar));
  if (wave() != cstar % kWaves) return -1;
  // the chunk's wave: index bins of kTokPerBin tokens over the chunk
  const int gstar = cstar / kWaves;
  const int c0 = cstar * G::kChunk;
  uint64_t* hb = fs.h[0].mass;  // this wave alone uses it from here on
  constexpr int kPer = kDrawBins / kWave;
  static_assert(kPer == 4, "four bins per lane");
  reinterpret_cast<ulonglong2*>(hb)[2 * lane()] = make_ulonglong2(0ull, 0ull);
  reinterpret_cast<ulonglong2*>(hb)[2 * lane() + 1] = make_ulonglong2(0ull, 0ull);
  MC_FOR(j, mc) {
    if (mc_group(j, capc) == gstar && mc.w[j] != 0ull) lds_add(&hb[(mc.idx[j] - c0) / kTokPerBin], mc.w[j]);
  }
  // lane l holds bins [4l, 4l + 4)
  const ulonglong2 q0 = reinterpret_cast<const ulonglong2*>(hb)[2 * lane()];
  const ulonglong2 q1 = reinterpret_cast<const ulonglong2*>(hb)[2 * lane() + 1];
  const uint64_t bv[kPer] = {q0.x, q0.y, q1.x, q1.y};
  const uint64_t s = (bv[0] + bv[1]) + (bv[2] + bv[3]);
  const uint64_t in2 = wave_scan_incl(s, (uint64_t)0, OpAdd{});
  const uint64_t h2 = __ballot(before + in2 - s <= t && t < before + in2);
  if (h2 == 0) return V - 1;
  const int L = __builtin_ctzll(h2);
  int bl = 0;
  uint64_t bf = 0, run = before + in2 - s;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    if (run <= t && t < run + bv[j]) {
      bl = kPer * lane() + j;
      bf = run;
    }
    run += bv[j];
  }
  const int b = uniform(lane_value(bl, L));
  const uint64_t bbefore = uniform(lane_value(bf, L));
  // the bin's kept tokens by offset
  if (lane() < kTokPerBin) fs.dspan[lane()] = 0ull;
  MC_FOR(j, mc) {
    if (mc_group(j, capc) == gstar && mc.w[j] != 0ull && (mc.idx[j] - c0) / kTokPerBin == b)
      fs.dspan[mc.idx[j] - c0 - b * kTokPerBin] = mc.w[j];
  }
  const uint64_t v = lane() < kTokPerBin ? fs.dspan[lane()] : 0ull;
  const uint64_t in3 = wave_scan_incl(v, (uint64_t)0, OpAdd{});
  const uint64_t h3 = __ballot(v != 0ull && bbefore + in3 - v <= t && t < bbefore + in3);
  if (h3 == 0) return V - 1;
  return c0 + b * kTokPerBin + __builtin_ctzll(h3);
}

// Top-k and/or top-p rows from the chunk candidates (sampling.py:75-90,
// :94-98).  id: the drawn token in the lanes of the wave that drew it, -1 in
// the others.
struct CandOut {
  int id;
  bool general;  // the candidates cannot decide the row exactly (uniform)
  double S;      // general: the full normaliser when known (top-p-only rows), else 0
};

template <typename TIn, bool TOPK>
__device__ __forceinline__ CandOut merge_cands(const SampleArgs& a, MCands& mc, const SegLoad& sg, const RowParams& rp,
                                               const PartSum& ps, FastSmem& fs, XWave& xw, int& hgen) {
  const int V = a.V;
  const double* tab = fs.exp_tab[wave()];
  const int* wc = fs.wcnt[wave()];
  auto count_cands = [&]() -> uint32_t {
    int nc = 0;
    for (int c = lane(); c < a.ws.C; c += kWave) nc += wc[c];
    return (uint32_t)uniform(wave_sum(nc));
  };
  const double T = rp.T;
  auto yexact = [&](double z) -> double { return T == 1.0 ? z : z / T; };

  // ---- top-k: k-th largest with multiplicity, keep y >= kth_y (:76-78)
  double z_lo = -INFINITY;
  uint32_t act = mc.valid;
  if (TOPK) {
    // every candidate lies in [the smallest chunk threshold, the row max]
    const double lo = ps.umin > -INFINITY ? ps.umin : -1.7976931348623157e308;
    const ZSel r = select_z<false>(act, mc, lo, ps.zmax, count_cands(), (uint64_t)rp.top_k, V, fs.rl[0], fs, xw, hgen);
    if (!r.found) return CandOut{V - 1, true, 0.0};
    const double kth_y = yexact(r.z);
    z_lo = r.z;
    for (int it = 0; it < 64; ++it) {
      const double zp = dbl_prev(z_lo);
      if (yexact(zp) >= kth_y) z_lo = zp;
      else break;
    }
    if (!(ps.umax < z_lo)) return CandOut{V - 1, true, 0.0};
  }

  // ---- softmax (:79-81): p = exp(y - ymax) / S, once per kept candidate
  const YScale ys{T, 1.0 / T};
  const double ymax = ys(ps.zmax);
  double s = 0.0;
  uint32_t nkept = 0;
  MC_FOR(j, mc) {
    const bool k = ((act >> j) & 1u) && mc.z[j] >= z_lo;
    const double e = k ? fast_exp_neg(ys(mc.z[j]) - ymax, tab) : 0.0;
    mc.w[j] = bits_of(e);  // the weight slot holds e until S is known
    nkept += k ? 1u : 0u;
    s += e;
  }
  double S;
  uint32_t nk;
  if (TOPK) {
    const auto sk = xw.post(bits_of(wave_sum(s)), (uint64_t)wave_sum(nkept), 0);
    S = 0.0;
    nk = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      S += dbl_of(sk[0][w]);
      nk += (uint32_t)sk[1][w];
    }
  } else {
    double ms[kSegPerLane], lex;
    S = seg_norm(sg, tab, ms, &lex).S;
    nk = count_cands();
  }
  const double invS = 1.0 / S;
  uint32_t pos = 0;
  MC_FOR(j, mc) {
    const double p = dbl_of(mc.w[j]) * invS;
    mc.w[j] = to_fx(p);
    if (p > 0.0) pos |= 1u << j;
  }

  // ---- top-p: first token (p desc, index asc) whose inclusive mass reaches
  // top_p (:82-90), in (z desc, index asc) order
  if (rp.topp) {
    const double lo = TOPK ? z_lo : (ps.umin > -INFINITY ? ps.umin : -1.7976931348623157e308);
    const ZSel r = select_z<true>(pos, mc, lo, ps.zmax, nk, topp_target(rp.top_p), V, fs.rl[1], fs, xw, hgen);
    if (r.giveup) return CandOut{V - 1, true, TOPK ? 0.0 : S};
    if (r.found) {
      MC_FOR(j, mc) {
        if (!(mc.z[j] > r.z || (mc.z[j] == r.z && mc.idx[j] <= r.idx))) mc.w[j] = 0ull;
      }
    }
    if (!TOPK && ps.umax > -INFINITY) {
      // the largest token left out must fall outside the nucleus
      const double pU = fast_exp_neg(ys(ps.umax) - ymax, tab) * invS;
      const double pC = r.found ? fast_exp_neg(ys(r.z) - ymax, tab) * invS : 0.0;
      if (!(r.found && pC > pU)) return CandOut{V - 1, true, S};
    }
  }

  // ---- draw in vocabulary order (:94-98)
  return CandOut{draw_chunks<TIn>(a, mc, rp.u, fs), false, 0.0};
}

// ------------------------------------------------- top-p rows from buckets
// Top-p rows with no top-k (sampling.py:79-90, then :94-98), from the
// chunks' candidate buckets (write_buckets): the bucket masses of all
// chunks, aligned on the absolute grid, give the bucket holding the cut
// and the mass above it; only that bucket's candidates are then ordered
// (p descending, token index ascending), and only the chunk holding the
// inverse-CDF point has its kept candidates read again for the draw.
// Used when the row has at most kWaves chunks: wave c handles chunk c.
struct BktLoad {
  uint64_t m[kBkt / kWave];  // the lane's buckets 4l .. 4l + 3 of its wave's chunk
  uint32_t n[kBkt / kWave];
  int hb;                    // lane c: chunk c's top bucket
  double ym;                 // lane c: chunk c's max y
};

__device__ __forceinline__ void load_buckets(const SampleArgs& a, int row, BktLoad& bl) {
  const int C = a.ws.C;
  const size_t rb = (size_t)row * C;
  constexpr int kB4 = kBkt / kWave;
  bl.hb = INT_MIN;
  bl.ym = -INFINITY;
  if (lane() < C) {
    bl.hb = a.ws.bhb[rb + lane()];
    bl.ym = a.ws.bymax[rb + lane()];
  }
#pragma unroll
  for (int j = 0; j < kB4; ++j) {
    bl.m[j] = 0ull;
    bl.n[j] = 0u;
  }
  if (wave() < C) {
    const size_t b = (rb + wave()) * kBkt + kB4 * lane();
    const ulonglong2 m0 = *reinterpret_cast<const ulonglong2*>(a.ws.bmass + b);
    const ulonglong2 m1 = *reinterpret_cast<const ulonglong2*>(a.ws.bmass + b + 2);
    const uint4 n0 = *reinterpret_cast<const uint4*>(a.ws.bcnt + b);
    bl.m[0] = m0.x;
    bl.m[1] = m0.y;
    bl.m[2] = m1.x;
    bl.m[3] = m1.y;
    bl.n[0] = n0.x;
    bl.n[1] = n0.y;
    bl.n[2] = n0.z;
    bl.n[3] = n0.w;
  }
}

template <typename TIn>
__device__ __forceinline__ CandOut merge_topp(const SampleArgs& a, int row, const RowParams& rp, const PartSum& ps,
                                              const SegLoad& sg, const BktLoad& bl, FastSmem& fs, XWave& xw,
                                              int& hgen) {
  using G = Geo<TIn>;
  const int C = a.ws.C, capc = a.ws.capc, V = a.V;
  constexpr int kB4 = kBkt / kWave;
  const double* tab = fs.exp_tab[wave()];
  double ms[kSegPerLane], lex;
  const SegNorm sn = seg_norm(sg, tab, ms, &lex);
  const double invS = 1.0 / sn.S;
  const uint64_t target = topp_target(rp.top_p);
  PLH_STAMP(row, 2);
  // the row's top bucket and this wave's chunk (INT_MIN: a chunk without
  // candidates)
  const int hbt = uniform(wave_max(bl.hb));
  if (hbt == INT_MIN) return CandOut{V - 1, true, sn.S};
  const int c = wave();
  const int hbc = c < C ? uniform(lane_value(bl.hb, c)) : INT_MIN;
  const bool mine = hbc != INT_MIN;
  const int dc = mine ? hbt - hbc : 0;  // the chunk's bucket lb is row bucket dc + lb (the last one open)
  // probability of a candidate of this chunk: e * Fc
  const double Fc = mine ? fast_exp_neg(uniform(lane_value(bl.ym, c)) - sn.ymax, tab) * invS : 0.0;
  // bucket masses in units of 2^-62 of probability, added into the row buckets
  // (zeroed at the kernel's start)
  wg_barrier();
  uint64_t wv[kB4];
#pragma unroll
  for (int j = 0; j < kB4; ++j) {
    wv[j] = bl.m[j] != 0ull ? (uint64_t)__double2ull_rn((double)bl.m[j] * (Fc * 1024.0)) : 0ull;
    if (wv[j] != 0ull) {
      const int r = min(dc + kB4 * lane() + j, kBkt - 1);
      lds_add(&fs.rowm[r], wv[j]);
    }
  }
  wg_barrier();
  // every wave: the row bucket where the running mass from the top reaches target
  uint64_t rv[kB4], rs = 0;
  {
    const ulonglong2 q0 = reinterpret_cast<const ulonglong2*>(fs.rowm)[2 * lane()];
    const ulonglong2 q1 = reinterpret_cast<const ulonglong2*>(fs.rowm)[2 * lane() + 1];
    rv[0] = q0.x;
    rv[1] = q0.y;
    rv[2] = q1.x;
    rv[3] = q1.y;
    rs = (rv[0] + rv[1]) + (rv[2] + rv[3]);
  }
  PLH_STAMP(row, 3);
  const uint64_t rin = wave_scan_incl(rs, (uint64_t)0, OpAdd{});
  const uint64_t hx = __ballot(rin - rs < target && rin >= target);
  if (hx == 0ull) return CandOut{V - 1, true, sn.S};
  const int lx = __builtin_ctzll(hx);
  int rl_ = 0;
  uint64_t ab = 0, run = rin - rs;
#pragma unroll
  for (int j = 0; j < kB4; ++j) {
    if (run < target && run + rv[j] >= target) {
      rl_ = kB4 * lane() + j;
      ab = run;
    }
    run += rv[j];
  }
  const int rstar = uniform(lane_value(rl_, lx));
  const uint64_t A = uniform(lane_value(ab, lx));
  // this chunk: mass above the cut bucket, and the list range of its
  // candidates in the cut bucket
  uint64_t above = 0;
  uint32_t cnt_before = 0, cnt_in = 0;
#pragma unroll
  for (int j = 0; j < kB4; ++j) {
    const int r = min(dc + kB4 * lane() + j, kBkt - 1);
    if (r < rstar) {
      above += wv[j];
      cnt_before += bl.n[j];
    } else if (r == rstar) {
      cnt_in += bl.n[j];
    }
  }
  above = wave_sum(above);
  const int p0 = uniform(wave_sum((int)cnt_before));
  const int p1 = p0 + uniform(wave_sum((int)cnt_in));
  // the cut bucket's candidates of this chunk: p = e * Fc
  MCands mc;
  mc.valid = 0;
  mc.jm = 0;
  const size_t cb = ((size_t)row * C + c) * capc;
#pragma unroll
  for (int j = 0; j < kMS; ++j) {
    mc.z[j] = 0.0;
    mc.w[j] = 0ull;
    mc.idx[j] = 0;
    const int pos = p0 + kWave * j + lane();
    if (mine && p0 + kWave * j < p1) {
      mc.jm |= 1u << j;
      if (pos < p1) {
        const double p = a.ws.cz[cb + pos] * Fc;
        mc.z[j] = p;
        mc.w[j] = to_fx(p);
        mc.idx[j] = a.ws.ci[cb + pos];
        mc.valid |= 1u << j;
      }
    }
  }
  if (lane() == 0 && c < C) {
    fs.cq0[c] = mine ? p0 : 0;
    fs.cq1[c] = mine ? p1 : 0;
  }
  // the cut among them, in (p desc, index asc) order (select_z orders by its
  // values, here p), starting from the mass above the bucket
  wg_barrier();
  PLH_STAMP(row, 4);
  uint32_t nx = 0;
  for (int k = lane(); k < C; k += kWave) nx += (uint32_t)(fs.cq1[k] - fs.cq0[k]);
  nx = (uint32_t)uniform((int)wave_sum(nx));
  // every p of the bucket lies in [exp(B / 8 - ymax), exp((B + 1) / 8 - ymax)] / S
  // (B = hbt - rstar; the last bucket is open below), with some slack
  const double yb = (double)(hbt - rstar) / kBktPerY - sn.ymax;
  const double plo = rstar == kBkt - 1 ? 0.0 : fast_exp_neg(yb, tab) * invS * (1.0 - 1e-9);
  const double phi = fast_exp_neg(fmin(yb + 1.0 / kBktPerY, 0.0), tab) * invS * (1.0 + 1e-9);
  const ZSel r = select_z<true>(mc.valid, mc, plo, phi, nx, target, V, fs.rl[1], fs, xw, hgen, A);
  PLH_STAMP(row, 5);
  if (!r.found) return CandOut{V - 1, true, sn.S};
  if (ps.umax > -INFINITY) {
    // the largest token left out must fall outside the nucleus
    const YScale ys{rp.T, 1.0 / rp.T};
    const double pU = fast_exp_neg(ys(ps.umax) - sn.ymax, tab) * invS;
    if (!(r.z > pU)) return CandOut{V - 1, true, sn.S};
  }
  // kept mass of each chunk: above the cut bucket, and its kept candidates in it
  uint64_t kx = 0;
  MC_FOR(j, mc) {
    if (((mc.valid >> j) & 1u) && (mc.z[j] > r.z || (mc.z[j] == r.z && mc.idx[j] <= r.idx))) kx += mc.w[j];
  }
  kx = wave_sum(kx);
  if (lane() == 0 && c < C) fs.csum[c] = mine ? above + kx : 0ull;
  for (int b = threadIdx.x; b < kDrawBins; b += kThreads) fs.h[0].mass[b] = 0ull;
  if (threadIdx.x < G::kChunk / kDrawBins) fs.dspan[threadIdx.x] = 0ull;
  wg_barrier();
  // every wave: the chunk holding the inverse-CDF point
  PLH_STAMP(row, 6);
  const uint64_t cs = lane() < C ? fs.csum[lane()] : 0ull;
  const uint64_t incl = wave_scan_incl(cs, (uint64_t)0, OpAdd{});
  const uint64_t tot = lane_value(incl, kWave - 1);
  if (tot == 0) return CandOut{V - 1, false, 0.0};
  const uint64_t t = (uint64_t)__double2ull_rd(rp.u * (double)tot);
  const uint64_t hc = __ballot(incl - cs <= t && t < incl && lane() < C);
  if (hc == 0) return CandOut{V - 1, false, 0.0};
  const int cstar = __builtin_ctzll(hc);
  const uint64_t before = uniform(lane_value(incl - cs, cstar));
  // its kept candidates (every thread: list positions tid, tid + 512), by
  // index bins of the chunk's tokens
  const double Fs = fast_exp_neg(uniform(lane_value(bl.ym, cstar)) - sn.ymax, tab) * invS;
  // the chunk's cut-bucket range: entries before q0 are above the cut bucket
  const int q0 = uniform(fs.cq0[cstar]);
  const int q1 = uniform(fs.cq1[cstar]);
  const size_t sb = ((size_t)row * C + cstar) * capc;
  const int c0 = cstar * G::kChunk;
  constexpr int kTokPerBin = G::kChunk / kDrawBins;
  constexpr int kPer = kCapChunk / kThreads;
  uint64_t dw[kPer];
  int di[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int pos = (int)threadIdx.x + k * kThreads;
    dw[k] = 0ull;
    di[k] = c0;
    if (pos < q1) {
      const double p = a.ws.cz[sb + pos] * Fs;
      const int id = a.ws.ci[sb + pos];
      const bool keep = pos < q0 || p > r.z || (p == r.z && id <= r.idx);
      dw[k] = keep ? to_fx(p) : 0ull;
      di[k] = id;
      if (dw[k] != 0ull) lds_add(&fs.h[0].mass[(id - c0) / kTokPerBin], dw[k]);
    }
  }
  wg_barrier();
  // every wave: the index bin, then its tokens by offset
  PLH_STAMP(row, 7);
  const ulonglong2 b0 = reinterpret_cast<const ulonglong2*>(fs.h[0].mass)[2 * lane()];
  const ulonglong2 b1 = reinterpret_cast<const ulonglong2*>(fs.h[0].mass)[2 * lane() + 1];
  const uint64_t bv[4] = {b0.x, b0.y, b1.x, b1.y};
  const uint64_t bs = (bv[0] + bv[1]) + (bv[2] + bv[3]);
  const uint64_t bin = wave_scan_incl(bs, (uint64_t)0, OpAdd{});
  const uint64_t hb2 = __ballot(before + bin - bs <= t && t < before + bin);
  if (hb2 == 0) return CandOut{V - 1, false, 0.0};
  const int L = __builtin_ctzll(hb2);
  int bsel = 0;
  uint64_t bf = 0, rr = before + bin - bs;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (rr <= t && t < rr + bv[j]) {
      bsel = 4 * lane() + j;
      bf = rr;
    }
    rr += bv[j];
  }
  const int bb = uniform(lane_value(bsel, L));
  const uint64_t bbefore = uniform(lane_value(bf, L));
#pragma unroll
  for (int k = 0; k < kPer; ++k)
    if (dw[k] != 0ull && (di[k] - c0) / kTokPerBin == bb) fs.dspan[di[k] - c0 - bb * kTokPerBin] = dw[k];
  wg_barrier();
  PLH_STAMP(row, 8);
  if (wave() != 0) return CandOut{-1, false, 0.0};
  const uint64_t v = lane() < kTokPerBin ? fs.dspan[lane()] : 0ull;
  const uint64_t in3 = wave_scan_incl(v, (uint64_t)0, OpAdd{});
  const uint64_t h3 = __ballot(v != 0ull && bbefore + in3 - v <= t && t < bbefore + in3);
  if (h3 == 0) return CandOut{V - 1, false, 0.0};
  return CandOut{c0 + bb * kTokPerBin + __builtin_ctzll(h3), false, 0.0};
}

template <typename TIn, bool VEC, bool NUC>
__global__ __launch_bounds__(kThreads) void k_sample_final(SampleArgs a) {
  __shared__ SmemAll sm;
  FastSmem& fs = sm.f;
  const int row = blockIdx.x;
  PLH_STAMP(row, 0);
  RowLoad rload;
  issue_row_params(a, row, rload);
  // the first 128 candidate slots of each chunk (all a top-k row usually
  // fills), read while the row's parameters are on their way
  MCands mc;
  const int sfirst = min(128, a.ws.capc);
  mc_load_first(a, row, mc, sfirst);
  // and the row's first wave parts (every mode reads them), in the same
  // round trip; the rest waits for the row's mode (more loads in flight at
  // once lengthen the round trip for every row)
  PartLoad pl;
  load_parts_first(a, row, pl);
  const RowParams rp = row_params_of(a, rload);
  if (NUC && rp.nucleus) return;  // the nucleus kernels own the row (k_nuc_window onwards)
  init_exp_table_wave(fs.exp_tab[wave()]);
  const bool cands = !rp.greedy && (rp.topk || (rp.topp && !(NUC && rp.nucleus)));
  if (cands) {  // ordered before their first use by the first barrier
    for (int b = threadIdx.x; b < kHB; b += kThreads) {
      fs.h[0].cnt[b] = 0u;
      fs.h[0].mass[b] = 0ull;
    }
    if (threadIdx.x < kDrawSpanMax) fs.dspan[threadIdx.x] = 0ull;
    if (threadIdx.x < kBkt) fs.rowm[threadIdx.x] = 0ull;
    if (threadIdx.x < 2) fs.rl[threadIdx.x].n = 0;
    if (threadIdx.x < 2 * kWave) {
      fs.rl[threadIdx.x / kWave].rank[threadIdx.x % kWave] = 0u;
      fs.rl[threadIdx.x / kWave].ahead[threadIdx.x % kWave] = 0ull;
    }
  }
  XWave xw{fs.xw, 0};
  int hgen = 0;
  // top-p rows with more than kWaves chunks read the rest of their
  // candidates (their chunks fill nearly all slots) now; a top-k chunk
  // with more than 128 candidates is read once the counts are in
  const bool bkt = cands && !rp.topk && a.ws.C <= kWaves;
  BktLoad bl;
  if (bkt) load_buckets(a, row, bl);
  const int smax = rp.topk ? sfirst : a.ws.capc;
  if (cands && !bkt && smax > sfirst) mc_load_range(a, row, mc, sfirst, smax);
  SegLoad sg;
  if (!rp.greedy && !rp.topk && !(NUC && rp.nucleus)) {  // nucleus rows only set their bin range here
    load_segs(a, row, (a.V + Geo<TIn>::kSeg - 1) / Geo<TIn>::kSeg, sg);
  }
  const PartSum ps = scan_parts(a, row, rp.greedy, cands, fs, pl);
  PLH_STAMP(row, 1);
  if (cands && !bkt) mc_validate(a, row, mc, fs.wcnt[wave()], smax);
  // a chunk that could not keep all its penalised tokens aside sends the
  // row to the general pipeline
  bool general = ps.flags != 0;
  int id = 0;
  PipeIn pin{false, 0.0, false, 0.0, false, 0.0};  // what the fast path already knows of the row
  if (general) {
  } else if (rp.greedy) {
    id = ps.best.i;
  } else if (!cands) {
    id = finish_temp<TIn>(a, row, rp, sg, fs, xw);
  } else {
    const CandOut o = rp.topk ? merge_cands<TIn, true>(a, mc, sg, rp, ps, fs, xw, hgen)
                      : bkt   ? merge_topp<TIn>(a, row, rp, ps, sg, bl, fs, xw, hgen)
                              : merge_cands<TIn, false>(a, mc, sg, rp, ps, fs, xw, hgen);
    general = o.general;
    if (!general) {
      // the id is known in the lanes of the wave that drew it
      if (lane() == 0 && o.id >= 0) a.out_ids[row] = o.id;
      PLH_STAMP(row, 9);
      return;
    }
    pin = PipeIn{true, ps.zmax, o.S > 0.0, o.S, false, 0.0};
  }
  if (general) {
    wg_barrier();
    if (threadIdx.x == 0) glb_add(a.fallback_rows, 1ull);
    id = row_general<TIn, VEC>(a, row, rp, sm.g, nullptr, pin);
  }
  PLH_STAMP(row, 9);
  if (threadIdx.x == 0) a.out_ids[row] = id;
}

// ================================================================ nucleus
// Rows with no top-k and top_p >= kNucTopP keep most of the vocabulary
// (top_p 0.99 over a Zipf-like distribution keeps ~90% of it), more than
// any candidate list holds.  With the caller's hint they take passes over
// all chunks instead of one workgroup per row: k_sample_chunks leaves the
// segment partials of the normaliser, each wave's smallest and largest
// finite logit, (penalised rows) each chunk's bitmap of penalised tokens,
// and each chunk's count histogram on a power-of-two grid of its own (the
// finest that fits the chunk's range in kNucBins bins); k_sample_final
// leaves such rows at once; then
//   k_nuc_window  picks the row's grid, no finer than any chunk's (or hands
//                 the row to the general pipeline when a chunk could not set
//                 its penalised tokens aside), adds the chunks' histograms
//                 into the row's bins and
//                 bounds each bin's mass by its count and the exp of its
//                 edges, which brackets the top-p cut (sampling.py:82-90) in a
//                 window of bins: the bins below it hold at most 1 - top_p
//                 of the mass (dropped), those above it more than that below
//                 them (kept);
//   k_nuc_cands   writes the window's tokens as candidates and sums, per
//                 segment, the mass on the row's smaller side of the window;
//   k_nuc_final   finds the cut among the candidates in (p desc, idx asc)
//                 order, starting from the mass above the window, then draws
//                 (sampling.py:94-98): the segment where the kept mass
//                 crosses u * total, rescanned from HBM.
// A row whose window does not fit its candidate slots, or whose cut falls
// outside the window, is finished by the general pipeline (in k_nuc_final).

// A nucleus row's grid, by every wave on its own from the same data (the
// same result in each): its bins span the row's finite penalised logits on
// a power-of-two grid no finer than any chunk's.  general: a chunk could not
// set its penalised tokens aside, or the row has one distinct finite value,
// none, or logits too large to bin (the general pipeline, k_nuc_final).
__device__ __forceinline__ void nuc_row_grid(const SampleArgs& a, int row, float* rz_out, int* base_out,
                                             int* general_out) {
  const int C = a.ws.C;
  const WavePart* pp = a.ws.part + (size_t)row * C * kWaves;
  double lo = INFINITY, hi = -INFINITY;
  int flags = 0;
  for (int j = lane(); j < C * kWaves; j += kWave) {
    const WavePart w = pp[j];
    lo = fmin(lo, w.umax);  // nucleus rows: the wave's smallest finite logit
    hi = fmax(hi, w.zmax);
    flags |= w.flags;
  }
  float crz = INFINITY;
  int bad = 0;
  for (int j = lane(); j < C; j += kWave) {
    const float r = a.ws.ngrid[(size_t)row * C + j].rz;
    if (r < 0.0f) bad = 1;
    if (r > 0.0f) crz = fminf(crz, r);
  }
  lo = wave_min(lo);
  hi = wave_max(hi);
  crz = wave_min(crz);
  bad = wave_max(bad | (flags != 0 ? 1 : 0));
  const NucGrid rg = nuc_fit((float)lo, (float)hi);
  const float rz = fminf(rg.rz, crz);
  *rz_out = rz;
  *base_out = rz > 0.0f ? __float2int_rd((float)lo * rz) : 0;
  *general_out = (hi - lo > 0.0 && hi - lo < INFINITY && rg.rz > 0.0f && !bad) ? 0 : 1;
}

// Bin of a nucleus row's token on the row's grid (NucRow rz, base), clamped
// to [0, kNucBins - 1].  Every kernel that bins a token uses this function.
struct NucBin {
  float rz;
  int base, top;
  __device__ __forceinline__ explicit NucBin(const NucRow& nr) : rz(nr.rz), base(nr.base) {
    // the clamp's upper end lives in a register: v_med3_i32 takes no
    // literal, and the compiler would otherwise rebuild it for every token
    top = kNucBins - 1;
    asm volatile("" : "+v"(top));
  }
  __device__ __forceinline__ int operator()(float zf) const {
    return min(max(__float2int_rd(zf * rz) - base, 0), top);
  }
  __device__ __forceinline__ int operator()(double z) const { return (*this)((float)z); }
  // bin 0's lower edge in z and the bins per unit of z
  __device__ __forceinline__ double lo() const { return (double)base / (double)rz; }
  __device__ __forceinline__ double scale() const { return (double)rz; }
};

// The calling lane's penalty bits (as chunk_pbits) from the chunk bitmap
// the first pass wrote.
template <typename TIn>
__device__ __forceinline__ uint32_t nuc_pbits(const SampleArgs& a, int g) {
  using G = Geo<TIn>;
  const uint32_t* bm = a.ws.npen + (size_t)g * kNucPenWords;
  uint32_t pb = 0;
  const int q0 = wave() * G::kSeg + lane() * G::kVW;
#pragma unroll
  for (int j = 0; j < kU; ++j) {
    const int q = q0 + j * G::kSpan;
    pb |= ((bm[q >> 5] >> (q & 31)) & ((1u << G::kVW) - 1u)) << (G::kVW * j);
  }
  return pb;
}

// p of a nucleus row's token: exp(y - ymax) / S.
__device__ __forceinline__ double nuc_p(double y, const NucRow& nr, const double* tab) {
  return fast_exp_neg(y - nr.ymax, tab) * nr.invS;
}

struct NucWinSmem {
  uint32_t rowh[kNucBins];  // the row's counts on its grid
  double exp_tab[kWaves][64];
  double redd[2 * kWaves];
  int redi[2 * kWaves];
  uint64_t redu[kWaves];
  uint64_t redu2[2 * kWaves];
};

// One workgroup per nucleus row: the normaliser from the segment partials
// and the window of candidate bins.  Bin b spans z in [lo + b / scale,
// lo + (b + 1) / scale) (NucBin's float lo and scale) up to rounding: a
// margin of 0.01 bin plus the float rounding of z on each edge, the bottom
// bin open below and the top one closed at ymax.  U(b) =
// mass bound of the bins below b from their upper edges, L(b + 1) = mass
// bound of the bins up to b from their lower edges; dlo = the largest b with
// U(b) <= (1 - top_p) S, dhi = the smallest b with L(b + 1) > (1 - top_p) S.
template <typename TIn>
__global__ __launch_bounds__(kThreads) void k_nuc_window(SampleArgs a) {
  using G = Geo<TIn>;
  __shared__ NucWinSmem sm;
  const int row = blockIdx.x;
  const RowParams rp = load_row_params(a, row);
  if (!rp.nucleus) return;
  NucRow nr{};
  nuc_row_grid(a, row, &nr.rz, &nr.base, &nr.general);
  nr.state = kNucActive;
  if (threadIdx.x == 0) {  // for k_nuc_cands and k_nuc_final (the window's fields follow below)
    NucRow& g = a.ws.nrow[row];
    g.rz = nr.rz;
    g.base = nr.base;
    g.general = nr.general;
    g.state = kNucActive;
  }
  if (nr.general != 0) return;
  init_exp_table_wave(sm.exp_tab[wave()]);
  const double* tab = sm.exp_tab[wave()];
  constexpr int kPer = kNucBins / kThreads;
  const int b0 = kPer * (int)threadIdx.x;
  // the row's counts: each chunk's histogram (its own grid, nested in the
  // row's: shift by the exponent difference) added into the row's bins
  for (int b = threadIdx.x; b < kNucBins; b += kThreads) sm.rowh[b] = 0u;
  {
    const int C = a.ws.C;
    const int erow = pow2_exp(nr.rz);
    const NucGrid* grids = a.ws.ngrid + (size_t)row * C;
    const uint32_t* hist = a.ws.nhist + (size_t)row * C * (kNucBins / 2);
    wg_barrier();
    constexpr int kWordsPerThread = kNucBins / 2 / kThreads;  // 2
    constexpr int kBatch = 8;                                 // chunks whose words are loaded at once
    for (int c0 = 0; c0 < C; c0 += kBatch) {
      uint32_t wv[kBatch][kWordsPerThread];
#pragma unroll
      for (int k = 0; k < kBatch; ++k)
#pragma unroll
        for (int w = 0; w < kWordsPerThread; ++w)
          wv[k][w] = c0 + k < C ? hist[(size_t)(c0 + k) * (kNucBins / 2) + threadIdx.x + w * kThreads] : 0u;
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        if (c0 + k >= C) break;
        const NucGrid gq = grids[c0 + k];
        if (!(gq.rz > 0.0f)) continue;
        const int sh = pow2_exp(gq.rz) - erow;  // >= 0: the row's grid is no finer
#pragma unroll
        for (int w = 0; w < kWordsPerThread; ++w) {
          const int j = 2 * ((int)threadIdx.x + w * kThreads);
          const uint32_t v = wv[k][w];
          if (v & 0xffffu) lds_add(&sm.rowh[min(max(((gq.q0 + j) >> sh) - nr.base, 0), kNucBins - 1)], v & 0xffffu);
          if (v >> 16) lds_add(&sm.rowh[min(max(((gq.q0 + j + 1) >> sh) - nr.base, 0), kNucBins - 1)], v >> 16);
        }
      }
    }
    wg_barrier();
  }
  uint32_t c[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) c[j] = sm.rowh[b0 + j];
  SegLoad sg;
  load_segs(a, row, (a.V + G::kSeg - 1) / G::kSeg, sg);
  double ms[kSegPerLane], lex;
  const SegNorm sn = seg_norm(sg, tab, ms, &lex);
  const double invT = 1.0 / rp.T;
  // NucBin bins z rounded to float on an exact grid: rounding z moves a
  // token by up to 2^-24 |z|, which the margin covers with room to spare
  const NucBin nbin(nr);
  const double flo = nbin.lo(), fsc = nbin.scale();
  const double mag = fmax(fabs(flo), fabs(flo + (double)kNucBins / fsc));
  const double mb = 0.01 + mag * fsc * 2.5e-7;
  double lo[kPer], hi[kPer], slo = 0.0, shi = 0.0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int b = b0 + j;
    const double y0 = b == 0 ? -INFINITY : (flo + ((double)b - mb) / fsc) * invT;
    const double y1 = b == kNucBins - 1 ? sn.ymax : (flo + ((double)b + 1.0 + mb) / fsc) * invT;
    lo[j] = c[j] ? (double)c[j] * fast_exp_neg(fmin(y0 - sn.ymax, 0.0), tab) * (1.0 - 1e-12) : 0.0;
    hi[j] = c[j] ? (double)c[j] * fast_exp_neg(fmin(y1 - sn.ymax, 0.0), tab) * (1.0 + 1e-12) : 0.0;
    slo += lo[j];
    shi += hi[j];
  }
  const double ilo = wave_scan_incl(slo, 0.0, OpAdd{}), ihi = wave_scan_incl(shi, 0.0, OpAdd{});
  if (lane() == kWave - 1) {
    sm.redd[wave()] = ilo;
    sm.redd[kWaves + wave()] = ihi;
  }
  wg_barrier();
  double l = wave_shift_up1(ilo, 0.0), u = wave_shift_up1(ihi, 0.0);
  for (int w = 0; w < wave(); ++w) {
    l += sm.redd[w];
    u += sm.redd[kWaves + w];
  }
  const double thr = (1.0 - rp.top_p) * sn.S;
  int mlo = -1, mhi = INT_MAX;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    if (u <= thr) mlo = b0 + j;
    l += lo[j];
    if (mhi == INT_MAX && l > thr) mhi = b0 + j;
    u += hi[j];
  }
  mlo = wave_max(mlo);
  mhi = wave_min(mhi);
  if (lane() == 0) {
    sm.redi[wave()] = mlo;
    sm.redi[kWaves + wave()] = mhi;
  }
  wg_barrier();
  int dlo = -1, dhi = INT_MAX;
  for (int w = 0; w < kWaves; ++w) {
    dlo = max(dlo, sm.redi[w]);
    dhi = min(dhi, sm.redi[kWaves + w]);
  }
  uint64_t n = 0, nb = 0, na = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int b = b0 + j;
    if (b >= dlo && b <= dhi) n += c[j];
    else if (b < dlo) nb += c[j];
    else na += c[j];
  }
  n = wave_sum(n);
  nb = wave_sum(nb);
  na = wave_sum(na);
  if (lane() == 0) {
    sm.redu[wave()] = n;
    sm.redu2[wave()] = nb;
    sm.redu2[kWaves + wave()] = na;
  }
  wg_barrier();
  if (threadIdx.x == 0) {
    uint64_t tot = 0, below = 0, abv = 0;
    for (int w = 0; w < kWaves; ++w) {
      tot += sm.redu[w];
      below += sm.redu2[w];
      abv += sm.redu2[kWaves + w];
    }
    NucRow& out = a.ws.nrow[row];
    out.above = abv < below ? 1 : 0;
    out.ymax = sn.ymax;
    out.S = sn.S;
    out.invS = 1.0 / sn.S;
    out.dlo = dlo;
    out.dhi = dhi;
    out.general = (dhi == INT_MAX || dhi < dlo || tot > (uint64_t)a.ws.C * a.ws.capc) ? 1 : 0;
  }
}

constexpr int kNucStage = 256;                   // tokens a wave stages before summing their mass
constexpr int kNucCandWave = kCapChunk / kWaves;  // window tokens a wave stages

// The window's tokens go to the candidate slots (p and id); the tokens on
// the row's smaller side of the window (nr.above) have their p summed per
// segment.  Both are first staged per wave in LDS (a ballot per token step,
// each lane's place from mbcnt), so the exps run densely over the staged
// tokens instead of in a branch nearly every wave would take.
template <typename TIn, bool VEC>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4))) void k_nuc_cands(SampleArgs a) {
  using G = Geo<TIn>;
  __shared__ ChunkSmem cm;
  __shared__ double stz[kWaves][kNucStage];
  __shared__ int over;
  const int C = a.ws.C;
  const int capc = a.ws.capc;
  const int g = chunk_block(C, a.B);
  if (g < 0) return;
  const int row = g / C;
  const RowParams rp = load_row_params(a, row);
  if (!rp.nucleus) return;
  const NucRow nr = a.ws.nrow[row];
  if (nr.state != kNucActive || nr.general != 0) return;
  const int c0 = (g - row * C) * G::kChunk;
  const TIn* x = reinterpret_cast<const TIn*>(a.logits) + (int64_t)row * a.ld;
  ChunkToks<TIn> tk;
  load_chunk<TIn, VEC>(x, a.V, c0, tk.v);
  init_exp_table_wave(cm.exp_tab[wave()]);
  const double* tab = cm.exp_tab[wave()];
  if (threadIdx.x == 0) {
    cm.cand_n = 0;
    over = 0;
  }
  if (rp.pen_active) set_aside_penalised<TIn>(tk, nuc_pbits<TIn>(a, g), rp.pen, c0, cm);
  wg_barrier();
  const YScale ys{rp.T, 1.0 / rp.T};
  const NucBin nb(nr);
  const bool abv = nr.above != 0;
  double* sz = stz[wave()];
  StageRaw* cs = cm.sraw + wave() * kNucCandWave;
  uint32_t* cc = cm.scode + wave() * kNucCandWave;
  double acc = 0.0;  // this lane's share of the side's mass
  int mn = 0, cn = 0;  // staged side tokens and window tokens (the same in every lane)
  auto flush = [&]() {
    for (int i = lane(); i < mn; i += kWave) acc += nuc_p(ys(sz[i]), nr, tab);
    mn = 0;
  };
  // the side's bins: above the window, or below it
  const int slo = abv ? nr.dhi + 1 : 0;
  const int shi = abv ? kNucBins - 1 : nr.dlo - 1;
  // z: the token's (penalised) logit; zf: z rounded to float, which is
  // what the bins see (exact for a register token).  A -inf token takes
  // bin -1, outside both ranges; the tests are plain compares, no branches.
  auto take = [&](double z, float zf, int idx) {
    const int b = z > -INFINITY ? nb(zf) : -1;
    const bool side = (b >= slo) & (b <= shi);
    const bool cand = (b >= nr.dlo) & (b <= nr.dhi);
    const uint64_t ms = __ballot(side);
    if (ms != 0ull) {
      if (side) sz[mbcnt(ms, mn)] = z;
      mn += __popcll(ms);
      if (mn > kNucStage - kWave) flush();
    }
    const uint64_t mc = __ballot(cand);
    if (mc != 0ull) {
      const int slot = mbcnt(mc, cn);
      if (cand && slot < kNucCandWave) {
        cs[slot].d = z;
        cc[slot] = (uint32_t)idx;
      }
      cn += __popcll(mc);
    }
  };
  tk.new_pass();
#pragma unroll
  for (int e = 0; e < G::kEpt; ++e) take((double)tk.rv(e), (float)tk.rv(e), c0 + slot_q<TIn>(e));
  const int npmax = wave_max(tk.np);
  for (int i = 0; i < npmax; ++i) {
    const double z = i < tk.np ? tk.pen_z(cm, i) : -INFINITY;
    take(z, (float)z, i < tk.np ? tk.pen_tok(cm, i) : 0);
  }
  flush();
  acc = wave_sum(acc);
  if (lane() == 0) a.ws.nexcl[(size_t)g * kWaves + wave()] = acc;
  // the staged window tokens: one reservation per wave, then to the slots
  int base = 0;
  if (lane() == 0 && cn > 0) base = lds_fetch_add(&cm.cand_n, cn);
  base = lane_value(base, 0);
  if (cn > kNucCandWave || base + cn > capc) {
    if (lane() == 0) over = 1;
  } else {
    double* cz = a.ws.cz + (size_t)g * capc;
    int32_t* ci = a.ws.ci + (size_t)g * capc;
    for (int i = lane(); i < cn; i += kWave) {
      cz[base + i] = nuc_p(ys(cs[i].d), nr, tab);
      ci[base + i] = (int)cc[i];
    }
  }
  wg_barrier();
  if (threadIdx.x == 0) a.ws.ncand[g] = over ? -1 : cm.cand_n;
}

template <typename TIn, bool VEC>
__global__ __launch_bounds__(kThreads) void k_nuc_final(SampleArgs a) {
  using G = Geo<TIn>;
  __shared__ SmemAll sm;
  FastSmem& fs = sm.f;
  const int row = blockIdx.x;
  const RowParams rp = load_row_params(a, row);
  // with the nucleus-only hint no merge kernel ran: a row that is not a
  // nucleus row is finished here, by the general pipeline below
  const bool other = !rp.nucleus;
  if (other && !a.nucleus_only) return;
  NucRow nr{};
  if (!other) {
    nr = a.ws.nrow[row];
    if (nr.state != kNucActive) return;
  }
  init_exp_table_wave(fs.exp_tab[wave()]);
  for (int b = threadIdx.x; b < kHB; b += kThreads) {  // ordered before use by the first barrier
    fs.h[0].cnt[b] = 0u;
    fs.h[0].mass[b] = 0ull;
  }
  if (threadIdx.x < 2) fs.rl[threadIdx.x].n = 0;
  if (threadIdx.x < 2 * kWave) {
    fs.rl[threadIdx.x / kWave].rank[threadIdx.x % kWave] = 0u;
    fs.rl[threadIdx.x / kWave].ahead[threadIdx.x % kWave] = 0ull;
  }
  XWave xw{fs.xw, 0};
  int hgen = 0;
  const double* tab = fs.exp_tab[wave()];
  const int V = a.V;
  const int C = a.ws.C;
  const int capc = a.ws.capc;
  const int csh = __ffs(capc) - 1;
  const int slots = C * capc;
  const int nseg = C * kWaves;
  bool general = other || nr.general != 0;
  int id = V - 1;
  if (!general) {
    // every candidate slot into registers; the chunks' counts per wave
    RegCands rc;
    gather_cands(a, row, rc);
    int* wc = fs.wcnt[wave()];
    int bad = 0;
    for (int c = lane(); c < C; c += kWave) {
      const int n = a.ws.ncand[(size_t)row * C + c];
      bad |= n < 0 ? 1 : 0;
      wc[c] = n < 0 ? 0 : n;
    }
    general = uniform(wave_max(bad)) != 0;
    if (!general) {
      rc.valid = 0;
      uint32_t pos = 0;
      uint64_t ws = 0;
#pragma unroll
      for (int q = 0; q < kPerT; ++q) {
        const int i = q * kThreads + (int)threadIdx.x;
        rc.w[q] = 0ull;
        if (i < slots && (i & (capc - 1)) < wc[i >> csh]) {
          rc.valid |= 1u << q;
          if (rc.v[q] > 0.0) pos |= 1u << q;
          rc.w[q] = to_fx(rc.v[q]);
          ws += rc.w[q];
        }
      }
      // the window's fixed-point mass (exact, in any slot order) and the
      // mass below it (segment sums in a fixed order)
      const auto sw = xw.post(wave_sum(ws), 0, 0);
      uint64_t wsum = 0;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) wsum += sw[0][w];
      double dl = 0.0;
      for (int s = lane(); s < nseg; s += kWave) dl += a.ws.nexcl[(size_t)row * nseg + s];
      const double side = uniform(wave_sum(dl));
      const bool abv = nr.above != 0;
      uint64_t above = to_fx(side);
      if (!abv) {
        const uint64_t below_and_in = above + wsum;
        above = below_and_in < kFxOne ? kFxOne - below_and_in : 0ull;
      }
      const uint64_t target = topp_target(rp.top_p);
      SelOut r{false, true, 0, 0};
      if (above < target)
        r = select_desc<true>(pos, rc, [](double p) { return pkey_of(p); }, target - above, V, fs.rl[1], fs, xw,
                              hgen);
      if (!r.found || r.giveup) {
        general = true;
      } else {
        // by segment (fixed point): the kept candidates when the side
        // summed is above the window, else the candidates past the cut
        Hist& h = next_hist(fs, hgen);
#pragma unroll
        for (int q = 0; q < kPerT; ++q) {
          if (((rc.valid >> q) & 1u) && rc.w[q] != 0ull) {
            const uint64_t k = pkey_of(rc.v[q]);
            const bool kept = k > r.key || (k == r.key && rc.idx[q] <= r.idx);
            if (kept == abv) lds_add(&h.mass[rc.idx[q] / G::kSeg], rc.w[q]);
          }
        }
        wg_barrier();
        // kept mass per segment: the mass above the window plus the kept
        // candidates, or the segment's share of the normaliser less the mass
        // below the window and the candidates past the cut
        const int nsv = (V + G::kSeg - 1) / G::kSeg;
        double ms[kSegPerLane];
        if (!abv) {
          SegLoad sg;
          load_segs(a, row, nsv, sg);
          double lex;
          seg_norm(sg, tab, ms, &lex);
        }
        double kk[kSegPerLane], ks = 0.0;
#pragma unroll
        for (int j = 0; j < kSegPerLane; ++j) {
          const int s = kSegPerLane * lane() + j;
          kk[j] = 0.0;
          if (s < nsv) {
            const double side_s = a.ws.nexcl[(size_t)row * nseg + s];
            const double cand_s = (double)h.mass[s] * (1.0 / kFxScale);
            kk[j] = abv ? side_s + cand_s : ms[j] * nr.invS - side_s - cand_s;
            if (!(kk[j] > 0.0)) kk[j] = 0.0;
          }
          ks += kk[j];
        }
        const double kin = wave_scan_incl(ks, 0.0, OpAdd{});
        const double t = rp.u * uniform(lane_value(kin, kWave - 1));
        double run = kin - ks, bl = 0.0;
        int kl = INT_MAX;
#pragma unroll
        for (int j = 0; j < kSegPerLane; ++j) {
          if (kl == INT_MAX && kk[j] > 0.0 && run + kk[j] > t) {
            kl = kSegPerLane * lane() + j;
            bl = run;
          }
          run += kk[j];
        }
        const uint64_t hits = __ballot(kl != INT_MAX);
        if (hits == 0) {
          general = true;
        } else {
          const int L = __builtin_ctzll(hits);
          const int kstar = uniform(lane_value(kl, L));
          const double before = uniform(lane_value(bl, L));
          const int s0 = kstar * G::kSeg;
          if (rp.pen_active) {  // the segment's words of its chunk's penalty bitmap
            const uint32_t* bm = a.ws.npen + ((size_t)row * C + kstar / kWaves) * kNucPenWords +
                                 (kstar % kWaves) * (G::kSeg / 32);
            for (int w = threadIdx.x; w < G::kSeg / 32; w += kThreads) fs.segbits[w] = bm[w];
            wg_barrier();
          }
          // thread t holds tokens s0 + kPer*t + q, in vocabulary order
          constexpr int kPer = G::kSeg / kThreads;
          const TIn* x = reinterpret_cast<const TIn*>(a.logits) + (int64_t)row * a.ld;
          const YScale ys{rp.T, 1.0 / rp.T};
          const NucBin nb(nr);
          const int q0 = kPer * (int)threadIdx.x;
          double e[kPer], es = 0.0;
#pragma unroll
          for (int q = 0; q < kPer; ++q) {
            e[q] = 0.0;
            const int p = s0 + q0 + q;
            if (p < V) {
              double z = (double)x[p];
              if (rp.pen_active && ((fs.segbits[(q0 + q) >> 5] >> ((q0 + q) & 31)) & 1u)) z = penalize(z, rp.pen);
              if (z > -INFINITY) {
                const int b = nb(z);
                if (b >= nr.dlo) {
                  const double pz = nuc_p(ys(z), nr, tab);
                  const uint64_t k = pkey_of(pz);
                  if (b > nr.dhi || k > r.key || (k == r.key && p <= r.idx)) e[q] = pz;
                }
              }
            }
            es += e[q];
          }
          double pex, ptot;
          xw_scan(xw, es, &pex, &ptot);
          double rr = pex;
          int hit = INT_MAX, last = -1;
#pragma unroll
          for (int q = 0; q < kPer; ++q) {
            rr += e[q];
            if (e[q] > 0.0) last = s0 + q0 + q;
            if (hit == INT_MAX && e[q] > 0.0 && before + rr > t) hit = s0 + q0 + q;
          }
          hit = xw_min(xw, hit);
          if (hit == INT_MAX) hit = xw_max(xw, last);  // rounding at the segment end
          if (hit < 0) general = true;
          else id = hit;
        }
      }
    }
  }
  if (general) {
    wg_barrier();
    if (threadIdx.x == 0) glb_add(a.fallback_rows, 1ull);
    id = row_general<TIn, VEC>(a, row, rp, sm.g, nullptr);
  }
  if (threadIdx.x == 0) a.out_ids[row] = id;
}

// ------------------------------------------------------------------- draw

template <typename TIn>
__global__ __launch_bounds__(kThreads) void k_draw(DrawArgs a) {
  __shared__ double redd[kWaves];
  __shared__ uint64_t redu[kWaves];
  __shared__ int redi[kWaves];
  const int row = blockIdx.x;
  const TIn* p = reinterpret_cast<const TIn*>(a.p) + (int64_t)row * a.ld;
  auto w = [&](int i) -> double {
    const double v = (double)p[i];
    return v > 0.0 ? v : 0.0;
  };
  const int id = draw_weights(w, a.V, a.uniforms[row], redd, redu, redi);
  if (threadIdx.x == 0) a.out_ids[row] = id;
}

// --------------------------------------------------------------- penalize

// apply_repetition_penalty on a copy (sampling.py:52-62), in the input's
// precision: float32 rows use float32 arithmetic, as numpy does for a
// float32 array and a Python float.
template <typename TIn>
__global__ __launch_bounds__(kThreads) void k_penalize(PenalizeArgs a) {
  const int row = blockIdx.x;
  const TIn* x = reinterpret_cast<const TIn*>(a.x) + (int64_t)row * a.ld;
  TIn* o = reinterpret_cast<TIn*>(a.out) + (int64_t)row * a.out_ld;
  for (int i = threadIdx.x; i < a.V; i += kThreads) o[i] = x[i];
  const double pen = a.rep_penalty[row];
  const int64_t h0 = a.hist_off != nullptr ? a.hist_off[row] : 0;
  const int64_t h1 = a.hist_off != nullptr ? a.hist_off[row + 1] : 0;
  if (pen == 1.0 || h1 <= h0 || a.hist_ids == nullptr) return;
  wg_barrier();
  const TIn pn = (TIn)pen;
  for (int64_t h = h0 + threadIdx.x; h < h1; h += kThreads) {
    const int id = a.hist_ids[h];
    if ((unsigned)id < (unsigned)a.V) {
      const TIn v = x[id];
      o[id] = v > (TIn)0 ? v / pn : v * pn;  // same value for a repeated id
    }
  }
}

// ----------------------------------------------------------------- append

// slab[pos[i]] = ids[i] (pos[i] >= 0): the sampled ids join their
// sequences' device-resident histories (llm_engine.py:284).
__global__ __launch_bounds__(256) void k_append(int32_t* slab, const int64_t* pos, const int32_t* ids, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) {
    const int64_t q = pos[i];
    if (q >= 0) slab[q] = ids[i];
  }
}

// ---------------------------------------------------------------- launch

namespace {

int chunks_of(int V, bool f64) {
  const int L = f64 ? Geo<double>::kChunk : Geo<float>::kChunk;
  return (V + L - 1) / L;
}

// Candidate slots per chunk: a power of two (>= 16) with C * capc <= kCandCap.
int capc_of(int C) {
  int c = kCapChunk;
  while (c > 16 && c * C > kCandCap) c >>= 1;
  return c;
}

size_t up256(size_t v) { return (v + 255) & ~(size_t)255; }

}  // namespace

size_t fast_ws_bytes(int B, int V, bool f64) {
  const size_t C = (size_t)chunks_of(V, f64), cap = (size_t)capc_of((int)C), n = (size_t)B * C;
  return up256(n * kWaves * sizeof(WavePart)) + 2 * up256(n * kWaves * sizeof(double)) + up256(n * cap * sizeof(double)) +
         up256(n * cap * sizeof(int32_t)) + up256((size_t)B * sizeof(NucRow)) +
         up256(n * (kNucBins / 2) * sizeof(uint32_t)) + up256(n * sizeof(NucGrid)) + up256(n * kWaves * sizeof(double)) + up256(n * sizeof(int32_t)) +
         up256(n * kNucPenWords * sizeof(uint32_t)) + up256(n * kBkt * sizeof(uint64_t)) +
         up256(n * kBkt * sizeof(uint32_t)) + up256(n * sizeof(double)) + up256(n * sizeof(int32_t));
}

ChunkWs fast_ws_layout(void* base, int B, int V, bool f64) {
  ChunkWs w{};
  w.C = chunks_of(V, f64);
  w.capc = capc_of(w.C);
  const size_t n = (size_t)B * w.C;
  char* p = static_cast<char*>(base);
  w.part = reinterpret_cast<WavePart*>(p);
  p += up256(n * kWaves * sizeof(WavePart));
  w.seg_m = reinterpret_cast<double*>(p);
  p += up256(n * kWaves * sizeof(double));
  w.seg_s = reinterpret_cast<double*>(p);
  p += up256(n * kWaves * sizeof(double));
  w.cz = reinterpret_cast<double*>(p);
  p += up256(n * w.capc * sizeof(double));
  w.ci = reinterpret_cast<int32_t*>(p);
  p += up256(n * w.capc * sizeof(int32_t));
  w.nrow = reinterpret_cast<NucRow*>(p);
  p += up256((size_t)B * sizeof(NucRow));
  w.nhist = reinterpret_cast<uint32_t*>(p);
  p += up256(n * (kNucBins / 2) * sizeof(uint32_t));
  w.ngrid = reinterpret_cast<NucGrid*>(p);
  p += up256(n * sizeof(NucGrid));
  w.nexcl = reinterpret_cast<double*>(p);
  p += up256(n * kWaves * sizeof(double));
  w.ncand = reinterpret_cast<int32_t*>(p);
  p += up256(n * sizeof(int32_t));
  w.npen = reinterpret_cast<uint32_t*>(p);
  p += up256(n * kNucPenWords * sizeof(uint32_t));
  w.bmass = reinterpret_cast<uint64_t*>(p);
  p += up256(n * kBkt * sizeof(uint64_t));
  w.bcnt = reinterpret_cast<uint32_t*>(p);
  p += up256(n * kBkt * sizeof(uint32_t));
  w.bymax = reinterpret_cast<double*>(p);
  p += up256(n * sizeof(double));
  w.bhb = reinterpret_cast<int32_t*>(p);
  return w;
}

hipError_t launch_sample_rows(const SampleArgs& a, bool f64, bool vec, hipStream_t s) {
  const dim3 grid(a.B), block(kThreads);
  if (f64) {
    if (vec) hipLaunchKernelGGL((k_sample_rows<double, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((k_sample_rows<double, false>), grid, block, 0, s, a);
  } else {
    if (vec) hipLaunchKernelGGL((k_sample_rows<float, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((k_sample_rows<float, false>), grid, block, 0, s, a);
  }
  return hipGetLastError();
}

hipError_t launch_sample_fast(const SampleArgs& a, bool f64, bool vec, int num_cu, hipStream_t s, hipEvent_t between) {
  (void)num_cu;
  const int total = kXcds * ((a.B + kXcds - 1) / kXcds) * a.ws.C;  // blocks of the chunk grids (chunk_block)
  const dim3 gf(a.B), block(kThreads);
  // the nucleus code is compiled only into the instantiations the hint selects
  using K = void (*)(SampleArgs);
  const K chunks[2][2][2] = {{{k_sample_chunks<float, false, false>, k_sample_chunks<float, false, true>},
                              {k_sample_chunks<float, true, false>, k_sample_chunks<float, true, true>}},
                             {{k_sample_chunks<double, false, false>, k_sample_chunks<double, false, true>},
                              {k_sample_chunks<double, true, false>, k_sample_chunks<double, true, true>}}};
  const K finals[2][2][2] = {{{k_sample_final<float, false, false>, k_sample_final<float, false, true>},
                              {k_sample_final<float, true, false>, k_sample_final<float, true, true>}},
                             {{k_sample_final<double, false, false>, k_sample_final<double, false, true>},
                              {k_sample_final<double, true, false>, k_sample_final<double, true, true>}}};
  const int nuc = a.nucleus ? 1 : 0;
  hipLaunchKernelGGL(chunks[f64][vec][nuc], dim3(total), block, 0, s, a);
  if (between != nullptr) {
    const hipError_t e = hipEventRecord(between, s);
    if (e != hipSuccess) return e;
  }
  // every row a nucleus row (the caller's hint): they would all leave the
  // merge kernel at once, so it is not launched (k_nuc_final finishes a row
  // that is not one with the general pipeline)
  if (!a.nucleus_only) hipLaunchKernelGGL(finals[f64][vec][nuc], gf, block, 0, s, a);
  if (a.nucleus) {
    auto cands = f64 ? (vec ? k_nuc_cands<double, true> : k_nuc_cands<double, false>)
                     : (vec ? k_nuc_cands<float, true> : k_nuc_cands<float, false>);
    auto fin = f64 ? (vec ? k_nuc_final<double, true> : k_nuc_final<double, false>)
                   : (vec ? k_nuc_final<float, true> : k_nuc_final<float, false>);
    hipLaunchKernelGGL(f64 ? k_nuc_window<double> : k_nuc_window<float>, gf, block, 0, s, a);
    hipLaunchKernelGGL(cands, dim3(total), block, 0, s, a);
    hipLaunchKernelGGL(fin, gf, block, 0, s, a);
  }
  return hipGetLastError();
}

hipError_t launch_append(int32_t* slab, const int64_t* pos, const int32_t* ids, int n, hipStream_t s) {
  hipLaunchKernelGGL(k_append, dim3((n + 255) / 256), dim3(256), 0, s, slab, pos, ids, n);
  return hipGetLastError();
}

hipError_t launch_draw(const DrawArgs& a, bool f64, hipStream_t s) {
  if (f64) hipLaunchKernelGGL((k_draw<double>), dim3(a.B), dim3(kThreads), 0, s, a);
  else hipLaunchKernelGGL((k_draw<float>), dim3(a.B), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_penalize(const PenalizeArgs& a, bool f64, hipStream_t s) {
  if (f64) hipLaunchKernelGGL((k_penalize<double>), dim3(a.B), dim3(kThreads), 0, s, a);
  else hipLaunchKernelGGL((k_penalize<float>), dim3(a.B), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace plh

#ifdef PLH_PHASE_STAMPS
// Profiling build only: copies the phase stamps of rows 0..255 (16 slots a
// row, shader clock ticks) to host memory.
extern "C" int plh_phase_stamps(unsigned long long* host) {
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(plh::g_phase), sizeof(plh::g_phase));
}
// Profiling build only: k_sample_final's real-time clocks (start, end) of
// rows 0..255.
extern "C" int plh_final_rt(unsigned long long* host) {
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(plh::g_frt), sizeof(plh::g_frt));
}
// Profiling build only: k_sample_chunks' stamps of chunks 0..4095: phase
// clocks (8 a chunk), real-time clocks (the start, then each wave's end: 9 a
// chunk) and hardware ids (HW_ID, XCC_ID: 2 a chunk).
extern "C" int plh_chunk_stamps(unsigned long long* phase, unsigned long long* rt, unsigned int* hw) {
  hipError_t e = hipMemcpyFromSymbol(phase, HIP_SYMBOL(plh::g_cphase), sizeof(plh::g_cphase));
  if (e == hipSuccess) e = hipMemcpyFromSymbol(rt, HIP_SYMBOL(plh::g_crt), sizeof(plh::g_crt));
  if (e == hipSuccess) e = hipMemcpyFromSymbol(hw, HIP_SYMBOL(plh::g_chw), sizeof(plh::g_chw));
  return (int)e;
}
#endif
