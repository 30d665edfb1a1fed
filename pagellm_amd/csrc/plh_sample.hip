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
//                                   histogram picks the threshold) and the
//                                   largest token left out; top-p-only rows
//                                   also leave the segment partials.
//                    Every chunk costs one 64 KB read whatever its row's
//                    mode, and the hardware dispatcher spreads the B x C
//                    workgroups over the CUs, so mixed batches stay
//                    balanced.
//   k_sample_final   one workgroup per row merges the partials: argmax;
//                    normaliser and the segment holding the inverse-CDF
//                    point (rescanned with the same arithmetic); or exact
//                    selection over the gathered candidates (k-th largest,
//                    top-p cut, fixed-point draw in vocabulary order).  A
//                    row the candidates cannot decide exactly is finished
//                    by the general pipeline in the same workgroup.
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

constexpr int kU = 8;             // 16-byte loads per thread per chunk
constexpr int kHB = 1024;         // histogram bins
constexpr int kSortMax = 2048;    // LDS sort list
constexpr int kCandCap = 8192;    // candidates one row gathers in LDS
constexpr int kCapChunk = 1024;   // candidate slots per chunk, at most
constexpr int kSelLevels = 4;

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

struct SortList {
  uint64_t key[kSortMax];
  uint64_t w[kSortMax];
  int idx[kSortMax];
};

// LDS of k_sample_final (the candidates themselves stay in registers).
struct FastSmem {
  double redd[kWaves];
  double redm[2 * kWaves];
  uint64_t redu[kWaves];
  int redi[kWaves];
  int ctl[8];
  uint64_t ctlu[4];
  double exp_tab[64];
  int cnt_c[64];
  uint32_t hcnt[kHB];
  uint64_t hmass[kHB];
  union {
    uint32_t segbits[kSegMax / 32];  // penalty bits of the rescanned segment
    SortList sl;                     // selection and draw
  } u;
};

union SmemAll {
  FastSmem f;
  Smem g;
};

// Workgroup barrier ordering LDS only (wg_barrier).
__device__ __forceinline__ void lds_barrier() { wg_barrier(); }

__device__ __forceinline__ RowParams load_row_params(const SampleArgs& a, int row) {
  RowParams rp;
  rp.T = a.temperature[row];
  rp.top_k = a.top_k[row];
  rp.top_p = a.top_p[row];
  rp.pen = a.rep_penalty[row];
  rp.u = a.uniforms != nullptr ? a.uniforms[row] : 0.0;
  rp.h0 = a.hist_off != nullptr ? a.hist_off[row] : 0;
  rp.h1 = a.hist_off != nullptr ? a.hist_off[row + 1] : 0;
  rp.greedy = rp.T == 0.0;  // SamplingParams.greedy (sampling.py:47-49)
  // sampling.py:56: no penalty when it is 1.0 or the context is empty
  rp.pen_active = rp.pen != 1.0 && rp.h1 > rp.h0 && a.hist_ids != nullptr;
  rp.topk = !rp.greedy && rp.top_k > 0 && rp.top_k < a.V;  // :76
  rp.topp = !rp.greedy && rp.top_p < 1.0;                  // :82
  return rp;
}

template <typename TIn, bool VEC>
__device__ __forceinline__ int row_general(const SampleArgs& a, int row, const RowParams& rp, Smem& sm,
                                           double* probs_out) {
  const TIn* x = reinterpret_cast<const TIn*>(a.logits) + (int64_t)row * a.ld;
  if (rp.pen_active) build_bitmap(sm.bitmap, 0, a.V, a.hist_ids, rp.h0, rp.h1);
  RowSource<TIn, VEC> src{x, a.V, sm.bitmap, rp.pen_active, rp.pen};
  const PipeIn in{false, 0.0, 0, false, 0.0, false, -INFINITY};
  return row_pipeline(src, rp, a.V, in, sm, probs_out).id;
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

// y = z / T as the segment partials compute it (multiplication by 1/T).
struct YScale {
  double T, invT;
  __device__ __forceinline__ double operator()(double z) const { return T == 1.0 ? z : z * invT; }
};

// ================================================================ chunks

typedef float f4_t __attribute__((ext_vector_type(4)));
typedef double d2_t __attribute__((ext_vector_type(2)));
template <typename TIn>
struct VecOf;
template <>
struct VecOf<float> {
  typedef f4_t T;
};
template <>
struct VecOf<double> {
  typedef d2_t T;
};

// Penalised tokens a wave keeps aside (their exact float64 value); a wave
// with more makes its chunk incomplete (the row takes the general
// pipeline).
constexpr int kPenPerWave = 128;

// LDS of k_sample_chunks: about 23 KB.
struct ChunkSmem {
  double redd[2 * kWaves];
  uint64_t redu[kWaves];
  int redi[kWaves];
  int ctl[8];
  uint64_t ctlu[4];
  double exp_tab[kWaves][64];  // one copy per wave
  uint32_t hcnt[kHB];
  uint32_t bitmap[Geo<float>::kChunk / 32];
  double pz[kWaves][kPenPerWave];
  int pt[kWaves][kPenPerWave];
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

template <typename TIn, bool VEC>
__device__ __forceinline__ void load_chunk(const TIn* x, int V, int c0, typename VecOf<TIn>::T (&v)[kU]) {
  using G = Geo<TIn>;
  using VT = typename VecOf<TIn>::T;
  const int off = c0 + wave() * G::kSeg + lane() * G::kVW;
  const bool full = VEC && c0 + G::kChunk <= V;  // uniform: no bounds checks needed
#pragma unroll
  for (int j = 0; j < kU; ++j) {
    const int p = off + j * G::kSpan;
    if (full || (VEC && p + G::kVW <= V)) {
      v[j] = __builtin_nontemporal_load(reinterpret_cast<const VT*>(x + p));
    } else {
#pragma unroll
      for (int s = 0; s < G::kVW; ++s) v[j][s] = (p + s < V) ? x[p + s] : (TIn)(-INFINITY);
    }
  }
}

// One bit per distinct history id inside the chunk (np.unique,
// sampling.py:59), then the calling lane's bits in register-slot order.
template <typename TIn>
__device__ __forceinline__ uint32_t chunk_pbits(const SampleArgs& a, const RowParams& rp, int c0, ChunkSmem& cm) {
  using G = Geo<TIn>;
  constexpr int kWords = G::kChunk / 32;
  for (int w = threadIdx.x; w < kWords; w += kThreads) cm.bitmap[w] = 0u;
  lds_barrier();
  for (int64_t h = rp.h0 + threadIdx.x; h < rp.h1; h += kThreads) {
    const int off = a.hist_ids[h] - c0;
    if ((unsigned)off < (unsigned)G::kChunk) lds_or(&cm.bitmap[off >> 5], 1u << (off & 31));
  }
  lds_barrier();
  uint32_t pb = 0;
  const int q0 = wave() * G::kSeg + lane() * G::kVW;
#pragma unroll
  for (int j = 0; j < kU; ++j) {
    const int q = q0 + j * G::kSpan;
    pb |= ((cm.bitmap[q >> 5] >> (q & 31)) & ((1u << G::kVW) - 1u)) << (G::kVW * j);
  }
  return pb;
}

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
  wg_barrier();
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
  int po = 0, np = 0;
  __device__ __forceinline__ double raw(int e) const { return (double)v[e / G::kVW][e % G::kVW]; }
  // Called at the start of each pass: the compiler must then widen the
  // registers again instead of keeping a float64 copy of the chunk alive
  // across passes (64 more VGPRs, which would cost occupancy).
  __device__ __forceinline__ void new_pass() {
#pragma unroll
    for (int j = 0; j < kU; ++j) asm volatile("" : "+v"(v[j]));
  }
  __device__ __forceinline__ double pen_z(const ChunkSmem& cm, int i) const { return cm.pz[wave()][po + i]; }
  __device__ __forceinline__ int pen_tok(const ChunkSmem& cm, int i) const { return cm.pt[wave()][po + i]; }
};

// Moves the calling wave's penalised tokens (bits pb of each lane) out of
// the registers: their penalised float64 value goes to the wave's LDS pool,
// the register slot to -inf.  Returns true when the pool overflows (the
// chunk is then incomplete).
template <typename TIn>
__device__ __forceinline__ bool set_aside_penalised(ChunkToks<TIn>& tk, uint32_t pb, double pen, int c0, ChunkSmem& cm) {
  using G = Geo<TIn>;
  const int n = __popc(pb);
  const int incl = wave_scan_incl(n, 0, OpAdd{});
  const int total = lane_value(incl, kWave - 1);
  tk.po = incl - n;
  tk.np = 0;
  if (total > kPenPerWave) return true;
  tk.np = n;
  if (pb != 0u) {
    int k = tk.po;
#pragma unroll
    for (int e = 0; e < G::kEpt; ++e) {
      if ((pb >> e) & 1u) {
        cm.pz[wave()][k] = penalize(tk.raw(e), pen);
        cm.pt[wave()][k] = c0 + slot_q<TIn>(e);
        ++k;
        tk.v[e / G::kVW][e % G::kVW] = (TIn)(-INFINITY);
      }
    }
  }
  return false;
}

// Candidates of one chunk: every finite z >= theta, with theta below the
// chunk's target-th largest token (all finite tokens when there are fewer).
//   top-k, k <= 512: the k-th largest of the workgroup's 512 per-thread
//     maxima is itself k tokens deep, so a histogram of those maxima alone
//     bounds the k-th largest token from below;
//   otherwise: a value histogram of all the chunk's tokens.
// theta is the lower edge of the histogram bin holding the target-th
// largest (cm.hcnt is zeroed at kernel start).  Each wave writes its
// candidates to a range of the chunk's slots and its part: the chunk's
// largest z, the largest finite z of its segment not written, the end of
// its slots.  lmax is the calling thread's largest z.
template <typename TIn>
__device__ __forceinline__ void chunk_candidates(ChunkToks<TIn>& tk, double lmax, const SampleArgs& a,
                                                 const RowParams& rp, int g, int c0, int flags, WavePart* wp,
                                                 ChunkSmem& cm) {
  constexpr int kEpt = Geo<TIn>::kEpt;
  const int capc = a.ws.capc;
  // top-p rows keep as many as the slots allow, less a margin for the
  // histogram bin that straddles the threshold
  const uint64_t keep = (uint64_t)(capc - capc / 16);
  const uint64_t target = rp.topk ? min((uint64_t)rp.top_k, keep) : keep;
  const bool by_max = rp.topk && target <= (uint64_t)kThreads;
  double lo = INFINITY, hi = lmax;
  if (by_max) {
    if (lmax > -INFINITY) lo = lmax;
  } else {
    tk.new_pass();
#pragma unroll
    for (int e = 0; e < kEpt; ++e) {
      const double z = tk.raw(e);
      if (z > -INFINITY) lo = fmin(lo, z);
    }
    for (int i = 0; i < tk.np; ++i) {
      const double z = tk.pen_z(cm, i);
      if (z > -INFINITY) lo = fmin(lo, z);
    }
  }
  block_minmax(&lo, &hi, cm.redd);
  lo = uniform(lo);
  hi = uniform(hi);
  double theta = -INFINITY;
  if (hi > -INFINITY) {
    const Affine af = make_affine(lo, hi, kHB);
    if (by_max) {
      if (lmax > -INFINITY) lds_add(&cm.hcnt[af.bin(lmax)], 1u);
    } else {
      tk.new_pass();
#pragma unroll
      for (int e = 0; e < kEpt; ++e) {
        const double z = tk.raw(e);
        if (z > -INFINITY) lds_add(&cm.hcnt[af.bin(z)], 1u);
      }
      for (int i = 0; i < tk.np; ++i) {
        const double z = tk.pen_z(cm, i);
        if (z > -INFINITY) lds_add(&cm.hcnt[af.bin(z)], 1u);
      }
    }
    lds_barrier();
    const Pick pk = pick_desc<false>(cm.hcnt, nullptr, kHB, 0, target, cm.redu, cm.ctl, cm.ctlu);
    // every z with bin(z) >= d is >= lo + (d - 0.01) / scale (bin(z) is
    // floor((z - lo) * scale) up to a few ulps); bin 0 starts at lo
    if (pk.found) theta = pk.d > 0 ? af.lo + ((double)uniform(pk.d) - 0.01) / af.scale : lo;
  }
  theta = uniform(theta);
  uint32_t pm = 0;
  double um = -INFINITY;
  tk.new_pass();
#pragma unroll
  for (int e = 0; e < kEpt; ++e) {
    const double z = tk.raw(e);
    const bool fin = z > -INFINITY;
    if (fin && z >= theta) pm |= 1u << e;
    else if (fin) um = fmax(um, z);
  }
  uint32_t qm = 0;  // penalised tokens kept
  for (int i = 0; i < tk.np; ++i) {
    const double z = tk.pen_z(cm, i);
    const bool fin = z > -INFINITY;
    if (fin && z >= theta) qm |= 1u << i;
    else if (fin) um = fmax(um, z);
  }
  // one LDS reservation per wave (cm.cand_n was reset before the barriers above)
  const int cnt = __popc(pm) + __popc(qm);
  const int incl = wave_scan_incl(cnt, 0, OpAdd{});
  const int wtot = lane_value(incl, kWave - 1);
  int base = 0;
  if (lane() == kWave - 1) base = lds_fetch_add(&cm.cand_n, incl);
  base = lane_value(base, kWave - 1);
  int slot = base + incl - cnt;
  double* cz = a.ws.cz + (size_t)g * capc;
  int32_t* ci = a.ws.ci + (size_t)g * capc;
  tk.new_pass();
#pragma unroll
  for (int e = 0; e < kEpt; ++e) {
    if ((pm >> e) & 1u) {
      if (slot < capc) {
        cz[slot] = tk.raw(e);
        ci[slot] = c0 + slot_q<TIn>(e);
      } else {
        um = fmax(um, tk.raw(e));
      }
      ++slot;
    }
  }
  for (int i = 0; i < tk.np; ++i) {
    if ((qm >> i) & 1u) {
      if (slot < capc) {
        cz[slot] = tk.pen_z(cm, i);
        ci[slot] = tk.pen_tok(cm, i);
      } else {
        um = fmax(um, tk.pen_z(cm, i));
      }
      ++slot;
    }
  }
  um = wave_max(um);
  if (lane() == 0) {
    wp->zmax = hi;
    wp->umax = um;
    wp->end = min(base + wtot, capc);
    wp->flags = flags;
  }
}

// One workgroup per 64 KB chunk (rows of any alignment: 16-byte
// non-temporal loads when the row allows, scalar loads otherwise).  The
// waves work on their own segments and write their own parts, so greedy and
// temperature chunks need no workgroup barrier; candidate chunks need the
// few of one value histogram.  Per row mode: greedy argmax, candidates,
// segment partials of the normaliser.
template <typename TIn, bool VEC>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4))) void k_sample_chunks(SampleArgs a) {
  using G = Geo<TIn>;
  __shared__ ChunkSmem cm;
  const int C = a.ws.C;
  const int g = blockIdx.x;
  const int row = g / C;
  const int c0 = (g - row * C) * G::kChunk;
  const RowParams rp = load_row_params(a, row);
  const TIn* x = reinterpret_cast<const TIn*>(a.logits) + (int64_t)row * a.ld;
  ChunkToks<TIn> tk;
  load_chunk<TIn, VEC>(x, a.V, c0, tk.v);
  const double* tab = cm.exp_tab[wave()];
  init_exp_table_wave(cm.exp_tab[wave()]);
  const bool cands = rp.topk || rp.topp;
  if (cands) {  // ordered before use by the first barrier of chunk_candidates
    for (int b = threadIdx.x; b < kHB; b += kThreads) cm.hcnt[b] = 0u;
    if (threadIdx.x == 0) cm.cand_n = 0;
  }
  int flags = 0;
  if (rp.pen_active) {
    const uint32_t pb = chunk_pbits<TIn>(a, rp, c0, cm);
    if (set_aside_penalised<TIn>(tk, pb, rp.pen, c0, cm)) flags = kChunkIncomplete;
  }
  WavePart* wp = a.ws.part + (size_t)g * kWaves + wave();
  if (rp.greedy) {
    ArgMax best{-INFINITY, INT_MAX};
    tk.new_pass();
#pragma unroll
    for (int e = 0; e < G::kEpt; ++e) best = argmax_merge(best, ArgMax{tk.raw(e), c0 + slot_q<TIn>(e)});
    for (int i = 0; i < tk.np; ++i) best = argmax_merge(best, ArgMax{tk.pen_z(cm, i), tk.pen_tok(cm, i)});
    best = wave_argmax(best);
    if (lane() == 0) {
      wp->best_z = best.v;
      wp->best_idx = best.i;
      wp->flags = flags;
    }
    return;
  }
  double lmax = -INFINITY;
  tk.new_pass();
#pragma unroll
  for (int e = 0; e < G::kEpt; ++e) lmax = fmax(lmax, tk.raw(e));
  for (int i = 0; i < tk.np; ++i) lmax = fmax(lmax, tk.pen_z(cm, i));
  if (cands) chunk_candidates<TIn>(tk, lmax, a, rp, g, c0, flags, wp, cm);
  else if (lane() == 0) wp->flags = flags;
  if (!rp.topk) {  // the full-vocabulary normaliser (sampling.py:79-81)
    // y = z / T is monotone in z, so the segment's max y is y(max z)
    const YScale ys{rp.T, 1.0 / rp.T};
    const double m = uniform(ys(wave_max(lmax)));
    double s = 0.0;
    if (m > -INFINITY) {
      tk.new_pass();
#pragma unroll
      for (int e = 0; e < G::kEpt; ++e) s += fast_exp_neg(ys(tk.raw(e)) - m, tab);
      for (int i = 0; i < tk.np; ++i) s += fast_exp_neg(ys(tk.pen_z(cm, i)) - m, tab);
    }
    s = wave_sum(s);
    if (lane() == 0) {
      a.ws.seg_m[(size_t)g * kWaves + wave()] = m;
      a.ws.seg_s[(size_t)g * kWaves + wave()] = s;
    }
  }
}

// ================================================================ finish

// Inclusive and exclusive scan of one double per thread, thread order,
// fixed association.
__device__ __forceinline__ double block_scan_d(double v, double* red, double* excl, double* total) {
  const double x = wave_scan_incl(v, 0.0, OpAdd{});
  const double xe = wave_shift_up1(x, 0.0);
  if (lane() == kWave - 1) red[wave()] = x;
  wg_barrier();
  double pre = 0.0, tot = 0.0;
  for (int w = 0; w < kWaves; ++w) {
    if (w < wave()) pre += red[w];
    tot += red[w];
  }
  wg_barrier();
  *excl = pre + xe;
  *total = tot;
  return pre + x;
}

// Candidates of one row, held in registers: thread t owns slots
// q * kThreads + t (q < kPerT) of the row's gathered list; bit q of `valid`
// marks a real candidate.  v[q] holds the penalised logit, later its exp.
constexpr int kPerT = kCandCap / kThreads;
struct RegCands {
  double v[kPerT];
  int idx[kPerT];
  uint32_t valid;
};

// Value-range selection over the register-resident candidates: slot q of
// each thread takes part when it is valid and elig(q) holds; val(q) places
// it in histogram bins (monotone in the order), key(q) orders exactly, token
// index ascending on equal keys.
//   MASS=false: the target-th largest key;
//   MASS=true : in (key desc, index asc) order the first candidate whose
//               inclusive weight wt(q) reaches target.
// Histogram levels narrow the active set until at most 64 candidates are
// left; one wave then ranks them (each lane counts the entries ahead of its
// own).  giveup: more than kSortMax candidates share one value at the cut
// (the caller falls back to the general pipeline).
struct SelOut {
  bool found;
  bool giveup;
  uint64_t key;
  int idx;
};

// Workgroup (min, max, count) in one barrier round.
__device__ __forceinline__ void block_range(double* lo, double* hi, uint32_t* cnt, FastSmem& fs) {
  double a = wave_min(*lo), b = wave_max(*hi);
  uint32_t n = wave_sum(*cnt);
  if (lane() == 0) {
    fs.redm[wave()] = a;
    fs.redm[kWaves + wave()] = b;
    reinterpret_cast<uint32_t*>(fs.redu)[wave()] = n;
  }
  wg_barrier();
  a = fs.redm[0];
  b = fs.redm[kWaves];
  n = reinterpret_cast<uint32_t*>(fs.redu)[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) {
    a = fmin(a, fs.redm[w]);
    b = fmax(b, fs.redm[kWaves + w]);
    n += reinterpret_cast<uint32_t*>(fs.redu)[w];
  }
  wg_barrier();
  *lo = a;
  *hi = b;
  *cnt = n;
}

__device__ __forceinline__ bool key_desc_idx_asc(uint64_t ka, int ia, uint64_t kb, int ib) {
  return ka > kb || (ka == kb && ia < ib);
}

// Histogram levels chosen so far (at most kSelLevels = 4), held in named
// fields so they stay in registers.
struct Levels {
  Affine a0, a1, a2, a3;
  int d0 = 0, d1 = 0, d2 = 0, d3 = 0;
  int n = 0;
  __device__ __forceinline__ bool match(double v) const {
    if (n > 0 && a0.bin(v) != d0) return false;
    if (n > 1 && a1.bin(v) != d1) return false;
    if (n > 2 && a2.bin(v) != d2) return false;
    if (n > 3 && a3.bin(v) != d3) return false;
    return true;
  }
  __device__ __forceinline__ void push(const Affine& a, int d) {
    if (n == 0) {
      a0 = a;
      d0 = d;
    } else if (n == 1) {
      a1 = a;
      d1 = d;
    } else if (n == 2) {
      a2 = a;
      d2 = d;
    } else {
      a3 = a;
      d3 = d;
    }
    ++n;
  }
};
static_assert(kSelLevels == 4, "Levels holds four histogram levels");

template <bool MASS, class Elig, class Val, class Key, class W>
__device__ __forceinline__ SelOut cand_select(const RegCands& rc, const Elig& elig, const Val& val, const Key& key,
                                              const W& wt, uint64_t target, FastSmem& fs) {
  Levels lv;
  uint64_t above = 0;
  SortList& sl = fs.u.sl;
  for (;;) {
    double lo = INFINITY, hi = -INFINITY;
    uint32_t cnt = 0, act = 0;
#pragma unroll
    for (int q = 0; q < kPerT; ++q) {
      if (((rc.valid >> q) & 1u) && elig(q)) {
        const double v = val(q);
        if (lv.match(v)) {
          lo = fmin(lo, v);
          hi = fmax(hi, v);
          ++cnt;
          act |= 1u << q;
        }
      }
    }
    block_range(&lo, &hi, &cnt, fs);
    if (cnt <= (uint32_t)kWave || !(hi > lo) || lv.n == kSelLevels) {
      if (cnt > (uint32_t)kSortMax) return SelOut{false, true, 0, 0};
      // list the active candidates: one LDS reservation per thread
      if (threadIdx.x == 0) fs.ctl[2] = 0;
      lds_barrier();
      int slot = act ? lds_fetch_add(&fs.ctl[2], __popc(act)) : 0;
#pragma unroll
      for (int q = 0; q < kPerT; ++q)
        if ((act >> q) & 1u) {
          sl.key[slot] = key(q);
          sl.idx[slot] = rc.idx[q];
          sl.w[slot] = MASS ? wt(q) : 0ull;
          ++slot;
        }
      lds_barrier();
      const int m = (int)cnt;
      if (m <= kWave) {
        // one wave: each lane holds one entry and counts the entries ahead of
        // it (rank) and their weight; the answer is the lane at rank pos, or
        // the lane whose weight takes the running total across target
        if (wave() == 0) {
          const int ln = lane();
          uint64_t k = 0ull, w = 0ull;
          int ix = INT_MAX;
          if (ln < m) {
            k = sl.key[ln];
            ix = sl.idx[ln];
            w = sl.w[ln];
          }
          int rank = 0;
          uint64_t ahead = 0;
#pragma unroll 8
          for (int j = 0; j < m; ++j) {
            const bool bj = key_desc_idx_asc(sl.key[j], sl.idx[j], k, ix);
            rank += bj ? 1 : 0;
            if (MASS && bj) ahead += sl.w[j];
          }
          bool hit;
          if (!MASS) hit = ln < m && (int64_t)rank == (int64_t)target - (int64_t)above - 1;
          else hit = ln < m && above + ahead < target && above + ahead + w >= target;
          const uint64_t b = __ballot(hit);
          if (ln == 0) fs.ctl[3] = b != 0 ? 1 : 0;
          if (hit) {
            fs.ctlu[2] = k;
            fs.ctl[4] = ix;
          }
        }
        lds_barrier();
        const bool found = fs.ctl[3] != 0;
        const SelOut r{found, !MASS && !found, found ? fs.ctlu[2] : 0ull, found ? fs.ctl[4] : 0};
        lds_barrier();
        return r;
      }
      lds_bitonic(sl.key, sl.idx, sl.w, m, 0ull, key_desc_idx_asc);
      if (!MASS) {
        const int pos = (int)(target - above - 1);
        if (pos < 0 || pos >= m) return SelOut{false, true, 0, 0};
        return SelOut{true, false, sl.key[pos], sl.idx[pos]};
      }
      // inclusive weight in sorted order, kSortMax / kThreads entries per thread
      constexpr int kPer = kSortMax / kThreads;
      const int i0 = kPer * (int)threadIdx.x;
      uint64_t wl[kPer], s = 0;
#pragma unroll
      for (int q = 0; q < kPer; ++q) {
        wl[q] = i0 + q < m ? sl.w[i0 + q] : 0ull;
        s += wl[q];
      }
      uint64_t tot;
      uint64_t run = above + block_excl_scan<uint64_t>(s, fs.redu, &tot);
      int hit = INT_MAX;
#pragma unroll
      for (int q = 0; q < kPer; ++q) {
        run += wl[q];
        if (hit == INT_MAX && i0 + q < m && run >= target) hit = i0 + q;
      }
      hit = block_min<int>(hit, fs.redi);
      if (hit == INT_MAX) return SelOut{false, false, 0, 0};
      return SelOut{true, false, sl.key[hit], sl.idx[hit]};
    }
    const Affine af = make_affine(lo, hi, kHB);
    for (int b = threadIdx.x; b < kHB; b += kThreads) {
      fs.hcnt[b] = 0u;
      fs.hmass[b] = 0ull;
    }
    lds_barrier();
#pragma unroll
    for (int q = 0; q < kPerT; ++q)
      if ((act >> q) & 1u) {
        const int b = af.bin(val(q));
        lds_add(&fs.hcnt[b], 1u);
        if (MASS) lds_add(&fs.hmass[b], wt(q));
      }
    lds_barrier();
    const Pick pk = pick_desc<MASS>(fs.hcnt, fs.hmass, kHB, above, target, fs.redu, fs.ctl, fs.ctlu);
    if (!pk.found) return SelOut{false, false, 0, 0};
    above = pk.above;
    lv.push(af, pk.d);
  }
}

// Inverse-CDF draw over the kept candidates in vocabulary order
// (sampling.py:94-98): with w(q) the fixed-point probability of kept
// candidates (0 otherwise), the first token whose running mass exceeds
// floor(u * total); V-1 when none does.
template <class W>
__device__ __forceinline__ int draw_kept(const RegCands& rc, int V, double u, const W& wt, FastSmem& fs) {
  auto wq = [&](int q) -> uint64_t { return ((rc.valid >> q) & 1u) ? wt(q) : 0ull; };
  uint64_t tot = 0;
#pragma unroll
  for (int q = 0; q < kPerT; ++q) tot += wq(q);
  tot = block_sum<uint64_t>(tot, fs.redu);
  if (tot == 0) return V - 1;
  const uint64_t t = (uint64_t)__double2ull_rd(u * (double)tot);
  for (int b = threadIdx.x; b < kHB; b += kThreads) fs.hmass[b] = 0ull;
  lds_barrier();
  auto ibin = [&](int idx) -> int { return (int)(((int64_t)idx * kHB) / V); };
#pragma unroll
  for (int q = 0; q < kPerT; ++q) {
    const uint64_t w = wq(q);
    if (w) lds_add(&fs.hmass[ibin(rc.idx[q])], w);
  }
  lds_barrier();
  // first index bin whose running mass exceeds t (kHB / kThreads bins per thread)
  constexpr int kPer = kHB / kThreads;
  const int b0 = kPer * (int)threadIdx.x;
  uint64_t hb[kPer], hs = 0;
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    hb[q] = fs.hmass[b0 + q];
    hs += hb[q];
  }
  uint64_t btot;
  uint64_t brun = block_excl_scan<uint64_t>(hs, fs.redu, &btot);
  // the running mass is non-decreasing: one bin takes it past t
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    if (brun <= t && brun + hb[q] > t) {
      fs.ctl[5] = b0 + q;
      fs.ctlu[0] = brun;
    }
    brun += hb[q];
  }
  if (threadIdx.x == 0) fs.ctl[2] = 0;
  wg_barrier();
  if (btot <= t) return V - 1;
  const int b = fs.ctl[5];
  const uint64_t before = fs.ctlu[0];
  SortList& sl = fs.u.sl;
  uint32_t mine = 0;
#pragma unroll
  for (int q = 0; q < kPerT; ++q)
    if (wq(q) && ibin(rc.idx[q]) == b) mine |= 1u << q;
  int slot = mine ? lds_fetch_add(&fs.ctl[2], __popc(mine)) : 0;
#pragma unroll
  for (int q = 0; q < kPerT; ++q)
    if ((mine >> q) & 1u) {
      sl.key[slot] = (uint64_t)rc.idx[q];
      sl.idx[slot] = rc.idx[q];
      sl.w[slot] = wq(q);
      ++slot;
    }
  lds_barrier();
  const int m = fs.ctl[2];  // at most V / kHB + 1 <= kThreads tokens
  if (m <= kWave) {
    // one wave: each lane sums the weight of the entries with a smaller
    // index; the hit is the lane whose weight takes the running mass past t
    if (wave() == 0) {
      const int ln = lane();
      uint64_t w = 0ull;
      int ix = INT_MAX;
      if (ln < m) {
        ix = sl.idx[ln];
        w = sl.w[ln];
      }
      uint64_t ahead = 0;
#pragma unroll 8
      for (int j = 0; j < m; ++j)
        if (sl.idx[j] < ix) ahead += sl.w[j];
      const bool hit = ln < m && before + ahead <= t && before + ahead + w > t;
      const uint64_t hbits = __ballot(hit);
      if (ln == 0 && hbits == 0) fs.ctl[3] = INT_MAX;
      if (hit) fs.ctl[3] = ix;
    }
    lds_barrier();
    const int hit = fs.ctl[3];
    return hit == INT_MAX ? V - 1 : hit;
  }
  auto idx_asc = [](uint64_t ka, int, uint64_t kb, int) { return ka < kb; };
  lds_bitonic(sl.key, sl.idx, sl.w, m, ~0ull, idx_asc);
  const uint64_t w = (int)threadIdx.x < m ? sl.w[threadIdx.x] : 0ull;
  uint64_t mt;
  const uint64_t ex = block_excl_scan<uint64_t>(w, fs.redu, &mt);
  const int hit = block_min<int>(((int)threadIdx.x < m && before + ex + w > t) ? sl.idx[threadIdx.x] : INT_MAX,
                                 fs.redi);
  return hit == INT_MAX ? V - 1 : hit;
}

// Greedy rows: argmax over the segment argmaxes (lowest index on ties).
__device__ __forceinline__ int finish_greedy(const SampleArgs& a, int row, FastSmem& fs) {
  const int P = a.ws.C * kWaves;
  ArgMax best{-INFINITY, INT_MAX};
  for (int c = threadIdx.x; c < P; c += kThreads) {
    const WavePart& p = a.ws.part[(size_t)row * P + c];
    best = argmax_merge(best, ArgMax{p.best_z, p.best_idx});
  }
  return block_argmax(best, fs.redd, fs.redi).i;
}

// The full distribution's segment partials, one per thread (nseg <=
// kThreads): *mk the segment max, *mass its sum rescaled to the largest
// segment max, which goes to *ymax.
__device__ __forceinline__ void segment_masses(const SampleArgs& a, int row, int nseg, FastSmem& fs, double* ymax,
                                               double* mk, double* mass) {
  const int k = threadIdx.x;
  const size_t b = (size_t)row * a.ws.C * kWaves;
  *mk = k < nseg ? a.ws.seg_m[b + k] : -INFINITY;
  const double sk = k < nseg ? a.ws.seg_s[b + k] : 0.0;
  *ymax = block_max(*mk, fs.redd);
  *mass = (k < nseg && *mk > -INFINITY) ? sk * fast_exp_neg(*mk - *ymax, fs.exp_tab) : 0.0;
}

// Temperature only: full-vocabulary softmax and draw (sampling.py:75-81,
// :94-98).  The segment holding the inverse-CDF point is rescanned from HBM
// with the arithmetic of the partials.
template <typename TIn>
__device__ __forceinline__ int finish_temp(const SampleArgs& a, int row, const RowParams& rp, FastSmem& fs) {
  using G = Geo<TIn>;
  const int V = a.V;
  const int nseg = (V + G::kSeg - 1) / G::kSeg;  // <= kThreads
  const YScale ys{rp.T, 1.0 / rp.T};
  const int k = threadIdx.x;
  double ymax, mk, mass;
  segment_masses(a, row, nseg, fs, &ymax, &mk, &mass);
  double ex, S;
  block_scan_d(mass, fs.redd, &ex, &S);
  const double t = rp.u * S;
  const int kstar = block_min<int>((k < nseg && ex + mass > t) ? k : INT_MAX, fs.redi);
  if (kstar == INT_MAX) return V - 1;
  if (k == kstar) {
    fs.ctlu[0] = (uint64_t)__double_as_longlong(ex);
    fs.ctlu[1] = (uint64_t)__double_as_longlong(mk);
  }
  const int s0 = kstar * G::kSeg;
  if (rp.pen_active) {
    for (int w = threadIdx.x; w < G::kSeg / 32; w += kThreads) fs.u.segbits[w] = 0u;
    wg_barrier();
    for (int64_t h = rp.h0 + threadIdx.x; h < rp.h1; h += kThreads) {
      const int off = a.hist_ids[h] - s0;
      if ((unsigned)off < (unsigned)G::kSeg) lds_or(&fs.u.segbits[off >> 5], 1u << (off & 31));
    }
  }
  wg_barrier();
  const double before = __longlong_as_double((long long)fs.ctlu[0]);
  const double ms = __longlong_as_double((long long)fs.ctlu[1]);
  const double sc = fast_exp_neg(ms - ymax, fs.exp_tab);
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
      if (rp.pen_active && ((fs.u.segbits[(q0 + q) >> 5] >> ((q0 + q) & 31)) & 1u)) z = penalize(z, rp.pen);
      e[q] = fast_exp_neg(ys(z) - ms, fs.exp_tab);
    }
    es += e[q];
  }
  double pex, ptot;
  block_scan_d(es, fs.redd, &pex, &ptot);
  double run = pex;
  int hit = INT_MAX, last = -1;
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    run += e[q];
    if (e[q] > 0.0) last = s0 + q0 + q;
    if (hit == INT_MAX && e[q] > 0.0 && before + run * sc > t) hit = s0 + q0 + q;
  }
  hit = block_min<int>(hit, fs.redi);
  if (hit == INT_MAX) hit = block_max<int>(last, fs.redi);  // rounding at the segment end
  return hit < 0 ? V - 1 : hit;
}

struct FastOut {
  int id;
  bool general;  // the candidates cannot decide the row exactly
};

// Top-k and/or top-p rows (sampling.py:75-90, :94-98) from the gathered
// chunk candidates.
template <typename TIn, bool TOPK>
__device__ __forceinline__ FastOut finish_cands(const SampleArgs& a, int row, const RowParams& rp, FastSmem& fs) {
  using G = Geo<TIn>;
  const int V = a.V;
  const int C = a.ws.C, capc = a.ws.capc;
  // gather every slot of the row first (slot i = q * kThreads + t, chunk
  // i / capc; consecutive lanes read consecutive addresses), then learn from
  // the chunk partials which slots hold candidates
  const int slots = C * capc;
  const size_t base = (size_t)row * slots;
  RegCands rc;
  rc.valid = 0;
#pragma unroll
  for (int q = 0; q < kPerT; ++q) {
    const int i = q * kThreads + (int)threadIdx.x;
    rc.v[q] = 0.0;
    rc.idx[q] = 0;
    if (i < slots) {
      rc.v[q] = a.ws.cz[base + i];
      rc.idx[q] = a.ws.ci[base + i];
    }
  }
  // a chunk's candidate count is the largest end over its waves
  if ((int)threadIdx.x < C) fs.cnt_c[threadIdx.x] = 0;
  wg_barrier();
  double u_l = -INFINITY, zm_l = -INFINITY;
  if ((int)threadIdx.x < C * kWaves) {
    const WavePart p = a.ws.part[(size_t)row * C * kWaves + threadIdx.x];
    lds_max(&fs.cnt_c[threadIdx.x / kWaves], p.end);
    u_l = p.umax;
    zm_l = p.zmax;
  }
  const double U = block_max(u_l, fs.redd);
  const double zmax = block_max(zm_l, fs.redd);
#pragma unroll
  for (int q = 0; q < kPerT; ++q) {
    const int i = q * kThreads + (int)threadIdx.x;
    if (i < slots) {
      const int c = i / capc;
      if (i - c * capc < fs.cnt_c[c]) rc.valid |= 1u << q;
    }
  }
  const double T = rp.T;
  auto yexact = [&](double z) -> double { return T == 1.0 ? z : z / T; };

  // ---- top-k: k-th largest with multiplicity, keep y >= kth_y (:76-78)
  double z_lo = -INFINITY;
  if (TOPK) {
    const SelOut r = cand_select<false>(rc, [](int) { return true; }, [&](int q) { return rc.v[q]; },
                                        [&](int q) { return key_of(rc.v[q]); }, [](int) { return 0ull; },
                                        (uint64_t)rp.top_k, fs);
    if (!r.found) return FastOut{V - 1, true};
    const double kth_z = val_of_key(r.key);
    const double kth_y = yexact(kth_z);
    z_lo = kth_z;
    for (int it = 0; it < 64; ++it) {
      const double zp = dbl_prev(z_lo);
      if (yexact(zp) >= kth_y) z_lo = zp;
      else break;
    }
    if (!(U < z_lo)) return FastOut{V - 1, true};
  }

  // ---- softmax (:79-81): each candidate's exp(y - ymax) once, in place of
  // z (0 outside the top-k set); p = e / S
  const YScale ys{T, 1.0 / T};
  const double ymax = ys(zmax);
  double s = 0.0;
#pragma unroll
  for (int q = 0; q < kPerT; ++q) {
    const double z = rc.v[q];
    const double e = (((rc.valid >> q) & 1u) && z >= z_lo) ? fast_exp_neg(ys(z) - ymax, fs.exp_tab) : 0.0;
    rc.v[q] = e;
    s += e;
  }
  double S;
  if (TOPK) {
    S = block_sum(s, fs.redd);
  } else {
    const int nseg = (V + G::kSeg - 1) / G::kSeg;
    double ysmax, mk, mass;
    segment_masses(a, row, nseg, fs, &ysmax, &mk, &mass);
    S = block_sum(mass, fs.redd);
  }
  const double invS = 1.0 / S;
  auto pq = [&](int q) -> double { return rc.v[q] * invS; };

  // ---- top-p: first token (p desc, index asc) whose inclusive mass reaches
  // top_p (:82-90); bins on the bit pattern of p (log-spaced)
  bool have_cut = false;
  uint64_t cut_key = 0;
  int cut_idx = INT_MAX;
  if (rp.topp) {
    const SelOut r = cand_select<true>(rc, [&](int q) { return rc.v[q] > 0.0; },
                                       [&](int q) { return (double)pkey_of(pq(q)); },
                                       [&](int q) { return pkey_of(pq(q)); }, [&](int q) { return to_fx(pq(q)); },
                                       topp_target(rp.top_p), fs);
    if (r.giveup) return FastOut{V - 1, true};
    if (r.found) {
      have_cut = true;
      cut_key = r.key;
      cut_idx = r.idx;
    }
    if (!TOPK && U > -INFINITY) {
      const double pU = fast_exp_neg(ys(U) - ymax, fs.exp_tab) * invS;
      if (!(have_cut && cut_key > pkey_of(pU))) return FastOut{V - 1, true};
    }
  }

  // ---- draw in vocabulary order (:94-98)
  auto wt = [&](int q) -> uint64_t {
    const double p = pq(q);
    if (!(p > 0.0)) return 0ull;
    if (have_cut) {
      const uint64_t k = pkey_of(p);
      if (!(k > cut_key || (k == cut_key && rc.idx[q] <= cut_idx))) return 0ull;
    }
    return to_fx(p);
  };
  return FastOut{draw_kept(rc, V, rp.u, wt, fs), false};
}

template <typename TIn, bool VEC>
__global__ __launch_bounds__(kThreads) void k_sample_final(SampleArgs a) {
  __shared__ SmemAll sm;
  FastSmem& fs = sm.f;
  const int row = blockIdx.x;
  const RowParams rp = load_row_params(a, row);
  init_exp_table(fs.exp_tab);
  wg_barrier();
  int id = 0;
  // a chunk that could not keep all its penalised tokens aside sends the
  // row to the general pipeline
  int fl = 0;
  for (int c = threadIdx.x; c < a.ws.C * kWaves; c += kThreads) fl |= a.ws.part[(size_t)row * a.ws.C * kWaves + c].flags;
  bool general = block_max<int>(fl, fs.redi) != 0;
  if (general) {
  } else if (rp.greedy) {
    id = finish_greedy(a, row, fs);
  } else if (!rp.topk && !rp.topp) {
    id = finish_temp<TIn>(a, row, rp, fs);
  } else {
    const FastOut o = rp.topk ? finish_cands<TIn, true>(a, row, rp, fs) : finish_cands<TIn, false>(a, row, rp, fs);
    id = o.id;
    general = o.general;
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
         up256(n * cap * sizeof(int32_t));
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
  const int total = a.B * a.ws.C;
  const dim3 gf(a.B), block(kThreads);
  if (vec) {
    if (f64) hipLaunchKernelGGL((k_sample_chunks<double, true>), dim3(total), block, 0, s, a);
    else hipLaunchKernelGGL((k_sample_chunks<float, true>), dim3(total), block, 0, s, a);
  } else {
    if (f64) hipLaunchKernelGGL((k_sample_chunks<double, false>), dim3(total), block, 0, s, a);
    else hipLaunchKernelGGL((k_sample_chunks<float, false>), dim3(total), block, 0, s, a);
  }
  if (between != nullptr) {
    const hipError_t e = hipEventRecord(between, s);
    if (e != hipSuccess) return e;
  }
  auto final_ = f64 ? (vec ? k_sample_final<double, true> : k_sample_final<double, false>)
                    : (vec ? k_sample_final<float, true> : k_sample_final<float, false>);
  hipLaunchKernelGGL(final_, gf, block, 0, s, a);
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
