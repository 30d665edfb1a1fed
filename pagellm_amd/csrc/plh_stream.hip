// Streaming sampler fast path for gfx950 (src/pagellm/engine/sampling.py:52-111),
// two launches:
//   k_stream_chunks  B x C workgroups: workgroup (row, c) reads the c-th
//          64 KB chunk of the row once (16-byte loads, 32 fp32 or 16 fp64
//          tokens per thread), penalises it, and leaves one record per wave
//          (its 1/8 of the chunk, a "segment"), plus the segment's candidate
//          tokens for rows that select:
//            greedy       the segment's argmax;
//            temperature  max y and sum exp(y - max) of the segment (y = z/T);
//            top-k        tokens >= the chunk's threshold theta, taken from
//                         the per-thread maxima so that it sits at or below
//                         the chunk's k-th largest token;
//            top-p        the segment's max and sum, and the tokens at or
//                         above a threshold picked from a value histogram
//                         so that the chunk keeps about ncand of them.
//   k_stream_merge   one workgroup per row selects exactly from the
//          records (k-th largest with ties, fixed-point top-p cut in
//          (p descending, index ascending) order, fixed-point or float64
//          inverse-CDF draw in vocabulary order) and writes the id.  A row
//          the records cannot decide exactly (a threshold above the cut, a
//          candidate overflow) is finished by the general pipeline in the
//          same workgroup.
#include <type_traits>

#include "plh_fast.h"
#include "plh_kernels.h"
#include "plh_pipeline.h"

namespace plh {

namespace {

constexpr int kUL = 8;             // 16-byte loads per thread per chunk
constexpr int kNB = 1024;          // bins of a chunk's value histogram
constexpr int kPenW = 128;         // penalised tokens one wave keeps aside
constexpr int kTopkMax = 512;      // largest top_k a chunk threshold covers
constexpr int kCPT = 20;           // candidates per merge thread (their 64-bit keys)
constexpr int kCandMax = kCPT * kThreads;
constexpr int kMB = 512;           // bins of one merge selection level
constexpr int kMBuf = 3;           // rotating merge histograms (one barrier per level)
constexpr int kFinal = 64;         // entries a selection ranks directly
constexpr double kRangeY = 40.0;   // histogram span below the chunk max, in units of y = z/T
constexpr int kMaxSegs = kMaxStreamChunks * kWaves;
constexpr uint32_t kPenBit = 0x80000000u;  // candidate id flag: the token was penalised

enum : int { kModeGreedy = 0, kModeTemp = 1, kModeTopK = 2, kModeTopP = 3, kModeGeneral = 4 };
enum : int { kRecIncomplete = 1, kRecOverflow = 2 };

template <typename TIn>
struct SGeo {
  static constexpr int VW = 16 / (int)sizeof(TIn);
  static constexpr int EPT = kUL * VW;       // tokens per thread
  static constexpr int SPAN = kWave * VW;    // tokens of one wave-wide load
  static constexpr int SEG = EPT * kWave;    // tokens of one wave's segment
  static constexpr int CH = SEG * kWaves;    // tokens of one chunk
};
constexpr int kMaxCh = SGeo<float>::CH;
constexpr int kMaxSeg = SGeo<float>::SEG;

typedef float sf4_t __attribute__((ext_vector_type(4)));
typedef double sd2_t __attribute__((ext_vector_type(2)));
template <typename TIn>
struct SVec;
template <>
struct SVec<float> {
  typedef sf4_t T;
};
template <>
struct SVec<double> {
  typedef sd2_t T;
};

// ------------------------------------------------------------------- LDS

struct ChunkLds {
  double red[2 * kWaves];
  int redi[2 * kWaves];
  uint32_t hist[kNB];
  uint32_t bitmap[kMaxCh / 32];
  double pz[kWaves][kPenW];
  int pt[kWaves][kPenW];
  double exp_tab[kWaves][64];
};

struct MergeLds {
  double exp_tab[64];
  uint32_t cnt[kMBuf][kMB];
  uint64_t mass[kMBuf][kMB];
  uint64_t segm[kMaxSegs];    // kept mass of each segment (fixed point)
  int segoff[kMaxSegs + 1];   // candidates before each segment
  uint64_t fkey[kFinal];      // the last level of a selection
  uint64_t fw[kFinal];
  int fidx[kFinal];
  int fn;
  double dscan[kThreads];     // draws: staged weights of a segment
  uint64_t uscan[kThreads];
  int iscan[kThreads];
  uint32_t segbits[kMaxSeg / 32];
  double redd[2 * kWaves];
  uint64_t redu[2 * kWaves];
  int redi[2 * kWaves];
  int ctl[8];
  uint64_t ctlu[4];
  double ctld[4];
};

union MergeSmem {
  MergeLds m;
  SmemCore g;  // the general pipeline (rows the records cannot decide)
};

// ------------------------------------------------------- device helpers

__device__ __forceinline__ RowParams stream_row_params(const SampleArgs& a, int row) {
  RowParams rp;
  rp.T = a.temperature[row];
  rp.top_k = a.top_k[row];
  rp.top_p = a.top_p[row];
  rp.pen = a.rep_penalty[row];
  rp.u = a.uniforms != nullptr ? a.uniforms[row] : 0.0;
  rp.h0 = a.hist_off != nullptr ? a.hist_off[a.hist_spans ? 2 * row : row] : 0;
  rp.h1 = a.hist_off != nullptr ? a.hist_off[a.hist_spans ? 2 * row + 1 : row + 1] : 0;
  rp.greedy = rp.T == 0.0;  // SamplingParams.greedy (sampling.py:47-49)
  rp.pen_active = rp.pen != 1.0 && rp.h1 > rp.h0 && a.hist_ids != nullptr;  // :56
  rp.topk = !rp.greedy && rp.top_k > 0 && rp.top_k < a.V;                  // :76
  rp.topp = !rp.greedy && rp.top_p < 1.0;                                   // :82
  rp.nucleus = false;
  return rp;
}

__device__ __forceinline__ int row_mode(const RowParams& rp) {
  if (rp.greedy) return kModeGreedy;
  if (rp.topk) return rp.top_k <= kTopkMax ? kModeTopK : kModeGeneral;
  if (rp.topp) return kModeTopP;
  return kModeTemp;
}

// ================================================================ chunks

template <typename TIn>
struct Toks {
  using G = SGeo<TIn>;
  typename SVec<TIn>::T v[kUL];
  int po = 0, np = 0;  // the thread's penalised tokens: entries [po, po + np) of its wave's pool
  __device__ __forceinline__ TIn rv(int e) const { return v[e / G::VW][e % G::VW]; }
  __device__ __forceinline__ void set(int e, TIn x) { v[e / G::VW][e % G::VW] = x; }
  // keeps the compiler from holding a widened copy of the registers across passes
  __device__ __forceinline__ void new_pass() {
#pragma unroll
    for (int j = 0; j < kUL; ++j) asm volatile("" : "+v"(v[j]));
  }
};

// Token id (within the row) of register slot e of the calling lane.
// The base is laundered through an empty asm so the compiler recomputes ids
// where they are needed instead of keeping the loads' 32 per-slot
// addresses alive through the whole chunk.
template <typename TIn>
__device__ __forceinline__ int slot_tok(int c0, int e) {
  using G = SGeo<TIn>;
  int base = c0 + wave() * G::SEG + lane() * G::VW;
  asm volatile("" : "+v"(base));
  return base + (e / G::VW) * G::SPAN + (e % G::VW);
}

template <typename TIn, bool VEC>
__device__ __forceinline__ void load_toks(const TIn* x, int V, int c0, Toks<TIn>& tk) {
  using G = SGeo<TIn>;
  using VT = typename SVec<TIn>::T;
  const int off = c0 + wave() * G::SEG + lane() * G::VW;
  const bool full = VEC && c0 + G::CH <= V;
#pragma unroll
  for (int j = 0; j < kUL; ++j) {
    const int p = off + j * G::SPAN;
    if (full || (VEC && p + G::VW <= V)) {
      tk.v[j] = __builtin_nontemporal_load(reinterpret_cast<const VT*>(x + p));
    } else {
#pragma unroll
      for (int s = 0; s < G::VW; ++s) tk.v[j][s] = (p + s < V) ? x[p + s] : (TIn)(-INFINITY);
    }
  }
}

// One bit per distinct history id inside the chunk (np.unique,
// sampling.py:59); returns the calling lane's bits in register-slot order.
template <typename TIn>
__device__ __forceinline__ uint32_t chunk_pen_bits(const SampleArgs& a, const RowParams& rp, int c0, ChunkLds& cm) {
  using G = SGeo<TIn>;
  constexpr int kWords = G::CH / 32;
  for (int w = threadIdx.x; w < kWords; w += kThreads) cm.bitmap[w] = 0u;
  wg_barrier();
  for (int64_t h0 = rp.h0; h0 < rp.h1; h0 += 8 * kThreads) {
    int id[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t h = h0 + j * kThreads + threadIdx.x;
      id[j] = h < rp.h1 ? a.hist_ids[h] : -1;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int off = id[j] - c0;
      if ((unsigned)off < (unsigned)G::CH) lds_or(&cm.bitmap[off >> 5], 1u << (off & 31));
    }
  }
  wg_barrier();
  uint32_t pb = 0;
  const int q0 = wave() * G::SEG + lane() * G::VW;
#pragma unroll
  for (int j = 0; j < kUL; ++j) {
    const int q = q0 + j * G::SPAN;
    pb |= ((cm.bitmap[q >> 5] >> (q & 31)) & ((1u << G::VW) - 1u)) << (G::VW * j);
  }
  return pb;
}

// Moves the lane's penalised tokens (bits pb) out of the registers into its
// wave's pool with their penalised float64 value (the register slot becomes
// -inf).  Returns true when the pool overflows.
template <typename TIn>
__device__ __forceinline__ bool set_aside(Toks<TIn>& tk, uint32_t pb, double pen, int c0, ChunkLds& cm) {
  using G = SGeo<TIn>;
  const int n = __popc(pb);
  const int incl = wave_scan_incl(n, 0, OpAdd{});
  const int total = lane_value(incl, kWave - 1);
  tk.po = incl - n;
  tk.np = 0;
  if (total > kPenW) return true;
  tk.np = n;
  if (pb != 0u) {
    int k = tk.po;
#pragma unroll
    for (int e = 0; e < G::EPT; ++e) {
      if ((pb >> e) & 1u) {
        cm.pz[wave()][k] = penalize((double)tk.rv(e), pen);
        cm.pt[wave()][k] = slot_tok<TIn>(c0, e);
        ++k;
        tk.set(e, (TIn)(-INFINITY));
      }
    }
  }
  return false;
}

// Smallest input-precision value t with (double)x >= theta <=> x >= t for
// finite x (every finite value when theta is -inf).
template <typename TIn>
__device__ __forceinline__ TIn in_thr(double theta) {
  if constexpr (sizeof(TIn) == 4) return fmaxf(__double2float_ru(theta), -3.402823466e38f);
  else return fmax(theta, -1.7976931348623157e308);
}

// Bins of a chunk's value histogram in the input precision: an Affine's
// bins, rounded to float for float inputs (the bounds rounded outward), so
// the pass over the register tokens needs no float64 arithmetic.  Any
// monotone binning serves: the bins only choose theta, and the candidates
// are exactly the tokens >= theta.
template <typename TIn>
struct HBin {
  Affine af;
  __device__ __forceinline__ explicit HBin(const Affine& a) : af(a) {}
  __device__ __forceinline__ int bin(TIn x) const { return af.bin(x); }
  __device__ __forceinline__ double lo() const { return af.lo; }
  __device__ __forceinline__ double scale() const { return af.scale; }
};
template <>
struct HBin<float> {
  float lo_f, scale_f;
  __device__ __forceinline__ explicit HBin(const Affine& a) {
    lo_f = __double2float_rd(a.lo);
    scale_f = (float)a.scale;
    if (!(scale_f < INFINITY)) scale_f = 0.0f;
  }
  __device__ __forceinline__ int bin(float x) const {
    return (int)__builtin_amdgcn_fmed3f((x - lo_f) * scale_f, 0.0f, (float)(kNB - 1));
  }
  __device__ __forceinline__ double lo() const { return (double)lo_f; }
  __device__ __forceinline__ double scale() const { return (double)scale_f; }
};

// Appends the flagged register slots of the calling wave (and its flagged
// pool entries) to the wave's candidate slots; returns the count or -1
// when they would overflow kCapW.
template <typename TIn, class Flag>
__device__ __forceinline__ int write_cands(const Toks<TIn>& tk, const Flag& flag, uint32_t pool_mask, int c0,
                                           const SampleArgs& a, size_t gw, const ChunkLds& cm) {
  using G = SGeo<TIn>;
  TIn* cv = reinterpret_cast<TIn*>(a.sw.cval) + gw * kCapW;
  int* ci = a.sw.cidx + gw * kCapW;
  int total = 0;
#pragma unroll
  for (int e = 0; e < G::EPT; ++e) total += flag(e, tk.rv(e)) ? 1 : 0;
  total += __popc(pool_mask);
  const int incl = wave_scan_incl(total, 0, OpAdd{});
  const int wtot = lane_value(incl, kWave - 1);
  if (wtot > kCapW) return -1;
  int slot = incl - total;
#pragma unroll
  for (int e = 0; e < G::EPT; ++e) {
    const TIn v = tk.rv(e);
    if (flag(e, v)) {
      cv[slot] = v;
      ci[slot] = slot_tok<TIn>(c0, e);
      ++slot;
    }
  }
  for (int i = 0; i < tk.np; ++i) {
    if ((pool_mask >> i) & 1u) {
      // the raw input value and the penalised flag: the merge recomputes the
      // penalised value with the same arithmetic
      const int tok = cm.pt[wave()][tk.po + i];
      cv[slot] = (TIn)0;
      ci[slot] = (int)((uint32_t)tok | kPenBit);
      ++slot;
    }
  }
  return wtot;
}

__device__ __forceinline__ void publish(const SampleArgs& a, size_t gw, double m, double s, double th, int n,
                                        int flags) {
  if (lane() == 0) a.sw.rec[gw] = WaveRec{m, s, th, n, flags};
}

// Each wave walks the kNB bins of cm.hist from bin 0 on its own: the first
// bin where the running count reaches k (INT_MAX if the total is below k).
__device__ __forceinline__ int hist_reach(const ChunkLds& cm, uint32_t k) {
  constexpr int PL = kNB / kWave;
  uint32_t s = 0;
#pragma unroll 1
  for (int i = 0; i < PL; ++i) s += cm.hist[lane() * PL + i];
  const uint32_t inc = wave_scan_incl(s, 0u, OpAdd{});
  uint32_t run = inc - s;
  int d = INT_MAX;
#pragma unroll 1
  for (int i = 0; i < PL; ++i) {
    const uint32_t cnt = cm.hist[lane() * PL + i];
    if (d == INT_MAX && run < k && run + cnt >= k) d = lane() * PL + i;
    run += cnt;
  }
  return wave_min(d);
}

template <typename TIn, bool VEC>
__device__ __forceinline__ void chunk_phase(const SampleArgs& a, int row, int c, ChunkLds& cm) {
  using G = SGeo<TIn>;
  // the chunk's loads go out first: the row's parameters arrive meanwhile
  const int c0 = c * G::CH;
  const TIn* x = reinterpret_cast<const TIn*>(a.logits) + (int64_t)row * a.ld;
  Toks<TIn> tk;
  load_toks<TIn, VEC>(x, a.V, c0, tk);
  const RowParams rp = stream_row_params(a, row);
  const int mode = row_mode(rp);
  const size_t gw = ((size_t)row * a.sw.C + c) * kWaves + wave();
  if (mode == kModeGeneral) {
    publish(a, gw, -INFINITY, 0.0, 0.0, 0, 0);
    return;
  }
  int flags = 0;
  if (rp.pen_active) {
    const uint32_t pb = chunk_pen_bits<TIn>(a, rp, c0, cm);
    if (set_aside<TIn>(tk, pb, rp.pen, c0, cm)) flags |= kRecIncomplete;
  }
  const double* pz = cm.pz[wave()] + tk.po;

  if (mode == kModeGreedy) {
    const int* pt = cm.pt[wave()] + tk.po;
    TIn m = (TIn)(-INFINITY);
#pragma unroll
    for (int e = 0; e < G::EPT; ++e) m = fmax(m, tk.rv(e));
    uint32_t eq = 0u;
#pragma unroll
    for (int e = 0; e < G::EPT; ++e) eq |= tk.rv(e) == m ? 1u << e : 0u;
    ArgMax best{-INFINITY, INT_MAX};
    if (eq != 0u && m > (TIn)(-INFINITY)) best = ArgMax{(double)m, slot_tok<TIn>(c0, __builtin_ctz(eq))};
    for (int i = 0; i < tk.np; ++i) best = argmax_merge(best, ArgMax{pz[i], pt[i]});
    best = wave_argmax(best);
    publish(a, gw, best.v, 0.0, 0.0, best.i, flags);
    return;
  }

  // the lane's largest and smallest finite token
  TIn lmx = (TIn)(-INFINITY), lmn = (TIn)INFINITY;
  tk.new_pass();
#pragma unroll
  for (int e = 0; e < G::EPT; ++e) {
    const TIn v = tk.rv(e);
    lmx = fmax(lmx, v);
    lmn = fmin(lmn, v > (TIn)(-INFINITY) ? v : (TIn)INFINITY);
  }
  double zmx = (double)lmx, zmn = (double)lmn;
  for (int i = 0; i < tk.np; ++i) {
    zmx = fmax(zmx, pz[i]);
    if (pz[i] > -INFINITY) zmn = fmin(zmn, pz[i]);
  }
  const double invT = 1.0 / rp.T;
  const double* tab = cm.exp_tab[wave()];
  cm.exp_tab[wave()][lane()] = kExp2Frac64[lane()];
  const double my = uniform(wave_max(zmx) * invT);  // the segment's max y (y is monotone in z)

  // the segment's normaliser partial (temperature and top-p rows)
  double s = 0.0;
  if (mode != kModeTopK && my > -INFINITY) {
    double s0 = 0.0, s1 = 0.0;
    tk.new_pass();
#pragma unroll
    for (int e = 0; e < G::EPT; e += 2) {
      s0 += exp_neg_term(fma((double)tk.rv(e), invT, -my), tab);
      s1 += exp_neg_term(fma((double)tk.rv(e + 1), invT, -my), tab);
      // each pair of terms is complete here: the table loads of later
      // tokens are not hoisted (they would be held as 64-bit registers)
      asm volatile("" : "+v"(s0), "+v"(s1));
    }
    for (int i = 0; i < tk.np; ++i) s0 += exp_neg_term(fma(pz[i], invT, -my), tab);
    s = wave_sum(s0 + s1);
  }
  if (mode == kModeTemp) {
    publish(a, gw, my, s, 0.0, 0, flags);
    return;
  }

  // ---- top-k and top-p: theta, at or below the chunk's target-th largest
  // token, so that every token >= theta is a candidate and every other one
  // is below theta.  Top-k (k <= 512): the k-th largest of the 512
  // per-thread maxima (a subset of the chunk's tokens); top-p: the bin of a
  // value histogram (every VW-th token, counted VW times) where the count
  // from the top reaches the chunk's candidate target.
  for (int b = threadIdx.x; b < kNB; b += kThreads) cm.hist[b] = 0u;
  const bool fin = zmx > -INFINITY;
  double lo, hi;
  int nf;
  {
    double l = mode == kModeTopK ? (fin ? zmx : INFINITY) : zmn;
    l = wave_min(l);
    const double h = wave_max(zmx);
    const int n1 = wave_sum(fin ? 1 : 0);
    if (lane() == 0) {
      cm.red[wave()] = l;
      cm.red[kWaves + wave()] = h;
      cm.redi[wave()] = n1;
    }
  }
  wg_barrier();
  lo = cm.red[0];
  hi = cm.red[kWaves];
  nf = cm.redi[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) {
    lo = fmin(lo, cm.red[w]);
    hi = fmax(hi, cm.red[kWaves + w]);
    nf += cm.redi[w];
  }
  lo = uniform(lo);
  hi = uniform(hi);
  nf = uniform(nf);
  double theta = -INFINITY;
  if (mode == kModeTopK) {
    const Affine af = make_affine(lo, hi, kNB);
    if (fin) lds_add(&cm.hist[kNB - 1 - af.bin(zmx)], 1u);  // bin 0 = highest
    wg_barrier();
    if (nf >= rp.top_k) {
      const int d = hist_reach(cm, (uint32_t)rp.top_k);
      const int ab = kNB - 1 - d;  // ascending bin of the k-th largest maximum
      // every z with af.bin(z) >= ab is >= lo + (ab - 0.01) / scale
      theta = (ab > 0 && af.scale > 0.0) ? lo + ((double)ab - 0.01) / af.scale : lo;
    }
  } else {
    // bins over [max(lo, hi - 40 T), hi] in z, affine; tokens further down
    // (each below e^-40 of the max) share the lowest bin
    const double span = fmin(hi - lo, kRangeY * rp.T);
    const Affine af = make_affine(hi - span, hi, kNB);
    const HBin<TIn> rf(af);
    if (hi > -INFINITY) {
      tk.new_pass();
#pragma unroll
      for (int j = 0; j < kUL; ++j) {
        const TIn v = tk.rv(j * G::VW);
        if (v > (TIn)(-INFINITY)) lds_add(&cm.hist[kNB - 1 - rf.bin(v)], (uint32_t)G::VW);
      }
      for (int i = 0; i < tk.np; ++i)
        if (pz[i] > -INFINITY) lds_add(&cm.hist[kNB - 1 - af.bin(pz[i])], 1u);
    }
    wg_barrier();
    const int d = hist_reach(cm, (uint32_t)a.sw.ncand);
    if (d != INT_MAX) {
      const int ab = kNB - 1 - d;
      theta = (ab > 0 && rf.scale() > 0.0) ? rf.lo() + ((double)ab - 0.01) / rf.scale() : rf.lo();
    }
  }
  theta = uniform(theta);
  const TIn tin = in_thr<TIn>(theta);
  uint32_t pm = 0u;
  for (int i = 0; i < tk.np; ++i)
    if (pz[i] > -INFINITY && pz[i] >= theta) pm |= 1u << i;
  tk.new_pass();
  const int n = write_cands<TIn>(tk, [&](int, TIn v) { return v >= tin && v > (TIn)(-INFINITY); }, pm, c0, a, gw, cm);
  if (n < 0) flags |= kRecOverflow;
  publish(a, gw, mode == kModeTopK ? wave_max(zmx) : my, s, theta, n < 0 ? 0 : n, flags);
}

// ================================================================ merges

struct RowRec {  // the merge thread's record (segment threadIdx.x of the row), if any
  double m, s, a;
  int n, flags;
};

__device__ __forceinline__ RowRec load_rec(const SampleArgs& a, int row, int nseg) {
  RowRec r{-INFINITY, 0.0, -INFINITY, 0, 0};
  const int t = threadIdx.x;
  if (t < nseg) {
    const WaveRec* p = a.sw.rec + (size_t)row * nseg + t;
    r.m = p->m;
    r.s = p->s;
    r.a = p->a;
    r.n = p->n;
    r.flags = p->flags;
  }
  return r;
}

// A row's candidates in a merge: entry s of thread t is candidate
// j = t + s * kThreads (in segment order, each segment's slots in order);
// only their 64-bit keys stay in registers, the rest is read back from the
// workspace by candidate number.
struct Cands {
  uint64_t key[kCPT];
  uint32_t act;  // bit s: entry s takes part in the current selection
};

// Workspace slot of candidate j (ml.segoff: the segments' exclusive prefix
// of candidate counts).
__device__ __forceinline__ size_t cand_slot(const MergeLds& ml, int row, int nseg, int j) {
  int lo = 0, hi = nseg - 1;  // the last segment g with segoff[g] <= j
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (ml.segoff[mid] <= j) lo = mid;
    else hi = mid - 1;
  }
  return ((size_t)row * nseg + lo) * kCapW + (size_t)(j - ml.segoff[lo]);
}

// Candidate j's token id and penalised logit z.
template <typename TIn>
__device__ __forceinline__ int cand_z(const SampleArgs& a, int row, double pen, size_t slot, double* z) {
  const uint32_t id = (uint32_t)a.sw.cidx[slot];
  const int tok = (int)(id & ~kPenBit);
  if (id & kPenBit) {
    const TIn* x = reinterpret_cast<const TIn*>(a.logits) + (int64_t)row * a.ld;
    *z = penalize((double)x[tok], pen);
  } else {
    *z = (double)reinterpret_cast<const TIn*>(a.sw.cval)[slot];
  }
  return tok;
}

struct SelOut {
  bool found;
  uint64_t key;     // the selected entry's key and token id
  int idx;
  uint64_t before;  // running total before it (from `above`)
};

// Among the active entries, ordered by (key descending, token id
// ascending), the entry at which the running total (entries counted, or
// for MASS their fixed-point weights: the key is a probability's bits),
// starting at `above`, first reaches `target`.  Levels of kMB bins of 2^sh
// consecutive keys narrow the active set (one barrier each: kMBuf rotating
// histograms, each zeroed two levels ahead) until at most kFinal entries
// remain, whose token ids are read and which every wave ranks directly.
// found == false with key 0: the active total is below target; with key
// ~0: undecided (more than kFinal entries share one key).  Deactivates
// every entry outside the final bin.
template <bool MASS>
__device__ __forceinline__ SelOut select_desc(Cands& cd, const SampleArgs& a, int row, int nseg, uint64_t above, uint64_t target,
                              MergeLds& ml, int& hg) {
  auto wgt = [&](int s) -> uint64_t { return MASS ? to_fx(__builtin_bit_cast(double, cd.key[s])) : 1ull; };
  uint64_t kmin = ~0ull, kmax = 0ull;
  int na = 0;
#pragma unroll
  for (int s = 0; s < kCPT; ++s)
    if ((cd.act >> s) & 1u) {
      kmin = min(kmin, cd.key[s]);
      kmax = max(kmax, cd.key[s]);
      ++na;
    }
  kmin = wave_min(kmin);
  kmax = wave_max(kmax);
  na = wave_sum(na);
  if (lane() == 0) {
    ml.redu[wave()] = kmin;
    ml.redu[kWaves + wave()] = kmax;
    ml.redi[wave()] = na;
  }
  wg_barrier();
  kmin = ml.redu[0];
  kmax = ml.redu[kWaves];
  na = ml.redi[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) {
    kmin = min(kmin, ml.redu[w]);
    kmax = max(kmax, ml.redu[kWaves + w]);
    na += ml.redi[w];
  }
  wg_barrier();  // the reduction slots are reused below
  kmin = uniform(kmin);
  kmax = uniform(kmax);
  na = uniform(na);
  SelOut out{false, 0, 0, above};
  if (na == 0) return out;
  for (int level = 0; level < 8 && na > kFinal; ++level) {
    const uint64_t spanm1 = kmax - kmin;
    int sh = 0;
    while ((spanm1 >> sh) >= (uint64_t)kMB) ++sh;
    const int cur = hg % kMBuf, nxt = (hg + 1) % kMBuf;
    ++hg;
    for (int b = threadIdx.x; b < kMB; b += kThreads) {
      ml.cnt[nxt][b] = 0u;
      ml.mass[nxt][b] = 0ull;
    }
#pragma unroll
    for (int s = 0; s < kCPT; ++s)
      if ((cd.act >> s) & 1u) {
        const int b = (int)((cd.key[s] - kmin) >> sh);
        lds_add(&ml.cnt[cur][b], 1u);
        if (MASS) lds_add(&ml.mass[cur][b], wgt(s));
      }
    wg_barrier();
    // each wave: the bins from the highest down, the first where the
    // running total reaches target
    constexpr int PL = kMB / kWave;
    auto binv = [&](int i) -> uint64_t {
      const int b = kMB - 1 - (lane() * PL + i);
      return MASS ? ml.mass[cur][b] : (uint64_t)ml.cnt[cur][b];
    };
    uint64_t sum = 0;
#pragma unroll 1
    for (int i = 0; i < PL; ++i) sum += binv(i);
    const uint64_t inc = wave_scan_incl<uint64_t>(sum, 0, OpAdd{});
    const uint64_t tot = lane_value(inc, kWave - 1);
    if (above + tot < target) {
      out.before = above + tot;
      return out;
    }
    uint64_t run = above + inc - sum, bef = 0;
    int d = INT_MAX;
#pragma unroll 1
    for (int i = 0; i < PL; ++i) {
      const uint64_t v = binv(i);
      if (d == INT_MAX && run + v >= target) {
        d = kMB - 1 - (lane() * PL + i);
        bef = run;
      }
      run += v;
    }
    const int dl = __builtin_ctzll(__ballot(d != INT_MAX) | (1ull << 63));
    d = lane_value(d, dl);
    above = lane_value(bef, dl);
    na = (int)ml.cnt[cur][d];
#pragma unroll
    for (int s = 0; s < kCPT; ++s)
      if (((cd.act >> s) & 1u) && (int)((cd.key[s] - kmin) >> sh) != d) cd.act &= ~(1u << s);
    kmin = kmin + ((uint64_t)d << sh);
    kmax = min(kmax, kmin + ((1ull << sh) - 1));
    if (sh == 0) break;  // one key: ties ranked by token id below
  }
  // final: gather the remaining entries with their token ids and rank them
  if (threadIdx.x == 0) ml.fn = 0;
  wg_barrier();
#pragma unroll
  for (int s = 0; s < kCPT; ++s)
    if ((cd.act >> s) & 1u) {
      const int slot = lds_fetch_add(&ml.fn, 1);
      if (slot < kFinal) {
        ml.fkey[slot] = cd.key[s];
        ml.fw[slot] = wgt(s);
        const int j = (int)threadIdx.x + s * kThreads;
        ml.fidx[slot] = (int)((uint32_t)a.sw.cidx[cand_slot(ml, row, nseg, j)] & ~kPenBit);
      }
    }
  wg_barrier();
  const int fn = ml.fn;
  if (fn > kFinal || fn != na) {
    out.key = ~0ull;
    return out;
  }
  uint64_t ahead = 0;
  const bool mine = lane() < fn;
  const uint64_t ki = mine ? ml.fkey[lane()] : 0ull;
  const int ii = mine ? ml.fidx[lane()] : INT_MAX;
  for (int j = 0; j < fn; ++j) {
    const uint64_t kj = ml.fkey[j];
    const int ij = ml.fidx[j];
    if (kj > ki || (kj == ki && ij < ii)) ahead += ml.fw[j];
  }
  const uint64_t wi = mine ? ml.fw[lane()] : 0ull;
  const bool hit = mine && above + ahead < target && above + ahead + wi >= target;
  const uint64_t hb = __ballot(hit);
  if (hb == 0ull) {
    const uint64_t ftot = wave_sum(wi);
    out.key = above + ftot < target ? 0ull : ~0ull;
    out.before = above + ftot;
    return out;
  }
  const int hl = __builtin_ctzll(hb);
  out.found = true;
  out.key = lane_value(ki, hl);
  out.idx = lane_value(ii, hl);
  out.before = lane_value(above + ahead, hl);
  return out;
}

// p(z) = exp(z / T - M) / S of a top-p row, with z / T - M as one fused
// multiply-add.  Every place that compares or sums these probabilities
// calls this one function, so they agree to the last bit (separately
// written expressions may be contracted differently by the compiler).
__device__ __forceinline__ double p_of_z(double z, double invT, double M, double S, const double* tab) {
  return fast_exp_neg(fma(z, invT, -M), tab) / S;
}

// (key, id) at or ahead of (ck, ci) in (key desc, id asc) order.
__device__ __forceinline__ bool at_or_ahead(uint64_t k, int i, uint64_t ck, int ci) {
  return k > ck || (k == ck && i <= ci);
}

// Draw inside one segment from candidates g's slots: keep(z, id) returns
// the candidate's fixed-point weight if it is kept, else 0; the token at
// which the running mass (from `prefix`, in vocabulary order) first
// exceeds target, the last kept one if rounding leaves it unreached.
template <typename TIn, class KW>
__device__ __forceinline__ int draw_in_segment(const SampleArgs& a, int row, int nseg, int g, int n, double pen, uint64_t prefix,
                               uint64_t target, const KW& keep, MergeLds& ml) {
  const int t = threadIdx.x;
  int my_id = INT_MAX;
  uint64_t my_w = 0;
  if (t < n) {
    const size_t slot = ((size_t)row * nseg + g) * kCapW + t;
    double z;
    my_id = cand_z<TIn>(a, row, pen, slot, &z);
    my_w = keep(z, my_id);
    ml.iscan[t] = my_id;
  }
  wg_barrier();
  // sorted by token id: entry t's rank is the number of smaller ids
  int rank = 0;
  if (t < n)
    for (int j = 0; j < n; ++j) rank += ml.iscan[j] < my_id ? 1 : 0;
  wg_barrier();
  if (t < n) {
    ml.iscan[rank] = my_id;
    ml.uscan[rank] = my_w;
  }
  wg_barrier();
  int found = INT_MAX, last = INT_MAX;
  uint64_t run = prefix;
  for (int base = 0; base < n; base += kWave) {
    const int j = base + lane();
    const uint64_t w = j < n ? ml.uscan[j] : 0ull;
    const uint64_t inc = wave_scan_incl<uint64_t>(w, 0, OpAdd{});
    const uint64_t hb = __ballot(j < n && w > 0ull && run + inc > target);
    if (hb != 0ull) {
      found = ml.iscan[base + __builtin_ctzll(hb)];
      break;
    }
    const uint64_t pos = __ballot(j < n && w > 0ull);
    if (pos != 0ull) last = ml.iscan[base + 63 - __builtin_clzll(pos)];
    run += lane_value(inc, kWave - 1);
  }
  return found != INT_MAX ? found : last;
}

// Draw inside one segment of a temperature row by rescanning its tokens
// from HBM (4 per thread), float64 weights exp(y - M) running from
// `prefix` in vocabulary order: the first token whose running weight
// exceeds target, else the last token of positive weight.
template <typename TIn>
__device__ __forceinline__ int draw_rescan_temp(const SampleArgs& a, const RowParams& rp, int row, int t0, int t1, double prefix,
                                double target, double invT, double M, const double* tab, MergeLds& ml) {
  const int ntok = t1 - t0;
  const bool pen = rp.pen_active;
  if (pen) {
    for (int w = threadIdx.x; w < kMaxSeg / 32; w += kThreads) ml.segbits[w] = 0u;
    wg_barrier();
    for (int64_t h = rp.h0 + threadIdx.x; h < rp.h1; h += kThreads) {
      const int off = a.hist_ids[h] - t0;
      if ((unsigned)off < (unsigned)ntok) lds_or(&ml.segbits[off >> 5], 1u << (off & 31));
    }
    wg_barrier();
  }
  const TIn* x = reinterpret_cast<const TIn*>(a.logits) + (int64_t)row * a.ld;
  constexpr int PT = 4;
  double w[PT], ts = 0.0;
#pragma unroll
  for (int k = 0; k < PT; ++k) {
    const int o = (int)threadIdx.x * PT + k;
    w[k] = 0.0;
    if (o < ntok) {
      double z = (double)x[t0 + o];
      if (pen && ((ml.segbits[o >> 5] >> (o & 31)) & 1u)) z = penalize(z, rp.pen);
      w[k] = fast_exp_neg(fma(z, invT, -M), tab);
    }
    ts += w[k];
  }
  // float64 scan in thread order (a fixed order: deterministic)
  const double inc = wave_scan_incl(ts, 0.0, OpAdd{});
  if (lane() == kWave - 1) ml.redd[wave()] = inc;
  wg_barrier();
  double pre = 0.0;
#pragma unroll
  for (int v = 0; v < kWaves; ++v)
    if (v < wave()) pre += ml.redd[v];
  wg_barrier();
  double run = prefix + pre + (inc - ts);
  int f = INT_MAX, last = -1;
#pragma unroll
  for (int k = 0; k < PT; ++k) {
    run += w[k];
    if (f == INT_MAX && w[k] > 0.0 && run > target) f = t0 + (int)threadIdx.x * PT + k;
    if (w[k] > 0.0) last = t0 + (int)threadIdx.x * PT + k;
  }
  f = block_min<int>(f, ml.redi);
  if (f != INT_MAX) return f;
  last = block_max<int>(last, ml.redi);
  return last >= 0 ? last : t1 - 1;
}

template <typename TIn, bool VEC>
__device__ __forceinline__ void merge_general(const SampleArgs& a, int row, const RowParams& rp, MergeSmem& sm) {
  uint32_t* bits = a.sw.gbits + (size_t)row * a.sw.gwords;
  if (rp.pen_active) build_bitmap_global(bits, a.V, a.hist_ids, rp.h0, rp.h1);
  const TIn* x = reinterpret_cast<const TIn*>(a.logits) + (int64_t)row * a.ld;
  // 8 tokens per thread per group: the pipeline then fits the streaming
  // kernel's register budget (it is the rare path)
  RowSource<TIn, VEC, true, 8> src{x, a.V, bits, rp.pen_active, rp.pen};
  const int id = row_pipeline(src, rp, a.V, PipeIn{false, 0.0, false, 0.0, false, 0.0}, sm.g, nullptr);
  if (threadIdx.x == 0) {
    a.out_ids[row] = id;
    if (a.fallback_rows != nullptr) glb_add(a.fallback_rows, 1ull);
  }
}

template <typename TIn, bool VEC>
__device__ __forceinline__ void merge_phase(const SampleArgs& a, int row, MergeSmem& sm) {
  using G = SGeo<TIn>;
  MergeLds& ml = sm.m;
  const int C = a.sw.C;
  const int nseg = C * kWaves;
  // the records and the row's parameters are loaded together
  const RowRec r = load_rec(a, row, nseg);
  const RowParams rp = stream_row_params(a, row);
  const int mode = row_mode(rp);
  if (mode == kModeGeneral) {
    merge_general<TIn, VEC>(a, row, rp, sm);
    return;
  }
  if (threadIdx.x < 64) ml.exp_tab[threadIdx.x] = kExp2Frac64[threadIdx.x];
  // a segment flagged (or a count no wave can have written): the row needs
  // the general pipeline
  const bool cand_mode = mode == kModeTopK || mode == kModeTopP;
  const int bad = block_max<int>(r.flags != 0 || (cand_mode && (r.n < 0 || r.n > kCapW)) ? 1 : 0, ml.redi);
  if (bad != 0) {
    merge_general<TIn, VEC>(a, row, rp, sm);
    return;
  }
  const int t = threadIdx.x;
  const bool has = t < nseg;

  if (mode == kModeGreedy) {
    const ArgMax best = block_argmax(has ? ArgMax{r.m, r.n} : ArgMax{-INFINITY, INT_MAX}, ml.redd, ml.redi);
    if (t == 0) a.out_ids[row] = best.i == INT_MAX ? 0 : best.i;
    return;
  }

  const double invT = 1.0 / rp.T;
  const double* tab = ml.exp_tab;
  double M = -INFINITY, S = 0.0;
  if (mode != kModeTopK) {
    // the full-vocabulary normaliser from the segment partials (sampling.py:79-81)
    M = block_max<double>(has ? r.m : -INFINITY, ml.redd);
  }

  if (mode == kModeTemp) {
    const double seg = (has && r.m > -INFINITY) ? r.s * fast_exp_neg(r.m - M, tab) : 0.0;
    // running totals of the segments in vocabulary order (thread order)
    const double inc = wave_scan_incl(seg, 0.0, OpAdd{});
    if (lane() == kWave - 1) ml.redd[wave()] = inc;
    wg_barrier();
    double pre = 0.0, St = 0.0;
#pragma unroll
    for (int v = 0; v < kWaves; ++v) {
      const double sv = ml.redd[v];
      if (v < wave()) pre += sv;
      St += sv;
    }
    wg_barrier();
    const double ex = pre + (inc - seg);
    const double target = rp.u * St;  // sampling.py:98: u * c[-1]
    const bool hit = has && seg > 0.0 && ex + seg > target;
    int g = block_min<int>(hit ? t : INT_MAX, ml.redi);
    if (g == INT_MAX) {  // rounding past the end: the last segment of positive mass
      g = block_max<int>(has && seg > 0.0 ? t : -1, ml.redi);
      if (g < 0) g = nseg - 1;
    }
    if (t == g) ml.ctld[0] = ex;
    wg_barrier();
    const double gpre = ml.ctld[0];
    wg_barrier();
    const int t0 = g * G::SEG, t1 = min(a.V, t0 + G::SEG);
    const int id = draw_rescan_temp<TIn>(a, rp, row, t0, t1, gpre, target, invT, M, tab, ml);
    if (t == 0) a.out_ids[row] = id;
    return;
  }

  // ---- candidate rows: counts and offsets
  const int cntv = has ? r.n : 0;
  uint64_t ntot64;
  const uint64_t off = block_excl_scan<uint64_t>((uint64_t)cntv, ml.redu, &ntot64);
  const int ntot = (int)ntot64;
  if (has) ml.segoff[t] = (int)off;
  if (t == 0) ml.segoff[nseg] = ntot;
  for (int b = t; b < kMB; b += kThreads) {
    ml.cnt[0][b] = 0u;
    ml.mass[0][b] = 0ull;
    ml.cnt[1][b] = 0u;
    ml.mass[1][b] = 0ull;
  }
  if (mode == kModeTopP) {
    // S (one barrier round, a fixed order)
    const double Sv = wave_sum((has && r.m > -INFINITY) ? r.s * fast_exp_neg(r.m - M, tab) : 0.0);
    if (lane() == 0) ml.redd[kWaves + wave()] = Sv;
  }
  wg_barrier();
  if (mode == kModeTopP) {
#pragma unroll
    for (int v = 0; v < kWaves; ++v) S += ml.redd[kWaves + v];
  }
  if (ntot > kCandMax || ntot == 0) {
    merge_general<TIn, VEC>(a, row, rp, sm);
    return;
  }
  // candidate keys: top-k orders y = z / T (sampling.py:75); top-p the
  // probabilities exp(y - M) / S (:80-81)
  Cands cd;
  cd.act = 0u;
  {
    int g = 0;
#pragma unroll
    for (int s = 0; s < kCPT; ++s) {
      const int j = t + s * kThreads;
      cd.key[s] = 0ull;
      if (j < ntot) {
        while (g + 1 < nseg && ml.segoff[g + 1] <= j) ++g;
        const size_t slot = ((size_t)row * nseg + g) * kCapW + (size_t)(j - ml.segoff[g]);
        double z;
        (void)cand_z<TIn>(a, row, rp.pen, slot, &z);
        cd.key[s] = mode == kModeTopK ? key_of(z / rp.T) : pkey_of(p_of_z(z, invT, M, S, tab));
        cd.act |= 1u << s;
      }
    }
  }
  const uint32_t all = cd.act;
  int hg = 0;
  uint64_t kthk = 0;
  double ymax = 0.0, SK = 0.0;
  if (mode == kModeTopK) {
    const SelOut kth = select_desc<false>(cd, a, row, nseg, 0, (uint64_t)rp.top_k, ml, hg);
    cd.act = all;
    if (!kth.found && kth.key != 0ull) {  // undecided (ties beyond the final stage)
      merge_general<TIn, VEC>(a, row, rp, sm);
      return;
    }
    // the candidates hold every token >= kth: each chunk's other tokens are
    // below its theta, which must map strictly below kth's y
    const double kth_y = kth.found ? val_of_key(kth.key) : -INFINITY;
    const bool ok_here = !has || !(r.a > -INFINITY) || !kth.found || (r.a / rp.T < kth_y);
    if (block_min<int>(ok_here ? 1 : 0, ml.redi) == 0) {
      merge_general<TIn, VEC>(a, row, rp, sm);
      return;
    }
    // kept: y >= kth (every candidate when the row has fewer than k finite tokens)
    kthk = kth.found ? kth.key : 0ull;
#pragma unroll
    for (int s = 0; s < kCPT; ++s)
      if (((cd.act >> s) & 1u) && cd.key[s] < kthk) cd.act &= ~(1u << s);
    // softmax over the kept set (sampling.py:79-81)
    uint64_t kmx = 0;
#pragma unroll
    for (int s = 0; s < kCPT; ++s)
      if ((cd.act >> s) & 1u) kmx = max(kmx, cd.key[s]);
    ymax = val_of_key(block_max<uint64_t>(kmx, ml.redu));
    double es = 0.0;
#pragma unroll
    for (int s = 0; s < kCPT; ++s)
      if ((cd.act >> s) & 1u) es += fast_exp_neg(val_of_key(cd.key[s]) - ymax, tab);
    SK = block_sum<double>(es, ml.redd);
#pragma unroll
    for (int s = 0; s < kCPT; ++s)
      if ((cd.act >> s) & 1u) cd.key[s] = pkey_of(fast_exp_neg(val_of_key(cd.key[s]) - ymax, tab) / SK);
  }
  const uint32_t kept1 = cd.act;

  // ---- top-p cut over the kept candidates (sampling.py:82-90)
  uint64_t cut_key = 0;
  int cut_idx = 0;
  const bool cut = rp.topp;
  if (cut) {
    const SelOut sel = select_desc<true>(cd, a, row, nseg, 0, topp_target(rp.top_p), ml, hg);
    cd.act = kept1;
    if (!sel.found) {
      merge_general<TIn, VEC>(a, row, rp, sm);
      return;
    }
    cut_key = sel.key;
    cut_idx = sel.idx;
    if (mode == kModeTopP) {
      // every token of the row at or ahead of the cut must be a candidate:
      // each chunk's other tokens are below its theta, so theta <= z of the
      // cut token suffices (then they are below the cut's z)
      const TIn* x = reinterpret_cast<const TIn*>(a.logits) + (int64_t)row * a.ld;
      double zc = (double)x[cut_idx];
      bool penc = false;
      if (rp.pen_active)
        for (int64_t h = rp.h0 + t; h < rp.h1; h += kThreads)
          if (a.hist_ids[h] == cut_idx) penc = true;
      penc = block_max<int>(penc ? 1 : 0, ml.redi) != 0;
      if (penc) zc = penalize(zc, rp.pen);
      const bool ok_here = !has || r.a <= zc;
      if (block_min<int>(ok_here ? 1 : 0, ml.redi) == 0) {
        merge_general<TIn, VEC>(a, row, rp, sm);
        return;
      }
    }
  }

  // ---- draw in vocabulary order (sampling.py:94-98): the kept mass of each
  // segment, the segment where the running mass crosses floor(u * total),
  // then that segment's kept candidates in token order
  for (int g = t; g < nseg; g += kThreads) ml.segm[g] = 0ull;
  wg_barrier();
  {
    int g = 0;
#pragma unroll
    for (int s = 0; s < kCPT; ++s) {
      const int j = t + s * kThreads;
      if ((cd.act >> s) & 1u) {
        while (g + 1 < nseg && ml.segoff[g + 1] <= j) ++g;
        bool keep = true;
        if (cut) {
          int id = INT_MAX;
          if (cd.key[s] == cut_key)  // ties at the cut are ranked by token id
            id = (int)((uint32_t)a.sw.cidx[((size_t)row * nseg + g) * kCapW + (j - ml.segoff[g])] & ~kPenBit);
          keep = cd.key[s] > cut_key || (cd.key[s] == cut_key && id <= cut_idx);
        }
        if (keep) lds_add(&ml.segm[g], to_fx(__builtin_bit_cast(double, cd.key[s])));
      }
    }
  }
  wg_barrier();
  const uint64_t segv = has ? ml.segm[t] : 0ull;
  uint64_t total;
  const uint64_t ex = block_excl_scan<uint64_t>(segv, ml.redu, &total);
  const uint64_t target = (uint64_t)__double2ull_rd(rp.u * (double)total);
  const bool hit = has && segv > 0 && ex + segv > target;
  int g = block_min<int>(hit ? t : INT_MAX, ml.redi);
  if (g == INT_MAX) g = block_max<int>(has && segv > 0 ? t : -1, ml.redi);
  if (g < 0) g = 0;
  if (t == g) ml.ctlu[0] = ex;
  wg_barrier();
  const uint64_t gpre = ml.ctlu[0];
  const int gn = ml.segoff[g + 1] - ml.segoff[g];
  wg_barrier();
  const double T = rp.T;
  const int id = draw_in_segment<TIn>(
      a, row, nseg, g, gn, rp.pen, gpre, target,
      [&](double z, int tok) -> uint64_t {
        double p;
        if (mode == kModeTopK) {
          const uint64_t k1 = key_of(z / T);
          if (k1 < kthk) return 0ull;
          p = fast_exp_neg(val_of_key(k1) - ymax, tab) / SK;
        } else {
          p = p_of_z(z, invT, M, S, tab);
        }
        if (cut && !at_or_ahead(pkey_of(p), tok, cut_key, cut_idx)) return 0ull;
        return to_fx(p);
      },
      ml);
  if (t == 0) a.out_ids[row] = id;
}

// Grid B * C: block b is chunk b % C of row b / C.
template <typename TIn, bool VEC>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4))) void k_stream_chunks(SampleArgs a) {
  __shared__ ChunkLds sm;
  const int row = (int)blockIdx.x / a.sw.C;
  chunk_phase<TIn, VEC>(a, row, (int)blockIdx.x - row * a.sw.C, sm);
}

// Grid B: block b merges row b.
template <typename TIn, bool VEC>
__global__ __launch_bounds__(kThreads) void k_stream_merge(SampleArgs a) {
  __shared__ MergeSmem sm;
  merge_phase<TIn, VEC>(a, (int)blockIdx.x, sm);
}

size_t up256s(size_t v) { return (v + 255) & ~(size_t)255; }

}  // namespace

int stream_chunk_tokens(bool f64) { return f64 ? SGeo<double>::CH : SGeo<float>::CH; }

size_t stream_ws_bytes(int B, int V, bool f64) {
  const int CH = stream_chunk_tokens(f64);
  const size_t C = (size_t)((V + CH - 1) / CH);
  const size_t nseg = (size_t)B * C * kWaves;
  const size_t nslot = nseg * kCapW;
  const size_t gwords = (size_t)((V + 31) / 32);
  return up256s(nseg * sizeof(WaveRec)) + up256s(nslot * (f64 ? 8 : 4)) + up256s(nslot * 4) +
         up256s((size_t)B * gwords * 4);
}

StreamWs stream_ws_layout(void* ws, int B, int V, bool f64) {
  StreamWs w{};
  const int CH = stream_chunk_tokens(f64);
  w.C = (V + CH - 1) / CH;
  const size_t nseg = (size_t)B * w.C * kWaves;
  const size_t nslot = nseg * kCapW;
  w.gwords = (V + 31) / 32;
  char* p = static_cast<char*>(ws);
  w.rec = reinterpret_cast<WaveRec*>(p);
  p += up256s(nseg * sizeof(WaveRec));
  w.cval = p;
  p += up256s(nslot * (f64 ? 8 : 4));
  w.cidx = reinterpret_cast<int32_t*>(p);
  p += up256s(nslot * 4);
  w.gbits = reinterpret_cast<uint32_t*>(p);
  // top-p rows: the candidates one chunk keeps, within both the merge's
  // register capacity and the chunk's slots
  // (the histogram counts every VW-th token: the chunk's actual count can
  // exceed the target by a few percent)
  w.ncand = min((int)(0.85 * kCandMax / w.C), (int)(0.6 * kWaves * kCapW));
  return w;
}

hipError_t launch_sample_stream(const SampleArgs& a, bool f64, bool vec, hipStream_t s, hipEvent_t between) {
  const dim3 gc(a.B * a.sw.C), gm(a.B), block(kThreads);
  if (f64) {
    if (vec) hipLaunchKernelGGL((k_stream_chunks<double, true>), gc, block, 0, s, a);
    else hipLaunchKernelGGL((k_stream_chunks<double, false>), gc, block, 0, s, a);
  } else {
    if (vec) hipLaunchKernelGGL((k_stream_chunks<float, true>), gc, block, 0, s, a);
    else hipLaunchKernelGGL((k_stream_chunks<float, false>), gc, block, 0, s, a);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (between != nullptr) {
    e = hipEventRecord(between, s);
    if (e != hipSuccess) return e;
  }
  if (f64) {
    if (vec) hipLaunchKernelGGL((k_stream_merge<double, true>), gm, block, 0, s, a);
    else hipLaunchKernelGGL((k_stream_merge<double, false>), gm, block, 0, s, a);
  } else {
    if (vec) hipLaunchKernelGGL((k_stream_merge<float, true>), gm, block, 0, s, a);
    else hipLaunchKernelGGL((k_stream_merge<float, false>), gm, block, 0, s, a);
  }
  return hipGetLastError();
}

}  // namespace plh
