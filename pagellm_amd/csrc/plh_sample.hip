// gfx950 kernels for the batched sampler (src/pagellm/engine/sampling.py:52-111).
//
//   k_sample_fast   one 512-thread workgroup per row, one pass over HBM.
//                   The row streams through registers with 16-byte
//                   non-temporal loads, one iteration (16384 tokens) ahead.
//                   Per row mode:
//                     greedy       argmax of the penalised logits;
//                     temperature  per-wave segment softmax partials, then
//                                  one 2048-token segment is rescanned for
//                                  the inverse-CDF draw;
//                     top-k        candidates >= a running lower bound of the
//                                  k-th largest, kept in LDS;
//                     top-p        segment partials for the normaliser plus
//                                  the largest tokens (a projected count) in
//                                  LDS.
//                   Selection inside LDS uses value-range histograms and
//                   small bitonic sorts; the draw is an exact fixed-point
//                   search in vocabulary order.  A row the candidates cannot
//                   decide exactly is finished by the general pipeline in
//                   the same workgroup.
//   k_sample_rows   the general pipeline for every row (and the only kernel
//                   that exports the processed distribution, probs()).
//   k_draw          inverse-CDF draw from given distributions (draw()).
//   k_penalize      repetition penalty on a copy (apply_repetition_penalty()).
#include "plh_fast.h"
#include "plh_kernels.h"
#include "plh_pipeline.h"

namespace plh {

constexpr int kU = 8;                              // 16-byte loads per thread per iteration
constexpr int kE = 4 * kU;                         // tokens per thread per iteration
constexpr int kSegLen = kE * kWave;                // 2048: one wave's contiguous share of an iteration
constexpr int kIterLen = kSegLen * kWaves;         // 16384 tokens per iteration
constexpr int kMaxSegs = kMaxVBitmap / kSegLen;    // 128
constexpr int kHB = 1024;                          // histogram bins
constexpr int kSortMax = 2048;                     // LDS sort list
constexpr int kCandBytes = 80 * 1024;              // candidate store
constexpr int kSelLevels = 4;

enum RowMode { kGreedy = 0, kTemp = 1, kTopK = 2, kTopP = 3 };

struct SortList {
  uint64_t key[kSortMax];
  uint64_t w[kSortMax];
  int idx[kSortMax];
};

struct FastSmem {
  double redd[kWaves];
  uint64_t redu[kWaves];
  int redi[kWaves];
  int ctl[8];
  uint64_t ctlu[4];
  double exp_tab[64];
  double seg_m[kMaxSegs];
  double seg_s[kMaxSegs];
  uint32_t hcnt[kHB];
  uint64_t hmass[kHB];
  union {
    uint32_t bitmap[kMaxVBitmap / 32];  // while streaming
    SortList sl;                        // while finishing
  } u;
  alignas(16) unsigned char cand[kCandBytes];
  int cand_n;
};

union SmemAll {
  FastSmem f;
  Smem g;
};

template <typename TIn>
constexpr int cand_cap() {
  return kCandBytes / (int)(sizeof(TIn) + 4);
}

// Workgroup barrier ordering LDS only: global loads issued ahead of it stay
// in flight.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

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

// ------------------------------------------------------------- streaming

typedef float f4_t __attribute__((ext_vector_type(4)));
typedef double d2_t __attribute__((ext_vector_type(2)));

template <typename TIn>
struct RawIter;
template <>
struct RawIter<float> {
  f4_t v[kU];
};
template <>
struct RawIter<double> {
  d2_t v[2 * kU];
};

// Token (j, s) of the calling lane in the iteration starting at `base`:
// base + wave*2048 + j*256 + 4*lane + s.  Each load instruction of a wave
// covers 1 KB of contiguous HBM.
__device__ __forceinline__ int lane_off(int base) { return base + wave() * kSegLen + 4 * lane(); }

template <bool VEC>
__device__ __forceinline__ void load_iter(const float* x, int V, int base, RawIter<float>& r) {
  const int off = lane_off(base);
  const bool full = VEC && base + kIterLen <= V;  // uniform: no bounds checks needed
#pragma unroll
  for (int j = 0; j < kU; ++j) {
    const int p = off + j * 256;
    if (full || (VEC && p + 3 < V)) {
      r.v[j] = __builtin_nontemporal_load(reinterpret_cast<const f4_t*>(x + p));
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) r.v[j][s] = (p + s < V) ? x[p + s] : -INFINITY;
    }
  }
}

template <bool VEC>
__device__ __forceinline__ void load_iter(const double* x, int V, int base, RawIter<double>& r) {
  const int off = lane_off(base);
  const bool full = VEC && base + kIterLen <= V;
#pragma unroll
  for (int j = 0; j < kU; ++j) {
    const int p = off + j * 256;
    if (full || (VEC && p + 3 < V)) {
      r.v[2 * j] = __builtin_nontemporal_load(reinterpret_cast<const d2_t*>(x + p));
      r.v[2 * j + 1] = __builtin_nontemporal_load(reinterpret_cast<const d2_t*>(x + p + 2));
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) r.v[2 * j + (s >> 1)][s & 1] = (p + s < V) ? x[p + s] : -INFINITY;
    }
  }
}

__device__ __forceinline__ double raw_at(const RawIter<float>& r, int e) { return (double)r.v[e >> 2][e & 3]; }
__device__ __forceinline__ double raw_at(const RawIter<double>& r, int e) { return r.v[e >> 1][e & 1]; }

// Validity (bit e: token e lies inside the row) and penalty (bit e: token e
// is in the history) masks of the calling lane for the iteration at `base`.
__device__ __forceinline__ void lane_bits(int base, int V, const RowParams& rp, const uint32_t* bitmap,
                                          uint32_t* vmask, uint32_t* pbits) {
  const int off = lane_off(base);
  uint32_t m = 0, pb = 0;
#pragma unroll
  for (int e = 0; e < kE; ++e)
    if (off + (e >> 2) * 256 + (e & 3) < V) m |= 1u << e;
  if (rp.pen_active) {
#pragma unroll
    for (int j = 0; j < kU; ++j) {
      const int p = off + j * 256;
      if (p < V) pb |= ((bitmap[p >> 5] >> (p & 31)) & 0xFu) << (4 * j);
    }
  }
  *vmask = m;
  *pbits = pb;
}

// Penalised logit of register slot e.
template <typename TIn>
__device__ __forceinline__ double zat(const RawIter<TIn>& r, int e, uint32_t pbits, double pen) {
  const double v = raw_at(r, e);
  return ((pbits >> e) & 1u) ? penalize(v, pen) : v;
}

__device__ __forceinline__ int tok_idx(int base, int e) { return lane_off(base) + (e >> 2) * 256 + (e & 3); }

// y = z / T as the segment partials compute it (multiplication by 1/T).
struct YScale {
  double T, invT;
  __device__ __forceinline__ double operator()(double z) const { return T == 1.0 ? z : z * invT; }
};

// Wave-wide softmax partial of one 2048-token segment: (max y, sum exp(y - max y)).
template <typename TIn>
__device__ __forceinline__ void segment_partial(const RawIter<TIn>& r, uint32_t vmask, uint32_t pbits, double pen,
                                                const YScale& ys, const double* tab, double* seg_m, double* seg_s,
                                                int seg) {
  double m = -INFINITY;
#pragma unroll
  for (int e = 0; e < kE; ++e)
    if ((vmask >> e) & 1u) m = fmax(m, ys(zat(r, e, pbits, pen)));
  m = wave_max(m);
  double s = 0.0;
  if (m > -INFINITY) {
#pragma unroll
    for (int e = 0; e < kE; ++e)
      if ((vmask >> e) & 1u) s += fast_exp_neg(ys(zat(r, e, pbits, pen)) - m, tab);
  }
  s = wave_sum(s);
  if (lane() == 0) {
    seg_m[seg] = m;
    seg_s[seg] = s;
  }
}

// ------------------------------------------------------------- selection

// The smallest value of the histogram bin that holds the target-th largest
// of the valid finite z in registers (-inf if there are fewer than target).
template <typename TIn>
__device__ __forceinline__ double theta_from_regs(const RawIter<TIn>& r, uint32_t vmask, uint32_t pbits, double pen,
                                                  uint64_t target, FastSmem& fs) {
  double lo = INFINITY, hi = -INFINITY;
#pragma unroll
  for (int e = 0; e < kE; ++e) {
    const double z = zat(r, e, pbits, pen);
    if (((vmask >> e) & 1u) && z > -INFINITY) {
      lo = fmin(lo, z);
      hi = fmax(hi, z);
    }
  }
  lo = block_min(lo, fs.redd);
  hi = block_max(hi, fs.redd);
  if (!(hi > -INFINITY)) return -INFINITY;
  const Affine af = make_affine(lo, hi, kHB);
  for (int b = threadIdx.x; b < kHB; b += kThreads) fs.hcnt[b] = 0u;
  lds_barrier();
#pragma unroll
  for (int e = 0; e < kE; ++e) {
    const double z = zat(r, e, pbits, pen);
    if (((vmask >> e) & 1u) && z > -INFINITY) lds_add(&fs.hcnt[af.bin(z)], 1u);
  }
  lds_barrier();
  const Pick pk = pick_desc<false>(fs.hcnt, fs.hmass, kHB, 0, target, fs.redu, fs.ctl, fs.ctlu);
  if (!pk.found) return -INFINITY;
  double m = INFINITY;
#pragma unroll
  for (int e = 0; e < kE; ++e) {
    const double z = zat(r, e, pbits, pen);
    if (((vmask >> e) & 1u) && z > -INFINITY && af.bin(z) == pk.d) m = fmin(m, z);
  }
  return block_min(m, fs.redd);
}

// Candidate store: value (the input type) and index, bit 31 set when the
// token's penalty applies.
template <typename TIn>
struct Cands {
  TIn* val;
  int* code;
  int cap;
  __device__ __forceinline__ double z(int c, double pen) const {
    double v = (double)val[c];
    return code[c] < 0 ? penalize(v, pen) : v;
  }
  __device__ __forceinline__ int idx(int c) const { return code[c] & 0x7fffffff; }
};

// Keep the candidates >= the smallest value of the histogram bin holding
// the target-th largest; in-place stable compaction, one round of kThreads
// entries at a time (a kept entry only moves down, into rounds already
// read).  Returns the new threshold; *umax gets the dropped maximum.
template <typename TIn>
__device__ __forceinline__ double compact_cands(const Cands<TIn>& cs, uint64_t target, double pen, double* umax,
                                                FastSmem& fs) {
  const int n = min(fs.cand_n, cs.cap);
  double lo = INFINITY, hi = -INFINITY;
  for (int c = threadIdx.x; c < n; c += kThreads) {
    const double z = cs.z(c, pen);
    if (z > -INFINITY) {
      lo = fmin(lo, z);
      hi = fmax(hi, z);
    }
  }
  lo = block_min(lo, fs.redd);
  hi = block_max(hi, fs.redd);
  const Affine af = make_affine(lo, hi, kHB);
  for (int b = threadIdx.x; b < kHB; b += kThreads) fs.hcnt[b] = 0u;
  lds_barrier();
  for (int c = threadIdx.x; c < n; c += kThreads) {
    const double z = cs.z(c, pen);
    if (z > -INFINITY) lds_add(&fs.hcnt[af.bin(z)], 1u);
  }
  lds_barrier();
  const Pick pk = pick_desc<false>(fs.hcnt, fs.hmass, kHB, 0, target, fs.redu, fs.ctl, fs.ctlu);
  double theta = -INFINITY;
  if (pk.found) {
    double m = INFINITY;
    for (int c = threadIdx.x; c < n; c += kThreads) {
      const double z = cs.z(c, pen);
      if (z > -INFINITY && af.bin(z) == pk.d) m = fmin(m, z);
    }
    theta = block_min(m, fs.redd);
  }
  int kept = 0;
  for (int r0 = 0; r0 < n; r0 += kThreads) {
    const int c = r0 + threadIdx.x;
    TIn v = TIn(0);
    int code = 0;
    bool keep = false;
    if (c < n) {
      v = cs.val[c];
      code = cs.code[c];
      const double z = cs.z(c, pen);
      keep = z >= theta;
      if (!keep) *umax = fmax(*umax, z);
    }
    uint32_t tot;
    const uint32_t ex = block_excl_scan<uint32_t>(keep ? 1u : 0u, reinterpret_cast<uint32_t*>(fs.redu), &tot);
    if (keep) {
      cs.val[kept + ex] = v;
      cs.code[kept + ex] = code;
    }
    kept += (int)tot;
    lds_barrier();
  }
  if (threadIdx.x == 0) fs.cand_n = kept;
  lds_barrier();
  return theta;
}


// Appends the valid tokens with z >= theta (one LDS atomic per wave and
// register slot).  Tokens that find the store full count as dropped.
template <typename TIn>
__device__ __forceinline__ void insert_cands(const Cands<TIn>& cs, const RawIter<TIn>& raw, uint32_t vmask,
                                             uint32_t pbits, double pen, int base, double theta, double* umax,
                                             FastSmem& fs) {
  const int off = lane_off(base);
#pragma unroll
  for (int e = 0; e < kE; ++e) {
    const double z = zat(raw, e, pbits, pen);
    const bool valid = (vmask >> e) & 1u;
    const bool pass = valid && z >= theta;
    const uint64_t mask = __ballot(pass);
    if (mask) {
      int first = 0;
      if (lane() == 0) first = lds_fetch_add(&fs.cand_n, (int)__popcll(mask));
      first = __shfl(first, 0);
      if (pass) {
        const int slot = first + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                                                __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
        if (slot < cs.cap) {
          if constexpr (sizeof(TIn) == 4) cs.val[slot] = raw.v[e >> 2][e & 3];
          else cs.val[slot] = raw.v[e >> 1][e & 1];
          cs.code[slot] = (off + (e >> 2) * 256 + (e & 3)) | (((pbits >> e) & 1u) ? (int)0x80000000 : 0);
        } else {
          *umax = fmax(*umax, z);
        }
      }
    }
    if (valid && !pass) *umax = fmax(*umax, z);
  }
}

// Inclusive and exclusive scan of one double per thread, thread order,
// fixed association.
__device__ __forceinline__ double block_scan_d(double v, double* red, double* excl, double* total) {
  double x = v;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const double y = __shfl_up(x, off);
    if (lane() >= off) x += y;
  }
  double xe = __shfl_up(x, 1);
  if (lane() == 0) xe = 0.0;
  if (lane() == kWave - 1) red[wave()] = x;
  __syncthreads();
  double pre = 0.0, tot = 0.0;
  for (int w = 0; w < kWaves; ++w) {
    if (w < wave()) pre += red[w];
    tot += red[w];
  }
  __syncthreads();
  *excl = pre + xe;
  *total = tot;
  return pre + x;
}

// Value-range selection over the candidate store: candidates with elig(c)
// take part; val(c) places them in histogram bins (monotone in the order),
// key(c) orders them exactly, token index ascending on equal keys.
//   MASS=false: the target-th largest key;
//   MASS=true : in (key desc, index asc) order the first candidate whose
//               inclusive weight wt(c) reaches target.
// giveup: more than kSortMax candidates share one value at the cut (the
// caller falls back to the general pipeline).
struct SelOut {
  bool found;
  bool giveup;
  uint64_t key;
  int idx;
};

template <bool MASS, typename TIn, class Elig, class Val, class Key, class W>
__device__ __forceinline__ SelOut cand_select(const Cands<TIn>& cs, int n, const Elig& elig, const Val& val,
                                              const Key& key, const W& wt, uint64_t target, FastSmem& fs) {
  Affine lv[kSelLevels];
  int dv[kSelLevels];
  int levels = 0;
  uint64_t above = 0;
  auto active = [&](int c, double v) -> bool {
    if (!elig(c)) return false;
    for (int l = 0; l < levels; ++l)
      if (lv[l].bin(v) != dv[l]) return false;
    return true;
  };
  SortList& sl = fs.u.sl;
  for (;;) {
    double lo = INFINITY, hi = -INFINITY;
    uint32_t cnt = 0;
    for (int c = threadIdx.x; c < n; c += kThreads) {
      const double v = val(c);
      if (active(c, v)) {
        lo = fmin(lo, v);
        hi = fmax(hi, v);
        ++cnt;
      }
    }
    lo = block_min(lo, fs.redd);
    hi = block_max(hi, fs.redd);
    cnt = block_sum<uint32_t>(cnt, reinterpret_cast<uint32_t*>(fs.redu));
    if (cnt <= (uint32_t)kSortMax || !(hi > lo) || levels == kSelLevels) {
      if (cnt > (uint32_t)kSortMax) return SelOut{false, true, 0, 0};
      if (threadIdx.x == 0) fs.ctl[2] = 0;
      lds_barrier();
      for (int c = threadIdx.x; c < n; c += kThreads) {
        if (active(c, val(c))) {
          const int s = lds_fetch_add(&fs.ctl[2], 1);
          sl.key[s] = key(c);
          sl.idx[s] = cs.idx(c);
          sl.w[s] = MASS ? wt(c) : 0ull;
        }
      }
      lds_barrier();
      const int m = (int)cnt;
      lds_bitonic(sl.key, sl.idx, sl.w, m, 0ull, [](uint64_t ka, int ia, uint64_t kb, int ib) {
        return ka > kb || (ka == kb && ia < ib);
      });
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
    for (int c = threadIdx.x; c < n; c += kThreads) {
      const double v = val(c);
      if (active(c, v)) {
        const int b = af.bin(v);
        lds_add(&fs.hcnt[b], 1u);
        if (MASS) lds_add(&fs.hmass[b], wt(c));
      }
    }
    lds_barrier();
    const Pick pk = pick_desc<MASS>(fs.hcnt, fs.hmass, kHB, above, target, fs.redu, fs.ctl, fs.ctlu);
    if (!pk.found) return SelOut{false, false, 0, 0};
    above = pk.above;
    lv[levels] = af;
    dv[levels] = pk.d;
    ++levels;
  }
}

// Inverse-CDF draw over the kept candidates in vocabulary order
// (sampling.py:94-98): with w(c) the fixed-point probability of kept
// candidates (0 otherwise), the first token whose running mass exceeds
// floor(u * total); V-1 when none does.
template <typename TIn, class W>
__device__ __forceinline__ int draw_kept(const Cands<TIn>& cs, int n, int V, double u, const W& wt, FastSmem& fs) {
  uint64_t tot = 0;
  for (int c = threadIdx.x; c < n; c += kThreads) tot += wt(c);
  tot = block_sum<uint64_t>(tot, fs.redu);
  if (tot == 0) return V - 1;
  const uint64_t t = (uint64_t)__double2ull_rd(u * (double)tot);
  for (int b = threadIdx.x; b < kHB; b += kThreads) fs.hmass[b] = 0ull;
  lds_barrier();
  auto ibin = [&](int idx) -> int { return (int)(((int64_t)idx * kHB) / V); };
  for (int c = threadIdx.x; c < n; c += kThreads) {
    const uint64_t w = wt(c);
    if (w) lds_add(&fs.hmass[ibin(cs.idx(c))], w);
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
  int mine = INT_MAX;
  uint64_t mine_before = 0;
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    if (mine == INT_MAX && brun + hb[q] > t) {
      mine = b0 + q;
      mine_before = brun;
    }
    brun += hb[q];
  }
  const int b = block_min<int>(mine, fs.redi);
  if (b == INT_MAX) return V - 1;
  if (mine == b) fs.ctlu[0] = mine_before;
  if (threadIdx.x == 0) fs.ctl[2] = 0;
  lds_barrier();
  const uint64_t before = fs.ctlu[0];
  SortList& sl = fs.u.sl;
  for (int c = threadIdx.x; c < n; c += kThreads) {
    const uint64_t w = wt(c);
    const int idx = cs.idx(c);
    if (w && ibin(idx) == b) {
      const int s = lds_fetch_add(&fs.ctl[2], 1);
      sl.key[s] = (uint64_t)idx;
      sl.idx[s] = idx;
      sl.w[s] = w;
    }
  }
  lds_barrier();
  const int m = fs.ctl[2];  // at most V / kHB + 1 <= kThreads tokens
  lds_bitonic(sl.key, sl.idx, sl.w, m, ~0ull, [](uint64_t ka, int, uint64_t kb, int) { return ka < kb; });
  const uint64_t w = (int)threadIdx.x < m ? sl.w[threadIdx.x] : 0ull;
  uint64_t mt;
  const uint64_t ex = block_excl_scan<uint64_t>(w, fs.redu, &mt);
  const int hit = block_min<int>(((int)threadIdx.x < m && before + ex + w > t) ? sl.idx[threadIdx.x] : INT_MAX,
                                 fs.redi);
  return hit == INT_MAX ? V - 1 : hit;
}

// ------------------------------------------------------------ row modes

template <typename TIn, bool VEC>
__device__ __forceinline__ int run_greedy(const TIn* x, int V, const RowParams& rp, FastSmem& fs) {
  RawIter<TIn> cur, nxt;
  load_iter<VEC>(x, V, 0, cur);
  ArgMax best{-INFINITY, INT_MAX};
  for (int base = 0; base < V; base += kIterLen) {
    if (base + kIterLen < V) load_iter<VEC>(x, V, base + kIterLen, nxt);
    uint32_t vm, pb;
    lane_bits(base, V, rp, fs.u.bitmap, &vm, &pb);
#pragma unroll
    for (int e = 0; e < kE; ++e)
      if ((vm >> e) & 1u) best = argmax_merge(best, ArgMax{zat(cur, e, pb, rp.pen), tok_idx(base, e)});
    cur = nxt;
  }
  best = block_argmax(best, fs.redd, fs.redi);
  return best.i;
}

// Temperature only: full-vocabulary softmax and draw (sampling.py:75-81, :94-98).
template <typename TIn, bool VEC>
__device__ __forceinline__ int run_temp(const TIn* x, int V, const RowParams& rp, FastSmem& fs) {
  const YScale ys{rp.T, 1.0 / rp.T};
  RawIter<TIn> cur, nxt;
  load_iter<VEC>(x, V, 0, cur);
  for (int base = 0; base < V; base += kIterLen) {
    if (base + kIterLen < V) load_iter<VEC>(x, V, base + kIterLen, nxt);
    uint32_t vm, pb;
    lane_bits(base, V, rp, fs.u.bitmap, &vm, &pb);
    segment_partial(cur, vm, pb, rp.pen, ys, fs.exp_tab, fs.seg_m, fs.seg_s, base / kSegLen + wave());
    cur = nxt;
  }
  lds_barrier();
  const int nseg = (V + kSegLen - 1) / kSegLen;
  const int k = threadIdx.x;
  const double mk = k < nseg ? fs.seg_m[k] : -INFINITY;
  const double ymax = block_max(mk, fs.redd);
  const double mass = (k < nseg && mk > -INFINITY) ? fs.seg_s[k] * fast_exp_neg(mk - ymax, fs.exp_tab) : 0.0;
  double ex, S;
  block_scan_d(mass, fs.redd, &ex, &S);
  const double t = rp.u * S;
  const int kstar = block_min<int>((k < nseg && ex + mass > t) ? k : INT_MAX, fs.redi);
  if (kstar == INT_MAX) return V - 1;
  if (k == kstar) fs.ctlu[0] = (uint64_t)__double_as_longlong(ex);
  lds_barrier();
  const double before = __longlong_as_double((long long)fs.ctlu[0]);
  const double ms = fs.seg_m[kstar];
  const double sc = fast_exp_neg(ms - ymax, fs.exp_tab);
  // rescan the segment with the stream's arithmetic: thread t holds tokens
  // kstar*kSegLen + kPer*t + q, in vocabulary order
  constexpr int kPer = kSegLen / kThreads;
  const int p0 = kstar * kSegLen + kPer * (int)threadIdx.x;
  double e[kPer], es = 0.0;
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    e[q] = 0.0;
    const int pos = p0 + q;
    if (pos < V) {
      double z = (double)x[pos];
      if (rp.pen_active && ((fs.u.bitmap[pos >> 5] >> (pos & 31)) & 1u)) z = penalize(z, rp.pen);
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
    if (e[q] > 0.0) last = p0 + q;
    if (hit == INT_MAX && e[q] > 0.0 && before + run * sc > t) hit = p0 + q;
  }
  hit = block_min<int>(hit, fs.redi);
  if (hit == INT_MAX) hit = block_max<int>(last, fs.redi);  // rounding at the segment end
  return hit < 0 ? V - 1 : hit;
}

struct FastOut {
  int id;
  bool general;  // the candidates cannot decide the row exactly
};

// Top-k and/or top-p rows (sampling.py:75-90, :94-98).
template <typename TIn, bool VEC, bool TOPK>
__device__ __forceinline__ FastOut run_cands(const TIn* x, int V, const RowParams& rp, FastSmem& fs) {
  constexpr int cap = cand_cap<TIn>();
  const Cands<TIn> cs{reinterpret_cast<TIn*>(fs.cand), reinterpret_cast<int*>(fs.cand + cap * sizeof(TIn)), cap};
  const YScale ys{rp.T, 1.0 / rp.T};
  constexpr bool topk = TOPK;
  // top-k keeps a running lower bound of the k-th largest; top-p keeps the
  // largest tokens, a count projected from the first iteration to ~0.7 cap
  const uint64_t keep_target = topk ? (uint64_t)rp.top_k : (uint64_t)(cap * 7 / 10);
  const uint64_t first_target =
      topk ? (uint64_t)rp.top_k
           : (V <= kIterLen ? keep_target : (uint64_t)max(1, (int)((double)keep_target * kIterLen / V)));
  double theta, umax = -INFINITY, zmax_l = -INFINITY;
  RawIter<TIn> cur, nxt;
  load_iter<VEC>(x, V, 0, cur);
  {  // threshold from the first iteration
    uint32_t vm, pb;
    lane_bits(0, V, rp, fs.u.bitmap, &vm, &pb);
    theta = theta_from_regs(cur, vm, pb, rp.pen, first_target, fs);
  }
  for (int base = 0; base < V; base += kIterLen) {
    if (base + kIterLen < V) load_iter<VEC>(x, V, base + kIterLen, nxt);
    uint32_t vm, pb;
    lane_bits(base, V, rp, fs.u.bitmap, &vm, &pb);
#pragma unroll
    for (int e = 0; e < kE; ++e)
      if ((vm >> e) & 1u) zmax_l = fmax(zmax_l, zat(cur, e, pb, rp.pen));
    if constexpr (!topk) segment_partial(cur, vm, pb, rp.pen, ys, fs.exp_tab, fs.seg_m, fs.seg_s, base / kSegLen + wave());
    insert_cands(cs, cur, vm, pb, rp.pen, base, theta, &umax, fs);
    cur = nxt;
    lds_barrier();
    if (fs.cand_n > cap - 2048) theta = fmax(theta, compact_cands(cs, keep_target, rp.pen, &umax, fs));
  }
  lds_barrier();
  const int n = min(fs.cand_n, cap);
  const double U = block_max(umax, fs.redd);
  const double zmax = block_max(zmax_l, fs.redd);
  const double T = rp.T;
  auto yexact = [&](double z) -> double { return T == 1.0 ? z : z / T; };
  const double ymax = yexact(zmax);
  auto zc = [&](int c) -> double { return cs.z(c, rp.pen); };

  // ---- top-k: k-th largest with multiplicity, keep y >= kth_y (:76-78)
  double z_lo = -INFINITY;
  if (topk) {
    const SelOut r = cand_select<false>(cs, n, [](int) { return true; }, zc, [&](int c) { return key_of(zc(c)); },
                                        [](int) { return 0ull; }, (uint64_t)rp.top_k, fs);
    if (!r.found) return FastOut{V - 1, true};
    const double kth_z = val_of_key(r.key);
    if (kth_z > -INFINITY) {
      const double kth_y = yexact(kth_z);
      z_lo = kth_z;
      for (int it = 0; it < 64; ++it) {
        const double zp = dbl_prev(z_lo);
        if (yexact(zp) >= kth_y) z_lo = zp; else break;
      }
    }
    if (!(U < z_lo)) return FastOut{V - 1, true};
  }
  auto elig = [&](int c) -> bool { return zc(c) >= z_lo; };

  // ---- softmax normaliser (:79-81)
  double S;
  if (topk) {
    double s = 0.0;
    for (int c = threadIdx.x; c < n; c += kThreads) {
      const double z = zc(c);
      if (z >= z_lo) s += fast_exp_neg(yexact(z) - ymax, fs.exp_tab);
    }
    S = block_sum(s, fs.redd);
  } else {
    const int nseg = (V + kSegLen - 1) / kSegLen;
    const int k = threadIdx.x;
    const double mk = k < nseg ? fs.seg_m[k] : -INFINITY;
    const double ysmax = block_max(mk, fs.redd);
    const double m = (k < nseg && mk > -INFINITY) ? fs.seg_s[k] * fast_exp_neg(mk - ysmax, fs.exp_tab) : 0.0;
    S = block_sum(m, fs.redd);
  }
  auto pc = [&](int c) -> double {
    const double z = zc(c);
    return z >= z_lo ? fast_exp_neg(yexact(z) - ymax, fs.exp_tab) / S : 0.0;
  };

  // ---- top-p: first token (p desc, index asc) whose inclusive mass reaches top_p (:82-90)
  bool have_cut = false;
  uint64_t cut_key = 0;
  int cut_idx = INT_MAX;
  if (rp.topp) {
    const SelOut r = cand_select<true>(cs, n, elig, [&](int c) { return yexact(zc(c)); },
                                       [&](int c) { return pkey_of(pc(c)); }, [&](int c) { return to_fx(pc(c)); },
                                       to_fx(rp.top_p), fs);
    if (r.giveup) return FastOut{V - 1, true};
    if (r.found) {
      have_cut = true;
      cut_key = r.key;
      cut_idx = r.idx;
    }
    if (!topk && U > -INFINITY) {
      const double pU = fast_exp_neg(yexact(U) - ymax, fs.exp_tab) / S;
      if (!(have_cut && cut_key > pkey_of(pU))) return FastOut{V - 1, true};
    }
  }

  // ---- draw in vocabulary order (:94-98)
  auto wt = [&](int c) -> uint64_t {
    const double p = pc(c);
    if (!(p > 0.0)) return 0ull;
    if (have_cut) {
      const uint64_t k = pkey_of(p);
      const int idx = cs.idx(c);
      if (!(k > cut_key || (k == cut_key && idx <= cut_idx))) return 0ull;
    }
    return to_fx(p);
  };
  return FastOut{draw_kept(cs, n, V, rp.u, wt, fs), false};
}

template <typename TIn, bool VEC>
__global__ __launch_bounds__(kThreads) void k_sample_fast(SampleArgs a) {
  __shared__ SmemAll sm;
  FastSmem& fs = sm.f;
  const int row = blockIdx.x;
  const int V = a.V;
  const RowParams rp = load_row_params(a, row);
  const TIn* x = reinterpret_cast<const TIn*>(a.logits) + (int64_t)row * a.ld;
  init_exp_table(fs.exp_tab);
  if (threadIdx.x == 0) fs.cand_n = 0;
  if (rp.pen_active) build_bitmap(fs.u.bitmap, 0, V, a.hist_ids, rp.h0, rp.h1);
  __syncthreads();
  int id;
  bool general = false;
  if (rp.greedy) {
    id = run_greedy<TIn, VEC>(x, V, rp, fs);
  } else if (!rp.topk && !rp.topp) {
    id = run_temp<TIn, VEC>(x, V, rp, fs);
  } else {
    const FastOut o = rp.topk ? run_cands<TIn, VEC, true>(x, V, rp, fs) : run_cands<TIn, VEC, false>(x, V, rp, fs);
    id = o.id;
    general = o.general;
  }
  if (general) {
    __syncthreads();
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
  __syncthreads();
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

hipError_t launch_sample_fast(const SampleArgs& a, bool f64, bool vec, hipStream_t s) {
  const dim3 grid(a.B), block(kThreads);
  if (f64) {
    if (vec) hipLaunchKernelGGL((k_sample_fast<double, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((k_sample_fast<double, false>), grid, block, 0, s, a);
  } else {
    if (vec) hipLaunchKernelGGL((k_sample_fast<float, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((k_sample_fast<float, false>), grid, block, 0, s, a);
  }
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
