// Per-row sampling pipeline for one 512-thread workgroup.
//
// The pipeline restates src/pagellm/engine/sampling.py:65-107 (penalty ->
// temperature -> top-k -> softmax -> top-p -> inverse-CDF draw, greedy
// argmax) over a logits row streamed from HBM once per pass, 32 consecutive
// tokens per thread per group with all of a group's loads in flight
// together.  It is the general path (any parameters, any distribution) and
// the path that exports the processed distribution.  Sorting is replaced by
// selection: top-k is an MSD radix select by count on order-preserving
// 64-bit keys of the penalised logits; the top-p cut is an MSD radix select
// by fixed-point probability mass on the same keys (p is non-decreasing in
// z, so (z descending, index ascending) is the reference's (p descending,
// index ascending) order except where two logits round to one p), which
// computes p only for the tokens still in play; the draw is an exact
// integer prefix scan in vocabulary order.
#pragma once

#include <limits.h>

#include "plh_device.h"
#include "plh_fast.h"

namespace plh {

constexpr int kBins = 2048;  // widest radix digit is 11 bits
constexpr int kSmall = 512;  // a bin this small is finished by an LDS sort
constexpr int kMaxVBitmap = 262144;  // penalty bitmap capacity (vocabulary size)

struct Smem {
  double redd[kWaves];
  uint64_t redu[kWaves];
  uint32_t redw[kWaves];
  int redi[kWaves];
  int ctl_i[16];
  uint64_t ctl_u[8];
  double ctl_d[8];
  uint32_t cnt[kBins];
  uint64_t mass[kBins];
  uint64_t lkey[kSmall];
  uint64_t lw[kSmall];
  int32_t lidx[kSmall];
  double exp_tab[64];
  uint32_t bitmap[kMaxVBitmap / 32];
};

struct RowParams {
  double T, top_p, pen, u;
  int top_k;
  int64_t h0, h1;  // history ids [h0, h1) of the CSR arrays
  bool greedy, pen_active, topk, topp;
  bool nucleus;  // the row takes the nucleus path of the fast kernels
};

// sampling.py:59-61: divide positive logits, multiply the others.
__device__ __forceinline__ double penalize(double x, double pen) { return x > 0.0 ? x / pen : x * pen; }

// Sets one bit per distinct history id in [lo, lo + n) of an LDS bitmap, so a
// repeated id is penalised once (np.unique, sampling.py:59).  Ids outside
// the range are ignored.
__device__ __forceinline__ void build_bitmap(uint32_t* bitmap, int lo, int n, const int32_t* ids, int64_t h0, int64_t h1) {
  const int words = (n + 31) >> 5;
  for (int w = threadIdx.x; w < words; w += kThreads) bitmap[w] = 0u;
  __syncthreads();
  for (int64_t h = h0 + threadIdx.x; h < h1; h += kThreads) {
    const int off = ids[h] - lo;
    if ((unsigned)off < (unsigned)n) lds_or(&bitmap[off >> 5], 1u << (off & 31));
  }
  __syncthreads();
}

// p(z) of the processed distribution for tokens that survived top-k
// (z >= z_lo); sampling.py:75-81, with y = z * (1 / T) and the table exp.
struct PCalc {
  double invT, ymax, invS, z_lo;
  const double* tab;
};

__device__ __forceinline__ double p_of(const PCalc& c, double z) {
  if (!(z >= c.z_lo)) return 0.0;
  return fast_exp_neg(z * c.invT - c.ymax, c.tab) * c.invS;
}

// ------------------------------------------------------------ source

// A logits row, penalised on the fly from an LDS bitmap.  group(base, f)
// covers tokens [base, base + kGroup): thread t owns the 32 consecutive
// tokens base + 32t .. base + 32t + 31, loaded before any is used; f(j, z,
// idx) is called for each of them in order (invalid ones: z = -inf, idx =
// INT_MAX).
template <typename TIn, bool VEC>
struct RowSource {
  static constexpr int kPer = 32;
  static constexpr int kGroup = kPer * kThreads;
  const TIn* x;  // row base
  int V;
  const uint32_t* bits;  // LDS penalty bitmap over [0, V)
  bool pen_on;           // false: no penalty, `bits` is not read
  double pen;

  __device__ __forceinline__ int n() const { return V; }

  template <class F>
  __device__ __forceinline__ void group(int base, const F& f) const {
    const int p0 = base + kPer * (int)threadIdx.x;
    TIn raw[kPer];
    if (VEC && p0 + kPer <= V) {
      if constexpr (sizeof(TIn) == 4) {
#pragma unroll
        for (int u = 0; u < kPer / 4; ++u) {
          const float4 v = *reinterpret_cast<const float4*>(x + p0 + 4 * u);
          raw[4 * u] = v.x; raw[4 * u + 1] = v.y; raw[4 * u + 2] = v.z; raw[4 * u + 3] = v.w;
        }
      } else {
#pragma unroll
        for (int u = 0; u < kPer / 2; ++u) {
          const double2 v = *reinterpret_cast<const double2*>(x + p0 + 2 * u);
          raw[2 * u] = v.x; raw[2 * u + 1] = v.y;
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < kPer; ++j) raw[j] = p0 + j < V ? x[p0 + j] : (TIn)(-INFINITY);
    }
    uint32_t pb = 0u;  // p0 is a multiple of 32: its bits are one word
    if (pen_on && p0 < V) pb = bits[p0 >> 5];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const bool valid = p0 + j < V;
      double z = (double)raw[j];
      if ((pb >> j) & 1u) z = penalize(z, pen);
      f(j, valid ? z : -INFINITY, valid ? p0 + j : INT_MAX);
    }
  }
};

// --------------------------------------------------------- radix select

// Histogram in sm.cnt (and sm.mass for MASS) over nb bins.  Walking the bins
// from the highest down, returns the bin d where the running total (starting
// at `above`) first reaches `target`, and the total of the bins above d.
struct BinPick {
  bool found;
  int d;
  uint64_t above;
};

template <bool MASS>
__device__ __forceinline__ BinPick pick_bin_desc(Smem& sm, int nb, uint64_t above, uint64_t target) {
  const int per = nb / kThreads;  // 4 or 2 bins per thread, highest bins first
  uint64_t v[4];
  uint64_t s = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[j] = 0;
    if (j < per) {
      const int d = nb - 1 - ((int)threadIdx.x * per + j);
      v[j] = MASS ? sm.mass[d] : (uint64_t)sm.cnt[d];
      s += v[j];
    }
  }
  uint64_t tot;
  const uint64_t ex = block_excl_scan<uint64_t>(s, sm.redu, &tot);
  if (above + tot < target) return BinPick{false, -1, above + tot};
  if (threadIdx.x == 0) sm.ctl_i[0] = INT_MAX;
  __syncthreads();
  uint64_t run = above + ex, myrun = 0;
  int myrank = INT_MAX;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (j < per && myrank == INT_MAX) {
      if (run + v[j] >= target) {
        myrank = (int)threadIdx.x * per + j;
        myrun = run;
      }
      run += v[j];
    }
  }
  if (myrank != INT_MAX) lds_min(&sm.ctl_i[0], myrank);
  __syncthreads();
  const int rk = sm.ctl_i[0];
  if (myrank == rk) sm.ctl_u[0] = myrun;
  __syncthreads();
  const BinPick r{true, nb - 1 - rk, sm.ctl_u[0]};
  __syncthreads();
  return r;
}

enum SelMode { kCount = 0, kMass = 1 };

struct SelResult {
  bool found;
  bool ties;        // more than kSmall elements share `key`; idx unresolved
  uint64_t key;
  int idx;
  uint64_t above;   // count or mass strictly before the result's key
  uint32_t tie_count;
};

// The gathered list (sm.ctl_i[2] entries, at most kSmall) sorted in (key
// desc, idx asc) order; the result of a selection whose earlier levels put
// `above` (count or mass) before the list.
template <int MODE>
__device__ __forceinline__ SelResult sorted_pick(uint64_t target, uint64_t above, Smem& sm) {
  const int n = min(sm.ctl_i[2], kSmall);
  int N = 2;
  while (N < n) N <<= 1;
  for (int i = threadIdx.x; i < N; i += kThreads)
    if (i >= n) {
      sm.lkey[i] = 0ull;
      sm.lidx[i] = INT_MAX;
      sm.lw[i] = 0ull;
    }
  __syncthreads();
  for (int k = 2; k <= N; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < N; i += kThreads) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const uint64_t ka = sm.lkey[i], kb = sm.lkey[ixj];
          const int ia = sm.lidx[i], ib = sm.lidx[ixj];
          const bool b_first = kb > ka || (kb == ka && ib < ia);
          const bool a_first = ka > kb || (ka == kb && ia < ib);
          const bool sw = ((i & k) == 0) ? b_first : a_first;
          if (sw) {
            sm.lkey[i] = kb; sm.lkey[ixj] = ka;
            sm.lidx[i] = ib; sm.lidx[ixj] = ia;
            const uint64_t t = sm.lw[i]; sm.lw[i] = sm.lw[ixj]; sm.lw[ixj] = t;
          }
        }
      }
      __syncthreads();
    }
  }
  SelResult r{true, false, 0, 0, above, 0};
  if (MODE == kCount) {
    const int pos = (int)(target - above - 1);  // 0 <= pos < n
    r.key = sm.lkey[pos];
    r.idx = sm.lidx[pos];
  } else {
    const int i = threadIdx.x;  // n <= kSmall == kThreads
    const uint64_t wi = i < n ? sm.lw[i] : 0ull;
    uint64_t tot;
    const uint64_t ex = block_excl_scan<uint64_t>(wi, sm.redu, &tot);
    if (threadIdx.x == 0) sm.ctl_i[3] = INT_MAX;
    __syncthreads();
    if (i < n && above + ex + wi >= target) lds_min(&sm.ctl_i[3], i);
    __syncthreads();
    const int pos = min(sm.ctl_i[3], n - 1);
    r.key = sm.lkey[pos];
    r.idx = sm.lidx[pos];
    // the mass before the result, for the kept total
    if (i == pos) sm.ctl_u[1] = above + ex;
    __syncthreads();
    r.above = sm.ctl_u[1];
  }
  __syncthreads();
  return r;
}


// `visit(fn)` calls fn(key, wfn, idx) once for every eligible element the
// calling thread owns, where wfn() returns the element's weight (only the
// kMass passes call it, and only for elements still in play); every thread
// of the workgroup must call visit.
//
// kCount: the target-th largest key (1-based, with multiplicity).
// kMass:  in (key descending, idx ascending) order, the first element whose
//         inclusive weight sum reaches target.
// found == false when the eligible total is below target (above then holds
// that total).
template <int MODE, class Visit>
__device__ __forceinline__ SelResult radix_select(const Visit& visit, uint64_t target, Smem& sm) {
  uint64_t prefix = 0, above = 0;
  uint32_t bincnt = 0;
  int done = 0;
  const int widths[6] = {11, 11, 11, 11, 10, 10};
  for (int pass = 0; pass < 6; ++pass) {
    const int w = widths[pass];
    const int shift = 64 - done - w;
    const int nb = 1 << w;
    const uint64_t dmask = (uint64_t)(nb - 1);
    for (int b = threadIdx.x; b < nb; b += kThreads) {
      sm.cnt[b] = 0u;
      if (MODE == kMass) sm.mass[b] = 0ull;
    }
    __syncthreads();
    visit([&](uint64_t key, auto wfn, int) {
      if (done > 0 && (key >> (64 - done)) != prefix) return;
      const int d = (int)((key >> shift) & dmask);
      lds_add(&sm.cnt[d], 1u);
      if (MODE == kMass) lds_add(&sm.mass[d], (uint64_t)wfn());
    });
    __syncthreads();
    const BinPick bp = pick_bin_desc<MODE == kMass>(sm, nb, above, target);
    if (!bp.found) return SelResult{false, false, 0, 0, bp.above, 0};
    above = bp.above;
    const int dstar = bp.d;
    bincnt = sm.cnt[dstar];
    prefix = (prefix << w) | (uint64_t)dstar;
    done += w;
    __syncthreads();
    if (bincnt <= (uint32_t)kSmall) break;
  }
  if (bincnt > (uint32_t)kSmall) {  // done == 64: every element of the bin has key == prefix
    return SelResult{true, true, prefix, -1, above, bincnt};
  }
  // Finish: gather the bin into LDS and sort it in (key desc, idx asc) order.
  if (threadIdx.x == 0) sm.ctl_i[2] = 0;
  __syncthreads();
  visit([&](uint64_t key, auto wfn, int idx) {
    if ((key >> (64 - done)) != prefix) return;
    const int slot = lds_fetch_add(&sm.ctl_i[2], 1);
    if (slot < kSmall) {
      sm.lkey[slot] = key;
      sm.lw[slot] = MODE == kMass ? (uint64_t)wfn() : 0ull;
      sm.lidx[slot] = idx;
    }
  });
  __syncthreads();
  return sorted_pick<MODE>(target, above, sm);
}

// Selection in (z descending, idx ascending) order over elements with value
// z:
//   kCount: the target-th element (1-based, with multiplicity);
//   kMass:  the first element whose inclusive weight sum reaches target.
// `visit(fn)` calls fn(z, wfn, idx) for every eligible element the calling
// thread owns (wfn() is its weight; only kMass calls it).  The first level
// bins z affinely over [zlo, zhi] (kBins bins; values outside clamp to the
// end bins), so the tokens of a smooth distribution spread over many bins
// instead of the few an exponent-led radix digit would give; later levels
// bin the exact 64-bit order keys of the elements still in play (kBins bins
// of 2^sh consecutive keys), until a bin holds at most kSmall elements,
// which are sorted.  Result keys are order keys (key_of(z)).  found ==
// false when the eligible total is below target (above then holds that
// total); ties: more than kSmall elements share one value.
template <int MODE, class Visit>
__device__ __forceinline__ SelResult value_select(const Visit& visit, double zlo, double zhi, uint64_t target,
                                                  Smem& sm) {
  const Affine af = make_affine(zlo, zhi, kBins);
  for (int b = threadIdx.x; b < kBins; b += kThreads) {
    sm.cnt[b] = 0u;
    if (MODE == kMass) sm.mass[b] = 0ull;
  }
  __syncthreads();
  visit([&](double z, auto wfn, int) {
    const int d = af.bin(z);
    lds_add(&sm.cnt[d], 1u);
    if (MODE == kMass) lds_add(&sm.mass[d], (uint64_t)wfn());
  });
  __syncthreads();
  BinPick bp = pick_bin_desc<MODE == kMass>(sm, kBins, 0, target);
  if (!bp.found) return SelResult{false, false, 0, 0, bp.above, 0};
  uint64_t above = bp.above;
  const int d0 = bp.d;
  uint32_t bincnt = sm.cnt[d0];
  __syncthreads();
  // exact key range [klo, khi] of the elements still in play
  uint64_t klo = 0, khi = ~0ull;
  bool keyed = false;
  auto in_play = [&](double z) -> bool {
    if (af.bin(z) != d0) return false;
    if (!keyed) return true;
    const uint64_t k = key_of(z);
    return k >= klo && k <= khi;
  };
  for (int lev = 0; bincnt > (uint32_t)kSmall; ++lev) {
    if (!keyed) {
      uint64_t lo = ~0ull, hi = 0ull;
      visit([&](double z, auto, int) {
        if (af.bin(z) != d0) return;
        const uint64_t k = key_of(z);
        lo = k < lo ? k : lo;
        hi = k > hi ? k : hi;
      });
      lo = wave_min(lo);
      hi = wave_max(hi);
      if (lane() == 0) {
        sm.redu[wave()] = lo;
        sm.lkey[wave()] = hi;
      }
      __syncthreads();
      klo = sm.redu[0];
      khi = sm.lkey[0];
      for (int w = 1; w < kWaves; ++w) {
        klo = sm.redu[w] < klo ? sm.redu[w] : klo;
        khi = sm.lkey[w] > khi ? sm.lkey[w] : khi;
      }
      __syncthreads();
      keyed = true;
    }
    if (klo == khi) return SelResult{true, true, klo, -1, above, bincnt};
    const uint64_t span = khi - klo;
    const int sh = span < (uint64_t)kBins ? 0 : 64 - __clzll((long long)span) - 11;
    for (int b = threadIdx.x; b < kBins; b += kThreads) {
      sm.cnt[b] = 0u;
      if (MODE == kMass) sm.mass[b] = 0ull;
    }
    __syncthreads();
    visit([&](double z, auto wfn, int) {
      if (!in_play(z)) return;
      const int d = (int)((key_of(z) - klo) >> sh);
      lds_add(&sm.cnt[d], 1u);
      if (MODE == kMass) lds_add(&sm.mass[d], (uint64_t)wfn());
    });
    __syncthreads();
    bp = pick_bin_desc<MODE == kMass>(sm, kBins, above, target);
    if (!bp.found) return SelResult{false, false, 0, 0, bp.above, 0};
    above = bp.above;
    bincnt = sm.cnt[bp.d];
    __syncthreads();
    const uint64_t nlo = klo + ((uint64_t)bp.d << sh);
    const uint64_t wid = (1ull << sh) - 1;
    khi = khi - nlo < wid ? khi : nlo + wid;
    klo = nlo;
  }
  // Finish: gather the bin into LDS and sort it in (key desc, idx asc) order.
  if (threadIdx.x == 0) sm.ctl_i[2] = 0;
  __syncthreads();
  visit([&](double z, auto wfn, int idx) {
    if (!in_play(z)) return;
    const int slot = lds_fetch_add(&sm.ctl_i[2], 1);
    if (slot < kSmall) {
      sm.lkey[slot] = key_of(z);
      sm.lw[slot] = MODE == kMass ? (uint64_t)wfn() : 0ull;
      sm.lidx[slot] = idx;
    }
  });
  __syncthreads();
  return sorted_pick<MODE>(target, above, sm);
}

// ----------------------------------------------------------------- draw

// Inverse-CDF draw over non-negative weights w(i), i < V (sampling.py:94-98):
// the first i whose running mass exceeds u * total, else V - 1.  Weights are
// normalised by their float64 total, then summed exactly in fixed point.
template <class W>
__device__ __forceinline__ int draw_weights(const W& wfn, int V, double u, double* redd, uint64_t* redu, int* redi) {
  double s = 0.0;
  for (int base = 0; base < V; base += (4 * kThreads))
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      const int i = base + 4 * (int)threadIdx.x + l;
      if (i < V) s += wfn(i);
    }
  const double Wt = block_sum(s, redd);
  if (!(Wt > 0.0)) return V - 1;
  uint64_t tf = 0;
  for (int base = 0; base < V; base += (4 * kThreads))
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      const int i = base + 4 * (int)threadIdx.x + l;
      if (i < V) tf += to_fx(wfn(i) / Wt);
    }
  tf = block_sum<uint64_t>(tf, redu);
  const uint64_t t_fx = (uint64_t)__double2ull_rd(u * (double)tf);
  uint64_t run = 0;
  for (int base = 0; base < V; base += (4 * kThreads)) {
    uint64_t w[4], ts = 0;
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      const int i = base + 4 * (int)threadIdx.x + l;
      w[l] = i < V ? to_fx(wfn(i) / Wt) : 0ull;
      ts += w[l];
    }
    uint64_t tt;
    const uint64_t ex = block_excl_scan<uint64_t>(ts, redu, &tt);
    if (run + tt > t_fx) {
      uint64_t c = run + ex;
      int my = INT_MAX;
#pragma unroll
      for (int l = 0; l < 4; ++l) {
        c += w[l];
        if (my == INT_MAX && c > t_fx) my = base + 4 * (int)threadIdx.x + l;
      }
      const int f = block_min<int>(my, redi);
      return f == INT_MAX ? V - 1 : f;
    }
    run += tt;
  }
  return V - 1;
}

// ------------------------------------------------------------- pipeline

struct PipeIn {
  bool have_max;  // zmax: the row's largest penalised logit
  double zmax;
  bool have_S;    // S: the full normaliser sum(exp(z / T - zmax / T)), no top-k
  double S;
  bool have_min;  // zmin: the row's smallest penalised logit (finite)
  double zmin;
};

template <class Src>
__device__ __forceinline__ int row_pipeline(Src& src, const RowParams& rp, int V, PipeIn in, Smem& sm,
                                            double* probs_out) {
  const int n = src.n();
  constexpr int kG = Src::kGroup;
  constexpr int kPer = Src::kPer;
  if (threadIdx.x < 64) sm.exp_tab[threadIdx.x] = kExp2Frac64[threadIdx.x];
  __syncthreads();

  // ---- max / argmax of the penalised logits (sampling.py:73, :79, :106),
  // and the smallest finite one (the range of the selection bins)
  double zmax = in.zmax, zmin = INFINITY;
  int argmax = 0;
  const bool need_min = !rp.greedy && (rp.topk || rp.topp);
  if (!in.have_max || rp.greedy) {
    ArgMax best{-INFINITY, INT_MAX};
    for (int base = 0; base < n; base += kG)
      src.group(base, [&](int, double z, int idx) {
        best = argmax_merge(best, ArgMax{z, idx});
        if (z > -INFINITY) zmin = fmin(zmin, z);
      });
    best = block_argmax(best, sm.redd, sm.redi);
    zmax = best.v;
    argmax = best.i;
    if (need_min) zmin = block_min(zmin, sm.redd);
  } else if (need_min && in.have_min) {
    zmin = in.zmin;
  } else if (need_min) {
    for (int base = 0; base < n; base += kG)
      src.group(base, [&](int, double z, int) {
        if (z > -INFINITY) zmin = fmin(zmin, z);
      });
    zmin = block_min(zmin, sm.redd);
  }
  if (rp.greedy) {  // sampling.py:71-74 / :102-106: no temperature, no uniform
    if (probs_out != nullptr)
      for (int i = threadIdx.x; i < V; i += kThreads) probs_out[i] = (i == argmax) ? 1.0 : 0.0;
    return argmax;
  }
  const double T = rp.T;
  const double invT = 1.0 / T;
  const double ymax = zmax * invT;

  // ---- top-k: kth = k-th largest (with multiplicity); keep y >= kth_y (:76-78)
  double z_lo = -INFINITY;
  if (rp.topk) {
    auto visit = [&](auto fn) {
      for (int base = 0; base < n; base += kG)
        src.group(base, [&](int, double z, int idx) {
          if (idx != INT_MAX) fn(z, [] { return 0ull; }, idx);
        });
    };
    const SelResult r = value_select<kCount>(visit, zmin, zmax, (uint64_t)rp.top_k, sm);
    const double kth_z = val_of_key(r.key);
    if (kth_z > -INFINITY) {
      const double kth_y = (T == 1.0) ? kth_z : kth_z / T;
      z_lo = kth_z;
      // smallest z whose y = z / T still reaches kth_y (division can merge
      // neighbouring values); a few steps at most
      for (int it = 0; it < 64; ++it) {
        const double zp = dbl_prev(z_lo);
        const double yp = (T == 1.0) ? zp : zp / T;
        if (yp >= kth_y) z_lo = zp; else break;
      }
    }
  }

  // ---- softmax normaliser over the survivors (:79-81)
  double S = in.S;
  if (!in.have_S || rp.topk) {
    const PCalc pc0{invT, ymax, 1.0, z_lo, sm.exp_tab};
    double s = 0.0;
    for (int base = 0; base < n; base += kG)
      src.group(base, [&](int, double z, int idx) {
        if (idx != INT_MAX) s += p_of(pc0, z);
      });
    S = block_sum(s, sm.redd);
  }
  const PCalc pc{invT, ymax, 1.0 / S, z_lo, sm.exp_tab};
  auto wt_of = [&](double z) -> uint64_t { return to_fx(p_of(pc, z)); };

  // ---- top-p: cut at the first token whose inclusive mass reaches top_p
  // (:82-90), selected on the logit keys
  bool have_cut = false;
  uint64_t cut_key = 0;
  int cut_idx = INT_MAX;
  uint64_t kept_tot = 0;  // fixed-point mass of the kept set, when known
  bool have_tot = false;
  if (rp.topp) {
    const uint64_t target = topp_target(rp.top_p);
    // tokens below z_lo (outside top-k) weigh nothing and never reach the cut
    auto visit = [&](auto fn) {
      for (int base = 0; base < n; base += kG)
        src.group(base, [&](int, double z, int idx) {
          if (idx != INT_MAX && z >= z_lo) fn(z, [&] { return wt_of(z); }, idx);
        });
    };
    const SelResult r = value_select<kMass>(visit, rp.topk ? z_lo : zmin, zmax, target, sm);
    if (!r.found) {
      kept_tot = r.above;  // every token is kept
      have_tot = true;
    } else {
      have_cut = true;
      cut_key = r.key;
      cut_idx = r.idx;
      const uint64_t w1 = wt_of(val_of_key(r.key));
      kept_tot = r.above + w1;
      have_tot = true;
      if (r.ties) {
        // r.tie_count tokens share key r.key; keep the lowest indices while
        // the mass before them stays below top_p
        uint64_t J = r.tie_count;
        if (w1 > 0) {
          const uint64_t need = (target - r.above - 1) / w1 + 1;
          J = need < J ? need : J;
        }
        kept_tot = r.above + J * w1;
        if (J >= r.tie_count) {
          cut_idx = INT_MAX;
        } else {
          const uint64_t tkey = r.key;
          auto vis2 = [&](auto fn) {
            for (int base = 0; base < n; base += kG)
              src.group(base, [&](int, double z, int idx) {
                if (idx != INT_MAX && key_of(z) == tkey) fn((uint64_t)(0x7fffffff - idx), [] { return 0ull; }, idx);
              });
          };
          const SelResult r2 = radix_select<kCount>(vis2, J, sm);
          cut_idx = 0x7fffffff - (int)r2.key;
        }
      }
    }
  }

  // a token survives top-p when it precedes or is the cut token in
  // (z descending, index ascending) order
  auto kept = [&](double z, int idx) -> bool {
    if (idx == INT_MAX || !(z >= z_lo)) return false;
    if (!have_cut) return true;
    const uint64_t k = key_of(z);
    return k > cut_key || (k == cut_key && idx <= cut_idx);
  };
  auto weight = [&](double z, int idx) -> uint64_t { return kept(z, idx) ? wt_of(z) : 0ull; };

  // ---- inverse-CDF draw in vocabulary order (:94-98)
  if (!have_tot) {
    uint64_t tot = 0;
    for (int base = 0; base < n; base += kG)
      src.group(base, [&](int, double z, int idx) { tot += weight(z, idx); });
    kept_tot = block_sum<uint64_t>(tot, sm.redu);
  }
  const uint64_t t_fx = (uint64_t)__double2ull_rd(rp.u * (double)kept_tot);
  uint64_t run = 0;
  int found = INT_MAX;
  for (int base = 0; base < n; base += kG) {
    uint64_t w[kPer], s = 0;
    int ix[kPer];
    src.group(base, [&](int j, double z, int idx) {
      w[j] = weight(z, idx);
      ix[j] = idx;
      s += w[j];
    });
    uint64_t group_tot;
    const uint64_t ex = block_excl_scan<uint64_t>(s, sm.redu, &group_tot);
    if (run + group_tot > t_fx) {
      uint64_t c = run + ex;
      int my = INT_MAX;
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        c += w[j];
        if (my == INT_MAX && c > t_fx) my = ix[j];
      }
      found = block_min<int>(my, sm.redi);
      break;
    }
    run += group_tot;
  }
  const int id = (found == INT_MAX) ? V - 1 : found;

  // ---- optional export of the processed distribution (probs())
  if (probs_out != nullptr) {
    double s2 = 1.0;
    if (have_cut) {
      double s = 0.0;
      for (int base = 0; base < n; base += kG)
        src.group(base, [&](int, double z, int idx) {
          if (kept(z, idx)) s += p_of(pc, z);
        });
      s2 = block_sum(s, sm.redd);
    }
    for (int base = 0; base < n; base += kG)
      src.group(base, [&](int, double z, int idx) {
        if (idx == INT_MAX) return;
        // top-p renormalises the kept mass (:89-90); without top-p p is final
        probs_out[idx] = have_cut ? (kept(z, idx) ? p_of(pc, z) / s2 : 0.0) : p_of(pc, z);
      });
  }
  return id;
}

}  // namespace plh
