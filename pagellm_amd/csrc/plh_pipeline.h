// Per-row sampling pipeline for one 512-thread workgroup.
//
// The pipeline restates src/pagellm/engine/sampling.py:65-107 (penalty ->
// temperature -> top-k -> softmax -> top-p -> inverse-CDF draw, greedy
// argmax) over an element source; RowSource streams a whole logits row from
// HBM once per pass.  It is the general path (any parameters, any
// distribution) and the path that exports the processed distribution.
// Sorting is replaced by selection: top-k is an MSD radix select by count on
// order-preserving 64-bit keys of the penalised logits; the top-p cut is an
// MSD radix select by fixed-point probability mass on the bits of p, in the
// reference's (p descending, index ascending) order; the draw is an exact
// integer prefix scan in vocabulary order.
#pragma once

#include <limits.h>

#include "plh_device.h"

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
  uint32_t bitmap[kMaxVBitmap / 32];
};

struct RowParams {
  double T, top_p, pen, u;
  int top_k;
  int64_t h0, h1;  // history ids [h0, h1) of the CSR arrays
  bool greedy, pen_active, topk, topp;
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

// p(z) of the processed distribution for elements that survived top-k
// (z >= z_lo); sampling.py:75-81.
struct PCalc {
  double T, ymax, S, z_lo;
};

__device__ __forceinline__ double p_of(const PCalc& c, double z) {
  if (!(z >= c.z_lo)) return 0.0;
  const double y = (c.T == 1.0) ? z : z / c.T;
  return exp(y - c.ymax) / c.S;
}

// ------------------------------------------------------------ sources

// Positions base + 4*tid + l (l = 0..3) of a tile of 4*kThreads elements.
template <typename TIn, bool VEC>
struct RowSource {
  const TIn* x;  // row base
  int V;
  const uint32_t* bits;  // LDS penalty bitmap over [0, V)
  bool pen_on;           // false: no penalty, `bits` is not read
  double pen;

  __device__ __forceinline__ int n() const { return V; }

  __device__ __forceinline__ void load4(int base, double z[4], int idx[4], bool valid[4], int addr[4]) const {
    const int p0 = base + 4 * (int)threadIdx.x;
    if (VEC && p0 + 3 < V) {
      if constexpr (sizeof(TIn) == 4) {
        const float4 v = *reinterpret_cast<const float4*>(x + p0);
        z[0] = v.x; z[1] = v.y; z[2] = v.z; z[3] = v.w;
      } else {
        const double2 a = *reinterpret_cast<const double2*>(x + p0);
        const double2 b = *reinterpret_cast<const double2*>(x + p0 + 2);
        z[0] = a.x; z[1] = a.y; z[2] = b.x; z[3] = b.y;
      }
#pragma unroll
      for (int l = 0; l < 4; ++l) valid[l] = true;
    } else {
#pragma unroll
      for (int l = 0; l < 4; ++l) {
        valid[l] = p0 + l < V;
        z[l] = valid[l] ? (double)x[p0 + l] : -INFINITY;
      }
    }
    if (pen_on && p0 < V) {
      const uint32_t w = bits[p0 >> 5] >> (p0 & 31);
#pragma unroll
      for (int l = 0; l < 4; ++l)
        if (valid[l] && ((w >> l) & 1u)) z[l] = penalize(z[l], pen);
    }
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      idx[l] = valid[l] ? p0 + l : INT_MAX;
      addr[l] = p0 + l;
    }
  }

  __device__ __forceinline__ void prepare_p(const PCalc&, Smem&) {}

  __device__ __forceinline__ void load4p(int base, double z[4], int idx[4], bool valid[4], double p[4],
                                         const PCalc& pc) const {
    int addr[4];
    load4(base, z, idx, valid, addr);
#pragma unroll
    for (int l = 0; l < 4; ++l) p[l] = valid[l] ? p_of(pc, z[l]) : 0.0;
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

// `visit(fn)` calls fn(key, weight, idx) once for every eligible element the
// calling thread owns; every thread of the workgroup must call visit.
//
// kCount: the target-th largest key (1-based, with multiplicity).
// kMass:  in (key descending, idx ascending) order, the first element whose
//         inclusive weight sum reaches target.
// found == false when the eligible total is below target.
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
    visit([&](uint64_t key, uint64_t wt, int) {
      if (done > 0 && (key >> (64 - done)) != prefix) return;
      const int d = (int)((key >> shift) & dmask);
      lds_add(&sm.cnt[d], 1u);
      if (MODE == kMass) lds_add(&sm.mass[d], wt);
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
  visit([&](uint64_t key, uint64_t wt, int idx) {
    if ((key >> (64 - done)) != prefix) return;
    const int slot = lds_fetch_add(&sm.ctl_i[2], 1);
    if (slot < kSmall) {
      sm.lkey[slot] = key;
      sm.lw[slot] = wt;
      sm.lidx[slot] = idx;
    }
  });
  __syncthreads();
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
  }
  __syncthreads();
  return r;
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
  bool have_max;
  double zmax;
  int argmax;
  bool have_S;
  double S;
  bool cand;  // source holds candidates only
  double U;   // cand: largest z among elements that are not candidates (-inf: none)
};

struct PipeOut {
  int id;
  bool insufficient;  // cand: the candidates cannot decide this row exactly
};

template <class Src>
__device__ __forceinline__ PipeOut row_pipeline(Src& src, const RowParams& rp, int V, PipeIn in, Smem& sm, double* probs_out) {
  const int n = src.n();
  constexpr int kTile = 4 * kThreads;
  PipeOut out{V - 1, false};

  // ---- max / argmax of the penalised logits (sampling.py:73, :79, :106)
  double zmax = in.zmax;
  int argmax = in.argmax;
  if (!in.have_max) {
    ArgMax best{-INFINITY, INT_MAX};
    for (int base = 0; base < n; base += kTile) {
      double z[4];
      int idx[4], addr[4];
      bool valid[4];
      src.load4(base, z, idx, valid, addr);
#pragma unroll
      for (int l = 0; l < 4; ++l)
        if (valid[l]) best = argmax_merge(best, ArgMax{z[l], idx[l]});
    }
    best = block_argmax(best, sm.redd, sm.redi);
    zmax = best.v;
    argmax = best.i;
  }
  if (rp.greedy) {  // sampling.py:71-74 / :102-106: no temperature, no uniform
    out.id = argmax;
    if (probs_out != nullptr)
      for (int i = threadIdx.x; i < V; i += kThreads) probs_out[i] = (i == argmax) ? 1.0 : 0.0;
    return out;
  }
  const double T = rp.T;
  const double ymax = (T == 1.0) ? zmax : zmax / T;

  // ---- top-k: kth = k-th largest (with multiplicity); keep y >= kth_y (:76-78)
  double z_lo = -INFINITY;
  if (rp.topk) {
    auto visit = [&](auto fn) {
      for (int base = 0; base < n; base += kTile) {
        double z[4];
        int idx[4], addr[4];
        bool valid[4];
        src.load4(base, z, idx, valid, addr);
#pragma unroll
        for (int l = 0; l < 4; ++l)
          if (valid[l]) fn(key_of(z[l]), 0ull, idx[l]);
      }
    };
    const SelResult r = radix_select<kCount>(visit, (uint64_t)rp.top_k, sm);
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
    if (in.cand && !(in.U < z_lo)) {
      out.insufficient = true;
      return out;
    }
  }

  // ---- softmax normaliser over the survivors (:79-81)
  double S = in.S;
  if (!in.have_S || rp.topk) {
    const PCalc pc0{T, ymax, 1.0, z_lo};
    double s = 0.0;
    for (int base = 0; base < n; base += kTile) {
      double z[4];
      int idx[4], addr[4];
      bool valid[4];
      src.load4(base, z, idx, valid, addr);
#pragma unroll
      for (int l = 0; l < 4; ++l)
        if (valid[l]) s += p_of(pc0, z[l]);
    }
    S = block_sum(s, sm.redd);
  }
  const PCalc pc{T, ymax, S, z_lo};
  src.prepare_p(pc, sm);

  // ---- top-p: cut at the first token whose inclusive mass reaches top_p (:82-90)
  bool have_cut = false;
  uint64_t cut_key = 0;
  int cut_idx = INT_MAX;
  if (rp.topp) {
    const uint64_t target = topp_target(rp.top_p);
    auto visit = [&](auto fn) {
      for (int base = 0; base < n; base += kTile) {
        double z[4], p[4];
        int idx[4];
        bool valid[4];
        src.load4p(base, z, idx, valid, p, pc);
#pragma unroll
        for (int l = 0; l < 4; ++l)
          if (valid[l]) fn(pkey_of(p[l]), to_fx(p[l]), idx[l]);
      }
    };
    const SelResult r = radix_select<kMass>(visit, target, sm);
    if (r.found) {
      have_cut = true;
      cut_key = r.key;
      cut_idx = r.idx;
      if (r.ties) {
        // r.tie_count tokens share probability key r.key; keep the lowest
        // indices while the mass before them stays below top_p
        const uint64_t w1 = to_fx(__longlong_as_double((long long)r.key));
        uint64_t J = r.tie_count;
        if (w1 > 0) {
          const uint64_t need = (target - r.above - 1) / w1 + 1;
          J = need < J ? need : J;
        }
        if (J >= r.tie_count) {
          cut_idx = INT_MAX;
        } else {
          const uint64_t tkey = r.key;
          auto vis2 = [&](auto fn) {
            for (int base = 0; base < n; base += kTile) {
              double z[4], p[4];
              int idx[4];
              bool valid[4];
              src.load4p(base, z, idx, valid, p, pc);
#pragma unroll
              for (int l = 0; l < 4; ++l)
                if (valid[l] && pkey_of(p[l]) == tkey) fn((uint64_t)(0x7fffffff - idx[l]), 0ull, idx[l]);
            }
          };
          const SelResult r2 = radix_select<kCount>(vis2, J, sm);
          cut_idx = 0x7fffffff - (int)r2.key;
        }
      }
    }
    if (in.cand && !rp.topk && in.U > -INFINITY) {
      const double pU = p_of(pc, in.U);
      if (!(have_cut && cut_key > pkey_of(pU))) {
        out.insufficient = true;
        return out;
      }
    }
  }

  // a token survives top-p when it precedes or is the cut token in
  // (p descending, index ascending) order
  auto kept = [&](double p, int idx) -> bool {
    if (!(p > 0.0)) return false;
    if (!have_cut) return true;
    const uint64_t k = pkey_of(p);
    return k > cut_key || (k == cut_key && idx <= cut_idx);
  };
  auto weight = [&](double p, int idx) -> uint64_t { return kept(p, idx) ? to_fx(p) : 0ull; };

  // ---- inverse-CDF draw in vocabulary order (:94-98)
  uint64_t tot = 0;
  for (int base = 0; base < n; base += kTile) {
    double z[4], p[4];
    int idx[4];
    bool valid[4];
    src.load4p(base, z, idx, valid, p, pc);
#pragma unroll
    for (int l = 0; l < 4; ++l)
      if (valid[l]) tot += weight(p[l], idx[l]);
  }
  tot = block_sum<uint64_t>(tot, sm.redu);
  const uint64_t t_fx = (uint64_t)__double2ull_rd(rp.u * (double)tot);
  uint64_t run = 0;
  int found = INT_MAX;
  for (int base = 0; base < n; base += kTile) {
    double z[4], p[4];
    int idx[4];
    bool valid[4];
    src.load4p(base, z, idx, valid, p, pc);
    uint64_t w[4], s = 0;
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      w[l] = valid[l] ? weight(p[l], idx[l]) : 0ull;
      s += w[l];
    }
    uint64_t tile_tot;
    const uint64_t ex = block_excl_scan<uint64_t>(s, sm.redu, &tile_tot);
    if (run + tile_tot > t_fx) {
      uint64_t c = run + ex;
      int my = INT_MAX;
#pragma unroll
      for (int l = 0; l < 4; ++l) {
        c += w[l];
        if (my == INT_MAX && c > t_fx) my = idx[l];
      }
      found = block_min<int>(my, sm.redi);
      break;
    }
    run += tile_tot;
  }
  out.id = (found == INT_MAX) ? V - 1 : found;

  // ---- optional export of the processed distribution (probs())
  if (probs_out != nullptr) {
    double s2 = 1.0;
    if (have_cut) {
      double s = 0.0;
      for (int base = 0; base < n; base += kTile) {
        double z[4], p[4];
        int idx[4];
        bool valid[4];
        src.load4p(base, z, idx, valid, p, pc);
#pragma unroll
        for (int l = 0; l < 4; ++l)
          if (valid[l] && kept(p[l], idx[l])) s += p[l];
      }
      s2 = block_sum(s, sm.redd);
    }
    for (int base = 0; base < n; base += kTile) {
      double z[4], p[4];
      int idx[4];
      bool valid[4];
      src.load4p(base, z, idx, valid, p, pc);
#pragma unroll
      for (int l = 0; l < 4; ++l) {
        if (!valid[l]) continue;
        // top-p renormalises the kept mass (:89-90); without top-p p is final
        probs_out[idx[l]] = have_cut ? (kept(p[l], idx[l]) ? p[l] / s2 : 0.0) : p[l];
      }
    }
  }
  return out;
}

}  // namespace plh
