// Building blocks of the fast path: a table-driven float64 exp and
// value-range histograms with a descending bin walk for selection.
#pragma once

#include <limits.h>

#include "plh_device.h"

namespace plh {

// ------------------------------------------------------------------- exp
// exp(d) for d <= 0 in float64, <= 2 ulp: d = k*ln2/64 + r with a two-part
// ln2/64 (Cody-Waite reduction), exp(r) by its degree-5 Taylor polynomial
// (|r| <= ln2/128, truncation < 4e-17), times 2^(k/64) from a 64-entry
// table of 2^(j/64) built on the device, scaled by 2^(k>>6) with ldexp.
// The split of ln2 is the classic fdlibm one (a 32-bit head, exact k*head
// for |k| < 2^21).
constexpr double kLn2Hi = 6.93147180369123816490e-01;
constexpr double kLn2Lo = 1.90821492927058770002e-10;

// The calling wave's own copy of the table (it needs no workgroup barrier
// before use: a wave's LDS accesses complete in order).
__device__ __forceinline__ void init_exp_table_wave(double* tab) {
  tab[lane()] = exp2((double)lane() / 64.0);
}

__device__ __forceinline__ double fast_exp_neg(double d, const double* tab) {
  // below -745.2 the result underflows: clamping to -1000 keeps k*ln2/64
  // exact and makes the final ldexp return 0 (also for -inf)
  d = fmax(d, -1000.0);
  const double kd = __builtin_rint(d * (64.0 / 0.6931471805599453));
  const int k = (int)kd;
  double r = fma(-kd, kLn2Hi / 64.0, d);
  r = fma(-kd, kLn2Lo / 64.0, r);
  double q = fma(r, 1.0 / 120.0, 1.0 / 24.0);
  q = fma(q, r, 1.0 / 6.0);
  q = fma(q, r, 0.5);
  q = fma(q, r, 1.0);
  q = fma(q, r, 1.0);
  return ldexp(tab[k & 63] * q, k >> 6);
}

// exp(d) for d <= 0 as a term of a normaliser sum: the reduction and
// polynomial of fast_exp_neg, with k = rint(d * 64 / ln2) from the
// magic-number rounding (adding 1.5 * 2^52 leaves k in the low mantissa
// bits) and 2^(k >> 6) added to the exponent field instead of an ldexp.  d
// is clamped at -708, where the scaled result is still normal: a term
// below e^-708 (including -inf) counts as e^-708 ~ 3e-308, which no sum
// holding a term of 1 can notice.
constexpr double kExpMagic = 6755399441055744.0;  // 1.5 * 2^52

__device__ __forceinline__ double exp_neg_term(double d, const double* tab) {
  d = fmax(d, -708.0);
  const double t = fma(d, 64.0 / 0.6931471805599453, kExpMagic);
  const int k = __double2loint(t);
  const double kd = t - kExpMagic;
  double r = fma(-kd, kLn2Hi / 64.0, d);
  r = fma(-kd, kLn2Lo / 64.0, r);
  double q = fma(r, 1.0 / 120.0, 1.0 / 24.0);
  q = fma(q, r, 1.0 / 6.0);
  q = fma(q, r, 0.5);
  q = fma(q, r, 1.0);
  q = fma(q, r, 1.0);
  const double v = tab[k & 63] * q;
  return __hiloint2double(__double2hiint(v) + ((k >> 6) << 20), __double2loint(v));
}

// ------------------------------------------------------- value histograms
// bin(v) = floor((v - lo) * scale) clamped to [0, nb-1]: monotone
// non-decreasing in v, so "bin(v) >= d" is a threshold rule on v.
struct Affine {
  double lo, scale;
  int nb;
  __device__ __forceinline__ int bin(double v) const {
    if (!(v > lo)) return 0;  // v <= lo (and -inf)
    const double t = (v - lo) * scale;
    if (t >= (double)(nb - 1)) return nb - 1;
    return t > 0.0 ? (int)t : 0;  // also NaN (+inf times a zero scale)
  }
};

__device__ __forceinline__ Affine make_affine(double lo, double hi, int nb) {
  Affine a;
  a.nb = nb;
  a.lo = lo;
  a.scale = (hi > lo && hi - lo < INFINITY) ? (double)(nb - 1) / (hi - lo) : 0.0;
  if (!(a.scale < INFINITY)) a.scale = 0.0;
  return a;
}

// Descending walk over nb histogram bins (counts and/or masses in LDS):
// the bin where the running total (from `above`) first reaches target.
struct Pick {
  bool found;
  int d;
  uint64_t above;
};

template <bool MASS>
__device__ __forceinline__ Pick pick_desc(const uint32_t* cnt, const uint64_t* mass, int nb, uint64_t above,
                                          uint64_t target, uint64_t* redu, int* ctl, uint64_t* ctlu) {
  const int per = (nb + kThreads - 1) / kThreads;  // nb <= 2 * kThreads
  uint64_t v[2];
  uint64_t s = 0;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    v[j] = 0;
    const int r = (int)threadIdx.x * per + j;
    if (j < per && r < nb) {
      const int d = nb - 1 - r;
      v[j] = MASS ? mass[d] : (uint64_t)cnt[d];
    }
    s += v[j];
  }
  uint64_t tot;
  const uint64_t ex = block_excl_scan<uint64_t>(s, redu, &tot);
  if (above >= target || above + tot < target) return Pick{false, -1, above + tot};
  // the running total is non-decreasing, so exactly one bin takes it from
  // below target to target or more
  uint64_t run = above + ex;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int r = (int)threadIdx.x * per + j;
    if (j < per && r < nb) {
      if (run < target && run + v[j] >= target) {
        ctl[0] = nb - 1 - r;
        ctlu[1] = run;
      }
      run += v[j];
    }
  }
  wg_barrier();
  const Pick p{true, ctl[0], ctlu[1]};
  wg_barrier();
  return p;
}

}  // namespace plh
