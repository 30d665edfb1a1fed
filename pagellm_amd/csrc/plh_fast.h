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

// 2^(j/64), j = 0..63, each the correctly rounded double (computed at 60
// significant digits).
__device__ const double kExp2Frac64[64] = {
  0x1.0000000000000p+0, 0x1.02c9a3e778061p+0, 0x1.059b0d3158574p+0, 0x1.0874518759bc8p+0,
  0x1.0b5586cf9890fp+0, 0x1.0e3ec32d3d1a2p+0, 0x1.11301d0125b51p+0, 0x1.1429aaea92de0p+0,
  0x1.172b83c7d517bp+0, 0x1.1a35beb6fcb75p+0, 0x1.1d4873168b9aap+0, 0x1.2063b88628cd6p+0,
  0x1.2387a6e756238p+0, 0x1.26b4565e27cddp+0, 0x1.29e9df51fdee1p+0, 0x1.2d285a6e4030bp+0,
  0x1.306fe0a31b715p+0, 0x1.33c08b26416ffp+0, 0x1.371a7373aa9cbp+0, 0x1.3a7db34e59ff7p+0,
  0x1.3dea64c123422p+0, 0x1.4160a21f72e2ap+0, 0x1.44e086061892dp+0, 0x1.486a2b5c13cd0p+0,
  0x1.4bfdad5362a27p+0, 0x1.4f9b2769d2ca7p+0, 0x1.5342b569d4f82p+0, 0x1.56f4736b527dap+0,
  0x1.5ab07dd485429p+0, 0x1.5e76f15ad2148p+0, 0x1.6247eb03a5585p+0, 0x1.6623882552225p+0,
  0x1.6a09e667f3bcdp+0, 0x1.6dfb23c651a2fp+0, 0x1.71f75e8ec5f74p+0, 0x1.75feb564267c9p+0,
  0x1.7a11473eb0187p+0, 0x1.7e2f336cf4e62p+0, 0x1.82589994cce13p+0, 0x1.868d99b4492edp+0,
  0x1.8ace5422aa0dbp+0, 0x1.8f1ae99157736p+0, 0x1.93737b0cdc5e5p+0, 0x1.97d829fde4e50p+0,
  0x1.9c49182a3f090p+0, 0x1.a0c667b5de565p+0, 0x1.a5503b23e255dp+0, 0x1.a9e6b5579fdbfp+0,
  0x1.ae89f995ad3adp+0, 0x1.b33a2b84f15fbp+0, 0x1.b7f76f2fb5e47p+0, 0x1.bcc1e904bc1d2p+0,
  0x1.c199bdd85529cp+0, 0x1.c67f12e57d14bp+0, 0x1.cb720dcef9069p+0, 0x1.d072d4a07897cp+0,
  0x1.d5818dcfba487p+0, 0x1.da9e603db3285p+0, 0x1.dfc97337b9b5fp+0, 0x1.e502ee78b3ff6p+0,
  0x1.ea4afa2a490dap+0, 0x1.efa1bee615a27p+0, 0x1.f50765b6e4540p+0, 0x1.fa7c1819e90d8p+0,
};

// The calling wave's own copy of the table (it needs no workgroup barrier
// before use: a wave's LDS accesses complete in order).
__device__ __forceinline__ void init_exp_table_wave(double* tab) { tab[lane()] = kExp2Frac64[lane()]; }

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

// exp(d) for d <= 0 as a term of a normaliser sum, relative error below
// 3e-15 for d >= -40 (the terms a sum holding a term of 1 can notice):
//   * k = rint(d * 64 / ln2) from the magic-number rounding (adding
//     1.5 * 2^52 leaves k in the low mantissa bits);
//   * r = d - k * ln2/64 with ln2/64 as one double: the constant's error,
//     |k| * 2^-60, stays below 3.3e-15 for |k| <= 3694 (d >= -40);
//   * exp(r) on |r| <= ln2/128 by the degree-4 polynomial interpolating exp
//     at the five Chebyshev nodes of that interval (relative error 2.4e-15;
//     kExpCheb4, from pagellm_amd/csrc/exp_poly.py);
//   * times 2^(k/64) from the table, scaled by 2^(k>>6) with ldexp.
// d is clamped at -708, where the scaled result is still normal: a term
// below e^-708 (including -inf) counts as e^-708 ~ 3e-308, which no sum
// holding a term of 1 can notice.
constexpr double kExpMagic = 6755399441055744.0;  // 1.5 * 2^52
constexpr double kLn2Over64 = 0x1.62e42fefa39efp-7;  // ln2 / 64 rounded to double
constexpr double kExpCheb4[4] = {0x1.fffffffffb135p-1, 0x1.fffffffffe5b9p-2, 0x1.55557e54ffd7ep-3,
                                 0x1.555570ac8d5b7p-5};  // r^1..r^4 (r^0: exactly 1)

__device__ __forceinline__ double exp_neg_term(double d, const double* tab) {
  d = fmax(d, -708.0);
  const double t = fma(d, 64.0 / 0.6931471805599453, kExpMagic);
  const int k = __double2loint(t);
  const double kd = t - kExpMagic;
  const double r = fma(-kd, kLn2Over64, d);
  double q = fma(r, kExpCheb4[3], kExpCheb4[2]);
  q = fma(q, r, kExpCheb4[1]);
  q = fma(q, r, kExpCheb4[0]);
  q = fma(q, r, 1.0);
  return ldexp(tab[k & 63] * q, k >> 6);
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
