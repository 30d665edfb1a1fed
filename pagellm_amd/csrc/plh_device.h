// Device primitives shared by the gfx950 sampler kernels: order-preserving
// keys, fixed-point masses, wave64/workgroup reductions and scans.
//
// Every reduction and scan here combines values in a fixed order (a DPP
// scan inside each wave, then the waves' partials left to right), so the
// kernels are deterministic run to run.  Integer (fixed-point) scans are
// exact, which is what the inverse-CDF draws and the top-p mass selection
// rely on.
//
// Cross-lane steps use DPP (data-parallel primitives: a VALU operand read
// from another lane of the same instruction) rather than ds_bpermute, whose
// every step is an LDS round trip.  The wave64 scan is the gfx9 sequence:
// row_shr 1, 2, 4, 8 inside each row of 16 lanes, then row_bcast15 into rows
// 1 and 3 and row_bcast31 into rows 2 and 3; lane 63 then holds the total.
// Callers invoke these from converged code (all 64 lanes active).
#pragma once

#include <hip/hip_runtime.h>
#include <limits.h>
#include <math.h>
#include <stdint.h>

namespace plh {

constexpr int kWave = 64;
constexpr int kThreads = 512;  // every kernel in this library runs 8 waves of 64
constexpr int kWaves = kThreads / kWave;

// 2^62: probabilities (each <= 1, sum ~1) become exact-addable integers.
constexpr double kFxScale = 4611686018427387904.0;
constexpr uint64_t kFxOne = 1ull << 62;  // kFxScale as an integer: probability 1

__device__ __forceinline__ int lane() { return threadIdx.x & (kWave - 1); }

// Workgroup barrier for LDS communication: the calling wave's LDS operations
// complete, then s_barrier.  Unlike __syncthreads() it carries no
// memory-model fence, so vector-memory loads in flight (into registers, or
// global->LDS loads into another buffer) stay in flight across it; the
// "memory" clobber keeps the compiler from moving memory accesses over it.
// Every barrier in this library orders LDS traffic only: no thread reads
// global memory written by another thread of its workgroup.
__device__ __forceinline__ void wg_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
__device__ __forceinline__ int wave() { return threadIdx.x >> 6; }

// Larger double -> larger key; -0.0 and +0.0 share a key (numpy compares them
// equal).  NaN is outside the supported input domain.
__device__ __forceinline__ uint64_t key_of(double d) {
  d = d + 0.0;
  const uint64_t u = (uint64_t)__double_as_longlong(d);
  return (u >> 63) ? ~u : (u | 0x8000000000000000ull);
}

__device__ __forceinline__ double val_of_key(uint64_t k) {
  const uint64_t u = (k >> 63) ? (k & 0x7fffffffffffffffull) : ~k;
  return __longlong_as_double((long long)u);
}

// Coarse 32-bit key: the order key of z rounded toward -inf to float.  It is
// monotone non-decreasing in z, and key32(a) < key32(b) implies a < b.
__device__ __forceinline__ uint32_t key32_of(double d) {
  float f = __double2float_rd(d);
  f = f + 0.0f;
  const uint32_t u = __float_as_uint(f);
  return (u >> 31) ? ~u : (u | 0x80000000u);
}

// Bits of a non-negative double are already order preserving.
__device__ __forceinline__ uint64_t pkey_of(double p) { return (uint64_t)__double_as_longlong(p + 0.0); }

__device__ __forceinline__ uint64_t to_fx(double p) {
  return p > 0.0 ? (uint64_t)__double2ull_rn(p * kFxScale) : 0ull;
}

// Fixed-point top-p target, at least 1 so that a top_p below 2^-62 still
// keeps the first token (its inclusive mass reaches any positive top_p).
__device__ __forceinline__ uint64_t topp_target(double top_p) {
  const uint64_t t = to_fx(top_p);
  return t > 0 ? t : 1ull;
}

// Largest double strictly below d (d finite).
__device__ __forceinline__ double dbl_prev(double d) {
  if (d == 0.0) return -4.9406564584124654e-324;
  const long long u = __double_as_longlong(d);
  return __longlong_as_double(d > 0.0 ? u - 1 : u + 1);
}

// ---------------------------------------------------------- LDS atomics
// Explicit address-space-3 atomics for workgroup-shared counters and
// histograms: they lower to ds_* instructions, never to flat atomics.
#define PLH_LDS(T, p) ((__attribute__((address_space(3))) T*)(p))

__device__ __forceinline__ void lds_add(uint32_t* p, uint32_t v) {
  __hip_atomic_fetch_add(PLH_LDS(uint32_t, p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_add(uint64_t* p, uint64_t v) {
  __hip_atomic_fetch_add(PLH_LDS(uint64_t, p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ int lds_fetch_add(int* p, int v) {
  return __hip_atomic_fetch_add(PLH_LDS(int, p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_or(uint32_t* p, uint32_t v) {
  __hip_atomic_fetch_or(PLH_LDS(uint32_t, p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_min(int* p, int v) {
  __hip_atomic_fetch_min(PLH_LDS(int, p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_max(int* p, int v) {
  __hip_atomic_fetch_max(PLH_LDS(int, p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Device-wide counters in global memory (address space 1), agent scope.
#define PLH_GLB(T, p) ((__attribute__((address_space(1))) T*)(p))

__device__ __forceinline__ uint32_t glb_fetch_add(uint32_t* p, uint32_t v) {
  return __hip_atomic_fetch_add(PLH_GLB(uint32_t, p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void glb_add(unsigned long long* p, unsigned long long v) {
  __hip_atomic_fetch_add(PLH_GLB(unsigned long long, p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------ reductions

// DPP controls (gfx9 encoding).
constexpr int kDppRowShr1 = 0x111, kDppRowShr2 = 0x112, kDppRowShr4 = 0x114, kDppRowShr8 = 0x118;
constexpr int kDppWaveShr1 = 0x138, kDppRowBcast15 = 0x142, kDppRowBcast31 = 0x143;

// One DPP move of a 4- or 8-byte value: lanes whose source is outside the
// pattern, or whose row is not in ROWM, receive `old`.
template <int CTRL, int ROWM, typename T>
__device__ __forceinline__ T dpp(T old, T src) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "4- or 8-byte values");
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old),
                                                             __builtin_bit_cast(int, src), CTRL, ROWM, 0xf, false));
  } else {
    const uint64_t o = __builtin_bit_cast(uint64_t, old), v = __builtin_bit_cast(uint64_t, src);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp((int)(uint32_t)o, (int)(uint32_t)v, CTRL, ROWM, 0xf, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp((int)(uint32_t)(o >> 32), (int)(uint32_t)(v >> 32), CTRL,
                                                              ROWM, 0xf, false);
    return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
  }
}

// A value the caller knows to be the same in every lane (a workgroup
// reduction read back from LDS, say), moved to scalar registers so that it
// costs no VGPRs.
__device__ __forceinline__ double uniform(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)u);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(u >> 32));
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ uint64_t uniform(uint64_t v) {
  return __builtin_bit_cast(uint64_t, uniform(__builtin_bit_cast(double, v)));
}

// Value of lane l (uniform).
template <typename T>
__device__ __forceinline__ T lane_value(T v, int l) {
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
  } else {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), l);
    return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
  }
}

// Inclusive scan over the 64 lanes with an associative op and its identity.
template <typename T, class Op>
__device__ __forceinline__ T wave_scan_incl(T v, T id, const Op& op) {
  v = op(v, dpp<kDppRowShr1, 0xf>(id, v));
  v = op(v, dpp<kDppRowShr2, 0xf>(id, v));
  v = op(v, dpp<kDppRowShr4, 0xf>(id, v));
  v = op(v, dpp<kDppRowShr8, 0xf>(id, v));
  v = op(v, dpp<kDppRowBcast15, 0xa>(id, v));
  v = op(v, dpp<kDppRowBcast31, 0xc>(id, v));
  return v;
}

// The inclusive value of the previous lane (id for lane 0).
template <typename T>
__device__ __forceinline__ T wave_shift_up1(T incl, T id) {
  return dpp<kDppWaveShr1, 0xf>(id, incl);
}

struct OpAdd {
  template <typename T>
  __device__ __forceinline__ T operator()(T a, T b) const { return a + b; }
};
struct OpMax {
  template <typename T>
  __device__ __forceinline__ T operator()(T a, T b) const { return b > a ? b : a; }
};
struct OpOr {
  template <typename T>
  __device__ __forceinline__ T operator()(T a, T b) const { return a | b; }
};
struct OpMin {
  template <typename T>
  __device__ __forceinline__ T operator()(T a, T b) const { return b < a ? b : a; }
};

// Wave reductions; every lane receives the result.
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
  return lane_value(wave_scan_incl(v, T(0), OpAdd{}), kWave - 1);
}

template <typename T>
__device__ __forceinline__ T wave_max(T v) {
  return lane_value(wave_scan_incl(v, v, OpMax{}), kWave - 1);
}

template <typename T>
__device__ __forceinline__ T wave_min(T v) {
  return lane_value(wave_scan_incl(v, v, OpMin{}), kWave - 1);
}

// All threads of the workgroup receive the result.  `red` holds kWaves slots.
template <typename T>
__device__ __forceinline__ T block_sum(T v, T* red) {
  v = wave_sum(v);
  if (lane() == 0) red[wave()] = v;
  wg_barrier();
  T r = red[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) r += red[w];
  wg_barrier();
  return r;
}

template <typename T>
__device__ __forceinline__ T block_max(T v, T* red) {
  v = wave_max(v);
  if (lane() == 0) red[wave()] = v;
  wg_barrier();
  T r = red[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) r = red[w] > r ? red[w] : r;
  wg_barrier();
  return r;
}

template <typename T>
__device__ __forceinline__ T block_min(T v, T* red) {
  v = wave_min(v);
  if (lane() == 0) red[wave()] = v;
  wg_barrier();
  T r = red[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) r = red[w] < r ? red[w] : r;
  wg_barrier();
  return r;
}

// (value, index) maximum; ties go to the lowest index, as numpy's argmax.
struct ArgMax {
  double v;
  int i;
};

__device__ __forceinline__ ArgMax argmax_merge(ArgMax a, ArgMax b) {
  return (b.v > a.v || (b.v == a.v && b.i < a.i)) ? b : a;
}

// Wave argmax (value, lowest index); every lane receives the result.
__device__ __forceinline__ ArgMax wave_argmax(ArgMax a) {
  const ArgMax id{-INFINITY, INT_MAX};
  auto step = [&](ArgMax o) { a = argmax_merge(a, o); };
  step(ArgMax{dpp<kDppRowShr1, 0xf>(id.v, a.v), dpp<kDppRowShr1, 0xf>(id.i, a.i)});
  step(ArgMax{dpp<kDppRowShr2, 0xf>(id.v, a.v), dpp<kDppRowShr2, 0xf>(id.i, a.i)});
  step(ArgMax{dpp<kDppRowShr4, 0xf>(id.v, a.v), dpp<kDppRowShr4, 0xf>(id.i, a.i)});
  step(ArgMax{dpp<kDppRowShr8, 0xf>(id.v, a.v), dpp<kDppRowShr8, 0xf>(id.i, a.i)});
  step(ArgMax{dpp<kDppRowBcast15, 0xa>(id.v, a.v), dpp<kDppRowBcast15, 0xa>(id.i, a.i)});
  step(ArgMax{dpp<kDppRowBcast31, 0xc>(id.v, a.v), dpp<kDppRowBcast31, 0xc>(id.i, a.i)});
  return ArgMax{lane_value(a.v, kWave - 1), lane_value(a.i, kWave - 1)};
}

__device__ __forceinline__ ArgMax block_argmax(ArgMax a, double* redd, int* redi) {
  // wave: a max-scan of (value, index) pairs (each DPP step moves both)
  const ArgMax id{-INFINITY, INT_MAX};
  auto step = [&](ArgMax o) { a = argmax_merge(a, o); };
  step(ArgMax{dpp<kDppRowShr1, 0xf>(id.v, a.v), dpp<kDppRowShr1, 0xf>(id.i, a.i)});
  step(ArgMax{dpp<kDppRowShr2, 0xf>(id.v, a.v), dpp<kDppRowShr2, 0xf>(id.i, a.i)});
  step(ArgMax{dpp<kDppRowShr4, 0xf>(id.v, a.v), dpp<kDppRowShr4, 0xf>(id.i, a.i)});
  step(ArgMax{dpp<kDppRowShr8, 0xf>(id.v, a.v), dpp<kDppRowShr8, 0xf>(id.i, a.i)});
  step(ArgMax{dpp<kDppRowBcast15, 0xa>(id.v, a.v), dpp<kDppRowBcast15, 0xa>(id.i, a.i)});
  step(ArgMax{dpp<kDppRowBcast31, 0xc>(id.v, a.v), dpp<kDppRowBcast31, 0xc>(id.i, a.i)});
  if (lane() == kWave - 1) {
    redd[wave()] = a.v;
    redi[wave()] = a.i;
  }
  wg_barrier();
  ArgMax r{redd[0], redi[0]};
#pragma unroll
  for (int w = 1; w < kWaves; ++w) r = argmax_merge(r, ArgMax{redd[w], redi[w]});
  wg_barrier();
  return r;
}

// Exclusive scan of one unsigned integer per thread in thread order; *total
// receives the sum over the workgroup.  Exact.
template <typename T>
__device__ __forceinline__ T block_excl_scan(T v, T* red, T* total) {
  const T x = wave_scan_incl(v, T(0), OpAdd{});
  if (lane() == kWave - 1) red[wave()] = x;
  wg_barrier();
  T pre = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const T s = red[w];
    if (w < wave()) pre += s;
    tot += s;
  }
  wg_barrier();
  *total = tot;
  return pre + (x - v);
}

}  // namespace plh
