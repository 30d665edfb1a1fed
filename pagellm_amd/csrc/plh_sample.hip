// gfx950 kernels for the batched sampler (src/pagellm/engine/sampling.py:52-111).
//
//   k_sample_rows   one workgroup per row, any parameters; streams the row as
//                   many times as the pipeline needs.  Also the only kernel
//                   that exports the processed distribution (probs()).
//   k_sample_split  the fast path: one workgroup per (row, 8192-element
//                   chunk).  Each chunk is read from HBM once, held in
//                   registers, penalised, reduced, and summarised (max and
//                   argmax, softmax partial sum, fixed-point tile masses, or a
//                   compacted candidate set for top-k / top-p).  The last
//                   workgroup of a row to arrive (agent-scope atomic counter)
//                   finishes the row from the summaries alone; a row whose
//                   candidates cannot decide it exactly is finished by the
//                   row-wise pipeline in that same workgroup.
//   k_draw          inverse-CDF draw from given distributions (draw()).
//   k_penalize      repetition penalty on a copy (apply_repetition_penalty()).
#include "plh_kernels.h"
#include "plh_pipeline.h"

namespace plh {

constexpr int kTile = 4 * kThreads;                // elements per tile (one 16-byte load per thread)
constexpr double kFx48 = 281474976710656.0;        // 2^48: a chunk's masses relative to its max

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
__device__ __forceinline__ int row_general(const SampleArgs& a, int row, const RowParams& rp, Smem& sm, double* probs_out) {
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

// ------------------------------------------------------------------ split

// Element e (0..15) of the calling thread sits at chunk offset
// (e / 4) * kTile + 4 * tid + e % 4: every load is a coalesced 16-byte access.
constexpr int kEPT = 4 * kChunkTiles;  // elements per thread

template <typename TIn, bool VEC>
__device__ __forceinline__ void load_chunk(const TIn* x, int cn, double z[kEPT]) {
  const int t4 = 4 * (int)threadIdx.x;
  if constexpr (sizeof(TIn) == 4) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    f4 raw[kChunkTiles];
#pragma unroll
    for (int j = 0; j < kChunkTiles; ++j) {
      const int p0 = j * kTile + t4;
      if (VEC && p0 + 3 < cn) {
        raw[j] = *reinterpret_cast<const f4*>(x + p0);
      } else {
#pragma unroll
        for (int l = 0; l < 4; ++l) raw[j][l] = (p0 + l < cn) ? x[p0 + l] : -INFINITY;
      }
    }
#pragma unroll
    for (int j = 0; j < kChunkTiles; ++j)
#pragma unroll
      for (int l = 0; l < 4; ++l) z[4 * j + l] = (double)raw[j][l];
  } else {
    typedef double d2 __attribute__((ext_vector_type(2)));
    d2 raw[2 * kChunkTiles];
#pragma unroll
    for (int j = 0; j < kChunkTiles; ++j) {
      const int p0 = j * kTile + t4;
      if (VEC && p0 + 3 < cn) {
        raw[2 * j] = *reinterpret_cast<const d2*>(x + p0);
        raw[2 * j + 1] = *reinterpret_cast<const d2*>(x + p0 + 2);
      } else {
#pragma unroll
        for (int l = 0; l < 4; ++l) raw[2 * j + (l >> 1)][l & 1] = (p0 + l < cn) ? x[p0 + l] : -INFINITY;
      }
    }
#pragma unroll
    for (int j = 0; j < kChunkTiles; ++j)
#pragma unroll
      for (int l = 0; l < 4; ++l) z[4 * j + l] = raw[2 * j + (l >> 1)][l & 1];
  }
}

__device__ __forceinline__ uint64_t fx48(double e) { return e > 0.0 ? (uint64_t)__double2ull_rn(e * kFx48) : 0ull; }

// exp(y - ymc) for the chunk softmax partials, y = z/T by multiplication with
// 1/T (the chunk partials only feed sums; exact y is used for decisions).
struct ChunkExp {
  double T, invT, ymc;
  __device__ __forceinline__ double operator()(double z) const {
    if (z == -INFINITY) return 0.0;
    const double y = (T == 1.0) ? z : z * invT;
    return exp(y - ymc);
  }
};

__device__ __forceinline__ ChunkExp chunk_exp(double T, double zmax_c) {
  ChunkExp c;
  c.T = T;
  c.invT = 1.0 / T;
  c.ymc = (zmax_c == -INFINITY) ? 0.0 : ((T == 1.0) ? zmax_c : zmax_c / T);
  return c;
}

// Temperature-only rows: locate u * (row mass) through the chunks' tile
// masses, then rescan the one tile that holds it (sampling.py:94-98).
template <typename TIn, bool VEC>
__device__ __forceinline__ int temp_finalize(const SampleArgs& a, int row, const RowParams& rp, double zmax, Smem& sm) {
  const ChunkSum* rs = a.sums + (size_t)row * a.G;
  const int G = a.G;
  const double T = rp.T;
  const double ymax = (T == 1.0) ? zmax : zmax / T;
  auto chunk_scale = [&](int c) -> double {
    const double zc = rs[c].zmax;
    if (zc == -INFINITY) return 0.0;
    const double ymc = (T == 1.0) ? zc : zc / T;
    return exp(ymc - ymax);
  };
  auto chunk_total = [&](int c) -> uint64_t {
    uint64_t t = 0;
#pragma unroll
    for (int j = 0; j < kChunkTiles; ++j) t += rs[c].tile[j];
    return t;
  };
  double M = 0.0;
  for (int c = 0; c < G; ++c) M += (double)chunk_total(c) * chunk_scale(c);
  const double t = rp.u * M;
  int cstar = -1;
  double before = 0.0;
  {
    double run = 0.0;
    for (int c = 0; c < G; ++c) {
      const double m = (double)chunk_total(c) * chunk_scale(c);
      if (run + m > t) {
        cstar = c;
        before = run;
        break;
      }
      run += m;
    }
  }
  if (cstar < 0) return a.V - 1;  // u * total rounded up to the total
  const uint64_t tc = chunk_total(cstar);
  const double tin = (t - before) / chunk_scale(cstar);
  uint64_t tfx = tin > 0.0 ? (uint64_t)__double2ull_rd(tin) : 0ull;
  if (tfx >= tc) tfx = tc - 1;
  int jstar = kChunkTiles - 1;
  uint64_t cum = 0;
  for (int j = 0; j < kChunkTiles; ++j) {
    const uint64_t tj = rs[cstar].tile[j];
    if (cum + tj > tfx) {
      jstar = j;
      break;
    }
    cum += tj;
  }
  // rescan tile jstar of chunk cstar with the chunk pass's exact arithmetic
  const int lo = cstar * kChunk;
  const int cn = min(kChunk, a.V - lo);
  const int tlo = jstar * kTile;
  const TIn* x = reinterpret_cast<const TIn*>(a.logits) + (int64_t)row * a.ld + lo;
  if (rp.pen_active) build_bitmap(sm.bitmap, lo + tlo, kTile, a.hist_ids, rp.h0, rp.h1);
  const ChunkExp ce = chunk_exp(T, rs[cstar].zmax);
  const int p0 = tlo + 4 * (int)threadIdx.x;
  uint64_t w[4], s = 0;
  const uint32_t bits = (rp.pen_active && p0 < cn) ? (sm.bitmap[(4 * threadIdx.x) >> 5] >> ((4 * threadIdx.x) & 31)) : 0u;
#pragma unroll
  for (int l = 0; l < 4; ++l) {
    w[l] = 0;
    if (p0 + l < cn) {
      double z = (double)x[p0 + l];
      if ((bits >> l) & 1u) z = penalize(z, rp.pen);
      w[l] = fx48(ce(z));
    }
    s += w[l];
  }
  uint64_t tile_tot;
  const uint64_t ex = block_excl_scan<uint64_t>(s, sm.redu, &tile_tot);
  uint64_t c = cum + ex;
  int my = INT_MAX;
#pragma unroll
  for (int l = 0; l < 4; ++l) {
    c += w[l];
    if (my == INT_MAX && c > tfx) my = lo + p0 + l;
  }
  const int found = block_min<int>(my, sm.redi);
  return found == INT_MAX ? a.V - 1 : found;
}

template <typename TIn, bool VEC>
__global__ __launch_bounds__(kThreads, 4) void k_sample_split(SampleArgs a) {
  __shared__ Smem sm;
  const int G = a.G;
  int row, chunk;
  if (a.xcd_map) {
    // consecutive workgroups land on different XCDs; keep a row's chunks on
    // one XCD so its history, summaries and candidates share that L2
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
    row = xcd + 8 * (slot / G);
    chunk = slot % G;
  } else {
    row = blockIdx.x / G;
    chunk = blockIdx.x % G;
  }
  if (row >= a.B) return;
  const int V = a.V;
  const int tid = threadIdx.x;
  const RowParams rp = load_row_params(a, row);
  const int lo = chunk * kChunk;
  const int cn = min(kChunk, V - lo);
  const TIn* x = reinterpret_cast<const TIn*>(a.logits) + (int64_t)row * a.ld + lo;

  double z[kEPT];
  load_chunk<TIn, VEC>(x, cn, z);
  // bit e: element e lies inside the row
  uint32_t vmask = 0;
#pragma unroll
  for (int e = 0; e < kEPT; ++e)
    if ((e >> 2) * kTile + 4 * tid + (e & 3) < cn) vmask |= 1u << e;

  // ---- repetition penalty, once per distinct history id (sampling.py:52-62)
  if (rp.pen_active) {
    build_bitmap(sm.bitmap, lo, cn, a.hist_ids, rp.h0, rp.h1);
#pragma unroll
    for (int j = 0; j < kChunkTiles; ++j) {
      const int p0 = j * kTile + 4 * tid;
      if (p0 < cn) {
        const uint32_t w = sm.bitmap[p0 >> 5] >> (p0 & 31);
        if (w & 0xFu) {
#pragma unroll
          for (int l = 0; l < 4; ++l)
            if ((w >> l) & 1u) z[4 * j + l] = penalize(z[4 * j + l], rp.pen);
        }
      }
    }
  }

  // ---- chunk max and argmax (lowest index on ties)
  ArgMax best{-INFINITY, INT_MAX};
#pragma unroll
  for (int e = 0; e < kEPT; ++e)
    if ((vmask >> e) & 1u) best = argmax_merge(best, ArgMax{z[e], lo + (e >> 2) * kTile + 4 * tid + (e & 3)});
  best = block_argmax(best, sm.redd, sm.redi);

  ChunkSum* cs = a.sums + (size_t)row * G + chunk;
  const bool temp_only = !rp.greedy && !rp.topk && !rp.topp;
  if (temp_only) {
    const ChunkExp ce = chunk_exp(rp.T, best.v);
    uint64_t tiles[kChunkTiles];
#pragma unroll
    for (int j = 0; j < kChunkTiles; ++j) {
      uint64_t s = 0;
#pragma unroll
      for (int l = 0; l < 4; ++l)
        if ((vmask >> (4 * j + l)) & 1u) s += fx48(ce(z[4 * j + l]));
      tiles[j] = block_sum<uint64_t>(s, sm.redu);
    }
    if (tid == 0) {
#pragma unroll
      for (int j = 0; j < kChunkTiles; ++j) cs->tile[j] = tiles[j];
    }
  } else if (!rp.greedy) {
    // ---- softmax partial for top-p rows without top-k (exp relative to the chunk max)
    double s_c = 0.0;
    if (!rp.topk) {
      const ChunkExp ce = chunk_exp(rp.T, best.v);
      double s = 0.0;
#pragma unroll
      for (int e = 0; e < kEPT; ++e)
        if ((vmask >> e) & 1u) s += ce(z[e]);
      s_c = block_sum(s, sm.redd);
    }
    // ---- retain candidates: everything with key32 >= L
    //   top-k rows: at least the chunk's top-k (whole coarse bins), at most cap
    //   top-p rows: at most cap, as many as two 11-bit digits resolve
    uint64_t L = 0;
    bool overflow = false;
    const int cap = a.cap;
    if (cn > cap) {
      const uint64_t target = rp.topk ? (uint64_t)rp.top_k : (uint64_t)cap + 1;
      if (target > (uint64_t)cn) {
        overflow = true;
      } else {
        uint32_t prefix = 0;
        uint64_t above = 0;
        int done = 0;
        const int widths[3] = {11, 11, 10};
        for (int pass = 0; pass < 3; ++pass) {
          const int w = widths[pass];
          const int shift = 32 - done - w;
          const int nb = 1 << w;
          for (int b = tid; b < nb; b += kThreads) sm.cnt[b] = 0u;
          __syncthreads();
#pragma unroll
          for (int e = 0; e < kEPT; ++e) {
            if ((vmask >> e) & 1u) {
              const uint32_t k = key32_of(z[e]);
              if (done == 0 || (k >> (32 - done)) == prefix) lds_add(&sm.cnt[(k >> shift) & (uint32_t)(nb - 1)], 1u);
            }
          }
          __syncthreads();
          const BinPick bp = pick_bin_desc<false>(sm, nb, above, target);
          const uint32_t bcnt = sm.cnt[bp.d];
          __syncthreads();
          const uint32_t np = (prefix << w) | (uint32_t)bp.d;
          const int nd = done + w;
          if (rp.topk) {
            if (bp.above + bcnt <= (uint64_t)cap) {  // keep the whole bin
              L = (uint64_t)np << (32 - nd);
              break;
            }
            if (nd == 32) {  // exact key with more ties than the capacity
              L = np;
              overflow = true;
              break;
            }
          } else if (pass == 1 || nd == 32) {  // keep strictly above the bin
            L = ((uint64_t)np + 1) << (32 - nd);
            break;
          }
          prefix = np;
          above = bp.above;
          done = nd;
        }
      }
    }
    // ---- ordered compaction of the retained elements (index order within the chunk)
    double umax = -INFINITY;
    uint64_t packed = 0;  // 16-bit retained count per tile
    uint32_t rmask = 0;
    if (!overflow) {
#pragma unroll
      for (int e = 0; e < kEPT; ++e) {
        if ((vmask >> e) & 1u) {
          if ((uint64_t)key32_of(z[e]) >= L) rmask |= 1u << e;
          else umax = z[e] > umax ? z[e] : umax;
        }
      }
#pragma unroll
      for (int j = 0; j < kChunkTiles; ++j) packed |= (uint64_t)__popc((rmask >> (4 * j)) & 0xFu) << (16 * j);
    }
    uint64_t ptot;
    const uint64_t pex = block_excl_scan<uint64_t>(packed, sm.redu, &ptot);
    umax = block_max(umax, sm.redd);
    int ncand = 0;
    if (!overflow) {
      const size_t cbase = ((size_t)row * G + chunk) * (size_t)cap;
      int base = 0;
#pragma unroll
      for (int j = 0; j < kChunkTiles; ++j) {
        int pos = base + (int)((pex >> (16 * j)) & 0xFFFFull);
#pragma unroll
        for (int l = 0; l < 4; ++l) {
          const int e = 4 * j + l;
          if ((rmask >> e) & 1u) {
            a.cz[cbase + pos] = z[e];
            a.cidx[cbase + pos] = lo + j * kTile + 4 * tid + l;
            ++pos;
          }
        }
        base += (int)((ptot >> (16 * j)) & 0xFFFFull);
      }
      ncand = base;
    }
    if (tid == 0) {
      cs->ncand = overflow ? -1 : ncand;
      cs->umax = umax;
      cs->s = s_c;
    }
  }
  if (tid == 0) {
    cs->zmax = best.v;
    cs->argmax = best.i;
  }

  // ---- arrival: the last chunk of the row finishes it
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const unsigned prev = glb_fetch_add(&a.row_count[row], 1u);
    sm.ctl_i[8] = (prev == (unsigned)(G - 1)) ? 1 : 0;
  }
  __syncthreads();
  if (sm.ctl_i[8] == 0) return;
  __threadfence();

  const ChunkSum* rs = a.sums + (size_t)row * G;
  ArgMax rb{-INFINITY, INT_MAX};
  for (int c = tid; c < G; c += kThreads) rb = argmax_merge(rb, ArgMax{rs[c].zmax, rs[c].argmax});
  rb = block_argmax(rb, sm.redd, sm.redi);

  int id = V - 1;
  bool general = false;
  if (rp.greedy) {
    id = rb.i;
  } else if (temp_only) {
    id = temp_finalize<TIn, VEC>(a, row, rp, rb.v, sm);
  } else {
    if (tid == 0) {
      int acc = 0, bad = 0;
      sm.cpref[0] = 0;
      for (int c = 0; c < G; ++c) {
        const int n = rs[c].ncand;
        if (n < 0) bad = 1;
        acc += n < 0 ? 0 : n;
        sm.cpref[c + 1] = acc;
      }
      sm.ctl_i[9] = bad;
    }
    __syncthreads();
    if (sm.ctl_i[9]) {
      general = true;
    } else {
      double U = -INFINITY;
      for (int c = tid; c < G; c += kThreads) U = rs[c].umax > U ? rs[c].umax : U;
      U = block_max(U, sm.redd);
      double S = 0.0;
      if (!rp.topk) {  // softmax normaliser over the whole row from the chunk partials
        const double ymax = (rp.T == 1.0) ? rb.v : rb.v / rp.T;
        for (int c = 0; c < G; ++c) {
          const double zc = rs[c].zmax;
          if (zc == -INFINITY) continue;
          const double ymc = (rp.T == 1.0) ? zc : zc / rp.T;
          S += rs[c].s * exp(ymc - ymax);
        }
      }
      const size_t rbase = (size_t)row * G * (size_t)a.cap;
      CandSource src{a.cz + rbase, a.cidx + rbase, a.cp + rbase, sm.cpref, G, a.cap, sm.cpref[G], false};
      const PipeIn in{true, rb.v, rb.i, !rp.topk, S, true, U};
      const PipeOut o = row_pipeline(src, rp, V, in, sm, nullptr);
      if (o.insufficient) general = true;
      else id = o.id;
    }
  }
  if (general) {
    if (tid == 0) glb_add(a.fallback_rows, 1ull);
    id = row_general<TIn, VEC>(a, row, rp, sm, nullptr);
  }
  if (tid == 0) {
    a.out_ids[row] = id;
    a.row_count[row] = 0u;
  }
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

hipError_t launch_sample_split(const SampleArgs& a, bool f64, bool vec, hipStream_t s) {
  const int rows = a.xcd_map ? 8 * ((a.B + 7) / 8) : a.B;
  const dim3 grid(rows * a.G), block(kThreads);
  if (f64) {
    if (vec) hipLaunchKernelGGL((k_sample_split<double, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((k_sample_split<double, false>), grid, block, 0, s, a);
  } else {
    if (vec) hipLaunchKernelGGL((k_sample_split<float, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((k_sample_split<float, false>), grid, block, 0, s, a);
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
