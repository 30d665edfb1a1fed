// gfx950 kernels for speculative decoding's accept/resample step
// (src/pagellm/engine/speculative.py:38-60).
//
// The k accept tests are k gathered scalars: accept x_i while
// u_i < min(1, p_i[x_i] / q_i[x_i]) (strict), stop at the first rejection.
// Only the stop position's rows are then streamed: on a rejection at i the
// residual max(p_i - q_i, 0) (or p_i when the residual is all zero), after k
// acceptances the bonus row p_k; the emitted token is an inverse-CDF draw
// over that row.
//
// A row's draw is spread over chunks of 4096 tokens, one workgroup each, so
// that a batch of a few dozen rows still fills the chip:
//   k_verify_parts  (row, chunk)  stop position; float64 chunk sums of the
//                                 residual and of p;
//   k_verify_draw   (row)         W and the running chunk totals in one fixed
//                                 order; the first chunk whose running total
//                                 exceeds u * W is rescanned in float64 for
//                                 the token.
// The float64 running sums add the weights in another order than numpy's
// cumsum; the token they give differs from the reference's only when u lies
// within ~1e-15 (relative) of a CDF boundary.  When the rescan's own
// rounding leaves the crossing just past the chunk's end, the chunk's last
// token of positive weight is taken (a neighbour of the boundary either
// way).
#include "plh_kernels.h"
#include "plh_pipeline.h"

namespace plh {

constexpr int kVPer = 8;                   // tokens per thread in a chunk
constexpr int kVChunk = kVPer * kThreads;  // tokens per chunk

__host__ __device__ constexpr int verify_chunks(int V) { return (V + kVChunk - 1) / kVChunk; }

// Stop position of row b (speculative.py:51-60): the first i < k whose
// draft id is out of range (-1) or whose accept test fails (i), else k.
// Computed by each calling wave on its own (k gathers per 64 tests).
template <typename TIn>
__device__ __forceinline__ int stop_position(const VerifyArgs& a, const TIn* P, const TIn* Q, int b) {
  const int k = a.k, V = a.V;
  for (int base = 0; base < k; base += kWave) {
    const int i = base + lane();
    bool bad = false, stop = false;
    if (i < k) {
      const int x = a.draft[(size_t)b * k + i];
      bad = x < 0 || x >= V;  // rejected by the host wrapper; never index with it
      if (!bad) {
        const double r = (double)P[(size_t)i * V + x] / (double)Q[(size_t)i * V + x];
        const double thr = r < 1.0 ? r : 1.0;  // Python min(1.0, r): NaN -> 1.0
        stop = !(a.accept_u[(size_t)b * k + i] < thr);
      }
    }
    const uint64_t m = __ballot(bad || stop);
    if (m != 0) {
      const int f = __builtin_ctzll(m);
      return lane_value((int)bad, f) ? -1 : base + f;
    }
  }
  return k;
}

// What the draw reads from row b's stop position s: the residual
// max(p_s - q_s, 0) unless it sums to zero (speculative.py:55-58), else
// max(p_s, 0); and its float64 total W.  W comes from the chunk sums in one
// fixed order (lane j adds chunks j, j + 64, ..., then the wave's sum tree),
// so every wave of every launch gets the same bits.
struct DrawTotal {
  bool resid;
  double W;
};

// The calling lane's share of row b's chunk sums (residual, p); loaded
// before the stop position is known (they do not depend on it).
struct PartLanes {
  double sr, sp;
};

__device__ __forceinline__ PartLanes load_part_lanes(const VerifyWs& ws, int b) {
  const int C = ws.C;
  const double* part = ws.part + (size_t)b * C * 2;
  // the first 64 chunks, one per lane, loaded unconditionally (lanes past
  // C read chunk C - 1 and drop it in finish_part_lanes): no branch whose
  // join would make the compiler wait for the loads here
  const int j = min(lane(), C - 1);
  return PartLanes{part[2 * j], part[2 * j + 1]};
}

__device__ __forceinline__ void finish_part_lanes(const VerifyWs& ws, int b, PartLanes& pl) {
  const int C = ws.C;
  const double* part = ws.part + (size_t)b * C * 2;
  if (lane() >= C) pl = PartLanes{0.0, 0.0};
  for (int j = lane() + kWave; j < C; j += kWave) {
    pl.sr += part[2 * j];
    pl.sp += part[2 * j + 1];
  }
}

__device__ __forceinline__ DrawTotal draw_total(const PartLanes& pl, int s, int k) {
  const double sr = wave_sum(pl.sr);
  const double sp = wave_sum(pl.sp);
  const bool resid = s < k && sr > 0.0;
  return DrawTotal{resid, resid ? sr : sp};
}

// The draw weight of one token from its p and q values (q is ignored unless
// the draw is over the residual); tokens past V weigh nothing.
__device__ __forceinline__ double draw_weight(double p, double q, bool resid, bool in_row) {
  const double v = p - (resid ? q : 0.0);
  return in_row && v > 0.0 ? v : 0.0;
}

template <typename TIn>
__global__ __launch_bounds__(kThreads) void k_verify_parts(VerifyArgs a, VerifyWs ws) {
  __shared__ double red[2][kWaves];
  const int C = ws.C;
  const int b = blockIdx.x / C, c = blockIdx.x - b * C;
  const int k = a.k, V = a.V;
  const TIn* P = reinterpret_cast<const TIn*>(a.p) + (size_t)b * (k + 1) * V;
  const TIn* Q = reinterpret_cast<const TIn*>(a.q) + (size_t)b * k * V;
  const int s = stop_position(a, P, Q, b);
  if (c == 0 && threadIdx.x == 0) ws.stop[b] = s;
  if (s < 0) return;
  const TIn* ps = P + (size_t)s * V;
  const int i0 = c * kVChunk + (int)threadIdx.x;
  double sr = 0.0, sp = 0.0;
  if (s < k) {
    const TIn* qs = Q + (size_t)s * V;
    TIn pv[kVPer], qv[kVPer];
#pragma unroll
    for (int l = 0; l < kVPer; ++l) {
      const int i = i0 + l * kThreads;
      pv[l] = i < V ? ps[i] : TIn(0);
      qv[l] = i < V ? qs[i] : TIn(0);
    }
#pragma unroll
    for (int l = 0; l < kVPer; ++l) {
      const double d = (double)pv[l] - (double)qv[l];
      sr += d > 0.0 ? d : 0.0;
      sp += (double)pv[l] > 0.0 ? (double)pv[l] : 0.0;
    }
  } else {
    TIn pv[kVPer];
#pragma unroll
    for (int l = 0; l < kVPer; ++l) {
      const int i = i0 + l * kThreads;
      pv[l] = i < V ? ps[i] : TIn(0);
    }
#pragma unroll
    for (int l = 0; l < kVPer; ++l) sp += (double)pv[l] > 0.0 ? (double)pv[l] : 0.0;
  }
  sr = wave_sum(sr);
  sp = wave_sum(sp);
  if (lane() == 0) {
    red[0][wave()] = sr;
    red[1][wave()] = sp;
  }
  wg_barrier();
  if (threadIdx.x == 0) {
    double tr = red[0][0], tp = red[1][0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) {
      tr += red[0][w];
      tp += red[1][w];
    }
    ws.part[2 * (size_t)blockIdx.x] = tr;
    ws.part[2 * (size_t)blockIdx.x + 1] = tp;
  }
}

template <typename TIn>
__global__ __launch_bounds__(kThreads) void k_verify_draw(VerifyArgs a, VerifyWs ws) {
  __shared__ double redd[kWaves];
  __shared__ int redi[kWaves];
  const int b = blockIdx.x;
  const int k = a.k, V = a.V, C = ws.C;
  // the chunk sums and the uniforms travel with the stop position (none of
  // their addresses depends on it); per-stop uniforms: lane i holds u_i
  PartLanes pl = load_part_lanes(ws, b);
  double ul = a.draw_u[a.draw_u_per_stop ? (size_t)b * (k + 1) + min(lane(), k) : (size_t)b];
  const int s_in = ws.stop[b];
  asm volatile("" : "+v"(ul), "+v"(pl.sr), "+v"(pl.sp));  // all of them in, before the branch on the stop
  finish_part_lanes(ws, b, pl);
  const int s = uniform(s_in);
  int32_t* out = a.out_tokens + (size_t)b * (k + 1);
  if (s < 0) {
    for (int i = threadIdx.x; i <= k; i += kThreads) out[i] = -1;
    if (threadIdx.x == 0) a.out_n_acc[b] = -1;
    return;
  }
  const double u = !a.draw_u_per_stop ? ul
                   : s < kWave        ? lane_value(ul, s)
                                      : a.draw_u[(size_t)b * (k + 1) + s];
  const DrawTotal d = draw_total(pl, s, k);
  int tok = V - 1;  // sampling.py:98: no mass takes the last id
  if (d.W > 0.0) {
    const double t = u * d.W;
    const double* part = ws.part + (size_t)b * C * 2 + (d.resid ? 0 : 1);
    // the first chunk whose running total exceeds t, else the last chunk
    // with mass (every wave alike, sums in one fixed order)
    int cs = -1, clast = -1;
    double before = 0.0, blast = 0.0, run = 0.0;
    for (int base = 0; base < C; base += kWave) {
      const int j = base + lane();
      const double v = j < C ? part[2 * j] : 0.0;
      const double incl = run + wave_scan_incl(v, 0.0, OpAdd{});
      const uint64_t pos = __ballot(j < C && v > 0.0);
      if (pos != 0) {
        const int f = 63 - __builtin_clzll(pos);
        clast = base + f;
        blast = lane_value(incl - v, f);
      }
      const uint64_t m = __ballot(j < C && incl > t);
      if (m != 0) {
        const int f = __builtin_ctzll(m);
        cs = base + f;
        before = lane_value(incl - v, f);
        break;
      }
      run = lane_value(incl, kWave - 1);
    }
    const bool crossed = cs >= 0;
    if (!crossed) {
      cs = clast;
      before = blast;
    }
    if (cs >= 0) {
      const TIn* ps = reinterpret_cast<const TIn*>(a.p) + ((size_t)b * (k + 1) + s) * V;
      const TIn* qs = s < k ? reinterpret_cast<const TIn*>(a.q) + ((size_t)b * k + s) * V : ps;
      const int i0 = cs * kVChunk + (int)threadIdx.x * kVPer;
      TIn pv[kVPer], qv[kVPer];
#pragma unroll
      for (int l = 0; l < kVPer; ++l) {
        const int i = min(i0 + l, V - 1);
        pv[l] = ps[i];
        qv[l] = qs[i];
      }
      double w[kVPer], ts = 0.0;
#pragma unroll
      for (int l = 0; l < kVPer; ++l) {
        w[l] = draw_weight((double)pv[l], (double)qv[l], d.resid, i0 + l < V);
        ts += w[l];
      }
      double tt;
      double cum = before + block_excl_scan<double>(ts, redd, &tt);
      int my = INT_MAX, mylast = -1;
#pragma unroll
      for (int l = 0; l < kVPer; ++l) {
        cum += w[l];
        if (crossed && my == INT_MAX && cum > t) my = i0 + l;
        if (w[l] > 0.0) mylast = i0 + l;
      }
      const int f = block_min<int>(my, redi);
      if (f != INT_MAX) {
        tok = f;
      } else {  // the crossing sits at the chunk's end (or u * W at the total)
        tok = block_max<int>(mylast, redi);
        if (tok < 0) tok = V - 1;
      }
    }
  }
  if (threadIdx.x == 0) {
    const int32_t* dr = a.draft + (size_t)b * k;
    for (int i = 0; i < s; ++i) out[i] = dr[i];
    out[s] = tok;
    for (int i = s + 1; i <= k; ++i) out[i] = -1;
    a.out_n_acc[b] = s;
  }
}

namespace {
size_t up256(size_t v) { return (v + 255) / 256 * 256; }
}  // namespace

size_t verify_ws_bytes(int B, int V) {
  const size_t n = (size_t)B * verify_chunks(V);
  return up256((size_t)B * sizeof(int32_t)) + up256(n * 2 * sizeof(double));
}

VerifyWs verify_ws_layout(void* base, int B, int V) {
  VerifyWs w{};
  w.C = verify_chunks(V);
  const size_t n = (size_t)B * w.C;
  char* p = static_cast<char*>(base);
  w.stop = reinterpret_cast<int32_t*>(p);
  p += up256((size_t)B * sizeof(int32_t));
  w.part = reinterpret_cast<double*>(p);
  return w;
}

template <typename TIn>
hipError_t launch_verify_t(const VerifyArgs& a, const VerifyWs& ws, hipStream_t s, hipEvent_t between) {
  const dim3 block(kThreads);
  const dim3 grid_parts((unsigned)((size_t)a.B * ws.C));
  hipLaunchKernelGGL((k_verify_parts<TIn>), grid_parts, block, 0, s, a, ws);
  if (between != nullptr) {
    const hipError_t e = hipEventRecord(between, s);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((k_verify_draw<TIn>), dim3(a.B), block, 0, s, a, ws);
  return hipGetLastError();
}

hipError_t launch_verify(const VerifyArgs& a, const VerifyWs& ws, bool f64, hipStream_t s, hipEvent_t between) {
  return f64 ? launch_verify_t<double>(a, ws, s, between) : launch_verify_t<float>(a, ws, s, between);
}

}  // namespace plh
