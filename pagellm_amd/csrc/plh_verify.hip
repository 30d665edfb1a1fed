// gfx950 kernel for speculative decoding's accept/resample step
// (src/pagellm/engine/speculative.py:38-60), one workgroup per sequence.
//
// The k accept tests are k gathered scalars: accept x_i while
// u_i < min(1, p_i[x_i] / q_i[x_i]) (strict), stop at the first rejection.
// Only the stop position's rows are then streamed: on a rejection at i the
// residual max(p_i - q_i, 0) (or p_i when the residual is all zero), after k
// acceptances the bonus row p_k; the emitted token is an inverse-CDF draw
// over that row.
#include "plh_kernels.h"
#include "plh_pipeline.h"

namespace plh {

template <typename TIn>
__global__ __launch_bounds__(kThreads) void k_verify(VerifyArgs a) {
  __shared__ double redd[kWaves];
  __shared__ uint64_t redu[kWaves];
  __shared__ int redi[kWaves];
  __shared__ int s_stop;
  const int b = blockIdx.x;
  const int k = a.k, V = a.V;
  const TIn* P = reinterpret_cast<const TIn*>(a.p) + (size_t)b * (k + 1) * V;
  const TIn* Q = reinterpret_cast<const TIn*>(a.q) + (size_t)b * k * V;
  if (threadIdx.x == 0) {
    int s = k;
    for (int i = 0; i < k; ++i) {
      const int x = a.draft[(size_t)b * k + i];
      if (x < 0 || x >= V) {  // rejected by the host wrapper; never index with it
        s = -1;
        break;
      }
      const double r = (double)P[(size_t)i * V + x] / (double)Q[(size_t)i * V + x];
      const double thr = r < 1.0 ? r : 1.0;  // Python min(1.0, r): NaN -> 1.0
      if (!(a.accept_u[(size_t)b * k + i] < thr)) {
        s = i;
        break;
      }
    }
    s_stop = s;
  }
  __syncthreads();
  const int s = s_stop;
  int32_t* out = a.out_tokens + (size_t)b * (k + 1);
  if (s < 0) {
    for (int i = threadIdx.x; i <= k; i += kThreads) out[i] = -1;
    if (threadIdx.x == 0) a.out_n_acc[b] = -1;
    return;
  }
  const double u = a.draw_u_per_stop ? a.draw_u[(size_t)b * (k + 1) + s] : a.draw_u[b];
  int tok;
  if (s < k) {
    const TIn* ps = P + (size_t)s * V;
    const TIn* qs = Q + (size_t)s * V;
    auto resid = [&](int i) -> double {
      const double d = (double)ps[i] - (double)qs[i];
      return d > 0.0 ? d : 0.0;
    };
    double sr = 0.0;
    for (int i = threadIdx.x; i < V; i += kThreads) sr += resid(i);
    sr = block_sum(sr, redd);
    if (sr > 0.0) {
      tok = draw_weights(resid, V, u, redd, redu, redi);
    } else {
      auto pw = [&](int i) -> double {
        const double v = (double)ps[i];
        return v > 0.0 ? v : 0.0;
      };
      tok = draw_weights(pw, V, u, redd, redu, redi);
    }
  } else {
    const TIn* pk = P + (size_t)k * V;
    auto pw = [&](int i) -> double {
      const double v = (double)pk[i];
      return v > 0.0 ? v : 0.0;
    };
    tok = draw_weights(pw, V, u, redd, redu, redi);
  }
  if (threadIdx.x == 0) {
    const int32_t* dr = a.draft + (size_t)b * k;
    for (int i = 0; i < s; ++i) out[i] = dr[i];
    out[s] = tok;
    for (int i = s + 1; i <= k; ++i) out[i] = -1;
    a.out_n_acc[b] = s;
  }
}

hipError_t launch_verify(const VerifyArgs& a, bool f64, hipStream_t s) {
  if (f64) hipLaunchKernelGGL((k_verify<double>), dim3(a.B), dim3(kThreads), 0, s, a);
  else hipLaunchKernelGGL((k_verify<float>), dim3(a.B), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace plh
