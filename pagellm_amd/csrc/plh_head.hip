// gfx950 kernels for the logits producer: the model's final RMSNorm and
// lm_head product, logits = rms_norm(h, norm, eps) @ lm_head
// (src/pagellm/model/transformer.py:79-82, :271), in float32 as the
// reference computes it, written straight into the sampler's logits buffer.
//
//   k_head_rmsnorm  one workgroup per row: r = 1 / sqrt(mean(h * h) + eps)
//                   in float32 (the squares summed in float64 and rounded
//                   once), act = (h * r) * norm, zero-padded to a multiple of
//                   32 columns;
//   k_head_gemm     out = act @ W on the fp32 matrix cores
//                   (v_mfma_f32_32x32x2_f32, products and sums in float32).
//                   A workgroup of 8 waves owns a 256-row x 256-column tile
//                   of out; each wave a 64 x 128 block, 2 x 4 MFMA tiles
//                   held in 128 accumulator registers.  The k dimension
//                   streams through LDS 32 at a time, double-buffered: the
//                   next stage's global loads are in flight while the
//                   matrix cores work on the current one.
#include "plh_device.h"
#include "plh_kernels.h"

namespace plh {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr int kHeadRows = 256;             // rows of out per workgroup
constexpr int kHeadCols = 256;             // vocabulary columns per workgroup
constexpr int kHeadK = 32;                 // k per LDS stage
constexpr int kAStride = kHeadK + 2;       // act tile row pitch (floats)
constexpr int kBStride = kHeadCols + 32;   // W tile row pitch (floats)

__host__ __device__ constexpr int head_kpad(int D) { return (D + kHeadK - 1) / kHeadK * kHeadK; }

__global__ __launch_bounds__(kThreads) void k_head_rmsnorm(HeadArgs a) {
  __shared__ double red[kWaves];
  const int n = blockIdx.x;
  const float* x = a.h + (size_t)n * a.ldh;
  double s = 0.0;
  for (int d = threadIdx.x; d < a.D; d += kThreads) {
    const float v = x[d];
    s += (double)(v * v);  // the float32 square, as numpy forms x * x
  }
  s = block_sum(s, red);
  // np.mean in float32, + eps as a float32 (a Python float is a weak
  // scalar), float32 sqrt and reciprocal (transformer.py:81)
  const float mean = (float)s / (float)a.D;
  const float r = 1.0f / sqrtf(mean + a.eps);
  float* out = a.act + (size_t)n * a.lda;
  const int Dp = head_kpad(a.D);
  for (int d = threadIdx.x; d < Dp; d += kThreads) out[d] = d < a.D ? (x[d] * r) * a.norm[d] : 0.0f;  // :82
}

struct HeadSmem {
  float a[2][kHeadRows * kAStride];
  float b[2][kHeadK * kBStride];
};

__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_head_gemm(HeadArgs a) {
  __shared__ HeadSmem sm;
  const int N = a.N, D = a.D, V = a.V;
  const int v0 = blockIdx.x * kHeadCols, n0 = blockIdx.y * kHeadRows;
  const int tid = threadIdx.x, l = lane(), w = wave();
  const int wn = w & 3, wv = w >> 2;

  // global -> register staging: act row tid/2, 16 columns from (tid%2)*16
  // (rows past N repeat row N-1; their results are not stored); W row
  // tid/16 of the stage, 16 columns from (tid%16)*16 (rows past D are zero)
  const float* ag = a.act + (size_t)min(n0 + (tid >> 1), N - 1) * a.lda + (tid & 1) * 16;
  const int br = tid >> 4, bc = (tid & 15) * 16;
  const bool bvec = v0 + kHeadCols <= V && (a.ldw & 3) == 0 && (reinterpret_cast<uintptr_t>(a.w) & 15) == 0;
  f32x4 pa[4], pb[4];
  auto load = [&](int kb) {
    const int k0 = kb * kHeadK;
#pragma unroll
    for (int j = 0; j < 4; ++j) pa[j] = *reinterpret_cast<const f32x4*>(ag + k0 + 4 * j);
    const int kr = k0 + br;
    const float* bg = a.w + (size_t)min(kr, D - 1) * a.ldw;
    if (bvec) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(bg + v0 + bc + 4 * j);
        pb[j] = kr < D ? v : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int v = v0 + bc + 4 * j + e;
          const float x = bg[min(v, V - 1)];
          pb[j][e] = (kr < D && v < V) ? x : 0.0f;
        }
    }
  };
  auto store = [&](int buf) {
    float* as = sm.a[buf] + (tid >> 1) * kAStride + (tid & 1) * 16;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      *reinterpret_cast<f32x2*>(as + 4 * j) = f32x2{pa[j][0], pa[j][1]};
      *reinterpret_cast<f32x2*>(as + 4 * j + 2) = f32x2{pa[j][2], pa[j][3]};
    }
    float* bs = sm.b[buf] + br * kBStride + bc;
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<f32x4*>(bs + 4 * j) = pb[j];
  };

  f32x16 acc[2][4];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mt][nt][r] = 0.0f;

  const int nkb = head_kpad(D) / kHeadK;
  load(0);
  store(0);
  wg_barrier();
  for (int kb = 0; kb < nkb; ++kb) {
    const int cur = kb & 1;
    if (kb + 1 < nkb) load(kb + 1);
    // operands of v_mfma_f32_32x32x2_f32 at k step t: lane l holds
    // A[row l%32][k 2t + l/32] and B[k 2t + l/32][column l%32]
    const float* as = sm.a[cur] + (wn * 64 + (l & 31)) * kAStride + (l >> 5);
    const float* bs = sm.b[cur] + (l >> 5) * kBStride + wv * 128 + (l & 31);
#pragma unroll
    for (int t = 0; t < kHeadK / 2; ++t) {
      const float fa0 = as[2 * t], fa1 = as[32 * kAStride + 2 * t];
      float fb[4];
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) fb[nt] = bs[2 * t * kBStride + 32 * nt];
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        acc[0][nt] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa0, fb[nt], acc[0][nt], 0, 0, 0);
        acc[1][nt] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa1, fb[nt], acc[1][nt], 0, 0, 0);
      }
    }
    if (kb + 1 < nkb) store(cur ^ 1);
    wg_barrier();
  }

  // accumulator r of lane l holds row 8*(r/4) + 4*(l/32) + r%4, column l%32
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const int v = v0 + wv * 128 + nt * 32 + (l & 31);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int n = n0 + wn * 64 + mt * 32 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
        if (n < N && v < V) a.out[(size_t)n * a.ldo + v] = acc[mt][nt][r];
      }
    }
}

size_t head_ws_bytes(int N, int D) { return (size_t)N * head_kpad(D) * sizeof(float); }

hipError_t launch_head(HeadArgs a, hipStream_t s) {
  a.lda = head_kpad(a.D);
  hipLaunchKernelGGL(k_head_rmsnorm, dim3(a.N), dim3(kThreads), 0, s, a);
  const dim3 grid((unsigned)((a.V + kHeadCols - 1) / kHeadCols), (unsigned)((a.N + kHeadRows - 1) / kHeadRows));
  hipLaunchKernelGGL(k_head_gemm, grid, dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace plh
