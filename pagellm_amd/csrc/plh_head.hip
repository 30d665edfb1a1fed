// gfx950 kernels for the logits producer: the model's final RMSNorm and
// lm_head product, logits = rms_norm(h, norm, eps) @ lm_head
// (src/pagellm/model/transformer.py:79-82, :271), in float32 as the
// reference computes it, written straight into the sampler's logits buffer.
//
//   k_head_rms      one workgroup per row: r = 1 / sqrt(mean(h * h) + eps)
//                   in float32 (the squares summed in float64 and rounded
//                   once);
//   k_head_act      act = (h * r) * norm, stored k-major and zero-padded to
//                   whole tiles (32 in k, 256 in n);
//   k_head_gemm     out = act @ W on the fp32 matrix cores
//                   (v_mfma_f32_32x32x2_f32, products and sums in float32).
//                   A workgroup of 8 waves (two per SIMD) owns a 256-row x
//                   256-column tile of out; each wave a 64 x 128 block,
//                   2 x 4 MFMA tiles held in 128 accumulator registers.
//                   Both operands are k-major in LDS (each half-wave reads
//                   32 consecutive floats per MFMA operand); k streams
//                   through LDS 32 at a time, double-buffered: the next
//                   stage is copied from HBM straight into LDS
//                   (global_load_lds_dwordx4) while the matrix cores work on
//                   the current one, and operand reads run two k steps ahead
//                   of the MFMAs.
#include "plh_device.h"
#include "plh_kernels.h"

namespace plh {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kHeadRows = 256;             // rows of out per workgroup
constexpr int kHeadCols = 256;             // vocabulary columns per workgroup
constexpr int kHeadK = 32;                 // k per LDS stage
constexpr int kTileStride = 256 + 32;      // LDS row pitch of both tiles (floats)

__host__ __device__ constexpr int head_kpad(int D) { return (D + kHeadK - 1) / kHeadK * kHeadK; }
__host__ __device__ constexpr int head_npad(int N) { return (N + kHeadRows - 1) / kHeadRows * kHeadRows; }

// r_n = 1 / sqrt(mean(h[n] * h[n]) + eps), one workgroup per row.
__global__ __launch_bounds__(kThreads) void k_head_rms(HeadArgs a) {
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
  if (threadIdx.x == 0) {
    const float mean = (float)s / (float)a.D;
    a.rinv[n] = 1.0f / sqrtf(mean + a.eps);
  }
}

// act[d][n] = (h[n][d] * r_n) * norm[d] (transformer.py:82), stored k-major
// ([Dp][lda], lda = N rounded up to the row tile) and zero outside
// d < D, n < N: a 32 (d) x 64 (n) block per workgroup, transposed through LDS
// so that both the reads of h and the writes of act are 16-byte and
// contiguous.
__global__ __launch_bounds__(kThreads) void k_head_act(HeadArgs a) {
  __shared__ float t[64][32 + 1];
  const int d0 = blockIdx.x * 32, n0 = blockIdx.y * 64;
  const int tid = threadIdx.x;
  {
    const int nl = tid >> 3, dl = (tid & 7) * 4;  // 64 rows x 8 groups of 4
    const int n = n0 + nl;
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (n < a.N) {
      const float r = a.rinv[n];
      const float* x = a.h + (size_t)n * a.ldh;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int d = d0 + dl + e;
        if (d < a.D) v[e] = (x[d] * r) * a.norm[d];
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) t[nl][dl + e] = v[e];
  }
  wg_barrier();
  {
    const int dl = tid >> 4, nl = (tid & 15) * 4;  // 32 rows x 16 groups of 4
    f32x4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = t[nl + e][dl];
    *reinterpret_cast<f32x4*>(a.act + (size_t)(d0 + dl) * a.lda + n0 + nl) = v;
  }
}

// 16-byte aligned, so that the stage stores are single ds_write_b128s
struct __attribute__((aligned(16))) HeadSmem {
  float a[2][kHeadK * kTileStride];  // act stage, [k][n]
  float b[2][kHeadK * kTileStride];  // W stage, [k][v]
};

// Wave layout: each wave owns kMT x 4 MFMA tiles (kMT * 32 rows x 128
// columns) of the workgroup's 256 x 256 tile.  kMT = 2: 8 waves, two per
// SIMD, 128 accumulators each; kMT = 4: 4 waves, one per SIMD, 256.
constexpr int kMT = 2;
constexpr int kWavesN = kHeadRows / (32 * kMT);
constexpr int kGemmWaves = kWavesN * 2;
constexpr int kGemmThreads = 64 * kGemmWaves;
constexpr int kStageRows = kGemmThreads / 64;   // stage rows one pass of the workgroup moves
constexpr int kStagePasses = kHeadK / kStageRows;
// The next stage goes to LDS one pass (two ds_write_b128) per k step,
// after steps kStoreStep .. kStoreStep + kStagePasses - 1, so that LDS
// writes never arrive as a burst in front of the operand reads.
constexpr int kStoreStep = 1;
constexpr int kAhead = 2;                        // k steps the operand reads run ahead
static_assert(kStoreStep + kStagePasses <= kHeadK / 2, "stage stores must end inside the k loop");

// One workgroup tile.  VEC: every W row segment of the tile is inside the
// matrix and 16-byte aligned (all tiles but a ragged last one); the two
// forms are separate code so that no branch joins inside the k loop.
// DMA (full tiles whose k stages all lie inside D): the stages go from HBM
// straight into LDS (global_load_lds_dwordx4: each wave's load fills one
// contiguous 1 KB LDS row, lane l at 16 l), with no registers or LDS
// stores on the way; the wave waits for its copies before the barrier that
// ends the stage.
template <bool VEC, bool DMA>
__device__ __forceinline__ void head_tile(const HeadArgs& a, HeadSmem& sm) {
  static_assert(!DMA || VEC, "the DMA form needs whole, aligned rows");
  const int N = a.N, D = a.D, V = a.V;
  const int v0 = blockIdx.x * kHeadCols, n0 = blockIdx.y * kHeadRows;
  const int tid = threadIdx.x, l = lane(), w = wave();
  const int wn = w % kWavesN, wv = w / kWavesN;  // this wave's block of the tile

  // global -> register staging, the same map for both tiles: stage row
  // (tid / 64) + kStageRows j, 4 columns from (tid % 64) * 4, so that each wave moves
  // one contiguous 1 KB row per load and per LDS store.  act is padded to
  // whole tiles; W rows past D are read clamped and zeroed at the store.
  const int sr = tid >> 6, sc = (tid & 63) * 4;
  const float* ag = a.act + (size_t)sr * a.lda + n0 + sc;
  // The loads only fill registers; what falls outside the matrix is zeroed
  // when the registers go to LDS, so that no wait for the loads precedes
  // the current stage's MFMAs.
  f32x4 pa[kStagePasses], pb[kStagePasses];
  auto load = [&](int kb) {
    const int k0 = kb * kHeadK;
#pragma unroll
    for (int j = 0; j < kStagePasses; ++j)
      pa[j] = *reinterpret_cast<const f32x4*>(ag + (size_t)(k0 + kStageRows * j) * a.lda);
#pragma unroll
    for (int j = 0; j < kStagePasses; ++j) {
      const float* bg = a.w + (size_t)min(k0 + sr + kStageRows * j, D - 1) * a.ldw;
      if constexpr (VEC) {
        pb[j] = *reinterpret_cast<const f32x4*>(bg + v0 + sc);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) pb[j][e] = bg[min(v0 + sc + e, V - 1)];
      }
    }
  };
  auto store = [&](int kb, int buf, int j) {
    {
      const int r = sr + kStageRows * j;
      *reinterpret_cast<f32x4*>(sm.a[buf] + r * kTileStride + sc) = pa[j];
      const bool kin = kb * kHeadK + r < D;
      f32x4 v = pb[j];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = (kin && v0 + sc + e < V) ? v[e] : 0.0f;
      *reinterpret_cast<f32x4*>(sm.b[buf] + r * kTileStride + sc) = v;
    }
  };

  f32x16 acc[kMT][4];
#pragma unroll
  for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mt][nt][r] = 0.0f;

  // the DMA form: stage kb into LDS buffer buf (the LDS row of each copy is
  // the same for the whole wave, as the instruction requires)
  auto dma = [&](int kb, int buf) {
    const int k0 = kb * kHeadK;
#pragma unroll
    for (int j = 0; j < kStagePasses; ++j) {
      const int r = sr + kStageRows * j;
      __builtin_amdgcn_global_load_lds(ag + (size_t)(k0 + kStageRows * j) * a.lda, sm.a[buf] + r * kTileStride, 16,
                                       0, 0);
      __builtin_amdgcn_global_load_lds(a.w + (size_t)(k0 + r) * a.ldw + v0 + sc, sm.b[buf] + r * kTileStride, 16, 0,
                                       0);
    }
  };
  auto dma_wait = [] { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); };

  const int nkb = head_kpad(D) / kHeadK;
  if constexpr (DMA) {
    dma(0, 0);
    dma_wait();
  } else {
    load(0);
#pragma unroll
    for (int j = 0; j < kStagePasses; ++j) store(0, 0, j);
  }
  wg_barrier();
  for (int kb = 0; kb < nkb; ++kb) {
    const int cur = kb & 1;
    if constexpr (DMA) {
      if (kb + 1 < nkb) dma(kb + 1, cur ^ 1);  // the other buffer's last reads were before the barrier
    } else {
      if (kb + 1 < nkb) load(kb + 1);
    }
    // operands of v_mfma_f32_32x32x2_f32 at k step t: lane l holds
    // A[row l%32][k 2t + l/32] and B[k 2t + l/32][column l%32]; both tiles
    // are k-major, so each half-wave reads 32 consecutive floats
    const float* as = sm.a[cur] + (l >> 5) * kTileStride + wn * 32 * kMT + (l & 31);
    const float* bs = sm.b[cur] + (l >> 5) * kTileStride + wv * 128 + (l & 31);
    // the operands of step t + kAhead are read from LDS while step t's
    // MFMAs run
    float fa[kAhead + 1][kMT], fb[kAhead + 1][4];
    auto frags = [&](int t, int slot) {
#pragma unroll
      for (int i = 0; i < kMT; ++i) fa[slot][i] = as[2 * t * kTileStride + 32 * i];
#pragma unroll
      for (int i = 0; i < 4; ++i) fb[slot][i] = bs[2 * t * kTileStride + 32 * i];
    };
#pragma unroll
    for (int t = 0; t < kAhead; ++t) frags(t, t);
#pragma unroll
    for (int t = 0; t < kHeadK / 2; ++t) {
      const int sl = t % (kAhead + 1);
      if (t + kAhead < kHeadK / 2) frags(t + kAhead, (t + kAhead) % (kAhead + 1));
      __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the MFMAs
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int mt = 0; mt < kMT; ++mt)
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[sl][mt], fb[sl][nt], acc[mt][nt], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      // the next stage goes to the other LDS buffer (its last reads were
      // before the previous barrier)
      if constexpr (!DMA) {
        if (t >= kStoreStep && t < kStoreStep + kStagePasses && kb + 1 < nkb)
          store(kb + 1, cur ^ 1, t - kStoreStep);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (DMA) dma_wait();
    wg_barrier();
  }

  // accumulator r of lane l holds row 8*(r/4) + 4*(l/32) + r%4, column l%32
#pragma unroll
  for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const int v = v0 + wv * 128 + nt * 32 + (l & 31);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int n = n0 + wn * 32 * kMT + mt * 32 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
        if (n < N && v < V) a.out[(size_t)n * a.ldo + v] = acc[mt][nt][r];
      }
    }
}

__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(kGemmWaves / 4, kGemmWaves / 4))) void
k_head_gemm(HeadArgs a) {
  __shared__ HeadSmem sm;
  const int v0 = blockIdx.x * kHeadCols;
  const bool vec = v0 + kHeadCols <= a.V && (a.ldw & 3) == 0 && (reinterpret_cast<uintptr_t>(a.w) & 15) == 0;
  if (vec && a.D % kHeadK == 0) head_tile<true, true>(a, sm);
  else if (vec) head_tile<true, false>(a, sm);
  else head_tile<false, false>(a, sm);
}

size_t head_ws_bytes(int N, int D) {
  return ((size_t)head_kpad(D) * head_npad(N) + (size_t)N) * sizeof(float) + 256;
}

hipError_t launch_head(HeadArgs a, hipStream_t s) {
  // workspace: act [Dp][lda] (k-major), then rinv [N]
  a.lda = head_npad(a.N);
  a.rinv = a.act + (size_t)head_kpad(a.D) * a.lda;
  hipLaunchKernelGGL(k_head_rms, dim3(a.N), dim3(kThreads), 0, s, a);
  hipLaunchKernelGGL(k_head_act, dim3((unsigned)(head_kpad(a.D) / 32), (unsigned)(a.lda / 64)), dim3(kThreads), 0, s,
                     a);
  const dim3 grid((unsigned)((a.V + kHeadCols - 1) / kHeadCols), (unsigned)(a.lda / kHeadRows));
  hipLaunchKernelGGL(k_head_gemm, grid, dim3(kGemmThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace plh
