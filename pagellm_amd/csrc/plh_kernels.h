// Internal launch interface between the C ABI (plh_api.hip) and the kernel
// translation units.  Not part of the public header.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace plh {

// Partial left by one wave of k_sample_chunks (its segment, 1/8 of a
// chunk) for k_sample_final.
struct WavePart {
  double zmax;    // largest finite penalised logit of the segment (-inf if none)
  double umax;    // bound on the tokens not kept as candidates: all are below it
                  // (nucleus rows: the smallest finite penalised logit, +inf if none)
  double best_z;  // greedy rows: the segment's argmax value ...
  int best_idx;   // ... and its token id
  int end;        // candidate rows: end of the wave's slots in its chunk's list
                  // (the chunk's candidate count is the largest end)
  int flags;      // kChunkIncomplete: the row needs the general pipeline
};
constexpr int kChunkIncomplete = 1;

// Per-row state of the nucleus path (rows with no top-k and a top_p of at
// least kNucTopP, when the caller asks for it): two passes over the row
// (segment partials and per-chunk count histograms of z, then the tokens of
// the bins that can hold the cut) instead of the general pipeline.  The
// row's bins lie on a power-of-two grid: bin b holds the tokens whose z,
// rounded to float, has floor(zf * rz) = base + b (zf * rz is exact).
struct NucRow {
  float rz;      // bins per unit of z, a power of two
  int base;      // floor(zf * rz) of the row's smallest finite penalised logit
  double ymax;   // largest y = z / T of the row
  double S;      // sum over the row of exp(y - ymax)
  double invS;
  int state;     // kNucActive while the nucleus kernels own the row
  int general;   // 1: k_nuc_final runs the general pipeline on the row
  int dlo, dhi;  // bins [dlo, dhi] hold the candidates
  int above;     // 1: nexcl sums the tokens above the window (fewer than those below)
};
constexpr int kNucActive = 1;
// A chunk's own histogram grid: bin j holds floor(zf * rz) = q0 + j; rz is
// the largest power of two that fits the chunk's span in kNucBins bins (0:
// the chunk holds no finite token).
struct NucGrid {
  float rz;
  int q0;
};
constexpr int kNucPenWords = 512;  // bitmap words of one chunk (16384 float tokens)
constexpr int kNucBins = 2048;
constexpr int kBkt = 256;          // candidate buckets of a top-p chunk
constexpr double kBktPerY = 8.0;   // buckets per unit of y (the last bucket is open below)

// Workspace of the two-launch fast path, carved from one device buffer.
struct ChunkWs {
  WavePart* part;   // [B * C * 8], entry (chunk * 8 + wave)
  double* seg_m;    // [B * C * 8] per-wave segment max of z / T
  double* seg_s;    // [B * C * 8] per-wave segment sum of exp(z / T - max)
  double* cz;       // [B * C * capc] candidate penalised logits
  int32_t* ci;      // [B * C * capc] candidate token ids
  NucRow* nrow;     // [B] nucleus path: per-row state
  uint32_t* nhist;  // [B * C * kNucBins / 2] nucleus path: each chunk's token counts per bin of its own
                    // grid, two 16-bit counts a word
  NucGrid* ngrid;   // [B * C] nucleus path: each chunk's grid (NucGrid)
  double* nexcl;    // [B * C * 8] nucleus path: per-segment mass on one side of the candidate bins
  int32_t* ncand;   // [B * C] nucleus path: candidates per chunk (-1: over capacity)
  uint32_t* npen;   // [B * C * kNucPenWords] nucleus path: each chunk's penalised-token bitmap
  // top-p rows (no top-k): each chunk's candidates in buckets of an absolute
  // grid of y = z / T (kBktPerY buckets per unit, bucket 0 the chunk's top),
  // written bucket by bucket, each with exp(y - the chunk's max y)
  uint64_t* bmass;  // [B * C * kBkt] per bucket: sum of exp(y - ymax_c) * 2^52
  uint32_t* bcnt;   // [B * C * kBkt] per bucket: candidates
  double* bymax;    // [B * C] the chunk's max y
  int32_t* bhb;     // [B * C] the chunk's top bucket: floor(ymax_c * kBktPerY)
  int C;            // chunks per row
  int capc;         // candidate slots per chunk
};

struct SampleArgs {
  const void* logits;
  int64_t ld;
  int B, V;
  const int32_t* hist_ids;
  const int64_t* hist_off;  // B+1 CSR offsets, or B (start, end) pairs
  int hist_spans;           // 1: hist_off holds (start, end) pairs
  const double* temperature;
  const int32_t* top_k;
  const double* top_p;
  const double* rep_penalty;
  const double* uniforms;
  int32_t* out_ids;
  double* out_probs;
  unsigned long long* fallback_rows;  // rows finished by the general path
  int nucleus;                        // 1: eligible rows take the nucleus path
  int nucleus_only;                   // 1 (with nucleus): no merge launch; other rows take the
                                      // general pipeline in k_nuc_final
  ChunkWs ws;                         // fast path only
};

struct DrawArgs {
  const void* p;
  int64_t ld;
  int B, V;
  const double* uniforms;
  int32_t* out_ids;
};

struct PenalizeArgs {
  const void* x;
  int64_t ld;
  void* out;
  int64_t out_ld;
  int B, V;
  const int32_t* hist_ids;
  const int64_t* hist_off;
  const double* rep_penalty;
};

struct VerifyArgs {
  const void* p;  // [B, k+1, V]
  const void* q;  // [B, k, V]
  int B, k, V;
  const int32_t* draft;     // [B, k]
  const double* accept_u;   // [B, k]
  const double* draw_u;     // [B] or [B, k+1]
  int draw_u_per_stop;
  int32_t* out_tokens;      // [B, k+1]
  int32_t* out_n_acc;       // [B]
};

struct VerifyWs {
  int32_t* stop;    // [B] stop position: first rejection, k, or -1
  double* part;     // [B * C * 2] chunk sums of the residual and of p
  int C;            // chunks per row
};

struct HeadArgs {
  const float* h;     // [N, ldh] final hidden states
  int64_t ldh;
  const float* norm;  // [D] RMSNorm weight
  float eps;
  const float* w;     // [D, ldw] lm_head, the reference's [D, V] layout
  int64_t ldw;
  float* out;         // [N, ldo] logits
  int64_t ldo;
  float* act;         // workspace [Dp, lda]: normalised rows, k-major, zero-padded
  int64_t lda;
  float* rinv;        // workspace [N]: 1 / rms of each row
  int N, D, V;
};

hipError_t launch_sample_rows(const SampleArgs& a, bool f64, bool vec, hipStream_t s);
// Fast path: workspace bytes for a [B, V] batch, its layout inside `base`
// (256-byte aligned), and the two launches.
size_t fast_ws_bytes(int B, int V, bool f64);
ChunkWs fast_ws_layout(void* base, int B, int V, bool f64);
// `vec`: every row starts 16-byte aligned (16-byte loads); `between`, when
// not null, is recorded on s between the two kernels.
hipError_t launch_sample_fast(const SampleArgs& a, bool f64, bool vec, int num_cu, hipStream_t s,
                              hipEvent_t between = nullptr);
hipError_t launch_draw(const DrawArgs& a, bool f64, hipStream_t s);
hipError_t launch_penalize(const PenalizeArgs& a, bool f64, hipStream_t s);
// Verify: workspace bytes for B rows of V tokens, its layout, and the two
// launches (stop positions and chunk sums, then the draw).
size_t verify_ws_bytes(int B, int V);
VerifyWs verify_ws_layout(void* base, int B, int V);
// `between`, when not null, is recorded on s between the two launches.
hipError_t launch_verify(const VerifyArgs& a, const VerifyWs& ws, bool f64, hipStream_t s,
                         hipEvent_t between = nullptr);
// Logits producer: workspace bytes (the normalised rows) and the two
// launches (RMSNorm, then the MFMA product into out).
size_t head_ws_bytes(int N, int D);
hipError_t launch_head(HeadArgs a, hipStream_t s);
hipError_t launch_append(int32_t* slab, const int64_t* pos, const int32_t* ids, int n, hipStream_t s);

}  // namespace plh
