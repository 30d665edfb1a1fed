/*
 * pagellm_hip.h - C ABI of libpagellm_hip.so, the MI355X (gfx950) sampler
 * for pagellm.
 *
 * Plain C types only: every tensor argument is a device pointer (from
 * plh_alloc, hipMalloc, or a torch tensor's data_ptr()) plus explicit sizes.
 * Every function returns PLH_OK (0) or a negative PLH_ERR_* code; the
 * message of the last failure on a context is available from
 * plh_last_error().  No C++ exception or abort() crosses this boundary.
 *
 * Threading: a plh_ctx is not thread-safe.  Use one context per host thread
 * (the reference samples from its single engine thread,
 * docs/adr/0004-single-engine-thread.md).  Work is queued on the context's
 * stream; plh_sync() waits for it.
 *
 * Randomness never comes from the device: callers pass uniforms in [0, 1)
 * drawn on the host from each sequence's numpy Generator
 * (src/pagellm/engine/sampling.py:110-111), in the reference's order.
 */
#ifndef PAGELLM_HIP_H
#define PAGELLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PLH_ABI_VERSION 1

/* status codes */
#define PLH_OK 0
#define PLH_ERR_INVALID_ARG -1
#define PLH_ERR_HIP -2
#define PLH_ERR_OUT_OF_MEMORY -3
#define PLH_ERR_UNSUPPORTED -4
#define PLH_ERR_NO_DEVICE -5

/* element types of logits / probability inputs */
#define PLH_F32 0
#define PLH_F64 1

/* plh_sample flags */
#define PLH_SAMPLE_ROWWISE 1 /* one workgroup per row (the general kernel) */
#define PLH_SAMPLE_HIST_SPANS 2 /* hist_off holds B (start, end) pairs into
                                   hist_ids instead of B+1 CSR offsets, so
                                   histories can live in fixed per-sequence
                                   slots that grow in place (plh_append_ids) */
#define PLH_SAMPLE_NUCLEUS 4 /* performance hint, same results: rows with no
                                top-k and top_p >= 0.98 (nuclei that hold most
                                of the vocabulary) take two streaming passes
                                over all chunks instead of the per-row general
                                pipeline; costs three extra launches */
#define PLH_SAMPLE_NUCLEUS_ONLY 8 /* performance hint, same results, with
                                     PLH_SAMPLE_NUCLEUS: every row is such a
                                     row, so the merge kernel is not launched;
                                     a row that is not one is finished by the
                                     general pipeline in the nucleus path */

/* plh_set_option options */
#define PLH_OPT_KERNEL_TIMING 1 /* value 1: bracket the fast path's kernels with
                                   HIP events (read by plh_kernel_times) */


typedef struct plh_ctx plh_ctx;

/* Version of this ABI (PLH_ABI_VERSION). */
int plh_abi_version(void);

/* Context on HIP device `device`, with its own stream.  No reference
 * counterpart: the reference samples on the host (sampling.py). */
int plh_create(plh_ctx** out, int device);
void plh_destroy(plh_ctx* ctx);
const char* plh_last_error(const plh_ctx* ctx);
/* Queue work on `stream` (a hipStream_t, e.g. torch's current stream); NULL
 * restores the context's own stream.  Moving to another stream records an
 * event on the stream being left that closes the calls queued there; the
 * next call on the new stream waits for it (calls on one stream record
 * nothing).  A stream stays in use until the context moves off it or is
 * destroyed: it must stay valid until then. */
int plh_set_stream(plh_ctx* ctx, void* stream);
int plh_set_option(plh_ctx* ctx, int option, int64_t value);
/* Rows the fast path (its merge kernel or the nucleus kernels) finished with
 * the general row-wise pipeline, cumulative since plh_create (waits for the
 * context's queued calls, on its stream and on the streams it left). */
int plh_fallback_rows(plh_ctx* ctx, int64_t* out);
/* While PLH_OPT_KERNEL_TIMING is on: device time of the fast path's
 * streaming kernel and merge kernel summed over the plh_sample calls made
 * since the last read, and their count.  Waits for those calls, then
 * resets.  No reference counterpart (measurement only). */
int plh_kernel_times(plh_ctx* ctx, double* stream_ms, double* merge_ms, int64_t* calls);

/* Device memory helpers so numpy callers need no other GPU library.
 * plh_h2d / plh_d2h return once the copy is complete. */
int plh_alloc(plh_ctx* ctx, void** out, size_t bytes);
int plh_free(plh_ctx* ctx, void* ptr);
int plh_h2d(plh_ctx* ctx, void* dst, const void* src, size_t bytes);
int plh_d2h(plh_ctx* ctx, void* dst, const void* src, size_t bytes);

/* Page-locked host memory, and a host-to-device copy that is only queued on
 * the context's stream (no wait): src must stay unchanged until the stream
 * has passed the copy, e.g. until the next plh_d2h or plh_sync returns.
 * For the small per-step inputs of a serving loop (one copy per step from
 * one page-locked buffer).  No reference counterpart (the reference's
 * inputs never leave the host). */
int plh_host_alloc(plh_ctx* ctx, void** out, size_t bytes);
int plh_host_free(plh_ctx* ctx, void* ptr);
int plh_h2d_async(plh_ctx* ctx, void* dst, const void* src, size_t bytes);
int plh_sync(plh_ctx* ctx);

/*
 * Batched sample(): replaces the per-sequence loop of
 * src/pagellm/engine/llm_engine.py:238-254 over
 * src/pagellm/engine/sampling.py:101-107 (sample), :65-91 (probs),
 * :94-98 (draw), :52-62 (apply_repetition_penalty).
 *
 *   logits      [B, ld] of `dtype` (PLH_F32 / PLH_F64); row b starts at b*ld;
 *               aligned to its element size (rows of any 16-byte alignment
 *               take the same kernels)
 *   hist_ids    int32 token ids, CSR over rows (the sequence's full history,
 *               prompt + outputs, llm_engine.py:283); may be NULL with
 *   hist_off    int64 [B+1] offsets into hist_ids, or NULL (no history);
 *               with PLH_SAMPLE_HIST_SPANS, int64 [2B]: row b's history is
 *               hist_ids[hist_off[2b] .. hist_off[2b+1])
 *   temperature float64 [B]  0 => greedy (SamplingParams.greedy, :47-49)
 *   top_k       int32 [B]    0 or >= V => disabled
 *   top_p       float64 [B]  1 => disabled
 *   rep_penalty float64 [B]  1 => disabled
 *   uniforms    float64 [B]  one uniform per non-greedy row (rng.random()
 *               of :98); ignored for greedy rows
 *   out_ids     int32 [B]    sampled token ids
 *   out_probs   float64 [B, V] or NULL: when given, the processed
 *               distribution (probs(), :65-91) is written too and the
 *               row-wise kernel is used
 *   flags       PLH_SAMPLE_* bits
 * Histories with an active penalty require V <= 262144.
 */
int plh_sample(plh_ctx* ctx, const void* logits, int dtype, int64_t ld, int B, int V,
               const int32_t* hist_ids, const int64_t* hist_off, const double* temperature,
               const int32_t* top_k, const double* top_p, const double* rep_penalty,
               const double* uniforms, int32_t* out_ids, double* out_probs, int flags);

/*
 * plh_sample without any allocation.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory during the call (code
 * under HIP graph capture, serving loops that forbid hipMalloc).  Same
 * arguments, kernels and results as plh_sample; the fast path's workspace
 * is a fixed 64 MiB array per GPU (a static device array, resolved when the
 * context is created), never the context's growable workspace, and the
 * kernel-timing option is ignored.  A batch whose workspace exceeds 64 MiB
 * returns PLH_ERR_INVALID_ARG (mixed128k, 256 x 128256 fp32, fits).  Every
 * call on one GPU shares that GPU's array.  Calls of one context are
 * ordered on it: when the context's stream changed since its last call,
 * the new stream first waits on an event that call recorded (created by
 * plh_create); under graph capture such a stream change returns
 * PLH_ERR_INVALID_ARG.  Calls of different contexts that overlap on one GPU
 * race.
 */
int plh_sample_noalloc(plh_ctx* ctx, const void* logits, int dtype, int64_t ld, int B, int V,
                       const int32_t* hist_ids, const int64_t* hist_off, const double* temperature,
                       const int32_t* top_k, const double* top_p, const double* rep_penalty,
                       const double* uniforms, int32_t* out_ids, double* out_probs, int flags);

/*
 * apply_repetition_penalty() on a copy: src/pagellm/engine/sampling.py:52-62.
 * out[b, :V] = x[b, :V] with every distinct id of row b's history mapped
 * through x > 0 ? x / penalty : x * penalty, computed in `dtype`.  No row
 * of `out` may overlap a row of `x` (PLH_ERR_INVALID_ARG): the penalty works
 * on a copy, as the reference's does (:58).  Interleaved rows of one buffer
 * (x = buf[:, :V], out = buf[:, V:2V], the same ld) are allowed.
 */
int plh_penalize(plh_ctx* ctx, const void* x, int dtype, int64_t ld, int B, int V,
                 const int32_t* hist_ids, const int64_t* hist_off, const double* rep_penalty,
                 void* out, int64_t out_ld);

/*
 * draw(): src/pagellm/engine/sampling.py:94-98 for B rows of non-negative
 * weights p[b, :V] (any scale): first i with cumsum(p)[i] > u[b] * sum(p),
 * else V-1.  float32 rows are widened exactly and drawn in float64
 * arithmetic (the reference's probs() hands draw() float64 rows).
 */
int plh_draw(plh_ctx* ctx, const void* p, int dtype, int64_t ld, int B, int V,
             const double* uniforms, int32_t* out_ids);

/*
 * Batched verify(): src/pagellm/engine/speculative.py:38-60.
 *   p           [B, k+1, V] target distributions (dtype)
 *   q           [B, k, V] draft distributions (dtype)
 *   draft       int32 [B, k] proposed tokens (0 <= id < V)
 *   accept_u    float64 [B, k]: test i accepts while accept_u < min(1, p/q)
 *   draw_u      float64 [B] (draw_u_per_stop = 0) or [B, k+1] (= 1, the
 *               uniform used when the walk stops at position s is
 *               draw_u[b, s])
 *   out_tokens  int32 [B, k+1]: accepted drafts, then the residual or bonus
 *               token, then -1 padding
 *   out_n_acc   int32 [B]: accepted draft count
 */
int plh_verify(plh_ctx* ctx, const void* p, const void* q, int dtype, int B, int k, int V,
               const int32_t* draft, const double* accept_u, const double* draw_u,
               int draw_u_per_stop, int32_t* out_tokens, int32_t* out_n_acc);

/*
 * Strided device-to-device copy on the context's stream: rows x row_bytes
 * from src (pitch src_pitch bytes) to dst (pitch dst_pitch bytes).  Places
 * a [B, V] block (for instance draft distributions exported by plh_sample)
 * at one position of a [B, k, V] buffer for plh_verify.  No counterpart in
 * the reference (host lists play this role there).
 */
int plh_copy_rows(plh_ctx* ctx, void* dst, int64_t dst_pitch, const void* src, int64_t src_pitch,
                  int64_t row_bytes, int rows);

/*
 * Appends sampled ids to device-resident histories: the step of
 * src/pagellm/engine/llm_engine.py:284 (seq.tokens.append(tok)) for a batch,
 * without a host round trip.  slab[pos[i]] = ids[i] for i < n; entries with
 * pos[i] < 0 are skipped.  slab, pos (int64 [n]) and ids (int32 [n], e.g.
 * plh_sample's out_ids) are device pointers; ordered on the context's stream.
 */
int plh_append_ids(plh_ctx* ctx, int32_t* slab, const int64_t* pos, const int32_t* ids, int n);

/*
 * The logits producer: the model's final RMSNorm and lm_head product,
 * replacing src/pagellm/model/transformer.py:271
 * (rms_norm(h, self.w["norm"], eps) @ self.w["lm_head"], rms_norm at :79-82)
 * for float32 models, written into a logits buffer plh_sample can read in
 * place:
 *   r_n = 1 / sqrt(mean_d(h[n, d]^2) + eps)      (float32, eps as a float32)
 *   out[n, v] = sum_d ((h[n, d] * r_n) * norm[d]) * W[d, v]
 * for n < N, v < V, with the products and sums in float32 on the matrix
 * cores.  h [N, ldh], norm [D], W [D, ldw] (row-major: the reference's
 * [D, V] lm_head) and out [N, ldo] are float32 device pointers; the
 * normalised rows live in the context's workspace.  Ordered on the
 * context's stream.
 */
int plh_rmsnorm_lm_head(plh_ctx* ctx, const float* h, int64_t ldh, int N, int D, const float* norm, double eps,
                        const float* W, int64_t ldw, int V, float* out, int64_t ldo);

#ifdef __cplusplus
}
#endif

#endif /* PAGELLM_HIP_H */
