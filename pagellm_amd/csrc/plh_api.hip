// C ABI of libpagellm_hip.so (declared in include/pagellm_hip.h): context,
// device memory helpers, argument validation and kernel launches.
#include <stdio.h>
#include <string.h>

#include <array>
#include <new>
#include <string>
#include <vector>

#include <cmath>

#include "pagellm_hip.h"
#include "plh_kernels.h"

struct plh_ctx {
  int device = 0;
  int num_cu = 0;
  hipStream_t own_stream = nullptr;
  hipStream_t stream = nullptr;
  unsigned long long* fallback = nullptr;
  // fast-path workspace, reused by every call on this context.  ws_stream:
  // the stream of the last call that used it; ws_open: that call is not yet
  // closed by ws_done, which plh_set_stream records on the stream it leaves
  // (one event per stream change instead of one per call: an event record
  // costs the queue ~3 us per two-kernel step)
  void* ws = nullptr;
  size_t ws_bytes = 0;
  hipEvent_t ws_done = nullptr;
  hipStream_t ws_stream = nullptr;
  bool ws_open = false;
  // plh_sample_noalloc: this device's copy of the file-scope scratch array;
  // scratch_stream, scratch_open and scratch_done as above, for this
  // context's noalloc calls
  void* scratch = nullptr;
  hipEvent_t scratch_done = nullptr;
  hipStream_t scratch_stream = nullptr;
  bool scratch_open = false;
  // PLH_OPT_KERNEL_TIMING: event triples (start, between, end) per timed call
  bool timing = false;
  std::vector<hipEvent_t> ev_free;
  std::vector<std::array<hipEvent_t, 3>> ev_pending;
  std::string err;
};

namespace {

constexpr int kMaxVBitmap = 262144;

int fail(plh_ctx* c, int code, const char* fmt, const char* detail = nullptr) {
  if (c != nullptr) {
    char buf[512];
    snprintf(buf, sizeof(buf), fmt, detail != nullptr ? detail : "");
    c->err = buf;
  }
  return code;
}

int hip_fail(plh_ctx* c, hipError_t e, const char* where) {
  if (c != nullptr) {
    c->err = std::string(where) + ": " + hipGetErrorString(e);
  }
  return e == hipErrorOutOfMemory ? PLH_ERR_OUT_OF_MEMORY : PLH_ERR_HIP;
}

#define PLH_HIP(ctx, call, where)                   \
  do {                                              \
    hipError_t e_ = (call);                         \
    if (e_ != hipSuccess) return hip_fail(ctx, e_, where); \
  } while (0)

int use_device(plh_ctx* c) {
  if (c == nullptr) return PLH_ERR_INVALID_ARG;
  PLH_HIP(c, hipSetDevice(c->device), "hipSetDevice");
  return PLH_OK;
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Makes the context's workspace at least `bytes` large and orders the
// current stream after the last call that used it (possibly on another
// stream).  Growing waits for that call and reallocates.
int reserve_ws(plh_ctx* c, size_t bytes) {
  if (bytes > c->ws_bytes) {
    if (c->ws_stream != nullptr) PLH_HIP(c, hipStreamSynchronize(c->ws_stream), "hipStreamSynchronize");
    if (c->ws != nullptr) {
      PLH_HIP(c, hipFree(c->ws), "hipFree");
      c->ws = nullptr;
      c->ws_bytes = 0;
    }
    const size_t sz = align_up(bytes + bytes / 4, 1u << 20);
    PLH_HIP(c, hipMalloc(&c->ws, sz), "hipMalloc(workspace)");
    c->ws_bytes = sz;
    c->ws_stream = nullptr;
    c->ws_open = false;
  }
  if (c->ws_stream != nullptr && c->ws_stream != c->stream)
    PLH_HIP(c, hipStreamWaitEvent(c->stream, c->ws_done, 0), "hipStreamWaitEvent");
  return PLH_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// PLH_OPT_KERNEL_TIMING: takes an event triple (start, between, end) for
// the call and records its start on the context's stream; the launch
// records `between` after its first kernel and the caller `end` after the
// last.  A no-op (null events) when timing is off.
int timing_begin(plh_ctx* c, std::array<hipEvent_t, 3>& ev) {
  if (!c->timing) return PLH_OK;
  for (auto& e : ev) {
    if (c->ev_free.empty()) {
      hipEvent_t n = nullptr;
      PLH_HIP(c, hipEventCreate(&n), "hipEventCreate");
      c->ev_free.push_back(n);
    }
    e = c->ev_free.back();
    c->ev_free.pop_back();
  }
  c->ev_pending.push_back(ev);
  PLH_HIP(c, hipEventRecord(ev[0], c->stream), "hipEventRecord");
  return PLH_OK;
}

constexpr size_t kScratchBytes = size_t(64) << 20;  // the no-allocation entry point's workspace, per GPU

}  // namespace

// Workspace of plh_sample_noalloc: one copy per GPU the library runs on,
// held until the process ends, zeroed when the code object loads.  In host
// code `scratch` names a host-side stand-in, never the device memory: host
// code uses only the address hipGetSymbolAddress returns for the current
// device (resolve_scratch).
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

// Called by plh_create with the context's device current: the device
// address of this device's scratch array, looked up afresh for every
// context (a reloaded code object gets a new address).
int resolve_scratch(plh_ctx* c) {
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || p == nullptr) return hip_fail(c, e != hipSuccess ? e : hipErrorInvalidSymbol, "hipGetSymbolAddress(scratch)");
  c->scratch = p;
  return PLH_OK;
}

// Orders a noalloc call after this context's previous one when the stream
// changed in between: outside graph capture the new stream waits on the
// event that closed the last call; under capture a stream change is
// refused (a captured wait on an outside event is not allowed).
int order_scratch(plh_ctx* c) {
  if (c->scratch_stream == nullptr || c->scratch_stream == c->stream) return PLH_OK;
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  PLH_HIP(c, hipStreamIsCapturing(c->stream, &st), "hipStreamIsCapturing");
  if (st != hipStreamCaptureStatusNone)
    return fail(c, PLH_ERR_INVALID_ARG, "plh_sample_noalloc: the stream changed since the last call while capturing%s");
  PLH_HIP(c, hipStreamWaitEvent(c->stream, c->scratch_done, 0), "hipStreamWaitEvent");
  return PLH_OK;
}

// plh_sample and plh_sample_noalloc: the same validation and kernels; the
// fast path's workspace is the context's (grown on demand) or, with
// noalloc, this device's scratch array (no allocation of any kind: no
// workspace growth, no timing events).
int sample_impl(plh_ctx* c, const void* logits, int dtype, int64_t ld, int B, int V, const int32_t* hist_ids,
                const int64_t* hist_off, const double* temperature, const int32_t* top_k, const double* top_p,
                const double* rep_penalty, const double* uniforms, int32_t* out_ids, double* out_probs, int flags,
                bool noalloc) {
  if (c == nullptr) return PLH_ERR_INVALID_ARG;
  if (B < 0 || V < 1) return fail(c, PLH_ERR_INVALID_ARG, "need B >= 0 and V >= 1%s");
  if (B == 0) return PLH_OK;
  if (dtype != PLH_F32 && dtype != PLH_F64) return fail(c, PLH_ERR_INVALID_ARG, "dtype must be PLH_F32 or PLH_F64%s");
  if (ld < V) return fail(c, PLH_ERR_INVALID_ARG, "ld must be >= V%s");
  if (logits == nullptr || temperature == nullptr || top_k == nullptr || top_p == nullptr ||
      rep_penalty == nullptr || out_ids == nullptr)
    return fail(c, PLH_ERR_INVALID_ARG, "null device pointer%s");
  if (hist_off != nullptr && hist_ids == nullptr)
    return fail(c, PLH_ERR_INVALID_ARG, "hist_off given without hist_ids%s");
  if (hist_off != nullptr && V > kMaxVBitmap)
    return fail(c, PLH_ERR_UNSUPPORTED, "repetition-penalty histories need V <= 262144%s");
  int rc = use_device(c);
  if (rc != PLH_OK) return rc;
  const size_t esize = dtype == PLH_F64 ? 8 : 4;
  if ((reinterpret_cast<uintptr_t>(logits) % esize) != 0)
    return fail(c, PLH_ERR_INVALID_ARG, "logits must be aligned to their element size%s");
  const bool vec = aligned16(logits) && ((size_t)ld * esize) % 16 == 0;
  plh::SampleArgs a{};
  a.logits = logits;
  a.ld = ld;
  a.B = B;
  a.V = V;
  a.hist_ids = hist_ids;
  a.hist_off = hist_off;
  a.hist_spans = (flags & PLH_SAMPLE_HIST_SPANS) ? 1 : 0;
  a.temperature = temperature;
  a.top_k = top_k;
  a.top_p = top_p;
  a.rep_penalty = rep_penalty;
  a.uniforms = uniforms;
  a.out_ids = out_ids;
  a.out_probs = out_probs;
  a.fallback_rows = c->fallback;
  a.nucleus = (flags & PLH_SAMPLE_NUCLEUS) ? 1 : 0;
  a.nucleus_only = a.nucleus && (flags & PLH_SAMPLE_NUCLEUS_ONLY) ? 1 : 0;
  const bool f64 = dtype == PLH_F64;
  // the fast path gathers per-row state in LDS sized for V <= 262144
  if (out_probs != nullptr || (flags & PLH_SAMPLE_ROWWISE) || V > kMaxVBitmap) {
    const hipError_t e = plh::launch_sample_rows(a, f64, vec, c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "plh_sample launch");
    return PLH_OK;
  }
  const size_t need = plh::fast_ws_bytes(B, V, f64);
  if (noalloc) {
    if (need > kScratchBytes) {
      char msg[160];
      snprintf(msg, sizeof(msg), "this batch needs %zu bytes of workspace; plh_sample_noalloc holds %zu%%s", need,
               kScratchBytes);
      return fail(c, PLH_ERR_INVALID_ARG, msg);
    }
    rc = order_scratch(c);
    if (rc != PLH_OK) return rc;
    a.ws = plh::fast_ws_layout(c->scratch, B, V, f64);
    const hipError_t e = plh::launch_sample_fast(a, f64, vec, c->num_cu, c->stream, nullptr);
    if (e != hipSuccess) return hip_fail(c, e, "plh_sample_noalloc launch");
    c->scratch_stream = c->stream;
    c->scratch_open = true;
    return PLH_OK;
  }
  rc = reserve_ws(c, need);
  if (rc != PLH_OK) return rc;
  a.ws = plh::fast_ws_layout(c->ws, B, V, f64);
  std::array<hipEvent_t, 3> ev{};
  rc = timing_begin(c, ev);
  if (rc != PLH_OK) return rc;
  const hipError_t e = plh::launch_sample_fast(a, f64, vec, c->num_cu, c->stream, ev[1]);
  if (e != hipSuccess) return hip_fail(c, e, "plh_sample launch");
  if (c->timing) PLH_HIP(c, hipEventRecord(ev[2], c->stream), "hipEventRecord");
  c->ws_stream = c->stream;
  c->ws_open = true;
  return PLH_OK;
}

}  // namespace

extern "C" {

int plh_abi_version(void) { return PLH_ABI_VERSION; }

int plh_create(plh_ctx** out, int device) {
  if (out == nullptr) return PLH_ERR_INVALID_ARG;
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return PLH_ERR_NO_DEVICE;
  if (device < 0 || device >= n) return PLH_ERR_INVALID_ARG;
  plh_ctx* c = new (std::nothrow) plh_ctx();
  if (c == nullptr) return PLH_ERR_OUT_OF_MEMORY;
  c->device = device;
  int rc = PLH_OK;
  do {
    if (hipSetDevice(device) != hipSuccess) { rc = PLH_ERR_HIP; break; }
    if (hipStreamCreateWithFlags(&c->own_stream, hipStreamNonBlocking) != hipSuccess) { rc = PLH_ERR_HIP; break; }
    c->stream = c->own_stream;
    if (hipMalloc(&c->fallback, sizeof(unsigned long long)) != hipSuccess) { rc = PLH_ERR_OUT_OF_MEMORY; break; }
    if (hipMemset(c->fallback, 0, sizeof(unsigned long long)) != hipSuccess) { rc = PLH_ERR_HIP; break; }
    if (hipEventCreateWithFlags(&c->ws_done, hipEventDisableTiming) != hipSuccess) { rc = PLH_ERR_HIP; break; }
    if (hipEventCreateWithFlags(&c->scratch_done, hipEventDisableTiming) != hipSuccess) { rc = PLH_ERR_HIP; break; }
    if (hipDeviceGetAttribute(&c->num_cu, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
        c->num_cu <= 0) { rc = PLH_ERR_HIP; break; }
    rc = resolve_scratch(c);
  } while (0);
  if (rc != PLH_OK) {
    plh_destroy(c);
    return rc;
  }
  *out = c;
  return PLH_OK;
}

void plh_destroy(plh_ctx* c) {
  if (c == nullptr) return;
  (void)hipSetDevice(c->device);
  if (c->stream != nullptr) (void)hipStreamSynchronize(c->stream);
  if (c->ws_stream != nullptr) (void)hipStreamSynchronize(c->ws_stream);
  if (c->ws != nullptr) (void)hipFree(c->ws);
  if (c->ws_done != nullptr) (void)hipEventDestroy(c->ws_done);
  if (c->scratch_done != nullptr) (void)hipEventDestroy(c->scratch_done);
  for (auto& t : c->ev_pending)
    for (hipEvent_t e : t) c->ev_free.push_back(e);
  for (hipEvent_t e : c->ev_free) (void)hipEventDestroy(e);
  if (c->fallback != nullptr) (void)hipFree(c->fallback);
  if (c->own_stream != nullptr) (void)hipStreamDestroy(c->own_stream);
  delete c;
}

const char* plh_last_error(const plh_ctx* c) { return c == nullptr ? "null context" : c->err.c_str(); }

int plh_set_stream(plh_ctx* c, void* stream) {
  if (c == nullptr) return PLH_ERR_INVALID_ARG;
  const hipStream_t s = stream != nullptr ? static_cast<hipStream_t>(stream) : c->own_stream;
  if (s == c->stream) return PLH_OK;
  // leaving a stream: an event closes the calls queued on it that used the
  // workspace or the scratch array; the next such call on another stream
  // waits for it (reserve_ws, order_scratch)
  if (c->ws_open || c->scratch_open) {
    const int rc = use_device(c);
    if (rc != PLH_OK) return rc;
  }
  if (c->ws_open && c->ws_stream == c->stream) {
    PLH_HIP(c, hipEventRecord(c->ws_done, c->stream), "hipEventRecord");
    c->ws_open = false;
  }
  if (c->scratch_open && c->scratch_stream == c->stream) {
    PLH_HIP(c, hipEventRecord(c->scratch_done, c->stream), "hipEventRecord");
    c->scratch_open = false;
  }
  c->stream = s;
  return PLH_OK;
}

int plh_set_option(plh_ctx* c, int option, int64_t value) {
  if (c == nullptr) return PLH_ERR_INVALID_ARG;
  switch (option) {
    case PLH_OPT_KERNEL_TIMING:
      if (value != 0 && value != 1) return fail(c, PLH_ERR_INVALID_ARG, "PLH_OPT_KERNEL_TIMING takes 0 or 1%s");
      c->timing = value != 0;
      return PLH_OK;
    default:
      return fail(c, PLH_ERR_INVALID_ARG, "unknown option%s");
  }
}

int plh_kernel_times(plh_ctx* c, double* stream_ms, double* merge_ms, int64_t* calls) {
  if (c == nullptr || stream_ms == nullptr || merge_ms == nullptr || calls == nullptr) return PLH_ERR_INVALID_ARG;
  int rc = use_device(c);
  if (rc != PLH_OK) return rc;
  double a = 0.0, b = 0.0;
  int64_t n = 0;
  for (auto& t : c->ev_pending) {
    PLH_HIP(c, hipEventSynchronize(t[2]), "hipEventSynchronize");
    float x = 0.f, y = 0.f;
    PLH_HIP(c, hipEventElapsedTime(&x, t[0], t[1]), "hipEventElapsedTime");
    PLH_HIP(c, hipEventElapsedTime(&y, t[1], t[2]), "hipEventElapsedTime");
    a += x;
    b += y;
    ++n;
  }
  for (auto& t : c->ev_pending)
    for (hipEvent_t e : t) c->ev_free.push_back(e);
  c->ev_pending.clear();
  *stream_ms = a;
  *merge_ms = b;
  *calls = n;
  return PLH_OK;
}

int plh_fallback_rows(plh_ctx* c, int64_t* out) {
  if (c == nullptr || out == nullptr) return PLH_ERR_INVALID_ARG;
  int rc = use_device(c);
  if (rc != PLH_OK) return rc;
  // this context's calls on a stream it has left are closed by their events
  if (c->ws_stream != nullptr && c->ws_stream != c->stream)
    PLH_HIP(c, hipStreamWaitEvent(c->stream, c->ws_done, 0), "hipStreamWaitEvent");
  if (c->scratch_stream != nullptr && c->scratch_stream != c->stream)
    PLH_HIP(c, hipStreamWaitEvent(c->stream, c->scratch_done, 0), "hipStreamWaitEvent");
  unsigned long long v = 0;
  PLH_HIP(c, hipMemcpyAsync(&v, c->fallback, sizeof(v), hipMemcpyDeviceToHost, c->stream), "hipMemcpyAsync");
  PLH_HIP(c, hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  *out = (int64_t)v;
  return PLH_OK;
}

int plh_alloc(plh_ctx* c, void** out, size_t bytes) {
  if (c == nullptr || out == nullptr) return PLH_ERR_INVALID_ARG;
  *out = nullptr;
  int rc = use_device(c);
  if (rc != PLH_OK) return rc;
  if (bytes == 0) bytes = 1;
  PLH_HIP(c, hipMalloc(out, bytes), "hipMalloc");
  return PLH_OK;
}

int plh_free(plh_ctx* c, void* p) {
  if (c == nullptr) return PLH_ERR_INVALID_ARG;
  if (p == nullptr) return PLH_OK;
  int rc = use_device(c);
  if (rc != PLH_OK) return rc;
  PLH_HIP(c, hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  PLH_HIP(c, hipFree(p), "hipFree");
  return PLH_OK;
}

int plh_h2d(plh_ctx* c, void* dst, const void* src, size_t bytes) {
  if (c == nullptr || (bytes > 0 && (dst == nullptr || src == nullptr))) return PLH_ERR_INVALID_ARG;
  int rc = use_device(c);
  if (rc != PLH_OK) return rc;
  if (bytes == 0) return PLH_OK;
  PLH_HIP(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync(H2D)");
  PLH_HIP(c, hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  return PLH_OK;
}

int plh_host_alloc(plh_ctx* c, void** out, size_t bytes) {
  if (c == nullptr || out == nullptr) return PLH_ERR_INVALID_ARG;
  *out = nullptr;
  int rc = use_device(c);
  if (rc != PLH_OK) return rc;
  const hipError_t e = hipHostMalloc(out, bytes > 0 ? bytes : 1, hipHostMallocDefault);
  if (e != hipSuccess) {
    *out = nullptr;
    return hip_fail(c, e, "hipHostMalloc");
  }
  return PLH_OK;
}

int plh_host_free(plh_ctx* c, void* p) {
  if (c == nullptr) return PLH_ERR_INVALID_ARG;
  if (p == nullptr) return PLH_OK;
  int rc = use_device(c);
  if (rc != PLH_OK) return rc;
  PLH_HIP(c, hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  PLH_HIP(c, hipHostFree(p), "hipHostFree");
  return PLH_OK;
}

int plh_h2d_async(plh_ctx* c, void* dst, const void* src, size_t bytes) {
  if (c == nullptr || (bytes > 0 && (dst == nullptr || src == nullptr))) return PLH_ERR_INVALID_ARG;
  int rc = use_device(c);
  if (rc != PLH_OK) return rc;
  if (bytes == 0) return PLH_OK;
  PLH_HIP(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync(H2D)");
  return PLH_OK;
}

int plh_d2h(plh_ctx* c, void* dst, const void* src, size_t bytes) {
  if (c == nullptr || (bytes > 0 && (dst == nullptr || src == nullptr))) return PLH_ERR_INVALID_ARG;
  int rc = use_device(c);
  if (rc != PLH_OK) return rc;
  if (bytes == 0) return PLH_OK;
  PLH_HIP(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream), "hipMemcpyAsync(D2H)");
  PLH_HIP(c, hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  return PLH_OK;
}

int plh_sync(plh_ctx* c) {
  int rc = use_device(c);
  if (rc != PLH_OK) return rc;
  PLH_HIP(c, hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  return PLH_OK;
}

int plh_sample(plh_ctx* c, const void* logits, int dtype, int64_t ld, int B, int V, const int32_t* hist_ids,
               const int64_t* hist_off, const double* temperature, const int32_t* top_k, const double* top_p,
               const double* rep_penalty, const double* uniforms, int32_t* out_ids, double* out_probs,
               int flags) {
  return sample_impl(c, logits, dtype, ld, B, V, hist_ids, hist_off, temperature, top_k, top_p, rep_penalty,
                     uniforms, out_ids, out_probs, flags, false);
}

int plh_sample_noalloc(plh_ctx* c, const void* logits, int dtype, int64_t ld, int B, int V,
                       const int32_t* hist_ids, const int64_t* hist_off, const double* temperature,
                       const int32_t* top_k, const double* top_p, const double* rep_penalty,
                       const double* uniforms, int32_t* out_ids, double* out_probs, int flags) {
  return sample_impl(c, logits, dtype, ld, B, V, hist_ids, hist_off, temperature, top_k, top_p, rep_penalty,
                     uniforms, out_ids, out_probs, flags, true);
}

int plh_penalize(plh_ctx* c, const void* x, int dtype, int64_t ld, int B, int V, const int32_t* hist_ids,
                 const int64_t* hist_off, const double* rep_penalty, void* out, int64_t out_ld) {
  if (c == nullptr) return PLH_ERR_INVALID_ARG;
  if (B < 0 || V < 1) return fail(c, PLH_ERR_INVALID_ARG, "need B >= 0 and V >= 1%s");
  if (B == 0) return PLH_OK;
  if (dtype != PLH_F32 && dtype != PLH_F64) return fail(c, PLH_ERR_INVALID_ARG, "dtype must be PLH_F32 or PLH_F64%s");
  if (ld < V || out_ld < V) return fail(c, PLH_ERR_INVALID_ARG, "ld and out_ld must be >= V%s");
  if (x == nullptr || out == nullptr || rep_penalty == nullptr)
    return fail(c, PLH_ERR_INVALID_ARG, "null device pointer%s");
  if (hist_off != nullptr && hist_ids == nullptr)
    return fail(c, PLH_ERR_INVALID_ARG, "hist_off given without hist_ids%s");
  {
    // the kernel copies x to out and then penalises out from x: in place, a
    // repeated id could read a value another thread has already penalised
    const size_t es = dtype == PLH_F64 ? 8 : 4;
    const uintptr_t x0 = reinterpret_cast<uintptr_t>(x), o0 = reinterpret_cast<uintptr_t>(out);
    const uintptr_t x1 = x0 + ((size_t)(B - 1) * (size_t)ld + (size_t)V) * es;
    const uintptr_t o1 = o0 + ((size_t)(B - 1) * (size_t)out_ld + (size_t)V) * es;
    bool overlap = x0 < o1 && o0 < x1;
    if (overlap && ld == out_ld) {
      // interleaved rows (x = buf[:, :V], out = buf[:, V:2V]) never touch:
      // row b' of out meets row b of x iff |d + (b' - b) * L| < V * es, with
      // d = o0 - x0 and L the row pitch; only the two m = b' - b nearest
      // -d / L can satisfy it
      const int64_t d = (int64_t)(o0 - x0), L = ld * (int64_t)es, w = (int64_t)V * (int64_t)es;
      const int64_t q = d >= 0 ? -(d / L) - 1 : (-d) / L;  // floor(-d / L) or one below it
      overlap = false;
      for (int64_t m = q - 1; m <= q + 2; ++m)
        if (m > -(int64_t)B && m < (int64_t)B && d + m * L < w && d + m * L > -w) overlap = true;
    }
    if (overlap) return fail(c, PLH_ERR_INVALID_ARG, "out must not overlap x (the penalty works on a copy)%s");
  }
  int rc = use_device(c);
  if (rc != PLH_OK) return rc;
  plh::PenalizeArgs a{x, ld, out, out_ld, B, V, hist_ids, hist_off, rep_penalty};
  const hipError_t e = plh::launch_penalize(a, dtype == PLH_F64, c->stream);
  if (e != hipSuccess) return hip_fail(c, e, "plh_penalize launch");
  return PLH_OK;
}

int plh_draw(plh_ctx* c, const void* p, int dtype, int64_t ld, int B, int V, const double* uniforms,
             int32_t* out_ids) {
  if (c == nullptr) return PLH_ERR_INVALID_ARG;
  if (B < 0 || V < 1) return fail(c, PLH_ERR_INVALID_ARG, "need B >= 0 and V >= 1%s");
  if (B == 0) return PLH_OK;
  if (dtype != PLH_F32 && dtype != PLH_F64) return fail(c, PLH_ERR_INVALID_ARG, "dtype must be PLH_F32 or PLH_F64%s");
  if (ld < V) return fail(c, PLH_ERR_INVALID_ARG, "ld must be >= V%s");
  if (p == nullptr || uniforms == nullptr || out_ids == nullptr)
    return fail(c, PLH_ERR_INVALID_ARG, "null device pointer%s");
  int rc = use_device(c);
  if (rc != PLH_OK) return rc;
  plh::DrawArgs a{p, ld, B, V, uniforms, out_ids};
  const hipError_t e = plh::launch_draw(a, dtype == PLH_F64, c->stream);
  if (e != hipSuccess) return hip_fail(c, e, "plh_draw launch");
  return PLH_OK;
}

int plh_verify(plh_ctx* c, const void* p, const void* q, int dtype, int B, int k, int V, const int32_t* draft,
               const double* accept_u, const double* draw_u, int draw_u_per_stop, int32_t* out_tokens,
               int32_t* out_n_acc) {
  if (c == nullptr) return PLH_ERR_INVALID_ARG;
  if (B < 0 || k < 0 || V < 1) return fail(c, PLH_ERR_INVALID_ARG, "need B >= 0, k >= 0 and V >= 1%s");
  if (B == 0) return PLH_OK;
  if (dtype != PLH_F32 && dtype != PLH_F64) return fail(c, PLH_ERR_INVALID_ARG, "dtype must be PLH_F32 or PLH_F64%s");
  if (p == nullptr || draw_u == nullptr || out_tokens == nullptr || out_n_acc == nullptr)
    return fail(c, PLH_ERR_INVALID_ARG, "null device pointer%s");
  if (k > 0 && (q == nullptr || draft == nullptr || accept_u == nullptr))
    return fail(c, PLH_ERR_INVALID_ARG, "null device pointer%s");
  int rc = use_device(c);
  if (rc != PLH_OK) return rc;
  plh::VerifyArgs a{p, q, B, k, V, draft, accept_u, draw_u, draw_u_per_stop ? 1 : 0, out_tokens, out_n_acc};
  rc = reserve_ws(c, plh::verify_ws_bytes(B, V));
  if (rc != PLH_OK) return rc;
  const plh::VerifyWs ws = plh::verify_ws_layout(c->ws, B, V);
  std::array<hipEvent_t, 3> ev{};
  rc = timing_begin(c, ev);
  if (rc != PLH_OK) return rc;
  const hipError_t e = plh::launch_verify(a, ws, dtype == PLH_F64, c->stream, ev[1]);
  if (e != hipSuccess) return hip_fail(c, e, "plh_verify launch");
  if (c->timing) PLH_HIP(c, hipEventRecord(ev[2], c->stream), "hipEventRecord");
  c->ws_stream = c->stream;
  c->ws_open = true;
  return PLH_OK;
}

int plh_copy_rows(plh_ctx* c, void* dst, int64_t dst_pitch, const void* src, int64_t src_pitch, int64_t row_bytes,
                  int rows) {
  if (c == nullptr) return PLH_ERR_INVALID_ARG;
  if (rows < 0 || row_bytes < 0 || dst_pitch < row_bytes || src_pitch < row_bytes)
    return fail(c, PLH_ERR_INVALID_ARG, "need rows, row_bytes >= 0 and pitches >= row_bytes%s");
  if (rows == 0 || row_bytes == 0) return PLH_OK;
  if (dst == nullptr || src == nullptr) return fail(c, PLH_ERR_INVALID_ARG, "null device pointer%s");
  int rc = use_device(c);
  if (rc != PLH_OK) return rc;
  PLH_HIP(c, hipMemcpy2DAsync(dst, (size_t)dst_pitch, src, (size_t)src_pitch, (size_t)row_bytes, (size_t)rows,
                              hipMemcpyDeviceToDevice, c->stream),
          "hipMemcpy2DAsync");
  return PLH_OK;
}

int plh_append_ids(plh_ctx* c, int32_t* slab, const int64_t* pos, const int32_t* ids, int n) {
  if (c == nullptr) return PLH_ERR_INVALID_ARG;
  if (n < 0) return fail(c, PLH_ERR_INVALID_ARG, "need n >= 0%s");
  if (n == 0) return PLH_OK;
  if (slab == nullptr || pos == nullptr || ids == nullptr) return fail(c, PLH_ERR_INVALID_ARG, "null device pointer%s");
  int rc = use_device(c);
  if (rc != PLH_OK) return rc;
  const hipError_t e = plh::launch_append(slab, pos, ids, n, c->stream);
  if (e != hipSuccess) return hip_fail(c, e, "plh_append_ids launch");
  return PLH_OK;
}

int plh_rmsnorm_lm_head(plh_ctx* c, const float* h, int64_t ldh, int N, int D, const float* norm, double eps,
                        const float* W, int64_t ldw, int V, float* out, int64_t ldo) {
  if (c == nullptr) return PLH_ERR_INVALID_ARG;
  if (N < 0 || D < 1 || V < 1) return fail(c, PLH_ERR_INVALID_ARG, "need N >= 0, D >= 1 and V >= 1%s");
  if (N == 0) return PLH_OK;
  if (ldh < D || ldw < V || ldo < V) return fail(c, PLH_ERR_INVALID_ARG, "need ldh >= D, ldw >= V and ldo >= V%s");
  if (h == nullptr || norm == nullptr || W == nullptr || out == nullptr)
    return fail(c, PLH_ERR_INVALID_ARG, "null device pointer%s");
  if (!(eps >= 0.0) || !std::isfinite(eps)) return fail(c, PLH_ERR_INVALID_ARG, "eps must be finite and >= 0%s");
  int rc = use_device(c);
  if (rc != PLH_OK) return rc;
  rc = reserve_ws(c, plh::head_ws_bytes(N, D));
  if (rc != PLH_OK) return rc;
  plh::HeadArgs a{};
  a.h = h;
  a.ldh = ldh;
  a.norm = norm;
  a.eps = (float)eps;
  a.w = W;
  a.ldw = ldw;
  a.out = out;
  a.ldo = ldo;
  a.act = static_cast<float*>(c->ws);
  a.N = N;
  a.D = D;
  a.V = V;
  const hipError_t e = plh::launch_head(a, c->stream);
  if (e != hipSuccess) return hip_fail(c, e, "plh_rmsnorm_lm_head launch");
  c->ws_stream = c->stream;
  c->ws_open = true;
  return PLH_OK;
}

}  // extern "C"
