// Internal launch interface between the C ABI (plh_api.hip) and the kernel
// translation units.  Not part of the public header.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace plh {

struct SampleArgs {
  const void* logits;
  int64_t ld;
  int B, V;
  const int32_t* hist_ids;
  const int64_t* hist_off;
  const double* temperature;
  const int32_t* top_k;
  const double* top_p;
  const double* rep_penalty;
  const double* uniforms;
  int32_t* out_ids;
  double* out_probs;
  unsigned long long* fallback_rows;  // rows finished by the general path
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

hipError_t launch_sample_rows(const SampleArgs& a, bool f64, bool vec, hipStream_t s);
hipError_t launch_sample_fast(const SampleArgs& a, bool f64, bool vec, hipStream_t s);
hipError_t launch_draw(const DrawArgs& a, bool f64, hipStream_t s);
hipError_t launch_penalize(const PenalizeArgs& a, bool f64, hipStream_t s);
hipError_t launch_verify(const VerifyArgs& a, bool f64, hipStream_t s);

}  // namespace plh
