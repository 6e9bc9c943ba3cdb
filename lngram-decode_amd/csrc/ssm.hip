// Diagonal SSM scan: s_t = a * s_{t-1} + (1 - a) * u_t, s_{-1} = s0 (or 0).
//
// Reduce-then-scan over time chunks of SSM_L steps, one wave per (batch,
// 64-channel group, chunk), lanes = channels so every step is one coalesced
// 256-byte row access:
//   k_ssm_chunk_end : zero-initial scan of each chunk -> its end state e_c
//   k_ssm_apply     : carry_c = a^L carry_{c-1} + e_{c-1} (short loop over the
//                     preceding chunk ends, fp64), then the chunk is re-scanned
//                     from carry_c with the plain fp32 recurrence.
#include "common.h"

namespace lng {

constexpr int SSM_L = 64;

__global__ __launch_bounds__(64) void k_ssm_chunk_end(const float* __restrict__ a, const float* __restrict__ u,
                                                      int64_t T, int32_t N, int32_t C, float* __restrict__ ends) {
  const int n = blockIdx.y * 64 + threadIdx.x;
  const int c = blockIdx.x;
  const int64_t b = blockIdx.z;
  if (n >= N) return;
  const float an = a[n], bn = 1.0f - an;
  const int64_t t0 = static_cast<int64_t>(c) * SSM_L;
  const int64_t t1 = t0 + SSM_L < T ? t0 + SSM_L : T;
  const float* ub = u + (b * T) * N + n;
  float x[SSM_L];
#pragma unroll
  for (int i = 0; i < SSM_L; ++i) x[i] = (t0 + i < t1) ? ub[(t0 + i) * N] : 0.f;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < SSM_L; ++i)
    if (t0 + i < t1) s = fmaf(an, s, bn * x[i]);
  ends[(b * C + c) * N + n] = s;
}

__global__ __launch_bounds__(64) void k_ssm_apply(const float* __restrict__ a, const float* __restrict__ u,
                                                  const float* __restrict__ s0, int64_t T, int32_t N, int32_t C,
                                                  const float* __restrict__ ends, float* __restrict__ s_out) {
  const int n = blockIdx.y * 64 + threadIdx.x;
  const int c = blockIdx.x;
  const int64_t b = blockIdx.z;
  if (n >= N) return;
  const float an = a[n], bn = 1.0f - an;
  // a^L in fp64 by repeated squaring (SSM_L is a power of two)
  double aL = an;
  for (int k = 1; k < SSM_L; k <<= 1) aL *= aL;
  double carry = s0 ? static_cast<double>(s0[b * N + n]) : 0.0;
  for (int q = 0; q < c; ++q) carry = aL * carry + static_cast<double>(ends[(b * C + q) * N + n]);
  const int64_t t0 = static_cast<int64_t>(c) * SSM_L;
  const int64_t t1 = t0 + SSM_L < T ? t0 + SSM_L : T;
  const float* ub = u + (b * T) * N + n;
  float* sb = s_out + (b * T) * N + n;
  float x[SSM_L];
#pragma unroll
  for (int i = 0; i < SSM_L; ++i) x[i] = (t0 + i < t1) ? ub[(t0 + i) * N] : 0.f;
  float s = static_cast<float>(carry);
#pragma unroll
  for (int i = 0; i < SSM_L; ++i) {
    if (t0 + i < t1) {
      s = fmaf(an, s, bn * x[i]);
      sb[(t0 + i) * N] = s;
    }
  }
}

}  // namespace lng

using namespace lng;

extern "C" {

size_t lng_ssm_workspace_bytes(int64_t B, int64_t T, int32_t N) {
  return static_cast<size_t>(B) * static_cast<size_t>(cdiv(T, SSM_L)) * static_cast<size_t>(N) * sizeof(float);
}

int lng_ssm_scan(const float* a, const float* u, const float* s0, int64_t B, int64_t T, int32_t N, float* workspace,
                 float* s, void* stream) {
  if (B < 0 || T < 0 || N <= 0) return fail(LNG_E_ARG, "ssm_scan: bad shape");
  if (B == 0 || T == 0) return LNG_OK;
  if (!workspace) return fail(LNG_E_ARG, "ssm_scan: workspace required (lng_ssm_workspace_bytes)");
  const int64_t C = cdiv(T, SSM_L);
  if (C > 65535 || B > 65535) return fail(LNG_E_ARG, "ssm_scan: sequence too long");
  dim3 grid(static_cast<unsigned>(C), static_cast<unsigned>(cdiv(N, 64)), static_cast<unsigned>(B));
  hipStream_t st = as_stream(stream);
  hipLaunchKernelGGL(k_ssm_chunk_end, grid, dim3(64), 0, st, a, u, T, N, static_cast<int32_t>(C), workspace);
  if (int rc = check_launch("ssm_chunk_end")) return rc;
  hipLaunchKernelGGL(k_ssm_apply, grid, dim3(64), 0, st, a, u, s0, T, N, static_cast<int32_t>(C), workspace, s);
  return check_launch("ssm_apply");
}

}  // extern "C"
