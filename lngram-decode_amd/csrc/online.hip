// Code-keyed online counts over a batch of query windows (drafting/drafters.py:117-142,
// OnlineCounts.mix): the committed (row at t, token t + 1) pairs of one sequence are the keys; a
// query row j matches pair t on every (route, order) whose key row equals the query's row, and only
// pairs with t <= deadline[j] count.  The match weights mix the next-token distribution p:
//
//   w[j, t] = #{(r, n) : key[t, r, n] == q[j, r, n] >= 0}          (t <= deadline[j], else 0)
//   tot = sum_t w[j, t];  n_eff = tot / (R * n_orders);  lam = n_eff / (n_eff + kappa)
//   out[j, v] = (1 - lam) p[j, v] + lam * (sum_{t : nxt[t] = v} w[j, t]) / max(tot, 1e-9)
//
// The drafter's own kernels do the same inside a draft step; this is the batched form for callers
// that hold their own windows (the offline drafting harness's OnlineCounts).
#include "common.h"

namespace lng {

// One wave per (query row, pair); lanes over the R * n_orders key entries.
__global__ __launch_bounds__(256) void k_online_match(const int32_t* __restrict__ keys, int32_t T,
                                                      const int32_t* __restrict__ q,
                                                      const int64_t* __restrict__ deadline, int32_t RK,
                                                      float* __restrict__ w) {
  const int lane = threadIdx.x & 63;
  const int j = blockIdx.y;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  float cnt = 0.f;
  if (static_cast<int64_t>(t) <= deadline[j]) {  // uniform across the wave
    const int32_t* kt = keys + static_cast<int64_t>(t) * RK;
    const int32_t* qj = q + static_cast<int64_t>(j) * RK;
    for (int i = lane; i < RK; i += 64) {
      const int32_t qq = qj[i];
      cnt += (qq >= 0 && kt[i] == qq) ? 1.f : 0.f;
    }
    cnt = wave_sum(cnt);
  }
  if (lane == 0) w[static_cast<int64_t>(j) * T + t] = cnt;
}

// One block per query row: the total in a fixed order, the base term for every token, then the
// count term added at the pairs' next tokens.
__global__ __launch_bounds__(256) void k_online_mix(const float* __restrict__ w, const int64_t* __restrict__ nxt,
                                                    int32_t T, int32_t RK, const float* __restrict__ p, int64_t V,
                                                    float kappa, float* __restrict__ out) {
  __shared__ float red[4];
  const int j = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float* wj = w + static_cast<int64_t>(j) * T;
  float s = 0.f;
  for (int t = tid; t < T; t += 256) s += wj[t];
  s = wave_sum(s);
  if (lane == 0) red[wave] = s;
  __syncthreads();
  const float tot = (red[0] + red[1]) + (red[2] + red[3]);
  const float n_eff = tot / static_cast<float>(RK);
  const float lam = n_eff / (n_eff + kappa);
  const float add = lam / fmaxf(tot, 1e-9f);
  const float* pj = p + static_cast<int64_t>(j) * V;
  float* oj = out + static_cast<int64_t>(j) * V;
  for (int64_t v = tid; v < V; v += 256) oj[v] = (1.f - lam) * pj[v];
  __threadfence();
  __syncthreads();
  for (int t = tid; t < T; t += 256) {
    const float wt = wj[t];
    const int64_t v = nxt[t];
    if (wt > 0.f && v >= 0 && v < V) atomicAdd(oj + v, wt * add);  // ids outside the vocabulary add nothing
  }
}

}  // namespace lng

using namespace lng;

extern "C" {

int lng_online_mix(const int32_t* keys, const int64_t* nxt, int32_t T, const int32_t* q, const int64_t* deadline,
                   int32_t N, int32_t R, int32_t n_orders, const float* p, int64_t V, float kappa, float* w_work,
                   float* out, void* stream) {
  if (T < 0 || N < 0 || R <= 0 || n_orders <= 0 || V <= 0 || !(kappa > 0.f))
    return fail(LNG_E_ARG, "online_mix: bad shape or kappa");
  if (N > 65535) return fail(LNG_E_ARG, "online_mix: at most 65535 query rows");
  if (p == out) return fail(LNG_E_ARG, "online_mix: out must not alias p");
  if (N == 0) return LNG_OK;
  hipStream_t s = as_stream(stream);
  const int32_t RK = R * n_orders;
  if (T > 0) {
    hipLaunchKernelGGL(k_online_match, dim3(static_cast<unsigned>(cdiv(T, 4)), static_cast<unsigned>(N)), dim3(256),
                       0, s, keys, T, q, deadline, RK, w_work);
    if (int rc = check_launch("online_match")) return rc;
  }
  hipLaunchKernelGGL(k_online_mix, dim3(static_cast<unsigned>(N)), dim3(256), 0, s, w_work, nxt, T, RK, p, V, kappa,
                     out);
  return check_launch("online_mix");
}

}  // extern "C"
