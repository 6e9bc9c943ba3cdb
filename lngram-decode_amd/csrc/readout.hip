// Route readout in its materialised form: sink-softmax attention over the R route
// slots with keys/values as produced by the memory projection.  Used by cached
// decode, tree verification, the draft head and the fp32 layer; the bf16 layer
// forward uses the fused kernel (readout_fused.hip).
#include "common.h"

namespace lng {

// ------------------------------------------------------------------ sink probabilities
__global__ __launch_bounds__(256) void k_sink_probs(const float* __restrict__ scores, int64_t M, int32_t R, float sink,
                                                    float* __restrict__ probs) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const float* s = scores + row * R;
  float m = sink;
  for (int r = lane; r < R; r += 64) m = fmaxf(m, s[r]);
  m = wave_max(m);
  float z = 0.f;
  for (int r = lane; r < R; r += 64) z += expf(s[r] - m);
  z = wave_sum(z) + expf(sink - m);
  for (int r = lane; r < R; r += 64) probs[row * R + r] = expf(s[r] - m) / z;
}

// ------------------------------------------------------------------ materialised sink attention
// One wave per (token, query head).  Scores are rounded to the storage type before
// the fp32 scale (the reference's matmul output), probabilities are rounded to the
// storage type before the value product, the output is rounded once.
template <typename T>
__global__ __launch_bounds__(256) void k_sink_attention(const T* __restrict__ q, const T* __restrict__ key,
                                                        const T* __restrict__ value, int64_t BT, int32_t KV, int32_t G,
                                                        int32_t R, int32_t hd, int64_t ks_bt, int64_t ks_h,
                                                        int64_t ks_r, int64_t vs_bt, int64_t vs_h, int64_t vs_r,
                                                        float scale, float sink, T* __restrict__ out) {
  extern __shared__ float sm[];  // 4 waves x R probabilities
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + wave;  // (bt, head)
  const int64_t H = static_cast<int64_t>(KV) * G;
  float* p = sm + wave * R;
  const bool ok = item < BT * H;
  const int64_t bt = ok ? item / H : 0;
  const int head = ok ? static_cast<int>(item % H) : 0;
  const int h = head / G;
  const T* qv = q + (bt * H + head) * hd;
  float m = sink;
  if (ok) {
    for (int r = lane; r < R; r += 64) {
      const T* kr = key + bt * ks_bt + h * ks_h + r * ks_r;
      float acc = 0.f;
      for (int d = 0; d < hd; ++d) acc = fmaf(to_f32(qv[d]), to_f32(kr[d]), acc);
      const float sc = round_to<T>(acc) * scale;
      p[r] = sc;
      m = fmaxf(m, sc);
    }
  }
  m = wave_max(m);
  float z = 0.f;
  if (ok)
    for (int r = lane; r < R; r += 64) {
      const float e = expf(p[r] - m);
      p[r] = e;
      z += e;
    }
  z = wave_sum(z) + expf(sink - m);
  __syncthreads();
  if (!ok) return;
  for (int d = lane; d < hd; d += 64) {
    float acc = 0.f;
    for (int r = 0; r < R; ++r) acc = fmaf(round_to<T>(p[r] / z), to_f32(value[bt * vs_bt + h * vs_h + r * vs_r + d]), acc);
    out[(bt * H + head) * hd + d] = from_f32<T>(acc);
  }
}

}  // namespace lng

using namespace lng;

extern "C" {

int lng_sink_probabilities(const float* scores, int64_t M, int32_t R, float sink_logit, float* probs, void* stream) {
  if (M < 0 || R <= 0) return fail(LNG_E_ARG, "sink_probabilities: bad shape");
  if (M == 0) return LNG_OK;
  hipLaunchKernelGGL(k_sink_probs, dim3(cdiv(M, 4)), dim3(256), 0, as_stream(stream), scores, M, R, sink_logit, probs);
  return check_launch("sink_probabilities");
}

int lng_sink_attention_strided(const void* query, const void* key, const void* value, int dtype, int64_t BT,
                               int32_t kv_heads, int32_t groups, int32_t R, int32_t head_dim, const int64_t* kstride,
                               const int64_t* vstride, float scale, float sink_logit, void* out, void* stream) {
  if (BT < 0 || kv_heads <= 0 || groups <= 0 || R <= 0 || head_dim <= 0)
    return fail(LNG_E_ARG, "sink_attention: bad shape");
  if (R > 4096) return fail(LNG_E_ARG, "sink_attention: too many routes");
  if (BT == 0) return LNG_OK;
  const int64_t items = BT * kv_heads * groups;
  const size_t lds = sizeof(float) * 4 * R;
  hipStream_t s = as_stream(stream);
  if (dtype == LNG_F32)
    hipLaunchKernelGGL(k_sink_attention<float>, dim3(cdiv(items, 4)), dim3(256), lds, s,
                       static_cast<const float*>(query), static_cast<const float*>(key),
                       static_cast<const float*>(value), BT, kv_heads, groups, R, head_dim, kstride[0], kstride[1],
                       kstride[2], vstride[0], vstride[1], vstride[2], scale, sink_logit, static_cast<float*>(out));
  else if (dtype == LNG_BF16)
    hipLaunchKernelGGL(k_sink_attention<bf16>, dim3(cdiv(items, 4)), dim3(256), lds, s,
                       static_cast<const bf16*>(query), static_cast<const bf16*>(key), static_cast<const bf16*>(value),
                       BT, kv_heads, groups, R, head_dim, kstride[0], kstride[1], kstride[2], vstride[0], vstride[1],
                       vstride[2], scale, sink_logit, static_cast<bf16*>(out));
  else
    return fail(LNG_E_DTYPE, "sink_attention: dtype must be f32 or bf16");
  return check_launch("sink_attention");
}

int lng_sink_attention(const void* query, const void* key, const void* value, int dtype, int64_t BT, int32_t kv_heads,
                       int32_t groups, int32_t R, int32_t head_dim, float scale, float sink_logit, void* out,
                       void* stream) {
  const int64_t ks[3] = {static_cast<int64_t>(kv_heads) * R * head_dim, static_cast<int64_t>(R) * head_dim, head_dim};
  return lng_sink_attention_strided(query, key, value, dtype, BT, kv_heads, groups, R, head_dim, ks, ks, scale,
                                    sink_logit, out, stream);
}

}  // extern "C"
