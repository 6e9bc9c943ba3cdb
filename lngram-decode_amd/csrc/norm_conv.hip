// RMSNorm rows and the readout's short causal convolution (+ residual).
//
// Rounding follows the reference: normalise in fp32, round to the storage type,
// multiply by the weight and round again; the conv accumulates in fp32 and
// rounds its output, SiLU and the residual add each round once more.
#include "common.h"

namespace lng {

// One wave per row; 4 rows per 256-thread block.
template <typename T>
__global__ __launch_bounds__(256) void k_rmsnorm(const T* __restrict__ x, const T* __restrict__ w, int64_t rows,
                                                 int32_t dim, float eps, T* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * dim;
  float ss = 0.f;
  for (int c = lane; c < dim; c += 64) {
    const float v = to_f32(xr[c]);
    ss = fmaf(v, v, ss);
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / static_cast<float>(dim) + eps);
  T* o = out + row * dim;
  for (int c = lane; c < dim; c += 64) o[c] = from_f32<T>(round_to<T>(to_f32(xr[c]) * r) * to_f32(w[c]));
}

constexpr int CONV_TT = 16;  // positions per block

// out[b,t,c] = [mixed +] SiLU(sum_j w[c,j] * xn[b, t - (K-1-j)*dil, c]), xn = RMSNorm(mixed).
// Block: one (b, 16-position tile).  Row scales of the tile and its causal halo
// are computed first (one wave per row), then threads sweep the channels.
template <typename T>
__global__ __launch_bounds__(256) void k_causal_conv(const T* __restrict__ mixed, const T* __restrict__ norm_w,
                                                     const T* __restrict__ conv_w, int64_t T_len, int32_t d, int32_t K,
                                                     int32_t dil, float eps, int residual, T* __restrict__ out) {
  extern __shared__ float scale[];  // [CONV_TT + (K-1)*dil]
  const int64_t b = blockIdx.y;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * CONV_TT;
  const int halo = (K - 1) * dil;
  const int nrow = CONV_TT + halo;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const T* base = mixed + b * T_len * d;
  for (int i = wave; i < nrow; i += 4) {
    const int64_t t = t0 - halo + i;
    float r = 0.f;
    if (t >= 0 && t < T_len) {
      float ss = 0.f;
      for (int c = lane; c < d; c += 64) {
        const float v = to_f32(base[t * d + c]);
        ss = fmaf(v, v, ss);
      }
      ss = wave_sum(ss);
      r = 1.0f / sqrtf(ss / static_cast<float>(d) + eps);
    }
    if (lane == 0) scale[i] = r;
  }
  __syncthreads();
  for (int c = threadIdx.x; c < d; c += blockDim.x) {
    const float nw = to_f32(norm_w[c]);
    for (int tt = 0; tt < CONV_TT; ++tt) {
      const int64_t t = t0 + tt;
      if (t >= T_len) break;
      float acc = 0.f;
      for (int j = 0; j < K; ++j) {
        const int lag = (K - 1 - j) * dil;
        const int64_t ts = t - lag;
        if (ts < 0) continue;
        const float xn = round_to<T>(round_to<T>(to_f32(base[ts * d + c]) * scale[tt + halo - lag]) * nw);
        acc = fmaf(to_f32(conv_w[c * K + j]), xn, acc);
      }
      const float y = round_to<T>(acc);
      const float act = round_to<T>(y / (1.0f + expf(-y)));
      out[(b * T_len + t) * d + c] = residual ? from_f32<T>(to_f32(base[t * d + c]) + act) : from_f32<T>(act);
    }
  }
}

}  // namespace lng

using namespace lng;

extern "C" {

int lng_rmsnorm(const void* x, const void* w, int dtype, int64_t rows, int32_t dim, float eps, void* out,
                void* stream) {
  if (rows < 0 || dim <= 0) return fail(LNG_E_ARG, "rmsnorm: bad shape");
  if (rows == 0) return LNG_OK;
  dim3 grid(static_cast<unsigned>(cdiv(rows, 4)));
  hipStream_t s = as_stream(stream);
  if (dtype == LNG_F32)
    hipLaunchKernelGGL(k_rmsnorm<float>, grid, dim3(256), 0, s, static_cast<const float*>(x),
                       static_cast<const float*>(w), rows, dim, eps, static_cast<float*>(out));
  else if (dtype == LNG_BF16)
    hipLaunchKernelGGL(k_rmsnorm<bf16>, grid, dim3(256), 0, s, static_cast<const bf16*>(x), static_cast<const bf16*>(w),
                       rows, dim, eps, static_cast<bf16*>(out));
  else
    return fail(LNG_E_DTYPE, "rmsnorm: dtype must be f32 or bf16");
  return check_launch("rmsnorm");
}

int lng_causal_conv(const void* mixed, const void* norm_w, const void* conv_w, int dtype, int64_t B, int64_t T,
                    int32_t d, int32_t K, int32_t dilation, float eps, int residual, void* out, void* stream) {
  if (B < 0 || T < 0 || d <= 0 || K <= 0 || dilation <= 0) return fail(LNG_E_ARG, "causal_conv: bad shape");
  if (mixed == out) return fail(LNG_E_ARG, "causal_conv: out must not alias mixed");
  if (B == 0 || T == 0) return LNG_OK;
  const int halo = (K - 1) * dilation;
  if (halo > 4096) return fail(LNG_E_ARG, "causal_conv: receptive field too large");
  dim3 grid(static_cast<unsigned>(cdiv(T, CONV_TT)), static_cast<unsigned>(B));
  const size_t lds = sizeof(float) * (CONV_TT + halo);
  hipStream_t s = as_stream(stream);
  if (dtype == LNG_F32)
    hipLaunchKernelGGL(k_causal_conv<float>, grid, dim3(256), lds, s, static_cast<const float*>(mixed),
                       static_cast<const float*>(norm_w), static_cast<const float*>(conv_w), T, d, K, dilation, eps,
                       residual, static_cast<float*>(out));
  else if (dtype == LNG_BF16)
    hipLaunchKernelGGL(k_causal_conv<bf16>, grid, dim3(256), lds, s, static_cast<const bf16*>(mixed),
                       static_cast<const bf16*>(norm_w), static_cast<const bf16*>(conv_w), T, d, K, dilation, eps,
                       residual, static_cast<bf16*>(out));
  else
    return fail(LNG_E_DTYPE, "causal_conv: dtype must be f32 or bf16");
  return check_launch("causal_conv");
}

}  // extern "C"
