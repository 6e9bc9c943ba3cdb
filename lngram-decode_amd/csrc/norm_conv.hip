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

// Kernel 4, dilation 3 (the configured short conv: dilation = max n-gram order 3).
// Block = (b, 16 positions), 128 threads x 8 channels (16-byte accesses).  Row scales of
// the 16 + 9 rows come first (one wave per row); then each thread slides over the rows
// keeping the last 10 normalised rows of its channels in registers.
constexpr int C43_TT = 16;
constexpr int C43_HALO = 9;

__device__ __forceinline__ void load8(const float* p, float (&v)[8]) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(p), b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[j] = a[j];
    v[4 + j] = b[j];
  }
}
__device__ __forceinline__ void load8(const bf16* p, float (&v)[8]) {
  const bf16x8 a = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = static_cast<float>(a[j]);
}
__device__ __forceinline__ void store8(float* p, const float (&v)[8]) {
  *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
  *reinterpret_cast<f32x4*>(p + 4) = f32x4{v[4], v[5], v[6], v[7]};
}
__device__ __forceinline__ void store8(bf16* p, const float (&v)[8]) {
  bf16x8 a;
#pragma unroll
  for (int j = 0; j < 8; ++j) a[j] = static_cast<bf16>(v[j]);
  *reinterpret_cast<bf16x8*>(p) = a;
}

template <typename T>
__global__ __launch_bounds__(128) void k_causal_conv_k4d3(const T* __restrict__ mixed, const T* __restrict__ norm_w,
                                                          const T* __restrict__ conv_w, int64_t T_len, int32_t d,
                                                          float eps, int residual, T* __restrict__ out) {
  __shared__ float scale[C43_TT + C43_HALO];
  const int64_t b = blockIdx.y;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * C43_TT;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const T* base = mixed + b * T_len * d;
  for (int i = wave; i < C43_TT + C43_HALO; i += 2) {
    const int64_t t = t0 - C43_HALO + i;
    float r = 0.f;
    if (t >= 0 && t < T_len) {
      float ss = 0.f;
      for (int c = lane * 8; c < d; c += 64 * 8) {
        float v[8];
        load8(base + t * d + c, v);
#pragma unroll
        for (int j = 0; j < 8; ++j) ss = fmaf(v[j], v[j], ss);
      }
      ss = wave_sum(ss);
      r = 1.0f / sqrtf(ss / static_cast<float>(d) + eps);
    }
    if (lane == 0) scale[i] = r;
  }
  __syncthreads();
  for (int c = threadIdx.x * 8; c < d; c += blockDim.x * 8) {
    float nw[8], w[4][8];
    load8(norm_w + c, nw);
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int k = 0; k < 4; ++k) w[k][j] = to_f32(conv_w[(c + j) * 4 + k]);
    float hist[10][8];  // hist[k] = normalised row at t - k
#pragma unroll
    for (int k = 0; k < 10; ++k)
#pragma unroll
      for (int j = 0; j < 8; ++j) hist[k][j] = 0.f;
#pragma unroll
    for (int step = 0; step < C43_TT + C43_HALO; ++step) {
      const int64_t t = t0 - C43_HALO + step;
#pragma unroll
      for (int k = 9; k > 0; --k)
#pragma unroll
        for (int j = 0; j < 8; ++j) hist[k][j] = hist[k - 1][j];
      float x[8];
      if (t >= 0 && t < T_len) {
        load8(base + t * d + c, x);
        const float s = scale[step];
#pragma unroll
        for (int j = 0; j < 8; ++j) hist[0][j] = round_to<T>(round_to<T>(x[j] * s) * nw[j]);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          hist[0][j] = 0.f;
          x[j] = 0.f;
        }
      }
      if (step >= C43_HALO && t < T_len) {
        float o[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          float acc = w[0][j] * hist[9][j];
          acc = fmaf(w[1][j], hist[6][j], acc);
          acc = fmaf(w[2][j], hist[3][j], acc);
          acc = fmaf(w[3][j], hist[0][j], acc);
          const float y = round_to<T>(acc);
          const float act = round_to<T>(y / (1.0f + expf(-y)));
          o[j] = residual ? x[j] + act : act;
        }
        store8(out + (b * T_len + t) * d + c, o);
      }
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
  hipStream_t s = as_stream(stream);
  if (K == 4 && dilation == 3 && d % 8 == 0 && (dtype == LNG_F32 || dtype == LNG_BF16)) {
    dim3 g43(static_cast<unsigned>(cdiv(T, C43_TT)), static_cast<unsigned>(B));
    if (dtype == LNG_F32)
      hipLaunchKernelGGL(k_causal_conv_k4d3<float>, g43, dim3(128), 0, s, static_cast<const float*>(mixed),
                         static_cast<const float*>(norm_w), static_cast<const float*>(conv_w), T, d, eps, residual,
                         static_cast<float*>(out));
    else
      hipLaunchKernelGGL(k_causal_conv_k4d3<bf16>, g43, dim3(128), 0, s, static_cast<const bf16*>(mixed),
                         static_cast<const bf16*>(norm_w), static_cast<const bf16*>(conv_w), T, d, eps, residual,
                         static_cast<bf16*>(out));
    return check_launch("causal_conv_k4d3");
  }
  dim3 grid(static_cast<unsigned>(cdiv(T, CONV_TT)), static_cast<unsigned>(B));
  const size_t lds = sizeof(float) * (CONV_TT + halo);
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
