// RMSNorm rows and the readout's short causal convolution (+ residual).
//
// The reference has two RMSNorms that round differently in bf16:
// - model.RMSNorm (ffnmem/model.py:39-48; h_norm, router features, draft head, SSM input):
//   normalise in fp32, round to the storage type, multiply by the weight, round again;
// - lngram_v2.RMSNorm (lngram_v2.py:36-53, F.rms_norm; the readout's query, memory and
//   short-conv norms): normalise and apply the weight in fp32, round once.
// The short conv normalises with the second; it accumulates its taps in fp32 and rounds its
// output, SiLU and the residual add each once more.
#include "common.h"

namespace lng {

// One wave per row; 4 rows per 256-thread block.
// One normalised element: FUSED = F.rms_norm (weight applied in fp32, one rounding), else
// model.RMSNorm (round, multiply by the weight, round).
template <typename T, bool FUSED>
__device__ __forceinline__ float norm_elem(float x, float r, float w) {
  return FUSED ? round_to<T>(x * r * w) : round_to<T>(round_to<T>(x * r) * w);
}

template <typename T, bool FUSED>
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
  for (int c = lane; c < dim; c += 64) o[c] = from_f32<T>(norm_elem<T, FUSED>(to_f32(xr[c]), r, to_f32(w[c])));
}

// Vectorised RMSNorm for dim = NV * 512 (bf16: 16-byte loads): one wave per row, the
// whole row is loaded into registers before the reduction (one memory latency per row).
template <int NV, bool FUSED>
__global__ __launch_bounds__(256) void k_rmsnorm_bf16_vec(const bf16* __restrict__ x, const bf16* __restrict__ w,
                                                          int64_t rows, float eps, bf16* __restrict__ out) {
  constexpr int dim = NV * 512;
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const bf16* xr = x + row * dim;
  bf16x8 v[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) v[i] = *reinterpret_cast<const bf16x8*>(xr + (i * 64 + lane) * 8);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float f = static_cast<float>(v[i][j]);
      ss = fmaf(f, f, ss);
    }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / static_cast<float>(dim) + eps);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const bf16x8 wv = *reinterpret_cast<const bf16x8*>(w + (i * 64 + lane) * 8);
    bf16x8 o;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      o[j] = static_cast<bf16>(norm_elem<bf16, FUSED>(static_cast<float>(v[i][j]), r, static_cast<float>(wv[j])));
    *reinterpret_cast<bf16x8*>(out + row * dim + (i * 64 + lane) * 8) = o;
  }
}

constexpr int CONV_TT = 16;  // positions per block

// Rows the convolutions read: B sequences of `len` rows (positions 0 .. len-1, batch stride
// `stride` rows, rows before position 0 are the zero left padding); outputs for positions
// p0 .. p0+n-1 of each sequence, p0 = pos0 (+ *pos0_dev), written to out[b * n + (t - p0)].  A
// whole sequence: stride = len = n, p0 = 0; a decode step: the cache, p0 = the cached length.
// Positions at or past `len` produce nothing.
struct ConvWin {
  int64_t stride, len, pos0, n;
  const int32_t* pos0_dev;
};
__device__ __forceinline__ int64_t conv_p0(const ConvWin& W) {
  return W.pos0 + (W.pos0_dev ? static_cast<int64_t>(*W.pos0_dev) : 0);
}

// out[b,t,c] = [mixed +] SiLU(sum_j w[c,j] * xn[b, t - (K-1-j)*dil, c]), xn = RMSNorm(mixed).
// Block: one (b, 16-position tile).  Row scales of the tile and its causal halo
// are computed first (one wave per row), then threads sweep the channels.
template <typename T>
__global__ __launch_bounds__(256) void k_causal_conv(const T* __restrict__ mixed, const T* __restrict__ norm_w,
                                                     const T* __restrict__ conv_w, ConvWin W, int32_t d, int32_t K,
                                                     int32_t dil, float eps, int residual, T* __restrict__ out) {
  extern __shared__ float scale[];  // [CONV_TT + (K-1)*dil]
  const int64_t b = blockIdx.y;
  const int64_t p0 = conv_p0(W);
  const int64_t t0 = p0 + static_cast<int64_t>(blockIdx.x) * CONV_TT;
  const int64_t T_len = min(W.len, p0 + W.n);  // rows read and outputs end here
  const int halo = (K - 1) * dil;
  const int nrow = CONV_TT + halo;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const T* base = mixed + b * W.stride * d;
  if (p0 < 0) return;
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
        const float xn = norm_elem<T, true>(to_f32(base[ts * d + c]), scale[tt + halo - lag], nw);
        acc = fmaf(to_f32(conv_w[c * K + j]), xn, acc);
      }
      const float y = round_to<T>(acc);
      const float act = round_to<T>(y / (1.0f + expf(-y)));
      out[(b * W.n + t - p0) * d + c] = residual ? from_f32<T>(to_f32(base[t * d + c]) + act) : from_f32<T>(act);
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
                                                          const T* __restrict__ conv_w, ConvWin W, int32_t d,
                                                          float eps, int residual, T* __restrict__ out) {
  __shared__ float scale[C43_TT + C43_HALO];
  const int64_t b = blockIdx.y;
  const int64_t p0 = conv_p0(W);
  const int64_t t0 = p0 + static_cast<int64_t>(blockIdx.x) * C43_TT;
  const int64_t T_len = min(W.len, p0 + W.n);  // rows read and outputs end here
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const T* base = mixed + b * W.stride * d;
  if (p0 < 0) return;
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
        for (int j = 0; j < 8; ++j) hist[0][j] = norm_elem<T, true>(x[j], s, nw[j]);
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
        store8(out + (b * W.n + t - p0) * d + c, o);
      }
    }
  }
}

// rowsq[m] = sum_c x[m, c]^2 of bf16 rows (the RMSNorm statistic of the short conv, in the one-
// partial layout k_causal_conv_k4d3_stream reads).  One wave per row, 16-byte loads.
__global__ __launch_bounds__(256) void k_row_sumsq_bf16(const bf16* __restrict__ x, int64_t rows, int32_t d,
                                                        float* __restrict__ rowsq) {
  const int lane = threadIdx.x & 63;
  const int64_t m = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (m >= rows) return;
  const bf16* xr = x + m * d;
  float ss = 0.f;
  for (int c = 8 * lane; c < d; c += 512) {
    const bf16x8 v = *reinterpret_cast<const bf16x8*>(xr + c);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float f = static_cast<float>(v[j]);
      ss = fmaf(f, f, ss);
    }
  }
  ss = wave_sum(ss);
  if (lane == 0) rowsq[m] = ss;
}

// bf16, kernel 4, dilation 3, single pass: block = (b, CF_TT positions) x all channels, d/4
// threads of 4 channels.  Each thread loads its 4 channels of the CF_TT + 9 rows (the causal
// halo included) once; a row's sum of squares is a bf16 dot product per lane, summed over 16
// lanes with DPP and over the block's 16-lane groups in LDS in a fixed order.  Then the rows are
// normalised in order and the outputs formed as soon as their last tap is ready.  The rounding
// sequence is F.rms_norm's then the reference conv's: normalise and scale by the weight in fp32,
// round once, taps in order with fp32 accumulation (v_dot2_f32_bf16 adds a tap pair's exact
// bf16 products with one rounding), round, SiLU (hardware exp2 and reciprocal), round, add the
// residual.  A normalised row r is rounded straight into the pairs (r - 3, r) and (r, r + 3),
// the operands of the dot products of the outputs that read it.
constexpr int CF_HALO = 9;
constexpr int CF_MAXG = 32;  // 16-lane groups per block: d <= 2048

typedef float f32x2 __attribute__((ext_vector_type(2)));

// v[k] summed over each 16-lane row of the wave, returned in every lane of the row (fixed
// order); the N sums advance step by step together, so no DPP read waits on the add before it
template <int CTRL, int N>
__device__ __forceinline__ void dpp_add_step(float (&v)[N]) {
#pragma unroll
  for (int k = 0; k < N; ++k)
    v[k] += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v[k]), CTRL, 0xF, 0xF, true));
}
template <int N>
__device__ __forceinline__ void row16_sums(float (&v)[N]) {
  dpp_add_step<0xB1>(v);   // xor 1
  dpp_add_step<0x4E>(v);   // xor 2
  dpp_add_step<0x141>(v);  // half-row mirror
  dpp_add_step<0x140>(v);  // row mirror
}

__device__ __forceinline__ bf16x2 pk2(float a, float b) { return __builtin_convertvector(f32x2{a, b}, bf16x2); }
__device__ __forceinline__ float lo_f(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float hi_f(uint32_t u) { return __uint_as_float(u & 0xFFFF0000u); }

template <int TT>
__global__ __launch_bounds__(512) void k_causal_conv_k4d3_fused(const bf16* __restrict__ mixed,
                                                                const bf16* __restrict__ norm_w,
                                                                const bf16* __restrict__ conv_w, ConvWin W,
                                                                uint32_t d4, float eps, int residual,
                                                                bf16* __restrict__ out) {
  constexpr int ROWS = TT + CF_HALO;
  __shared__ float part[CF_MAXG][ROWS];
  __shared__ float srow[ROWS];
  const int tid = threadIdx.x, lane = tid & 63;
  const int ngrp = static_cast<int>(blockDim.x >> 4);
  // XCD-aware order: blocks go to the 8 XCDs round-robin (block b to XCD b % 8); when the grid
  // divides evenly, XCD x takes the x-th eighth of the (sequence, tile) order, so the 9-row causal
  // halo of a tile was fetched into the same L2 by the tile before it (21.9 -> 20.7 us at
  // B8 x T2048 x d1024)
  int tile_t = static_cast<int>(blockIdx.x), tile_b = static_cast<int>(blockIdx.y);
  const int64_t nb = static_cast<int64_t>(gridDim.x) * gridDim.y;
  if ((nb & 7) == 0) {
    const int64_t bid = tile_t + static_cast<int64_t>(gridDim.x) * tile_b;
    const int64_t tile = (bid & 7) * (nb >> 3) + (bid >> 3);
    tile_t = static_cast<int>(tile % gridDim.x);
    tile_b = static_cast<int>(tile / gridDim.x);
  }
  const int64_t p0 = conv_p0(W);
  if (p0 < 0) return;
  const int t0 = static_cast<int>(p0) + tile_t * TT;
  const int T = static_cast<int>(min(W.len, p0 + W.n));  // rows read and outputs end here
  const size_t row0 = static_cast<size_t>(tile_b) * W.stride;
  const size_t orow0 = static_cast<size_t>(tile_b) * W.n - p0;  // output row of position t: orow0 + t
  const uint32_t d = d4 * 4u;
  const bool active = static_cast<uint32_t>(tid) < d4;
  const uint32_t c = (active ? static_cast<uint32_t>(tid) : 0u) * 4u;
  auto clamp_t = [&](int tp) { return tp < 0 ? 0 : (tp >= T ? T - 1 : tp); };
  uint2 x[ROWS];  // channels c .. c+3 of row t0 - 9 + r
#pragma unroll
  for (int r = 0; r < ROWS; ++r)
    x[r] = *reinterpret_cast<const uint2*>(mixed + (row0 + clamp_t(t0 - CF_HALO + r)) * d + c);
  const uint2 nwv = *reinterpret_cast<const uint2*>(norm_w + c);
  const uint4 cw01 = *reinterpret_cast<const uint4*>(conv_w + static_cast<size_t>(c) * 4);      // channels c, c+1
  const uint4 cw23 = *reinterpret_cast<const uint4*>(conv_w + static_cast<size_t>(c) * 4 + 8);  // channels c+2, c+3
  const float live = active ? 1.f : 0.f;
#pragma unroll
  for (int r0 = 0; r0 < ROWS; r0 += 3) {
    float ss[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      const int r = r0 + k < ROWS ? r0 + k : ROWS - 1;
      const float a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x[r].x),
                                                      __builtin_bit_cast(bf16x2, x[r].x), 0.f, false);
      ss[k] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x[r].y), __builtin_bit_cast(bf16x2, x[r].y), a,
                                              false) * live;
    }
    row16_sums(ss);
#pragma unroll
    for (int k = 0; k < 3; ++k)
      if (r0 + k < ROWS && (lane & 15) == 0) part[tid >> 4][r0 + k] = ss[k];
  }
  __syncthreads();
  if (tid < ROWS) {
    float ss = 0.f;
    for (int g = 0; g < ngrp; ++g) ss += part[g][tid];
    // rows before the sequence start are the zero left padding
    srow[tid] = t0 - CF_HALO + tid < 0 ? 0.f : 1.0f / sqrtf(ss / static_cast<float>(d) + eps);
  }
  __syncthreads();
  if (!active) return;
  const float nw[4] = {lo_f(nwv.x), hi_f(nwv.x), lo_f(nwv.y), hi_f(nwv.y)};
  // tap pairs of channel c + j: (w0, w1) and (w2, w3)
  const uint32_t wa[4] = {cw01.x, cw01.z, cw23.x, cw23.z};
  const uint32_t wb[4] = {cw01.y, cw01.w, cw23.y, cw23.w};
  float yn[ROWS][4];   // normalised rows times the weight, fp32 (rounded once, into q)
  bf16x2 q[ROWS][4];   // q[r][j] = (yn[r][j], yn[r + 3][j]) rounded to bf16
#pragma unroll
  for (int r = 0; r < ROWS; ++r) {
    const float s = srow[r];
    const float xf[4] = {lo_f(x[r].x), hi_f(x[r].x), lo_f(x[r].y), hi_f(x[r].y)};
#pragma unroll
    for (int j = 0; j < 4; ++j) yn[r][j] = xf[j] * s * nw[j];
    if (r >= 3) {
#pragma unroll
      for (int j = 0; j < 4; ++j) q[r - 3][j] = pk2(yn[r - 3][j], yn[r][j]);
    }
    if (r >= CF_HALO) {
      // output t = t0 + i reads rows i, i+3 (taps 0, 1) and i+6, i+9 (taps 2, 3); row i + 9 = r
      const int i = r - CF_HALO;
      const int t = t0 + i;
      if (t < T) {
        float y[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float a = __builtin_amdgcn_fdot2_f32_bf16(q[i][j], __builtin_bit_cast(bf16x2, wa[j]), 0.f, false);
          y[j] = __builtin_amdgcn_fdot2_f32_bf16(q[i + 6][j], __builtin_bit_cast(bf16x2, wb[j]), a, false);
        }
        const uint32_t yp0 = __builtin_bit_cast(uint32_t, pk2(y[0], y[1]));
        const uint32_t yp1 = __builtin_bit_cast(uint32_t, pk2(y[2], y[3]));
        const float yr[4] = {lo_f(yp0), hi_f(yp0), lo_f(yp1), hi_f(yp1)};
        float act[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float e = __builtin_amdgcn_exp2f(-yr[j] * 1.4426950408889634f);
          act[j] = yr[j] * __builtin_amdgcn_rcpf(1.0f + e);
        }
        uint2 o;
        if (residual) {
          const uint32_t ap0 = __builtin_bit_cast(uint32_t, pk2(act[0], act[1]));
          const uint32_t ap1 = __builtin_bit_cast(uint32_t, pk2(act[2], act[3]));
          o.x = __builtin_bit_cast(uint32_t, pk2(xf[0] + lo_f(ap0), xf[1] + hi_f(ap0)));
          o.y = __builtin_bit_cast(uint32_t, pk2(xf[2] + lo_f(ap1), xf[3] + hi_f(ap1)));
        } else {
          o.x = __builtin_bit_cast(uint32_t, pk2(act[0], act[1]));
          o.y = __builtin_bit_cast(uint32_t, pk2(act[2], act[3]));
        }
        *reinterpret_cast<uint2*>(out + (orow0 + t) * d + c) = o;
      }
    }
  }
}

// bf16, kernel 4, dilation 3, with the row sums of squares formed by the producing GEMM
// (rowsq[p][m], P <= MAXP partials per row m = b*T + t, summed in the fixed order p = 0, 1, ...).
// One wave streams one (sequence, 256-channel group, SL-position range): lane l owns channels
// 4l .. 4l+3 of the group; a block holds WPB consecutive such tiles.  All SL + 9 rows (the range and its causal halo) are requested at
// kernel entry; each output is formed as soon as its four rows have arrived, so the arithmetic of
// the early rows overlaps the loads of the later ones, with no block barrier and no reduction in
// the kernel.  Lane r (< SL + 9) turns the partials of row t0 - 9 + r into that row's scale,
// which the wave reads back as a scalar.  The rounding sequence is k_causal_conv_k4d3_fused's.
// Ranges are numbered so that consecutive ranges of a sequence land on one XCD (blocks go to the
// 8 XCDs round-robin), where a range's halo rows were fetched by the range before it.
constexpr int CS_SL = 16;   // 16 positions + 9 halo rows, 4 waves a block: 18.7 us at B8 x T2048 x d1024
constexpr int CS_WPB = 4;  // (32 positions: 20.6 us; one-wave blocks: 21.2 us; 64 positions: 24.3 us)
constexpr int CS_MAXP = 16;

template <int SL, int MAXP, bool RESIDUAL>
__global__ __launch_bounds__(64 * CS_WPB) void k_causal_conv_k4d3_stream(const bf16* __restrict__ mixed,
                                                                const float* __restrict__ rowsq, int32_t P,
                                                                const bf16* __restrict__ norm_w,
                                                                const bf16* __restrict__ conv_w, int32_t T,
                                                                int32_t d, int32_t G, int32_t R, int64_t B_tiles,
                                                                int64_t M, float eps, bf16* __restrict__ out) {
  constexpr int ROWS = SL + CF_HALO;
  const int lane = threadIdx.x & 63;
  // the host keeps the tile count below 2^31 (and pads it to whole blocks: tiles past the end exit)
  const uint32_t ntiles = static_cast<uint32_t>(B_tiles);
  uint32_t tile = blockIdx.x * CS_WPB + (threadIdx.x >> 6);
  const uint32_t nb = gridDim.x * CS_WPB;
  if ((nb & 7) == 0) tile = (tile & 7) * (nb >> 3) + (tile >> 3);
  tile = __builtin_amdgcn_readfirstlane(tile);
  if (tile >= ntiles) return;  // no barrier follows
  const uint32_t gr = tile / static_cast<uint32_t>(G);
  const int cg = static_cast<int>(tile - gr * static_cast<uint32_t>(G));
  const uint32_t bb = gr / static_cast<uint32_t>(R);
  const int rg = static_cast<int>(gr - bb * static_cast<uint32_t>(R));
  const int t0 = rg * SL;
  const int c = cg * 256 + 4 * lane;
  const bool active = c < d;
  const int cc = active ? c : 0;
  // Rows are addressed through one buffer resource per sequence (T * d * 2 < 2^31 bytes, checked
  // by the host) and 32-bit byte offsets: a row before the sequence start (negative offset) or at
  // or past its end lies outside the resource, so its loads read zero and its stores are dropped
  // by the hardware -- no clamping, 64-bit address arithmetic or store branches per row.  Rows past
  // the end feed only outputs past the end; rows before the start are the zero left padding.
  const uint32_t seq_bytes = static_cast<uint32_t>(T) * static_cast<uint32_t>(d) * 2u;
  const size_t seq0 = static_cast<size_t>(bb) * static_cast<size_t>(T) * static_cast<size_t>(d);
  const __amdgpu_buffer_rsrc_t xr =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16*>(mixed + seq0), 0, static_cast<int>(seq_bytes), BUF_DW3);
  const __amdgpu_buffer_rsrc_t yr_out =
      __builtin_amdgcn_make_buffer_rsrc(out + seq0, 0, static_cast<int>(seq_bytes), BUF_DW3);
  const uint32_t rstride = static_cast<uint32_t>(d) * 2u;
  // unsigned offsets: a row before the start wraps above 2^31; lanes past d start at 2^31, which no
  // row step (ROWS * d * 2 < 2^30, checked by the host) brings back below T * d * 2
  const uint32_t voff = active ? static_cast<uint32_t>(t0 - CF_HALO) * rstride + 2u * static_cast<uint32_t>(c)
                               : 0x80000000u;
  // the partials first (every lane loads, unconditionally, so the row loads are not held back
  // behind them), then the rows; lane r's partials are row t0 - 9 + r's (clamped into the sequence)
  const int tl = t0 - CF_HALO + (lane < ROWS ? lane : 0);
  const int tlc = tl < 0 ? 0 : (tl >= T ? T - 1 : tl);
  const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(rowsq), 0, static_cast<int>(static_cast<uint32_t>(P) * static_cast<uint32_t>(M) * 4u), BUF_DW3);
  const int32_t poff = (static_cast<int32_t>(bb) * T + tlc) * 4;
  const int32_t pstep = static_cast<int32_t>(M) * 4;
  float pv[MAXP];
#pragma unroll
  for (int q = 0; q < MAXP; ++q)
    pv[q] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(pr, poff + (q < P ? q : 0) * pstep, 0, 0));
  uint2 x[ROWS];  // channels cc .. cc+3 of row t0 - 9 + r (zero outside the sequence)
#pragma unroll
  for (int r = 0; r < ROWS; ++r) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(xr, static_cast<int>(voff + r * rstride), 0, 0);
    x[r] = uint2{static_cast<uint32_t>(v[0]), static_cast<uint32_t>(v[1])};
  }
  const uint2 nwv = *reinterpret_cast<const uint2*>(norm_w + cc);
  const uint4 cw01 = *reinterpret_cast<const uint4*>(conv_w + static_cast<size_t>(cc) * 4);      // channels c, c+1
  const uint4 cw23 = *reinterpret_cast<const uint4*>(conv_w + static_cast<size_t>(cc) * 4 + 8);  // channels c+2, c+3
  const float nw[4] = {lo_f(nwv.x), hi_f(nwv.x), lo_f(nwv.y), hi_f(nwv.y)};
  const uint32_t wa[4] = {cw01.x, cw01.z, cw23.x, cw23.z};
  const uint32_t wb[4] = {cw01.y, cw01.w, cw23.y, cw23.w};
  // lane r's scale is row t0 - 9 + r's; rows before the sequence start are the zero left padding
  float ss = 0.f;
#pragma unroll
  for (int q = 0; q < MAXP; ++q) ss += q < P ? pv[q] : 0.f;
  const float s = tl < 0 ? 0.f : 1.0f / sqrtf(ss / static_cast<float>(d) + eps);
  float yn[ROWS][4];
  bf16x2 q[ROWS][4];  // q[r][j] = (yn[r][j], yn[r + 3][j]) rounded to bf16
#pragma unroll
  for (int r = 0; r < ROWS; ++r) {
    const float sr = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, s), r));
    const float xf[4] = {lo_f(x[r].x), hi_f(x[r].x), lo_f(x[r].y), hi_f(x[r].y)};
#pragma unroll
    for (int j = 0; j < 4; ++j) yn[r][j] = xf[j] * sr * nw[j];
    if (r >= 3) {
#pragma unroll
      for (int j = 0; j < 4; ++j) q[r - 3][j] = pk2(yn[r - 3][j], yn[r][j]);
    }
    if (r >= CF_HALO) {
      // output t0 + i reads rows i, i+3 (taps 0, 1) and i+6, i+9 (taps 2, 3); every lane forms it
      // and the resource drops the stores past the sequence end and past d
      const int i = r - CF_HALO;
      float y[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float a = __builtin_amdgcn_fdot2_f32_bf16(q[i][j], __builtin_bit_cast(bf16x2, wa[j]), 0.f, false);
        y[j] = __builtin_amdgcn_fdot2_f32_bf16(q[i + 6][j], __builtin_bit_cast(bf16x2, wb[j]), a, false);
      }
      const uint32_t yp0 = __builtin_bit_cast(uint32_t, pk2(y[0], y[1]));
      const uint32_t yp1 = __builtin_bit_cast(uint32_t, pk2(y[2], y[3]));
      const float yr[4] = {lo_f(yp0), hi_f(yp0), lo_f(yp1), hi_f(yp1)};
      float act[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float e = __builtin_amdgcn_exp2f(-yr[j] * 1.4426950408889634f);
        act[j] = yr[j] * __builtin_amdgcn_rcpf(1.0f + e);
      }
      uint32_t o0, o1;
      if (RESIDUAL) {
        const uint32_t ap0 = __builtin_bit_cast(uint32_t, pk2(act[0], act[1]));
        const uint32_t ap1 = __builtin_bit_cast(uint32_t, pk2(act[2], act[3]));
        o0 = __builtin_bit_cast(uint32_t, pk2(xf[0] + lo_f(ap0), xf[1] + hi_f(ap0)));
        o1 = __builtin_bit_cast(uint32_t, pk2(xf[2] + lo_f(ap1), xf[3] + hi_f(ap1)));
      } else {
        o0 = __builtin_bit_cast(uint32_t, pk2(act[0], act[1]));
        o1 = __builtin_bit_cast(uint32_t, pk2(act[2], act[3]));
      }
      typedef int i32x2 __attribute__((ext_vector_type(2)));
      __builtin_amdgcn_raw_buffer_store_b64(i32x2{static_cast<int>(o0), static_cast<int>(o1)}, yr_out,
                                            static_cast<int>(voff + r * rstride), 0, 0);
    }
  }
}

template <int SL, int MAXP>
static void conv_stream_kernel(dim3 grid, dim3 block, hipStream_t s, bool residual, const bf16* mx, const float* rowsq,
                               int32_t P, const bf16* nw, const bf16* cw, int32_t T, int32_t d, int32_t G, int32_t R,
                               int64_t nb, int64_t M, float eps, bf16* o) {
  if (residual)
    hipLaunchKernelGGL((k_causal_conv_k4d3_stream<SL, MAXP, true>), grid, block, 0, s, mx, rowsq, P, nw, cw, T, d, G, R,
                       nb, M, eps, o);
  else
    hipLaunchKernelGGL((k_causal_conv_k4d3_stream<SL, MAXP, false>), grid, block, 0, s, mx, rowsq, P, nw, cw, T, d, G,
                       R, nb, M, eps, o);
}

// the short conv over whole sequences with the row statistics of the producing GEMM
template <int SL>
static int launch_conv_stream(const bf16* mx, const float* rowsq, int32_t n_partials, const bf16* nw, const bf16* cw,
                              int64_t B, int64_t T, int32_t d, float eps, bool residual, bf16* o, hipStream_t s) {
  const int32_t G = static_cast<int32_t>(cdiv(d, 256)), R = static_cast<int32_t>(cdiv(T, SL));
  const int64_t nb = B * G * R;
  if (nb >= (int64_t{1} << 31)) return fail(LNG_E_ARG, "causal_conv_rowsq: too many tiles");
  const int64_t M = B * T;
  const int32_t Ti = static_cast<int32_t>(T);
  const dim3 grid(static_cast<unsigned>(cdiv(nb, CS_WPB))), block(64 * CS_WPB);
  if (n_partials <= 2)
    conv_stream_kernel<SL, 2>(grid, block, s, residual, mx, rowsq, n_partials, nw, cw, Ti, d, G, R, nb, M, eps, o);
  else if (n_partials <= 8)
    conv_stream_kernel<SL, 8>(grid, block, s, residual, mx, rowsq, n_partials, nw, cw, Ti, d, G, R, nb, M, eps, o);
  else
    conv_stream_kernel<SL, CS_MAXP>(grid, block, s, residual, mx, rowsq, n_partials, nw, cw, Ti, d, G, R, nb, M, eps,
                                    o);
  return LNG_OK;
}

template <bool FUSED>
int rmsnorm_launch(const void* x, const void* w, int dtype, int64_t rows, int32_t dim, float eps, void* out,
                          hipStream_t s) {
  dim3 grid(static_cast<unsigned>(cdiv(rows, 4)));
  if (dtype == LNG_BF16 && dim % 512 == 0 && dim <= 2048) {
    const bf16* xp = static_cast<const bf16*>(x);
    const bf16* wp = static_cast<const bf16*>(w);
    bf16* op = static_cast<bf16*>(out);
    if (dim == 512)
      hipLaunchKernelGGL((k_rmsnorm_bf16_vec<1, FUSED>), grid, dim3(256), 0, s, xp, wp, rows, eps, op);
    else if (dim == 1024)
      hipLaunchKernelGGL((k_rmsnorm_bf16_vec<2, FUSED>), grid, dim3(256), 0, s, xp, wp, rows, eps, op);
    else if (dim == 1536)
      hipLaunchKernelGGL((k_rmsnorm_bf16_vec<3, FUSED>), grid, dim3(256), 0, s, xp, wp, rows, eps, op);
    else
      hipLaunchKernelGGL((k_rmsnorm_bf16_vec<4, FUSED>), grid, dim3(256), 0, s, xp, wp, rows, eps, op);
    return check_launch("rmsnorm_bf16_vec");
  }
  if (dtype == LNG_F32)
    hipLaunchKernelGGL((k_rmsnorm<float, FUSED>), grid, dim3(256), 0, s, static_cast<const float*>(x),
                       static_cast<const float*>(w), rows, dim, eps, static_cast<float*>(out));
  else if (dtype == LNG_BF16)
    hipLaunchKernelGGL((k_rmsnorm<bf16, FUSED>), grid, dim3(256), 0, s, static_cast<const bf16*>(x),
                       static_cast<const bf16*>(w), rows, dim, eps, static_cast<bf16*>(out));
  else
    return fail(LNG_E_DTYPE, "rmsnorm: dtype must be f32 or bf16");
  return check_launch("rmsnorm");
}

}  // namespace lng

using namespace lng;

extern "C" {

int lng_rmsnorm(const void* x, const void* w, int dtype, int64_t rows, int32_t dim, float eps, int32_t mode,
                void* out, void* stream) {
  if (rows < 0 || dim <= 0) return fail(LNG_E_ARG, "rmsnorm: bad shape");
  if (mode != LNG_NORM_MODEL && mode != LNG_NORM_FUSED) return fail(LNG_E_ARG, "rmsnorm: unknown rounding mode");
  if (rows == 0) return LNG_OK;
  return mode == LNG_NORM_FUSED ? rmsnorm_launch<true>(x, w, dtype, rows, dim, eps, out, as_stream(stream))
                                : rmsnorm_launch<false>(x, w, dtype, rows, dim, eps, out, as_stream(stream));
}

int lng_causal_conv_rowsq(const void* mixed, const float* rowsq, int32_t n_partials, const void* norm_w,
                          const void* conv_w, int64_t B, int64_t T, int32_t d, int32_t K, int32_t dilation, float eps,
                          int residual, void* out, void* stream) {
  if (B < 0 || T < 0 || d <= 0 || d % 4 || n_partials <= 0) return fail(LNG_E_ARG, "causal_conv_rowsq: bad shape");
  if (K != 4 || dilation != 3) return fail(LNG_E_ARG, "causal_conv_rowsq: kernel 4 / dilation 3 only");
  if (mixed == out) return fail(LNG_E_ARG, "causal_conv_rowsq: out must not alias mixed");
  if (n_partials > CS_MAXP) return fail(LNG_E_ARG, "causal_conv_rowsq: at most 16 partials");
  if (B * T == 0) return LNG_OK;
  // one sequence and the partials fit one buffer resource each (byte offsets below 2^31), and a
  // wave's row steps stay below 2^30 bytes
  if (T * d >= (int64_t{1} << 30) || d > 65536 || static_cast<int64_t>(n_partials) * B * T >= (int64_t{1} << 29))
    return fail(LNG_E_ARG, "causal_conv_rowsq: tensor too large");
  const bf16* mx = static_cast<const bf16*>(mixed);
  const bf16* nw = static_cast<const bf16*>(norm_w);
  const bf16* cw = static_cast<const bf16*>(conv_w);
  bf16* o = static_cast<bf16*>(out);
  const int rc =
      launch_conv_stream<CS_SL>(mx, rowsq, n_partials, nw, cw, B, T, d, eps, residual != 0, o, as_stream(stream));
  if (rc) return rc;
  return check_launch("causal_conv_rowsq");
}

}  // extern "C"

namespace lng {

// Launch of the causal conv over window W (see ConvWin) of B sequences.
static int conv_launch(const void* mixed, const void* norm_w, const void* conv_w, int dtype, int64_t B, const ConvWin& W,
                       int32_t d, int32_t K, int32_t dilation, float eps, int residual, void* out, hipStream_t s) {
  const int64_t n = W.n;
  const int halo = (K - 1) * dilation;
  if (halo > 4096) return fail(LNG_E_ARG, "causal_conv: receptive field too large");
  if (K == 4 && dilation == 3 && d % 4 == 0 && d <= 2048 && dtype == LNG_BF16 && B <= 65535 && W.len < INT32_MAX) {
    // 16 positions (25 rows with the halo, 103 VGPRs): 4 waves per SIMD hide the load phase
    // better than 32-position blocks, whose halo share is smaller (21.5 against 22.8 us at
    // B8 x T2048 x d1024)
    constexpr int TT = 16;
    dim3 g43(static_cast<unsigned>(cdiv(n, TT)), static_cast<unsigned>(B));
    const int threads = static_cast<int>(cdiv(d / 4, 64) * 64);
    hipLaunchKernelGGL(k_causal_conv_k4d3_fused<TT>, g43, dim3(threads), 0, s, static_cast<const bf16*>(mixed),
                       static_cast<const bf16*>(norm_w), static_cast<const bf16*>(conv_w), W,
                       static_cast<uint32_t>(d / 4), eps, residual, static_cast<bf16*>(out));
    return check_launch("causal_conv_k4d3_bf16");
  }
  if (K == 4 && dilation == 3 && d % 8 == 0 && (dtype == LNG_F32 || dtype == LNG_BF16)) {
    dim3 g43(static_cast<unsigned>(cdiv(n, C43_TT)), static_cast<unsigned>(B));
    if (dtype == LNG_F32)
      hipLaunchKernelGGL(k_causal_conv_k4d3<float>, g43, dim3(128), 0, s, static_cast<const float*>(mixed),
                         static_cast<const float*>(norm_w), static_cast<const float*>(conv_w), W, d, eps, residual,
                         static_cast<float*>(out));
    else
      hipLaunchKernelGGL(k_causal_conv_k4d3<bf16>, g43, dim3(128), 0, s, static_cast<const bf16*>(mixed),
                         static_cast<const bf16*>(norm_w), static_cast<const bf16*>(conv_w), W, d, eps, residual,
                         static_cast<bf16*>(out));
    return check_launch("causal_conv_k4d3");
  }
  dim3 grid(static_cast<unsigned>(cdiv(n, CONV_TT)), static_cast<unsigned>(B));
  const size_t lds = sizeof(float) * (CONV_TT + halo);
  if (dtype == LNG_F32)
    hipLaunchKernelGGL(k_causal_conv<float>, grid, dim3(256), lds, s, static_cast<const float*>(mixed),
                       static_cast<const float*>(norm_w), static_cast<const float*>(conv_w), W, d, K, dilation, eps,
                       residual, static_cast<float*>(out));
  else if (dtype == LNG_BF16)
    hipLaunchKernelGGL(k_causal_conv<bf16>, grid, dim3(256), lds, s, static_cast<const bf16*>(mixed),
                       static_cast<const bf16*>(norm_w), static_cast<const bf16*>(conv_w), W, d, K, dilation, eps,
                       residual, static_cast<bf16*>(out));
  else
    return fail(LNG_E_DTYPE, "causal_conv: dtype must be f32 or bf16");
  return check_launch("causal_conv");
}

// ---------------------------------------------------------------- the conv over listed rows
// The short conv with each output's window given as row indices instead of a position range:
// output (b, i) reads tap j from row slots[i * (back + 1) + j * dil] of sequence b and its
// residual from row slots[i * (back + 1) + back], back = (K - 1) * dil, oldest first (a draft
// tree's ancestor windows, drafting/tree.py:186-194).  A slot outside [0, len) is a zero row (the
// left padding).  Each shape runs the arithmetic of the sequence kernel that conv_launch picks for
// it, so an output equals the sequence conv's at a position whose window holds the same rows.

__device__ __forceinline__ int64_t slot_row(const int32_t* slots, int64_t i, int back, int k, int64_t len) {
  const int32_t s = slots[i * (back + 1) + k];
  return (s >= 0 && s < len) ? s : -1;
}

// bf16, kernel 4, dilation 3: k_causal_conv_k4d3_fused's thread layout, row sums (dot products per
// lane, 16-lane DPP sums, 16-lane groups in LDS in order) and tap pairs.  Block (i, b), d/4
// threads of 4 channels (rounded up to whole waves).
__global__ __launch_bounds__(512) void k_conv_k4d3_slots_bf16(const bf16* __restrict__ rows,
                                                              const bf16* __restrict__ norm_w,
                                                              const bf16* __restrict__ conv_w,
                                                              const int32_t* __restrict__ slots, int64_t stride,
                                                              int64_t len, int64_t n, uint32_t d4, float eps,
                                                              int residual, bf16* __restrict__ out) {
  __shared__ float part[CF_MAXG][4];
  __shared__ float srow[4];
  const int tid = threadIdx.x, lane = tid & 63;
  const int ngrp = static_cast<int>(blockDim.x >> 4);
  const int64_t i = blockIdx.x, b = blockIdx.y;
  const uint32_t d = d4 * 4u;
  const bool active = static_cast<uint32_t>(tid) < d4;
  const uint32_t c = (active ? static_cast<uint32_t>(tid) : 0u) * 4u;
  int64_t rw[4];
  uint2 x[4];  // channels c .. c+3 of the rows of taps 0..3 (zero for a padding slot)
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    rw[k] = slot_row(slots, i, CF_HALO, 3 * k, len);
    x[k] = rw[k] >= 0 ? *reinterpret_cast<const uint2*>(rows + (b * stride + rw[k]) * d + c) : uint2{0u, 0u};
  }
  const uint2 nwv = *reinterpret_cast<const uint2*>(norm_w + c);
  const uint4 cw01 = *reinterpret_cast<const uint4*>(conv_w + static_cast<size_t>(c) * 4);
  const uint4 cw23 = *reinterpret_cast<const uint4*>(conv_w + static_cast<size_t>(c) * 4 + 8);
  const float live = active ? 1.f : 0.f;
  float ss[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x[k].x),
                                                    __builtin_bit_cast(bf16x2, x[k].x), 0.f, false);
    ss[k] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x[k].y), __builtin_bit_cast(bf16x2, x[k].y), a,
                                            false) * live;
  }
  row16_sums(ss);
  if ((lane & 15) == 0) {
#pragma unroll
    for (int k = 0; k < 4; ++k) part[tid >> 4][k] = ss[k];
  }
  __syncthreads();
  if (tid < 4) {
    float s = 0.f;
    for (int g = 0; g < ngrp; ++g) s += part[g][tid];
    srow[tid] = rw[tid] < 0 ? 0.f : 1.0f / sqrtf(s / static_cast<float>(d) + eps);
  }
  __syncthreads();
  if (!active) return;
  const float nw[4] = {lo_f(nwv.x), hi_f(nwv.x), lo_f(nwv.y), hi_f(nwv.y)};
  const uint32_t wa[4] = {cw01.x, cw01.z, cw23.x, cw23.z};
  const uint32_t wb[4] = {cw01.y, cw01.w, cw23.y, cw23.w};
  float yn[4][4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float s = srow[k];
    const float xf[4] = {lo_f(x[k].x), hi_f(x[k].x), lo_f(x[k].y), hi_f(x[k].y)};
#pragma unroll
    for (int j = 0; j < 4; ++j) yn[k][j] = xf[j] * s * nw[j];
  }
  float y[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float a = __builtin_amdgcn_fdot2_f32_bf16(pk2(yn[0][j], yn[1][j]), __builtin_bit_cast(bf16x2, wa[j]), 0.f,
                                                    false);
    y[j] = __builtin_amdgcn_fdot2_f32_bf16(pk2(yn[2][j], yn[3][j]), __builtin_bit_cast(bf16x2, wb[j]), a, false);
  }
  const uint32_t yp0 = __builtin_bit_cast(uint32_t, pk2(y[0], y[1]));
  const uint32_t yp1 = __builtin_bit_cast(uint32_t, pk2(y[2], y[3]));
  const float yr[4] = {lo_f(yp0), hi_f(yp0), lo_f(yp1), hi_f(yp1)};
  float act[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float e = __builtin_amdgcn_exp2f(-yr[j] * 1.4426950408889634f);
    act[j] = yr[j] * __builtin_amdgcn_rcpf(1.0f + e);
  }
  uint2 o;
  if (residual) {
    const float xs[4] = {lo_f(x[3].x), hi_f(x[3].x), lo_f(x[3].y), hi_f(x[3].y)};
    const uint32_t ap0 = __builtin_bit_cast(uint32_t, pk2(act[0], act[1]));
    const uint32_t ap1 = __builtin_bit_cast(uint32_t, pk2(act[2], act[3]));
    o.x = __builtin_bit_cast(uint32_t, pk2(xs[0] + lo_f(ap0), xs[1] + hi_f(ap0)));
    o.y = __builtin_bit_cast(uint32_t, pk2(xs[2] + lo_f(ap1), xs[3] + hi_f(ap1)));
  } else {
    o.x = __builtin_bit_cast(uint32_t, pk2(act[0], act[1]));
    o.y = __builtin_bit_cast(uint32_t, pk2(act[2], act[3]));
  }
  *reinterpret_cast<uint2*>(out + (b * n + i) * d + c) = o;
}

// Other shapes: K4D3 = k_causal_conv_k4d3<T>'s row sums (8 consecutive elements a lane, 512 apart)
// and tap order; otherwise k_causal_conv<T>'s (one element a lane, 64 apart).  Block (i, b) of 256
// threads; a wave per tap row for the row scales, then the threads sweep the channels.
template <typename T, bool K4D3>
__global__ __launch_bounds__(256) void k_conv_slots(const T* __restrict__ rows, const T* __restrict__ norm_w,
                                                    const T* __restrict__ conv_w, const int32_t* __restrict__ slots,
                                                    int64_t stride, int64_t len, int64_t n, int32_t d, int32_t K,
                                                    int32_t dil, float eps, int residual, T* __restrict__ out) {
  extern __shared__ float tap_scale[];  // [K]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t i = blockIdx.x, b = blockIdx.y;
  const int back = (K - 1) * dil;
  const T* base = rows + b * stride * d;
  for (int k = wave; k < K; k += 4) {
    const int64_t r = slot_row(slots, i, back, k * dil, len);
    float sc = 0.f;
    if (r >= 0) {
      float ss = 0.f;
      if (K4D3) {
        for (int c = lane * 8; c < d; c += 64 * 8) {
          float v[8];
          load8(base + r * d + c, v);
#pragma unroll
          for (int j = 0; j < 8; ++j) ss = fmaf(v[j], v[j], ss);
        }
      } else {
        for (int c = lane; c < d; c += 64) {
          const float v = to_f32(base[r * d + c]);
          ss = fmaf(v, v, ss);
        }
      }
      ss = wave_sum(ss);
      sc = 1.0f / sqrtf(ss / static_cast<float>(d) + eps);
    }
    if (lane == 0) tap_scale[k] = sc;
  }
  __syncthreads();
  const int64_t self = slot_row(slots, i, back, back, len);
  for (int c = threadIdx.x; c < d; c += blockDim.x) {
    const float nw = to_f32(norm_w[c]);
    float acc = 0.f;
    for (int k = 0; k < K; ++k) {
      const int64_t r = slot_row(slots, i, back, k * dil, len);
      const float xn = r >= 0 ? norm_elem<T, true>(to_f32(base[r * d + c]), tap_scale[k], nw) : 0.f;
      if (K4D3)
        acc = k == 0 ? to_f32(conv_w[c * K]) * xn : fmaf(to_f32(conv_w[c * K + k]), xn, acc);
      else if (r >= 0)
        acc = fmaf(to_f32(conv_w[c * K + k]), xn, acc);
    }
    const float y = round_to<T>(acc);
    const float act = round_to<T>(y / (1.0f + expf(-y)));
    const float xs = self >= 0 ? to_f32(base[self * d + c]) : 0.f;
    out[(b * n + i) * d + c] = residual ? from_f32<T>(xs + act) : from_f32<T>(act);
  }
}

static int conv_slots_launch(const void* rows, const void* norm_w, const void* conv_w, int dtype, int64_t B,
                             int64_t stride, int64_t len, const int32_t* slots, int64_t n, int32_t d, int32_t K,
                             int32_t dil, float eps, int residual, void* out, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(n), static_cast<unsigned>(B));
  // the same shape tests as conv_launch, in the same order
  if (K == 4 && dil == 3 && d % 4 == 0 && d <= 2048 && dtype == LNG_BF16 && len < INT32_MAX) {
    const int threads = static_cast<int>(cdiv(d / 4, 64) * 64);
    hipLaunchKernelGGL(k_conv_k4d3_slots_bf16, grid, dim3(threads), 0, s, static_cast<const bf16*>(rows),
                       static_cast<const bf16*>(norm_w), static_cast<const bf16*>(conv_w), slots, stride, len, n,
                       static_cast<uint32_t>(d / 4), eps, residual, static_cast<bf16*>(out));
    return check_launch("causal_conv_slots_k4d3_bf16");
  }
  const bool k4d3 = K == 4 && dil == 3 && d % 8 == 0;
  const size_t lds = sizeof(float) * K;
  if (dtype == LNG_F32) {
    const float *x = static_cast<const float*>(rows), *nw = static_cast<const float*>(norm_w),
                *cw = static_cast<const float*>(conv_w);
    if (k4d3)
      hipLaunchKernelGGL((k_conv_slots<float, true>), grid, dim3(256), lds, s, x, nw, cw, slots, stride, len, n, d, K,
                         dil, eps, residual, static_cast<float*>(out));
    else
      hipLaunchKernelGGL((k_conv_slots<float, false>), grid, dim3(256), lds, s, x, nw, cw, slots, stride, len, n, d, K,
                         dil, eps, residual, static_cast<float*>(out));
  } else if (dtype == LNG_BF16) {
    const bf16 *x = static_cast<const bf16*>(rows), *nw = static_cast<const bf16*>(norm_w),
               *cw = static_cast<const bf16*>(conv_w);
    if (k4d3)
      hipLaunchKernelGGL((k_conv_slots<bf16, true>), grid, dim3(256), lds, s, x, nw, cw, slots, stride, len, n, d, K,
                         dil, eps, residual, static_cast<bf16*>(out));
    else
      hipLaunchKernelGGL((k_conv_slots<bf16, false>), grid, dim3(256), lds, s, x, nw, cw, slots, stride, len, n, d, K,
                         dil, eps, residual, static_cast<bf16*>(out));
  } else {
    return fail(LNG_E_DTYPE, "causal_conv_slots: dtype must be f32 or bf16");
  }
  return check_launch("causal_conv_slots");
}

}  // namespace lng

extern "C" {

int lng_causal_conv(const void* mixed, const void* norm_w, const void* conv_w, int dtype, int64_t B, int64_t T,
                    int32_t d, int32_t K, int32_t dilation, float eps, int residual, void* out, void* stream) {
  if (B < 0 || T < 0 || d <= 0 || K <= 0 || dilation <= 0) return fail(LNG_E_ARG, "causal_conv: bad shape");
  if (mixed == out) return fail(LNG_E_ARG, "causal_conv: out must not alias mixed");
  if (B == 0 || T == 0) return LNG_OK;
  const ConvWin W{T, T, 0, T, nullptr};
  return conv_launch(mixed, norm_w, conv_w, dtype, B, W, d, K, dilation, eps, residual, out, as_stream(stream));
}

int lng_causal_conv_at(const void* rows, const void* norm_w, const void* conv_w, int dtype, int64_t B, int64_t stride,
                       int64_t len, int64_t pos0, const int32_t* pos0_dev, int64_t n, int32_t d, int32_t K,
                       int32_t dilation, float eps, int residual, void* out, void* stream) {
  if (B < 0 || n < 0 || d <= 0 || K <= 0 || dilation <= 0 || len < 0 || stride < len || pos0 < 0)
    return fail(LNG_E_ARG, "causal_conv_at: bad shape");
  if (!pos0_dev && pos0 + n > len) return fail(LNG_E_RANGE, "causal_conv_at: outputs past the rows");
  if (rows == out) return fail(LNG_E_ARG, "causal_conv_at: out must not alias the rows");
  if (B == 0 || n == 0) return LNG_OK;
  const ConvWin W{stride, len, pos0, n, pos0_dev};
  return conv_launch(rows, norm_w, conv_w, dtype, B, W, d, K, dilation, eps, residual, out, as_stream(stream));
}

int lng_causal_conv_slots(const void* rows, const void* norm_w, const void* conv_w, int dtype, int64_t B,
                          int64_t stride, int64_t len, const int32_t* slots, int64_t n, int32_t back, int32_t d,
                          int32_t K, int32_t dilation, float eps, int residual, void* out, void* stream) {
  if (B < 0 || n < 0 || d <= 0 || K <= 0 || dilation <= 0 || len < 0 || stride < len)
    return fail(LNG_E_ARG, "causal_conv_slots: bad shape");
  if (back != (K - 1) * dilation) return fail(LNG_E_ARG, "causal_conv_slots: back must be (K - 1) * dilation");
  if (B > 65535 || n > 0x7FFFFFFF) return fail(LNG_E_ARG, "causal_conv_slots: B <= 65535 sequences");
  if (K > 64) return fail(LNG_E_ARG, "causal_conv_slots: kernel size at most 64");
  if (rows == out) return fail(LNG_E_ARG, "causal_conv_slots: out must not alias the rows");
  if (B == 0 || n == 0) return LNG_OK;
  if (!slots) return fail(LNG_E_ARG, "causal_conv_slots: null slots");
  return conv_slots_launch(rows, norm_w, conv_w, dtype, B, stride, len, slots, n, d, K, dilation, eps, residual, out,
                           as_stream(stream));
}

int lng_row_sumsq(const void* x, int64_t rows, int32_t d, float* rowsq, void* stream) {
  if (rows < 0 || d <= 0 || d % 8 || !x || !rowsq) return fail(LNG_E_ARG, "row_sumsq: bf16 rows with d % 8 == 0");
  if (rows == 0) return LNG_OK;
  hipLaunchKernelGGL(k_row_sumsq_bf16, dim3(static_cast<unsigned>(cdiv(rows, 4))), dim3(256), 0, as_stream(stream),
                     static_cast<const bf16*>(x), rows, d, rowsq);
  return check_launch("row_sumsq");
}

}  // extern "C"
