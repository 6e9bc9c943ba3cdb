// Route readout: sink-softmax attention over the R route slots.
//
// k_sink_attention is the materialised form (query/key/value in the layout of
// _manual_gqa) used by cached decode, tree verification and the fp32 layer.
// k_readout_fused is the metric kernel: it gathers the route tokens from the
// n-gram tables by code, never materialises keys or values, and computes
//   score_{hg,r} = s_r * (qkw_hg . x_r),   qkw_hg = scale * w_mem . Wk[h]^T q_hg
//   o_hg         = Wv[h] (w_mem . sum_r p_{hg,r} s_r x_r / l_hg)
// on MFMA with an online softmax seeded by the sink (m, l) = (b0, 1).
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

// ------------------------------------------------------------------ fused gather + readout (bf16, SB shape)
constexpr int FR_TOK = 4;    // tokens per block (one per wave in the route phase)
constexpr int FR_H = 16;     // query heads
constexpr int FR_HD = 64;    // head dim
constexpr int FR_DT = 256;   // route token dim (2 orders x 128)
constexpr int FR_LD = FR_DT + 8;  // padded LDS row (bf16)

__device__ __forceinline__ bf16x8 ld16(const bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }
__device__ __forceinline__ bf16x8 zero8() {
  bf16x8 z;
#pragma unroll
  for (int j = 0; j < 8; ++j) z[j] = static_cast<bf16>(0.f);
  return z;
}

constexpr int FR_MAXR = 256;     // routes whose codes fit the per-wave LDS code cache

// Row sources of one route chunk (32 routes = 2 tiles of 16) for this lane:
// lane (li, lg) covers route c0 + 16*tt + li, features 64*lg .. 64*lg+63 of the
// 256-wide route token (lg 0,1: 2-gram row halves; lg 2,3: 3-gram row halves).
// The codes of the token at t, t-1, t-2 sit in LDS (cs[k][r] = code at t-k), so a
// row address never waits on a dependent global load.
struct FusedCtx {
  const uint8_t* cs;  // [3][FR_MAXR] in LDS
  const bf16* table2;
  const bf16* table3;
  int64_t t;
  int32_t R;
  int li, lg;
  bool tok_ok;
  __device__ __forceinline__ const bf16* src(int rho) const {
    if (!tok_ok || rho >= R) return nullptr;
    if (lg < 2) {
      if (t < 1) return nullptr;
      const int64_t c0 = cs[rho], c1 = cs[FR_MAXR + rho];
      const int64_t row = static_cast<int64_t>(rho) * 256 + c1 + 16 * c0;
      return table2 + row * 128 + 64 * lg;
    }
    if (t < 2) return nullptr;
    const int64_t c0 = cs[rho], c1 = cs[FR_MAXR + rho], c2 = cs[2 * FR_MAXR + rho];
    const int64_t row = static_cast<int64_t>(rho) * 4096 + c2 + 16 * c1 + 256 * c0;
    return table3 + row * 128 + 64 * (lg - 2);
  }
  __device__ __forceinline__ void load(int c0, bf16x8 (&x)[2][8]) const {
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const bf16* s = src(c0 + 16 * tt + li);
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) x[tt][kk] = s ? ld16(s + 8 * kk) : zero8();
    }
  }
};

// LDS: one 32-row region per wave/token, reused as qkw (rows 0..15, phase A -> B), the
// route chunk being transposed (rows 0..31, phase B) and u (rows 0..15, phase B -> C),
// plus the token's codes.  70.6 KB per block: two blocks (8 waves) per CU.
__global__ __launch_bounds__(256, 2) void k_readout_fused(const bf16* __restrict__ q, const uint8_t* __restrict__ codes,
                                                          int64_t B, int64_t T, int32_t R,
                                                          const bf16* __restrict__ table2,
                                                          const bf16* __restrict__ table3,
                                                          const bf16* __restrict__ wk_t, const bf16* __restrict__ wv,
                                                          const bf16* __restrict__ w_mem, float eps, float scale,
                                                          float sink, bf16* __restrict__ head_out) {
  __shared__ __attribute__((aligned(16))) bf16 xs[FR_TOK][32][FR_LD];
  __shared__ uint8_t csh[FR_TOK][3 * FR_MAXR];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int64_t ntok = B * T;
  const int64_t tok0 = static_cast<int64_t>(blockIdx.x) * FR_TOK;

  // ---------------- stage 0: this wave's token codes (t, t-1, t-2) into LDS, first gather in flight
  const int64_t tok = tok0 + w;
  const bool tok_ok = tok < ntok;
  const int64_t tpos = tok_ok ? tok % T : 0;
  for (int r = lane; r < R; r += 64) {
    csh[w][r] = tok_ok ? (codes[tok * R + r] & 15) : 0;
    csh[w][FR_MAXR + r] = (tok_ok && tpos >= 1) ? (codes[(tok - 1) * R + r] & 15) : 0;
    csh[w][2 * FR_MAXR + r] = (tok_ok && tpos >= 2) ? (codes[(tok - 2) * R + r] & 15) : 0;
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  __builtin_amdgcn_wave_barrier();
  FusedCtx ctx{csh[w], table2, table3, tpos, R, li, lg, tok_ok};
  bf16x8 xa[2][8];
  ctx.load(0, xa);

  // ---------------- phase A: qkw[t][4h+g][f] = scale * w_mem[f] * (Wk[h]^T q[t][4h+g])[f], wave = head h
  {
    const int h = w;
    const int64_t tq = tok0 + (li >> 2);
    const int hg = h * 4 + (li & 3);
    bf16x8 bq[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      bq[ks] = tq < ntok ? ld16(q + tq * (FR_H * FR_HD) + hg * FR_HD + 32 * ks + 8 * lg) : zero8();
#pragma unroll 4
    for (int ft = 0; ft < 16; ++ft) {
      f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const bf16x8 a = ld16(wk_t + (static_cast<int64_t>(h) * FR_DT + 16 * ft + li) * FR_HD + 32 * ks + 8 * lg);
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bq[ks], d, 0, 0, 0);
      }
      const int f = 16 * ft + 4 * lg;
      bf16x4 o;
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = static_cast<bf16>(d[i] * to_f32(w_mem[f + i]) * scale);
      *reinterpret_cast<bf16x4*>(&xs[li >> 2][hg][f]) = o;
    }
  }
  __syncthreads();

  // ---------------- phase B: one token per wave, routes in chunks of 32
  bf16x8 qb[8];
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) qb[kk] = *reinterpret_cast<const bf16x8*>(&xs[w][li][64 * lg + 8 * kk]);

  float m_run = sink, l_part = 0.f;
  f32x4 acc[16];
#pragma unroll
  for (int ft = 0; ft < 16; ++ft) acc[ft] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto process = [&](int c0, bf16x8 (&x)[2][8]) {
    float sr[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      float ss = 0.f;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float v = static_cast<float>(x[tt][kk][j]);
          ss = fmaf(v, v, ss);
        }
      ss += __shfl_xor(ss, 16, 64);
      ss += __shfl_xor(ss, 32, 64);
      sr[tt] = 1.0f / sqrtf(ss * (1.0f / FR_DT) + eps);  // route c0 + 16tt + li
    }
    f32x4 sc[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      sc[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) sc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x[tt][kk], qb[kk], sc[tt], 0, 0, 0);
    }
    // sc[tt][i]: route c0 + 16tt + 4lg + i, head hg = li
    float sD[2][4], s[2][4];
    float cmax = -INFINITY;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sD[tt][i] = __shfl(sr[tt], 4 * lg + i, 64);
        const int r = c0 + 16 * tt + 4 * lg + i;
        s[tt][i] = r < R ? sc[tt][i] * sD[tt][i] : -INFINITY;
        cmax = fmaxf(cmax, s[tt][i]);
      }
    cmax = fmaxf(cmax, __shfl_xor(cmax, 16, 64));
    cmax = fmaxf(cmax, __shfl_xor(cmax, 32, 64));
    const float m_new = fmaxf(m_run, cmax);
    const float alpha = expf(m_run - m_new);
    m_run = m_new;
    float psum = 0.f;
    bf16x8 pa;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = expf(s[tt][i] - m_new);
        psum += p;
        pa[4 * tt + i] = static_cast<bf16>(p * sD[tt][i]);
      }
    l_part = l_part * alpha + psum;
    float aD[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) aD[i] = __shfl(alpha, 4 * lg + i, 64);
#pragma unroll
    for (int ft = 0; ft < 16; ++ft)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[ft][i] *= aD[i];
    // route chunk to LDS (row layout), then transposed reads as the B operand of P.X;
    // the registers are refilled with the next chunk while the MFMAs below run
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) *reinterpret_cast<bf16x8*>(&xs[w][16 * tt + li][64 * lg + 8 * kk]) = x[tt][kk];
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    if (c0 + 32 < R) ctx.load(c0 + 32, x);
    // ds_read_b64_tr_b16: lane i of each 16-lane group receives element i%4 of the 8-byte
    // chunks addressed by lanes i/4 + 4c (c = 0..3), i.e. X[4g + c][16ft + i] here.  The
    // two halves are joined with a shuffle: element-wise bit casts of the returned
    // vector are miscompiled (every element becomes element 0).
#pragma unroll
    for (int ft = 0; ft < 16; ++ft) {
      const int col = 16 * ft + 4 * (li & 3);
      const bf16x4 b0 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
          (__attribute__((address_space(3))) bf16x4*)(&xs[w][4 * lg + (li >> 2)][col]));
      const bf16x4 b1 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
          (__attribute__((address_space(3))) bf16x4*)(&xs[w][16 + 4 * lg + (li >> 2)][col]));
      const bf16x8 b = __builtin_shufflevector(b0, b1, 0, 1, 2, 3, 4, 5, 6, 7);
      acc[ft] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, b, acc[ft], 0, 0, 0);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
  };

  for (int c0 = 0; c0 < R; c0 += 32) process(c0, xa);

  // normalise and stage u = w_mem . U / l for the value projection
  float lt = l_part + __shfl_xor(l_part, 16, 64);
  lt += __shfl_xor(lt, 32, 64);
  lt += expf(sink - m_run);
  const float inv = 1.0f / lt;
  float iD[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) iD[i] = __shfl(inv, 4 * lg + i, 64);
#pragma unroll
  for (int ft = 0; ft < 16; ++ft) {
    const int f = 16 * ft + li;
    const float wm = to_f32(w_mem[f]);
#pragma unroll
    for (int i = 0; i < 4; ++i) xs[w][4 * lg + i][f] = static_cast<bf16>(acc[ft][i] * iD[i] * wm);
  }
  __syncthreads();

  // ---------------- phase C: o[t][4h+g][d] = Wv[h][d] . u[t][4h+g], wave = head h
  {
    const int h = w;
    const int64_t tc = tok0 + (li >> 2);
    const int hg = h * 4 + (li & 3);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        const bf16x8 a = ld16(wv + (static_cast<int64_t>(h) * FR_HD + 16 * dt + li) * FR_DT + 32 * ks + 8 * lg);
        const bf16x8 b = *reinterpret_cast<const bf16x8*>(&xs[li >> 2][hg][32 * ks + 8 * lg]);
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, d, 0, 0, 0);
      }
      if (tc < ntok) {
        bf16x4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = static_cast<bf16>(d[i]);
        *reinterpret_cast<bf16x4*>(head_out + tc * (FR_H * FR_HD) + hg * FR_HD + 16 * dt + 4 * lg) = o;
      }
    }
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

int lng_memory_readout_fused(const void* q, const uint8_t* codes, int64_t B, int64_t T, int32_t R, const void* table2,
                             const void* table3, const void* wk_t, const void* wv, const void* w_mem, float eps,
                             float scale, float sink_logit, void* head_out, void* stream) {
  if (B < 0 || T < 0 || R <= 0) return fail(LNG_E_ARG, "memory_readout_fused: bad shape");
  if (R > FR_MAXR) return fail(LNG_E_ARG, "memory_readout_fused: at most 256 routes");
  const int64_t ntok = B * T;
  if (ntok == 0) return LNG_OK;
  const int64_t blocks = cdiv(ntok, FR_TOK);
  if (blocks > 0x7fffffffLL) return fail(LNG_E_ARG, "memory_readout_fused: too many tokens");
  hipLaunchKernelGGL(k_readout_fused, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, as_stream(stream),
                     static_cast<const bf16*>(q), codes, B, T, R, static_cast<const bf16*>(table2),
                     static_cast<const bf16*>(table3), static_cast<const bf16*>(wk_t), static_cast<const bf16*>(wv),
                     static_cast<const bf16*>(w_mem), eps, scale, sink_logit, static_cast<bf16*>(head_out));
  return check_launch("memory_readout_fused");
}

}  // extern "C"
