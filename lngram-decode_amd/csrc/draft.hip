// Self-drafting readers on gfx950: router codes of new positions, the draft readout over the
// shared n-gram table, full-vocabulary scoring with top-k, code-keyed online counts, the tree
// verification gather, and the per-level orchestration of a draft tree.
//
// State lives in caller-owned device buffers described by lng_drafter (include/lngram_hip.h):
// token ids, route codes and SSM states per row.  Rows 0 .. L-1 are the committed positions
// (L is read from device memory, so a captured launch sequence stays valid as L grows);
// rows past the committed capacity hold hypothetical / tree positions.  A row is named by a
// spec: v >= 0 is absolute row v, v < 0 is committed row L + v (-1 = the last committed
// token), LNG_ROW_NONE is "no position" (before the sequence start).
//
// Readout math (the per-token algorithm of drafting/cpu_drafter.py:208-244, restructured):
//   qkw[qh]   = r_e * QK[qh] e (+ QKS[qh] s)       QK = scale diag(mem_norm) Wk[h]^T W_q[qh] diag(q_norm)
//   score     = s_x * (qkw[qh] . x_r)               x_r = route token, s_x = rsqrt(mean(x_r^2) + eps)
//   u[qh]     = sum_r p_r s_x x_r                   sink-seeded softmax over routes
//   hid       = OV u                                OV = W_o blockdiag(Wv[h] diag(mem_norm))
//   logits    = E (RMSNorm(hid) * out_norm)
#include <algorithm>
#include <atomic>
#include <climits>
#include <vector>

#include "common.h"

namespace lng {

constexpr int DR_MAXP = 16;     // positions per readout launch
constexpr int DR_MAXN = 4;      // window length (max n-gram order)
constexpr int DR_MAXK = 8;      // top-k
constexpr int DR_MAXCH = 64;    // children written per select
constexpr int DR_RC = 32;       // routes per attention block
constexpr int DR_VB = 64;       // vocabulary rows per logits block
constexpr int DR_TB = 32;       // pair positions per online-count block
constexpr int DR_ADV_CHUNK = 1024;  // positions per advance launch (range form)

struct DrWin {
  int32_t n;
  int32_t slot[DR_MAXP][DR_MAXN];  // oldest first; the last slot is the position itself
};

struct DrAdv {
  int32_t n;
  int32_t range;          // != 0: rows base .. base+n-1 (absolute), prev of the first = prev0
  int32_t base, prev0;
  int32_t row[DR_MAXP], prev[DR_MAXP];
};

struct DrChildren {
  int32_t n;
  int32_t row[DR_MAXCH];
  int8_t parent[DR_MAXCH];
  int8_t rank[DR_MAXCH];
};

__device__ __forceinline__ int32_t dr_resolve(int32_t v, int32_t L) {
  if (v == LNG_ROW_NONE) return -1;
  if (v >= 0) return v;
  const int32_t t = L + v;
  return t >= 0 ? t : -1;
}

// Embedding element c of token tok (zero for an id outside [0, V): never read out of bounds).
__device__ __forceinline__ bool dr_tok_ok(const lng_drafter& D, int64_t tok) { return tok >= 0 && tok < D.V; }

template <typename T>
__device__ __forceinline__ float ldf(const void* p, int64_t i) {
  return to_f32(static_cast<const T*>(p)[i]);
}

__device__ __forceinline__ float ld_any(const void* p, int dt, int64_t i) {
  return dt == LNG_BF16 ? ldf<bf16>(p, i) : (dt == LNG_F16 ? ldf<_Float16>(p, i) : ldf<float>(p, i));
}

// Four / eight consecutive elements of a float, bf16 or fp16 row as fp32 (8- / 16-byte aligned for
// the 2-byte types, 16- / 32-byte for fp32).
__device__ __forceinline__ f32x4 bf2f4(uint32_t a, uint32_t b) {
  return f32x4{__uint_as_float(a << 16), __uint_as_float(a & 0xffff0000u), __uint_as_float(b << 16),
               __uint_as_float(b & 0xffff0000u)};
}
__device__ __forceinline__ f32x4 h2f4(uint32_t a, uint32_t b) {
  return f32x4{static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(a & 0xffffu))),
               static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(a >> 16))),
               static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(b & 0xffffu))),
               static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(b >> 16)))};
}
__device__ __forceinline__ f32x4 ld4_any(const void* p, int dt, int64_t i) {
  if (dt == LNG_F32) return *reinterpret_cast<const f32x4*>(static_cast<const float*>(p) + i);
  const uint2 v = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p) + i);
  return dt == LNG_BF16 ? bf2f4(v.x, v.y) : h2f4(v.x, v.y);
}
template <typename T>
__device__ __forceinline__ void ld8f(const T* p, f32x4& a, f32x4& b);
template <>
__device__ __forceinline__ void ld8f<float>(const float* p, f32x4& a, f32x4& b) {
  a = reinterpret_cast<const f32x4*>(p)[0];
  b = reinterpret_cast<const f32x4*>(p)[1];
}
template <>
__device__ __forceinline__ void ld8f<bf16>(const bf16* p, f32x4& a, f32x4& b) {
  const u32x4 v = *reinterpret_cast<const u32x4*>(p);
  a = bf2f4(v.x, v.y);
  b = bf2f4(v.z, v.w);
}
template <>
__device__ __forceinline__ void ld8f<_Float16>(const _Float16* p, f32x4& a, f32x4& b) {
  const u32x4 v = *reinterpret_cast<const u32x4*>(p);
  a = h2f4(v.x, v.y);
  b = h2f4(v.z, v.w);
}
__device__ __forceinline__ float dot4(f32x4 a, f32x4 b, float acc) {
  acc = fmaf(a.x, b.x, acc);
  acc = fmaf(a.y, b.y, acc);
  acc = fmaf(a.z, b.z, acc);
  return fmaf(a.w, b.w, acc);
}

// Sum over a block of 256 threads (4 waves); `red` holds >= 4 floats.
__device__ __forceinline__ float block_sum256(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// ------------------------------------------------------------------ SSM step inputs
// u[j, n] = W_in[n] . RMSNorm(E[tok_j]) * ssm_norm      grid (cdiv(N, 16), cdiv(P, 4))
__global__ __launch_bounds__(256) void k_draft_ssm_u(lng_drafter D, DrAdv A, float* __restrict__ u) {
  __shared__ float xs[4][LNG_DR_MAX_D];
  __shared__ float red[4];
  const int d = D.d;
  const int j0 = blockIdx.y * 4;
  const int L = *D.length;
  for (int jj = 0; jj < 4; ++jj) {
    const int j = j0 + jj;
    if (j >= A.n) break;
    const int32_t row = A.range ? A.base + j : dr_resolve(A.row[j], L);
    const int64_t tok = row >= 0 ? D.tokens[row] : -1;
    const bool ok = dr_tok_ok(D, tok);
    float ss = 0.f;
    for (int c = threadIdx.x; c < d; c += 256) {
      const float v = ok ? ld_any(D.emb, D.emb_dtype, tok * d + c) : 0.f;
      xs[jj][c] = v;
      ss = fmaf(v, v, ss);
    }
    ss = block_sum256(ss, red);
    const float r = 1.0f / sqrtf(ss / static_cast<float>(d) + D.ssm_eps);
    for (int c = threadIdx.x; c < d; c += 256) xs[jj][c] = xs[jj][c] * r * D.ssm_norm[c];
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  for (int q = 0; q < 4; ++q) {
    const int n = blockIdx.x * 16 + w * 4 + q;
    if (n >= D.ssm_dim) break;
    const float* wr = D.ssm_w_in + static_cast<int64_t>(n) * d;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int c = lane; c < d; c += 64) {
      const float wv = wr[c];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) acc[jj] = fmaf(wv, xs[jj][c], acc[jj]);
    }
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const float s = wave_sum(acc[jj]);
      const int j = j0 + jj;
      if (lane == 0 && j < A.n) u[static_cast<int64_t>(j) * D.ssm_dim + n] = s;
    }
  }
}

// s[row_j] = a * s[prev_j] + (1 - a) * u[j], positions in order (a chain within the batch reads
// the state this thread wrote for the earlier position).   grid (cdiv(N, 256))
__global__ __launch_bounds__(256) void k_draft_ssm_scan(lng_drafter D, DrAdv A, const float* __restrict__ u) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= D.ssm_dim) return;
  const int L = *D.length;
  const float a = D.ssm_decay[n];
  for (int j = 0; j < A.n; ++j) {
    const int32_t row = A.range ? A.base + j : dr_resolve(A.row[j], L);
    const int32_t pv = A.range ? (j == 0 ? dr_resolve(A.prev0, L) : A.base + j - 1) : dr_resolve(A.prev[j], L);
    if (row < 0) continue;
    const float sp = pv >= 0 ? D.ssm[static_cast<int64_t>(pv) * D.ssm_dim + n] : 0.f;
    D.ssm[static_cast<int64_t>(row) * D.ssm_dim + n] = a * sp + (1.f - a) * u[static_cast<int64_t>(j) * D.ssm_dim + n];
  }
}

// ------------------------------------------------------------------ router codes
// codes[row_j] = pack(router . concat(RMSNorm(E[prev] or start) * prev_norm, RMSNorm(E[tok]) * cur_norm
//                                      [, s[row_j]]) > 0)          grid (cdiv(R, 4), cdiv(P, 4))
__global__ __launch_bounds__(256) void k_draft_codes(lng_drafter D, DrAdv A) {
  __shared__ float fs[4][2 * LNG_DR_MAX_D + LNG_DR_MAX_N];
  __shared__ float red[4];
  __shared__ float lg[4][16];
  const int d = D.d;
  const int F = 2 * d + (D.router_ssm ? D.ssm_dim : 0);
  const int j0 = blockIdx.y * 4;
  const int L = *D.length;
  int32_t rows[4];
  for (int jj = 0; jj < 4; ++jj) {
    const int j = j0 + jj;
    rows[jj] = -1;
    if (j >= A.n) continue;
    const int32_t row = A.range ? A.base + j : dr_resolve(A.row[j], L);
    const int32_t pv = A.range ? (j == 0 ? dr_resolve(A.prev0, L) : A.base + j - 1) : dr_resolve(A.prev[j], L);
    if (row < 0) continue;
    rows[jj] = row;
    const int64_t tok = D.tokens[row];
    for (int half = 0; half < 2; ++half) {
      const bool use_start = half == 0 && pv < 0;
      const int64_t t = half == 0 ? (pv >= 0 ? D.tokens[pv] : 0) : tok;
      const bool ok = dr_tok_ok(D, t);
      const float* nw = half == 0 ? D.router_prev_norm : D.router_cur_norm;
      float ss = 0.f;
      for (int c = threadIdx.x; c < d; c += 256) {
        const float v = use_start ? D.router_start[c] : (ok ? ld_any(D.emb, D.emb_dtype, t * d + c) : 0.f);
        fs[jj][half * d + c] = v;
        ss = fmaf(v, v, ss);
      }
      ss = block_sum256(ss, red);
      const float r = 1.0f / sqrtf(ss / static_cast<float>(d) + D.router_eps);
      for (int c = threadIdx.x; c < d; c += 256) fs[jj][half * d + c] = fs[jj][half * d + c] * r * nw[c];
    }
    if (D.router_ssm)
      for (int c = threadIdx.x; c < D.ssm_dim; c += 256) fs[jj][2 * d + c] = D.ssm[static_cast<int64_t>(row) * D.ssm_dim + c];
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int bits = D.bits;
  // wave w: route blockIdx.x*4 + w, its `bits` logits for the 4 positions
  const int r = blockIdx.x * 4 + w;
  if (r < D.R) {
    for (int b = 0; b < bits; ++b) {
      const int64_t o = static_cast<int64_t>(r) * bits + b;
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
      for (int c = lane; c < F; c += 64) {
        const float wv = ld_any(D.router, D.router_dtype, o * F + c);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) acc[jj] = fmaf(wv, fs[jj][c], acc[jj]);
      }
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const float s = wave_sum(acc[jj]);
        if (lane == 0) lg[jj][w * 4 + b] = s;
      }
    }
    if (lane < 4 && rows[lane] >= 0) {
      int code = 0;
      for (int b = 0; b < bits; ++b) code |= (lg[lane][w * 4 + b] > 0.f ? 1 : 0) << b;
      D.codes[static_cast<int64_t>(rows[lane]) * D.R + r] = static_cast<uint8_t>(code);
    }
  }
}

// ------------------------------------------------------------------ readout
// Row of route r, order index oi, for the window w of position j (-1 when any slot is missing).
__device__ __forceinline__ int64_t dr_row(const lng_drafter& D, const int32_t* slot_rows, int oi, int r) {
  const int n = D.orders[oi];
  int64_t addr = 0;
  for (int k = 0; k < n; ++k) {
    const int32_t row = slot_rows[D.maxn - n + k];
    if (row < 0) return -1;
    addr |= static_cast<int64_t>(D.codes[static_cast<int64_t>(row) * D.R + r] & ((1 << D.bits) - 1)) << (k * D.bits);
  }
  return static_cast<int64_t>(r) * (int64_t{1} << (D.bits * n)) + addr;
}

// qkw[j, qh*Dt + i] = r_j * QK[qh*Dt + i] . e_j (+ QKS[..] . s_j)        grid (cdiv(QH*Dt, 32))
__global__ __launch_bounds__(256) void k_draft_qkw(lng_drafter D, DrWin W, float* __restrict__ qkw) {
  extern __shared__ float es[];  // [P][d] then [P][N]
  __shared__ float red[4];
  __shared__ float rj[DR_MAXP];
  const int d = D.d, P = W.n;
  const int L = *D.length;
  const int N = D.query_ssm ? D.ssm_dim : 0;
  float* ss_s = es + P * d;
  for (int j = 0; j < P; ++j) {
    const int32_t row = dr_resolve(W.slot[j][D.maxn - 1], L);
    const int64_t tok = row >= 0 ? D.tokens[row] : -1;
    const bool ok = dr_tok_ok(D, tok);
    float ss = 0.f;
    for (int c = threadIdx.x; c < d; c += 256) {
      const float v = ok ? ld_any(D.emb, D.emb_dtype, tok * d + c) : 0.f;
      es[j * d + c] = v;
      ss = fmaf(v, v, ss);
    }
    ss = block_sum256(ss, red);
    if (threadIdx.x == 0) rj[j] = 1.0f / sqrtf(ss / static_cast<float>(d) + D.draft_eps);
    for (int c = threadIdx.x; c < N; c += 256)
      ss_s[j * N + c] = row >= 0 ? D.ssm[static_cast<int64_t>(row) * D.ssm_dim + c] : 0.f;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int QD = D.q_heads * D.dt;
  for (int q = 0; q < 8; ++q) {
    const int o = blockIdx.x * 32 + w * 8 + q;
    if (o >= QD) break;
    const float* wr = D.qk + static_cast<int64_t>(o) * d;
    float acc[DR_MAXP];
#pragma unroll
    for (int j = 0; j < DR_MAXP; ++j) acc[j] = 0.f;
    for (int c = lane; c < d; c += 64) {
      const float wv = wr[c];
#pragma unroll
      for (int j = 0; j < DR_MAXP; ++j)
        if (j < P) acc[j] = fmaf(wv, es[j * d + c], acc[j]);
    }
    float accs[DR_MAXP];
#pragma unroll
    for (int j = 0; j < DR_MAXP; ++j) accs[j] = 0.f;
    if (N) {
      const float* sr = D.qks + static_cast<int64_t>(o) * N;
      for (int c = lane; c < N; c += 64) {
        const float wv = sr[c];
#pragma unroll
        for (int j = 0; j < DR_MAXP; ++j)
          if (j < P) accs[j] = fmaf(wv, ss_s[j * N + c], accs[j]);
      }
    }
#pragma unroll
    for (int j = 0; j < DR_MAXP; ++j) {
      if (j < P) {
        const float a = wave_sum(acc[j]);
        const float b = wave_sum(accs[j]);
        if (lane == 0) qkw[static_cast<int64_t>(j) * QD + o] = rj[j] * a + b;
      }
    }
  }
}

// Partial sink-free softmax over one chunk of DR_RC routes for every query head of position j:
// part[((j * nch + c) * QH + qh) * (Dt + 2) + {0..Dt-1, Dt, Dt+1}] = (U, m, l)
//                                                                   grid (nch, P)
__global__ __launch_bounds__(256) void k_draft_attend(lng_drafter D, DrWin W, const float* __restrict__ qkw,
                                                      float* __restrict__ part) {
  __shared__ float xs[DR_RC][LNG_DR_MAX_DT];
  __shared__ float sx[DR_RC];
  __shared__ float sc[LNG_DR_MAX_QH][DR_RC];
  __shared__ int64_t rowsh[DR_RC][DR_MAXN];
  __shared__ int32_t slot_rows[DR_MAXN];
  const int j = blockIdx.y, c = blockIdx.x;
  const int nch = gridDim.x;
  const int L = *D.length;
  const int Dt = D.dt, QH = D.q_heads, md = D.mem_dim;
  const int r0 = c * DR_RC;
  const int nr = min(DR_RC, D.R - r0);
  if (threadIdx.x < DR_MAXN) slot_rows[threadIdx.x] = threadIdx.x < D.maxn ? dr_resolve(W.slot[j][threadIdx.x], L) : -1;
  __syncthreads();
  for (int e = threadIdx.x; e < nr * D.n_orders; e += 256) {
    const int rr = e / D.n_orders, oi = e % D.n_orders;
    rowsh[rr][oi] = dr_row(D, slot_rows, oi, r0 + rr);
  }
  __syncthreads();
  // gather route tokens (order oi fills dims oi*md .. +md)
  for (int e = threadIdx.x; e < nr * Dt; e += 256) {
    const int rr = e / Dt, i = e % Dt;
    const int oi = i / md;
    const int64_t row = rowsh[rr][oi];
    xs[rr][i] = row >= 0 ? ld_any(D.tables[oi], D.table_dtype, row * md + (i % md)) : 0.f;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  for (int rr = w; rr < nr; rr += 4) {
    float ss = 0.f;
    for (int i = lane; i < Dt; i += 64) ss = fmaf(xs[rr][i], xs[rr][i], ss);
    ss = wave_sum(ss);
    const float s = 1.0f / sqrtf(ss / static_cast<float>(Dt) + D.mem_eps);
    if (lane == 0) sx[rr] = s;
    const float* qv = qkw + static_cast<int64_t>(j) * QH * Dt;
    for (int qh = 0; qh < QH; ++qh) {
      float a = 0.f;
      for (int i = lane; i < Dt; i += 64) a = fmaf(qv[qh * Dt + i], xs[rr][i], a);
      a = wave_sum(a);
      if (lane == 0) sc[qh][rr] = s * a;
    }
  }
  __syncthreads();
  // per head: m, l over the chunk; U = sum_r e^{score - m} s_r x_r
  for (int e = threadIdx.x; e < QH * Dt; e += 256) {
    const int qh = e / Dt, i = e % Dt;
    float m = -INFINITY;
    for (int rr = 0; rr < nr; ++rr) m = fmaxf(m, sc[qh][rr]);
    float l = 0.f, u = 0.f;
    for (int rr = 0; rr < nr; ++rr) {
      const float p = expf(sc[qh][rr] - m);
      l += p;
      u = fmaf(p * sx[rr], xs[rr][i], u);
    }
    float* o = part + ((static_cast<int64_t>(j) * nch + c) * QH + qh) * (Dt + 2);
    o[i] = u;
    if (i == 0) {
      o[Dt] = m;
      o[Dt + 1] = l;
    }
  }
}

// hid[j, o] = OV[o] . u_j, u_j = merged (sink-seeded) softmax of the chunk partials.
//                                                                   grid (cdiv(d, 16))
__global__ __launch_bounds__(256) void k_draft_hidden(lng_drafter D, int32_t P, int32_t nch,
                                                      const float* __restrict__ part, float* __restrict__ hid) {
  extern __shared__ float us[];  // [P][QH*Dt]
  __shared__ float scale_c[DR_MAXP][LNG_DR_MAX_QH][LNG_DR_MAX_CH];
  const int Dt = D.dt, QH = D.q_heads, QD = QH * Dt;
  const float b0 = D.sink_logit;
  for (int e = threadIdx.x; e < P * QH; e += 256) {
    const int j = e / QH, qh = e % QH;
    float M = b0;
    for (int c = 0; c < nch; ++c) M = fmaxf(M, part[((static_cast<int64_t>(j) * nch + c) * QH + qh) * (Dt + 2) + Dt]);
    float l = expf(b0 - M);
    for (int c = 0; c < nch; ++c) {
      const float* o = part + ((static_cast<int64_t>(j) * nch + c) * QH + qh) * (Dt + 2);
      const float f = expf(o[Dt] - M);
      l = fmaf(o[Dt + 1], f, l);
      scale_c[j][qh][c] = f;
    }
    for (int c = 0; c < nch; ++c) scale_c[j][qh][c] /= l;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < P * QD; e += 256) {
    const int j = e / QD, k = e % QD;
    const int qh = k / Dt, i = k % Dt;
    float u = 0.f;
    for (int c = 0; c < nch; ++c)
      u = fmaf(part[((static_cast<int64_t>(j) * nch + c) * QH + qh) * (Dt + 2) + i], scale_c[j][qh][c], u);
    us[j * QD + k] = u;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  for (int q = 0; q < 4; ++q) {
    const int o = blockIdx.x * 16 + w * 4 + q;
    if (o >= D.d) break;
    const float* wr = D.ov + static_cast<int64_t>(o) * QD;
    float acc[DR_MAXP];
#pragma unroll
    for (int j = 0; j < DR_MAXP; ++j) acc[j] = 0.f;
    for (int k = lane; k < QD; k += 64) {
      const float wv = wr[k];
#pragma unroll
      for (int j = 0; j < DR_MAXP; ++j)
        if (j < P) acc[j] = fmaf(wv, us[j * QD + k], acc[j]);
    }
#pragma unroll
    for (int j = 0; j < DR_MAXP; ++j) {
      if (j < P) {
        const float a = wave_sum(acc[j]);
        if (lane == 0) hid[static_cast<int64_t>(j) * D.d + o] = a;
      }
    }
  }
}

// logits[j, v] = E[v] . (RMSNorm(hid_j) * out_norm); per block and position: max, sum of
// exponentials and the block's top-k by (logit desc, index asc):
// lpart[(j * nblk + b) * (2 + 2K)] = {max, sumexp, K logits, K indices (as float bits)}
// Each wave scores four vocabulary rows at a time with 16-byte loads (d % 8 == 0; else one
// element per lane and load).  need (optional, [P]): the launch is skipped unless a position has
// need[j] != 0 (the shortlist left it to the whole vocabulary).
//                                                                   grid (cdiv(V, 64))
template <typename TE, int PM>
__global__ __launch_bounds__(256) void k_draft_logits(lng_drafter D, int32_t P, int32_t K,
                                                      const float* __restrict__ hid, float* __restrict__ logits,
                                                      float* __restrict__ lpart, const int32_t* __restrict__ need) {
  extern __shared__ __attribute__((aligned(16))) float hs[];  // [P][d]
  __shared__ float red[4];
  __shared__ float lt[DR_MAXP][DR_VB];
  if (need) {
    bool any = false;
    for (int j = 0; j < P; ++j) any = any || need[j] != 0;
    if (!any) return;
  }
  const int d = D.d;
  const int64_t V = D.V;
  for (int j = 0; j < P; ++j) {
    float ss = 0.f;
    for (int c = threadIdx.x; c < d; c += 256) {
      const float v = hid[static_cast<int64_t>(j) * d + c];
      hs[j * d + c] = v;
      ss = fmaf(v, v, ss);
    }
    ss = block_sum256(ss, red);
    const float r = 1.0f / sqrtf(ss / static_cast<float>(d) + D.draft_eps);
    for (int c = threadIdx.x; c < d; c += 256) hs[j * d + c] = hs[j * d + c] * r * D.out_norm[c];
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const TE* E = static_cast<const TE*>(D.emb);
  if (d % 8 == 0) {
    for (int q0 = 0; q0 < DR_VB / 4; q0 += 4) {
      const int vl0 = w * (DR_VB / 4) + q0;
      const int64_t v0 = static_cast<int64_t>(blockIdx.x) * DR_VB + vl0;
      float acc[4][PM];
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int jj = 0; jj < PM; ++jj) acc[u][jj] = 0.f;
      for (int c8 = lane; c8 < d / 8; c8 += 64) {
        f32x4 ea[4], eb[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if (v0 + u < V) {
            ld8f<TE>(E + (v0 + u) * d + 8 * c8, ea[u], eb[u]);
          } else {
            ea[u] = f32x4{0.f, 0.f, 0.f, 0.f};
            eb[u] = ea[u];
          }
        }
#pragma unroll
        for (int jj = 0; jj < PM; ++jj) {
          if (jj < P) {
            const f32x4 h0 = *reinterpret_cast<const f32x4*>(hs + jj * d + 8 * c8);
            const f32x4 h1 = *reinterpret_cast<const f32x4*>(hs + jj * d + 8 * c8 + 4);
#pragma unroll
            for (int u = 0; u < 4; ++u) acc[u][jj] = dot4(eb[u], h1, dot4(ea[u], h0, acc[u][jj]));
          }
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int vl = vl0 + u;
        const int64_t v = v0 + u;
#pragma unroll
        for (int jj = 0; jj < PM; ++jj) {
          if (jj >= P) continue;
          const float a = wave_sum(acc[u][jj]);
          if (lane == 0) {
            lt[jj][vl] = v < V ? a : -INFINITY;
            if (v < V) logits[static_cast<int64_t>(jj) * V + v] = a;
          }
        }
      }
    }
  } else {
    for (int q = 0; q < DR_VB / 4; ++q) {
      const int vl = w * (DR_VB / 4) + q;
      const int64_t v = static_cast<int64_t>(blockIdx.x) * DR_VB + vl;
      if (v >= V) {
        if (lane < DR_MAXP) lt[lane][vl] = -INFINITY;
        continue;
      }
      float acc[PM];
#pragma unroll
      for (int jj = 0; jj < PM; ++jj) acc[jj] = 0.f;
      for (int c = lane; c < d; c += 64) {
        const float ev = to_f32(E[v * d + c]);
#pragma unroll
        for (int jj = 0; jj < PM; ++jj)
          if (jj < P) acc[jj] = fmaf(ev, hs[jj * d + c], acc[jj]);
      }
#pragma unroll
      for (int jj = 0; jj < PM; ++jj) {
        if (jj < P) {
          const float a = wave_sum(acc[jj]);
          if (lane == 0) {
            lt[jj][vl] = a;
            logits[static_cast<int64_t>(jj) * V + v] = a;
          }
        }
      }
    }
  }
  __syncthreads();
  // wave w summarises positions w, w+4, ...
  const int nblk = gridDim.x;
  for (int j = w; j < P; j += 4) {
    const float x = lt[j][lane];
    const float m = wave_max(x);
    const float s = wave_sum(x == -INFINITY ? 0.f : expf(x - m));
    float* o = lpart + (static_cast<int64_t>(j) * nblk + blockIdx.x) * (2 + 2 * K);
    if (lane == 0) {
      o[0] = m;
      o[1] = s;
    }
    // top-K by (value desc, index asc) with K wave argmax rounds
    float cur = x;
    const int idx = static_cast<int>(blockIdx.x) * DR_VB + lane;
    for (int k = 0; k < K; ++k) {
      float bv = cur;
      int bi = cur == -INFINITY ? INT_MAX : idx;
      for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        if (ov > bv || (ov == bv && oi < bi)) {
          bv = ov;
          bi = oi;
        }
      }
      if (lane == 0) {
        o[2 + k] = bi == INT_MAX ? -INFINITY : bv;
        o[2 + K + k] = __int_as_float(bi == INT_MAX ? -1 : bi);
      }
      if (idx == bi) cur = -INFINITY;
    }
  }
}

// Online counts: w[j, t] = sum over orders and routes of [key row at pair t == query row of j]
// for pairs t = 0 .. L-2 (row at t, token t+1); sc[j, tokens[t+1]] += w.
//                                                 grid (cdiv(max pairs, 32), P), block = 256 (routes)
__global__ __launch_bounds__(256) void k_draft_online_match(lng_drafter D, DrWin W, int32_t* __restrict__ wout,
                                                            int32_t* __restrict__ sc, int32_t ld_w) {
  __shared__ int32_t slot_rows[DR_MAXN];
  __shared__ int32_t qaddr[4][256];
  __shared__ int32_t red[4][DR_TB];
  const int j = blockIdx.y;
  const int L = *D.length;
  const int npairs = L - 1;
  const int t0 = blockIdx.x * DR_TB;
  if (t0 >= npairs) return;
  if (threadIdx.x < DR_MAXN) slot_rows[threadIdx.x] = threadIdx.x < D.maxn ? dr_resolve(W.slot[j][threadIdx.x], L) : -1;
  __syncthreads();
  const int r = threadIdx.x;
  const bool rv = r < D.R;
  for (int oi = 0; oi < D.n_orders; ++oi) {
    const int64_t q = rv ? dr_row(D, slot_rows, oi, r) : -1;
    qaddr[oi][r] = q < 0 ? -1 : static_cast<int32_t>(q - static_cast<int64_t>(r) * (int64_t{1} << (D.bits * D.orders[oi])));
  }
  __syncthreads();
  // sliding window of the last maxn codes of route r ending at t
  int32_t win[DR_MAXN];
  for (int k = 0; k < DR_MAXN; ++k) {
    const int t = t0 - (D.maxn - 1) + k;
    win[k] = (rv && k < D.maxn && t >= 0) ? (D.codes[static_cast<int64_t>(t) * D.R + r] & ((1 << D.bits) - 1)) : 0;
  }
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  for (int tt = 0; tt < DR_TB; ++tt) {
    const int t = t0 + tt;
    if (t >= npairs) break;
    if (tt > 0) {
      for (int k = 0; k + 1 < DR_MAXN; ++k) win[k] = win[k + 1];
      win[D.maxn - 1] = rv ? (D.codes[static_cast<int64_t>(t) * D.R + r] & ((1 << D.bits) - 1)) : 0;
    }
    int m = 0;
    for (int oi = 0; oi < D.n_orders; ++oi) {
      const int n = D.orders[oi];
      if (t < n - 1) continue;
      int32_t addr = 0;
      for (int k = 0; k < n; ++k) addr |= win[D.maxn - n + k] << (k * D.bits);
      m += (rv && qaddr[oi][r] >= 0 && qaddr[oi][r] == addr) ? 1 : 0;
    }
    // sum over routes
    int s = m;
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if (lane == 0) red[w][tt] = s;
  }
  __syncthreads();
  if (threadIdx.x < DR_TB) {
    const int t = t0 + threadIdx.x;
    if (t < npairs) {
      const int s = (red[0][threadIdx.x] + red[1][threadIdx.x]) + (red[2][threadIdx.x] + red[3][threadIdx.x]);
      wout[static_cast<int64_t>(j) * ld_w + t] = s;
      if (s > 0) atomicAdd(&sc[static_cast<int64_t>(j) * D.V + D.tokens[t + 1]], s);
    }
  }
}

// Select the top-K of position j (grid (P), 256 threads): by logit, or with online counts by the
// mixed probability p = (1 - lam) softmax + lam sc / tot (scores reported as log p).  Writes
// ids/scores [P, K] and the children's tokens; restores sc to zero.
__global__ __launch_bounds__(256) void k_draft_select(lng_drafter D, int32_t K, int32_t nblk, int32_t online,
                                                      float kappa, const float* __restrict__ logits,
                                                      const float* __restrict__ lpart, const int32_t* __restrict__ w,
                                                      int32_t ld_w, int32_t* __restrict__ sc, DrChildren C,
                                                      int64_t* __restrict__ ids, float* __restrict__ scores,
                                                      const int32_t* __restrict__ need) {
  __shared__ float redf[4];
  __shared__ float bvs[4];
  __shared__ int bis[4];
  __shared__ int64_t sel_id[DR_MAXK];
  __shared__ float sel_sc[DR_MAXK];
  const int j = blockIdx.x;
  if (need && !need[j]) return;  // the shortlist drafted this position
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const float* lp = lpart + static_cast<int64_t>(j) * nblk * (2 + 2 * K);
  // global max and sum of exponentials
  float m = -INFINITY;
  for (int b = threadIdx.x; b < nblk; b += 256) m = fmaxf(m, lp[b * (2 + 2 * K)]);
  m = wave_max(m);
  __syncthreads();
  if (lane == 0) redf[wv] = m;
  __syncthreads();
  const float M = fmaxf(fmaxf(redf[0], redf[1]), fmaxf(redf[2], redf[3]));
  float s = 0.f;
  for (int b = threadIdx.x; b < nblk; b += 256) s += lp[b * (2 + 2 * K)] == -INFINITY ? 0.f : lp[b * (2 + 2 * K) + 1] * expf(lp[b * (2 + 2 * K)] - M);
  const float S = block_sum256(s, redf);
  // online counts: total weight and mixing factor
  const int L = *D.length;
  const int npairs = online ? L - 1 : 0;
  float tot = 0.f;
  if (online) {
    int ti = 0;
    for (int t = threadIdx.x; t < npairs; t += 256) ti += w[static_cast<int64_t>(j) * ld_w + t];
    tot = block_sum256(static_cast<float>(ti), redf);
  }
  const bool mix = online != 0;
  const float n_eff = tot / static_cast<float>(D.R * D.n_orders);
  const float lam = tot > 0.f ? n_eff / (n_eff + kappa) : 0.f;
  int32_t* scj = sc + static_cast<int64_t>(j) * D.V;
  const float* lgj = logits + static_cast<int64_t>(j) * D.V;
  // score of token v: log of the mixed probability (online) or the logit
  auto score_of = [&](int64_t v, float cnt) {
    if (!mix) return lgj[v];
    const float p = (1.f - lam) * expf(lgj[v] - M) / S + (tot > 0.f ? lam * cnt / tot : 0.f);
    return logf(p);
  };
  // candidates A: the blocks' top-K entries by logit (tokens with online counts are taken by
  // their owner below); read every count before any is cleared
  constexpr int PER = 16;
  float a_val[PER];
  int64_t a_id[PER];
  int na = 0, overflow = 0;
  const int nA = nblk * K;
  for (int e = threadIdx.x; e < nA; e += 256) {
    const int b = e / K, k = e % K;
    const int id = __float_as_int(lp[b * (2 + 2 * K) + 2 + K + k]);
    if (id < 0) continue;
    if (mix && scj[id] > 0) continue;
    if (na == PER) {
      overflow = 1;
      break;
    }
    a_val[na] = mix ? score_of(id, 0.f) : lp[b * (2 + 2 * K) + 2 + k];
    a_id[na] = id;
    ++na;
  }
  __syncthreads();
  // candidates B: one owner per online token (the exchange that sees the count), which also
  // returns the count buffer to zero
  float o_val[PER];
  int64_t o_id[PER];
  int no = 0;
  if (mix) {
    for (int t = threadIdx.x; t < npairs; t += 256) {
      if (w[static_cast<int64_t>(j) * ld_w + t] <= 0) continue;
      const int64_t v = D.tokens[t + 1];
      const int cnt = atomicExch(&scj[v], 0);
      if (cnt <= 0) continue;
      if (no == PER) {
        overflow = 1;
        continue;
      }
      o_val[no] = score_of(v, static_cast<float>(cnt));
      o_id[no] = v;
      ++no;
    }
  }
  // K rounds of block argmax by (score desc, id asc) over this thread's candidates
  for (int k = 0; k < K; ++k) {
    float bv = -INFINITY;
    int64_t bi = INT64_MAX;
    for (int e = 0; e < na; ++e)
      if (a_val[e] > bv || (a_val[e] == bv && a_id[e] < bi)) {
        bv = a_val[e];
        bi = a_id[e];
      }
    for (int e = 0; e < no; ++e)
      if (o_val[e] > bv || (o_val[e] == bv && o_id[e] < bi)) {
        bv = o_val[e];
        bi = o_id[e];
      }
    for (int off = 32; off > 0; off >>= 1) {
      const float ov = __shfl_xor(bv, off, 64);
      const int64_t oi = __shfl_xor(bi, off, 64);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
    __syncthreads();
    if (lane == 0) {
      bvs[wv] = bv;
      bis[wv] = static_cast<int>(bi == INT64_MAX ? INT_MAX : bi);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      float v = bvs[0];
      int i = bis[0];
      for (int q = 1; q < 4; ++q)
        if (bvs[q] > v || (bvs[q] == v && bis[q] < i)) {
          v = bvs[q];
          i = bis[q];
        }
      sel_id[k] = i == INT_MAX ? -1 : i;
      sel_sc[k] = i == INT_MAX ? -INFINITY : v;
    }
    __syncthreads();
    const int64_t win_id = sel_id[k];
    for (int e = 0; e < na; ++e)
      if (a_id[e] == win_id) a_val[e] = -INFINITY, a_id[e] = INT64_MAX;
    for (int e = 0; e < no; ++e)
      if (o_id[e] == win_id) o_val[e] = -INFINITY, o_id[e] = INT64_MAX;
  }
  if (threadIdx.x < K) {
    ids[static_cast<int64_t>(j) * K + threadIdx.x] = sel_id[threadIdx.x];
    scores[static_cast<int64_t>(j) * K + threadIdx.x] = sel_sc[threadIdx.x];
  }
  if (overflow && threadIdx.x == 0) ids[static_cast<int64_t>(j) * K] = -2;  // host reports the overflow
  for (int e = threadIdx.x; e < C.n; e += 256) {
    if (C.parent[e] != j) continue;
    const int64_t t = sel_id[C.rank[e]];
    D.tokens[C.row[e]] = t >= 0 ? t : sel_id[0];
  }
}

// ------------------------------------------------------------------ sketch shortlist
// RefDrafter._shortlist + _readout (cpu_drafter.py:179-206, :238-244; drafter.cpp:438-474): the
// candidates of a position are the tokens of its rows' count-sketch slots (every order with a
// sketch, every route), each with its counts summed over the slots that name it; ordered by
// (total desc, id asc) and cut to `cap`, then padded with the fallback tokens not yet present, in
// their order.  The drafts are the top-k of the candidates' logits, ties in candidate order (a
// stable descending sort); an empty list scores the whole vocabulary.  One block per position:
// the slots (n_orders * R * K <= 8192) are summed per token in an LDS hash table (open addressing
// keyed by token id, 64-bit totals, 2^tbits >= n_orders * R * K slots).  The list is cut by an
// exact radix select, 8 bits per pass from the top, on the key total << idbits | (2^idbits - 1 -
// id): it orders like (total desc, id asc) and is unique per token, so the keys at or above the
// selected threshold are exactly the list, which is then ranked.  Totals too wide for that key
// (above 2^(64 - idbits)) take the list one maximum at a time instead.
constexpr int SL_SLOTS = 8192;
constexpr int SL_MAXCAP = 256;
constexpr int SL_MAXFB = 1024;
constexpr int SL_MAXR = 256;
constexpr int SL_LOADS = 24;  // sketch slots each thread has in flight
constexpr int32_t SL_EMPTY = -1;
constexpr int32_t SL_TAKEN = 0x40000000;  // flag on a slot's id once the token is in the list

struct SlArgs {
  const int32_t* ids[DR_MAXN];     // per order index: [R * 2^(bits*n), K] token ids (null: no sketch)
  const int64_t* counts[DR_MAXN];  // same shape: counts (0 = empty slot)
  const int32_t* fallback;
  int32_t K, cap, n_fallback;
  int32_t tbits;                   // log2 of the hash table's slots (8 .. 13)
};

// Probe sequence of a token: start sl_hash, step sl_step (odd, so it visits every slot of the
// power-of-two table); double hashing keeps the probe chains short at load factors near 0.7.
__device__ __forceinline__ uint32_t sl_hash(int32_t id, int tbits) {
  return (static_cast<uint32_t>(id) * 2654435761u) >> (32 - tbits);
}
__device__ __forceinline__ uint32_t sl_step(int32_t id, int tbits) {
  return ((static_cast<uint32_t>(id) * 0x85EBCA6Bu) >> (32 - tbits)) | 1u;
}

// (total, id) a beats (total b, id b): larger total, then smaller id
__device__ __forceinline__ bool sl_better(unsigned long long ta, int32_t ia, unsigned long long tb, int32_t ib) {
  return ta > tb || (ta == tb && ia < ib);
}

// Eight consecutive row elements in their storage form (one or two 16-byte loads), converted
// when used.
template <typename T>
struct Raw8;
template <>
struct Raw8<bf16> {
  u32x4 v;
  __device__ __forceinline__ void load(const bf16* p) { v = *reinterpret_cast<const u32x4*>(p); }
  __device__ __forceinline__ void zero() { v = u32x4{0u, 0u, 0u, 0u}; }
  __device__ __forceinline__ void get(f32x4& a, f32x4& b) const {
    a = bf2f4(v.x, v.y);
    b = bf2f4(v.z, v.w);
  }
};
template <>
struct Raw8<_Float16> {
  u32x4 v;
  __device__ __forceinline__ void load(const _Float16* p) { v = *reinterpret_cast<const u32x4*>(p); }
  __device__ __forceinline__ void zero() { v = u32x4{0u, 0u, 0u, 0u}; }
  __device__ __forceinline__ void get(f32x4& a, f32x4& b) const {
    a = h2f4(v.x, v.y);
    b = h2f4(v.z, v.w);
  }
};
template <>
struct Raw8<float> {
  f32x4 x, y;
  __device__ __forceinline__ void load(const float* p) {
    x = reinterpret_cast<const f32x4*>(p)[0];
    y = reinterpret_cast<const f32x4*>(p)[1];
  }
  __device__ __forceinline__ void zero() {
    x = f32x4{0.f, 0.f, 0.f, 0.f};
    y = x;
  }
  __device__ __forceinline__ void get(f32x4& a, f32x4& b) const {
    a = x;
    b = y;
  }
};

// Logits of candidates ids[0 .. n) against the normalised hidden state hn (LDS, d floats, d % 8
// == 0, d / 8 <= 64 * CPL): wave w scores rows w*G .. w*G+G-1 (then 4G further on) with every
// row's loads (CPL 16-byte pieces per lane) issued before the first product, so a group of
// candidates costs one memory round trip.
template <typename TE, int CPL>
__device__ void sl_score(const lng_drafter& D, const int32_t* ids, int n, const float* hn, float* out) {
  constexpr int G = (sizeof(TE) == 4 ? 16 : 32) / CPL;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int d = D.d, d8 = d >> 3;
  const TE* E = static_cast<const TE*>(D.emb);
  f32x4 h0[CPL], h1[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int c8 = lane + 64 * c;
    h0[c] = c8 < d8 ? *reinterpret_cast<const f32x4*>(hn + 8 * c8) : f32x4{0.f, 0.f, 0.f, 0.f};
    h1[c] = c8 < d8 ? *reinterpret_cast<const f32x4*>(hn + 8 * c8 + 4) : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  for (int i0 = w * G; i0 < n; i0 += 4 * G) {
    Raw8<TE> raw[G][CPL];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int32_t id = i0 + g < n ? ids[i0 + g] : -1;
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const int c8 = lane + 64 * c;
        if (id >= 0 && c8 < d8)
          raw[g][c].load(E + static_cast<int64_t>(id) * d + 8 * c8);
        else
          raw[g][c].zero();
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float acc = 0.f;
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        f32x4 a, b;
        raw[g][c].get(a, b);
        acc = dot4(b, h1[c], dot4(a, h0[c], acc));
      }
      const float sum = wave_sum(acc);
      if (lane == 0 && i0 + g < n) out[i0 + g] = ids[i0 + g] >= 0 ? sum : -INFINITY;
    }
  }
}

// The candidate list of position j (RefDrafter._shortlist): sl[0 .. n) in LDS, n returned (0: empty
// list).  Called by every thread of a 256-thread block; the hash table and selection state are
// this function's own LDS.
__device__ int sl_build(const lng_drafter& D, const DrWin& W, const SlArgs& S, int j, int32_t* sl) {
  __shared__ __attribute__((aligned(16))) int32_t hkey[SL_SLOTS];
  __shared__ __attribute__((aligned(16))) unsigned long long hval[SL_SLOTS];
  __shared__ int64_t rowsh[DR_MAXN * SL_MAXR];  // per (order, route): first element of the sketch row
  __shared__ int32_t fb[SL_MAXFB];
  __shared__ unsigned long long selk[SL_MAXCAP];
  __shared__ int32_t hist[256];
  __shared__ int32_t slot_rows[DR_MAXN];
  __shared__ const int32_t* idp[DR_MAXN];
  __shared__ const int64_t* cnp[DR_MAXN];
  __shared__ unsigned long long red_t[4];
  __shared__ int32_t red_i[4], red_s[4];
  __shared__ int32_t rad[4];  // selected digit, keys above it, keys in it; list length
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int L = *D.length;
  const int R = D.R, SK = S.K, cap = S.cap, tb = S.tbits, TS = 1 << tb, TM = TS - 1;
  for (int e = 4 * tid; e < TS; e += 1024) {
    *reinterpret_cast<int4*>(&hkey[e]) = int4{SL_EMPTY, SL_EMPTY, SL_EMPTY, SL_EMPTY};
    *reinterpret_cast<ulonglong2*>(&hval[e]) = ulonglong2{0ull, 0ull};
    *reinterpret_cast<ulonglong2*>(&hval[e + 2]) = ulonglong2{0ull, 0ull};
  }
  for (int e = tid; e < S.n_fallback; e += 256) fb[e] = S.fallback[e];
  if (tid < DR_MAXN) slot_rows[tid] = tid < D.maxn ? dr_resolve(W.slot[j][tid], L) : -1;
  if (tid == 0) {
#pragma unroll
    for (int o = 0; o < DR_MAXN; ++o) {
      idp[o] = S.ids[o];
      cnp[o] = S.counts[o];
    }
  }
  __syncthreads();
  for (int e = tid; e < D.n_orders * R; e += 256) {
    const int o = e / R, r = e % R;
    const int64_t row = idp[o] ? dr_row(D, slot_rows, o, r) : -1;
    rowsh[e] = row >= 0 ? row * SK : -1;
  }
  __syncthreads();
  // sum the counts per token, SL_LOADS slots in flight per thread (at most TS distinct tokens:
  // every probe sequence ends); slot e is element e % K of sketch row e / K (order, route)
  const int M = D.n_orders * R * SK;
  const bool k_pow2 = (SK & (SK - 1)) == 0;
  const int k_shift = __ffs(SK) - 1;
  for (int e0 = 0; e0 < M; e0 += 256 * SL_LOADS) {
    int32_t idv[SL_LOADS];
    int64_t cv[SL_LOADS];
#pragma unroll
    for (int u = 0; u < SL_LOADS; ++u) {
      const int e = e0 + u * 256 + tid;
      idv[u] = -1;
      cv[u] = 0;
      if (e < M) {
        const int rr = k_pow2 ? e >> k_shift : e / SK;
        const int q = e - rr * SK;
        const int o = (rr >= R) + (rr >= 2 * R) + (rr >= 3 * R);
        const int64_t base = rowsh[rr];
        if (base >= 0) {
          cv[u] = cnp[o][base + q];
          idv[u] = idp[o][base + q];
        }
      }
    }
#pragma unroll
    for (int u = 0; u < SL_LOADS; ++u) {
      const int32_t id = idv[u];
      if (cv[u] <= 0 || id < 0 || id >= D.V) continue;
      uint32_t h = sl_hash(id, tb);
      const uint32_t st = sl_step(id, tb);
      bool placed = false;
      for (int p = 0; p < TS && !placed; ++p) {  // a free or matching slot always exists (TS >= M)
        const int32_t prev = atomicCAS(&hkey[h], SL_EMPTY, id);
        placed = prev == SL_EMPTY || prev == id;
        if (!placed) h = (h + st) & TM;
      }
      if (placed) atomicAdd(&hval[h], static_cast<unsigned long long>(cv[u]));
    }
  }
  __syncthreads();
  // the list: every slot's (id, total) into registers once (thread tid owns slots 1024 g + 4 tid
  // .. +3, read 16 bytes at a time); distinct tokens and largest total
  constexpr int KQ = SL_SLOTS / 256;
  int32_t kid[KQ];
  unsigned long long key[KQ];
  unsigned long long tmax = 0ull;
  int cnt = 0;
#pragma unroll
  for (int g = 0; g < KQ / 4; ++g) {
    const int e = (g << 10) + 4 * tid;
    int4 k4 = int4{SL_EMPTY, SL_EMPTY, SL_EMPTY, SL_EMPTY};
    ulonglong2 t01 = ulonglong2{0ull, 0ull}, t23 = t01;
    if (e < TS) {
      k4 = *reinterpret_cast<const int4*>(&hkey[e]);
      t01 = *reinterpret_cast<const ulonglong2*>(&hval[e]);
      t23 = *reinterpret_cast<const ulonglong2*>(&hval[e + 2]);
    }
    kid[4 * g] = k4.x;
    kid[4 * g + 1] = k4.y;
    kid[4 * g + 2] = k4.z;
    kid[4 * g + 3] = k4.w;
    key[4 * g] = t01.x;
    key[4 * g + 1] = t01.y;
    key[4 * g + 2] = t23.x;
    key[4 * g + 3] = t23.y;
  }
#pragma unroll
  for (int q = 0; q < KQ; ++q) {
    if (kid[q] < 0) key[q] = 0ull;
    tmax = key[q] > tmax ? key[q] : tmax;
    cnt += kid[q] >= 0 ? 1 : 0;
  }
  for (int off = 32; off >= 1; off >>= 1) {
    const unsigned long long ot = __shfl_xor(tmax, off, 64);
    tmax = ot > tmax ? ot : tmax;
    cnt += __shfl_xor(cnt, off, 64);
  }
  if (lane == 0) {
    red_t[w] = tmax;
    red_i[w] = cnt;
  }
  __syncthreads();
  tmax = red_t[0];
  cnt = red_i[0];
  for (int q = 1; q < 4; ++q) {
    tmax = red_t[q] > tmax ? red_t[q] : tmax;
    cnt += red_i[q];
  }
  const int ib = D.V > 1 ? 32 - __clz(D.V - 1) : 1;  // bits of a token id
  const int nb = (tmax ? 64 - __clzll(static_cast<long long>(tmax)) : 0) + ib;
  int m = 0;
  if (nb <= 64) {
    const unsigned long long vmask = (1ull << ib) - 1ull;
#pragma unroll
    for (int q = 0; q < KQ; ++q)
      key[q] = kid[q] >= 0 ? (key[q] << ib) | (vmask - static_cast<unsigned long long>(kid[q])) : 0ull;
    const int want = min(cap, cnt);
    unsigned long long thr = ~0ull;
    if (want > 0) {
      // passes of at most 8 bits from the top, none straddling the total / id boundary: the total
      // passes see few distinct digits (one atomic per distinct digit and wave), the id passes
      // spread over the bins
      unsigned long long prefix = 0ull, pmask = 0ull;
      int rem = want;  // keys still to take among those matching prefix
      int hi = nb;
      for (;;) {
        const int lo = hi > ib ? ib : 0;
        const int width = min(8, hi - lo), shift = hi - width;
        const unsigned long long dm = (1ull << width) - 1ull;
        hist[tid] = 0;
        __syncthreads();
        if (shift >= ib && width <= 3) {
          // a pass over the totals sees few distinct digits: counted per wave with ballots
          int c8[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
          for (int q = 0; q < KQ; ++q) {
            const unsigned long long k = key[q];
            const int dg = (k && (k & pmask) == prefix) ? static_cast<int>((k >> shift) & dm) : -1;
#pragma unroll
            for (int t = 0; t < 8; ++t) c8[t] += __popcll(__ballot(dg == t));
          }
          int mine = 0;
#pragma unroll
          for (int t = 0; t < 8; ++t) mine = lane == t ? c8[t] : mine;
          if (lane < 8 && mine) atomicAdd(&hist[lane], mine);
        } else {
#pragma unroll
          for (int q = 0; q < KQ; ++q) {
            const unsigned long long k = key[q];
            if (k && (k & pmask) == prefix) atomicAdd(&hist[static_cast<int>((k >> shift) & dm)], 1);
          }
        }
        __syncthreads();
        if (w == 0) {
          // lane l holds bins 4l .. 4l+3; suf = keys in bins >= 4l (non-increasing in l)
          const int h0 = hist[4 * lane], h1 = hist[4 * lane + 1], h2 = hist[4 * lane + 2], h3 = hist[4 * lane + 3];
          const int s4 = (h0 + h1) + (h2 + h3);
          int suf = s4;
          for (int off = 1; off < 64; off <<= 1) {
            const int t = __shfl_down(suf, off, 64);
            if (lane + off < 64) suf += t;
          }
          const unsigned long long bal = __ballot(suf >= rem);
          const int ls = 63 - __clzll(static_cast<long long>(bal));
          if (lane == ls) {
            int above = suf - s4, b = 4 * lane + 3, hb = h3;
            if (above + h3 < rem) {
              above += h3;
              b = 4 * lane + 2;
              hb = h2;
              if (above + h2 < rem) {
                above += h2;
                b = 4 * lane + 1;
                hb = h1;
                if (above + h1 < rem) {
                  above += h1;
                  b = 4 * lane;
                  hb = h0;
                }
              }
            }
            rad[0] = b;
            rad[1] = above;
            rad[2] = hb;
          }
        }
        __syncthreads();
        rem -= rad[1];
        prefix |= static_cast<unsigned long long>(rad[0]) << shift;
        pmask |= dm << shift;
        if (rad[2] == rem || shift == 0) {  // every key in the digit's bin is taken
          thr = prefix;
          break;
        }
        hi = shift;
      }
    }
    if (tid == 0) rad[3] = 0;
    __syncthreads();
#pragma unroll
    for (int q = 0; q < KQ; ++q) {
      const unsigned long long k = key[q];
      if (k && k >= thr) {
        const int pos = atomicAdd(&rad[3], 1);  // keys are unique: exactly `want` pass
        if (pos < SL_MAXCAP) selk[pos] = k;
        hkey[((q >> 2) << 10) + 4 * tid + (q & 3)] |= SL_TAKEN;
      }
    }
    __syncthreads();
    m = min(rad[3], cap);
    for (int i = tid; i < m; i += 256) {
      const unsigned long long k = selk[i];
      int rank = 0;
      for (int i2 = 0; i2 < m; ++i2) rank += selk[i2] > k ? 1 : 0;
      sl[rank] = static_cast<int32_t>(vmask - (k & vmask));
    }
  } else {
    // one maximum of (total desc, id asc) at a time
    for (; m < cap; ++m) {
      unsigned long long bt = 0ull;
      int32_t bi = INT_MAX, bs = -1;
      for (int e = tid; e < TS; e += 256) {
        const int32_t k = hkey[e];
        if (k < 0 || (k & SL_TAKEN)) continue;
        if (sl_better(hval[e], k, bt, bi)) {
          bt = hval[e];
          bi = k;
          bs = e;
        }
      }
      for (int off = 32; off >= 1; off >>= 1) {
        const unsigned long long ot = __shfl_xor(bt, off, 64);
        const int32_t oi = __shfl_xor(bi, off, 64), os = __shfl_xor(bs, off, 64);
        if (sl_better(ot, oi, bt, bi)) {
          bt = ot;
          bi = oi;
          bs = os;
        }
      }
      if (lane == 0) {
        red_t[w] = bt;
        red_i[w] = bi;
        red_s[w] = bs;
      }
      __syncthreads();
      bt = red_t[0];
      bi = red_i[0];
      bs = red_s[0];
      for (int q = 1; q < 4; ++q)
        if (sl_better(red_t[q], red_i[q], bt, bi)) {
          bt = red_t[q];
          bi = red_i[q];
          bs = red_s[q];
        }
      __syncthreads();
      if (bs < 0) break;  // no candidate left (uniform)
      if (tid == 0) {
        sl[m] = bi;
        hkey[bs] = bi | SL_TAKEN;
      }
      __syncthreads();
    }
  }
  __syncthreads();
  // fallback padding: first occurrences not in the list, in order
  int added = 0;
  for (int f0 = 0; f0 < S.n_fallback && m + added < cap; f0 += 256) {
    const int jf = f0 + tid;
    bool ok = false;
    int32_t f = -1;
    if (jf < S.n_fallback) {
      f = fb[jf];
      ok = f >= 0 && f < D.V;
      if (ok) {
        uint32_t h = sl_hash(f, tb);
        const uint32_t st = sl_step(f, tb);
        for (int p = 0; p < TS; ++p) {  // a full table has no empty slot to end on
          const int32_t k = hkey[h];
          if (k == SL_EMPTY) break;
          if ((k & ~SL_TAKEN) == f) {
            ok = !(k & SL_TAKEN);
            break;
          }
          h = (h + st) & TM;
        }
      }
      for (int i = 0; ok && i < jf; ++i) ok = fb[i] != f;
    }
    const unsigned long long bal = __ballot(ok);
    const int before = __popcll(bal & ((1ull << lane) - 1ull));
    if (lane == 0) red_s[w] = __popcll(bal);
    __syncthreads();
    int base = 0, tot = 0;
    for (int q = 0; q < 4; ++q) {
      base += q < w ? red_s[q] : 0;
      tot += red_s[q];
    }
    if (ok) {
      const int pos = m + added + base + before;
      if (pos < cap) sl[pos] = f;
    }
    added += tot;
    __syncthreads();
  }
  return min(cap, m + added);
}

// top-K of the candidates sl[0 .. n) by (logit sll desc, candidate index asc), by wave 0, into
// sel_id / sel_sc (-1 / -inf past the list)
__device__ void sl_topk(const int32_t* sl, const float* sll, int n, int K, int64_t* sel_id, float* sel_sc) {
  const int lane = threadIdx.x & 63;
  if (threadIdx.x >= 64) return;
  constexpr int NQ = SL_MAXCAP / 64;
  float v[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) v[q] = lane + 64 * q < n ? sll[lane + 64 * q] : 0.f;
  unsigned used = 0u;
  for (int k = 0; k < K; ++k) {
    float bv = -INFINITY;
    int bi = INT_MAX;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int i = lane + 64 * q;
      if (i >= n || ((used >> q) & 1u)) continue;
      if (v[q] > bv || (v[q] == bv && i < bi)) {
        bv = v[q];
        bi = i;
      }
    }
    for (int off = 32; off >= 1; off >>= 1) {
      const float ov = __shfl_xor(bv, off, 64);
      const int oi = __shfl_xor(bi, off, 64);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if (bi != INT_MAX && (bi & 63) == lane) used |= 1u << (bi >> 6);
    if (lane == 0) {
      sel_id[k] = bi == INT_MAX ? -1 : sl[bi];
      sel_sc[k] = bi == INT_MAX ? -INFINITY : bv;
    }
  }
}

// ids / scores [P, K] and the children's tokens from the selected drafts of position j
__device__ void sl_write(const lng_drafter& D, int j, int K, const DrChildren& C, const int64_t* sel_id,
                         const float* sel_sc, int64_t* ids, float* scores) {
  const int tid = threadIdx.x;
  if (tid < K) {
    ids[static_cast<int64_t>(j) * K + tid] = sel_id[tid];
    scores[static_cast<int64_t>(j) * K + tid] = sel_sc[tid];
  }
  for (int e = tid; e < C.n; e += 256) {
    if (C.parent[e] != j) continue;
    const int64_t t = sel_id[C.rank[e]];
    D.tokens[C.row[e]] = t >= 0 ? t : sel_id[0];
  }
}

// The shortlist drafts of P positions given their full-vocabulary logits [P, V] and top-k: the
// candidates' logits are read from the logits; an empty list keeps the full-vocabulary top-k
// (full_ids / full_sc).                                            grid (P)
__global__ __launch_bounds__(256) void k_draft_shortlist(lng_drafter D, DrWin W, SlArgs S,
                                                         const float* __restrict__ logits,
                                                         const int64_t* __restrict__ full_ids,
                                                         const float* __restrict__ full_sc, int32_t K, DrChildren C,
                                                         int64_t* __restrict__ ids, float* __restrict__ scores,
                                                         int32_t* __restrict__ sl_out, float* __restrict__ sll_out) {
  __shared__ int32_t sl[SL_MAXCAP];
  __shared__ float sll[SL_MAXCAP];
  __shared__ int64_t sel_id[DR_MAXK];
  __shared__ float sel_sc[DR_MAXK];
  const int j = blockIdx.x, tid = threadIdx.x, cap = S.cap;
  const int n_sl = sl_build(D, W, S, j, sl);
  const float* lg = logits + static_cast<int64_t>(j) * D.V;
  for (int i = tid; i < cap; i += 256) {
    int32_t id = -1;
    if (n_sl > 0)
      id = i < n_sl ? sl[i] : -1;
    else
      id = i < D.V ? i : -1;  // empty list: the whole vocabulary, cut to cap
    const float v = id >= 0 ? lg[id] : -INFINITY;
    sll[i] = v;
    if (sl_out) sl_out[static_cast<int64_t>(j) * cap + i] = id;
    if (sll_out) sll_out[static_cast<int64_t>(j) * cap + i] = v;
  }
  __syncthreads();
  if (n_sl == 0) {
    if (tid < K) {
      sel_id[tid] = full_ids[static_cast<int64_t>(j) * K + tid];
      sel_sc[tid] = full_sc[static_cast<int64_t>(j) * K + tid];
    }
  } else {
    sl_topk(sl, sll, n_sl, K, sel_id, sel_sc);
  }
  __syncthreads();
  sl_write(D, j, K, C, sel_id, sel_sc, ids, scores);
}

// The drafts of P positions scored over their candidate lists from the readout's hidden states:
// lists [P][1 + cap] (length, then the ids, as the attention launch's list blocks wrote them),
// hid [P, d] (RMSNorm * out_norm, then E[id] . h).  A position with an empty list gets
// need_full[j] = 1 and no drafts (the full-vocabulary kernels that follow write them), every other
// position need_full[j] = 0.  shortlist / shortlist_logits (optional): as lng_drafter_shortlist
// (an empty list reports tokens 0 .. cap-1 with their logits).          grid (P)
template <typename TE>
__global__ __launch_bounds__(256) void k_sl_score(lng_drafter D, int32_t cap, const int32_t* __restrict__ lists,
                                                  const float* __restrict__ hid, int32_t K, DrChildren C,
                                                  int64_t* __restrict__ ids, float* __restrict__ scores,
                                                  int32_t* __restrict__ sl_out, float* __restrict__ sll_out,
                                                  int32_t* __restrict__ need_full) {
  __shared__ int32_t sl[SL_MAXCAP];
  __shared__ float sll[SL_MAXCAP];
  __shared__ int64_t sel_id[DR_MAXK];
  __shared__ float sel_sc[DR_MAXK];
  __shared__ float red_f[4];
  __shared__ __attribute__((aligned(16))) float hn[LNG_DR_MAX_D];
  const int j = blockIdx.x, tid = threadIdx.x, d = D.d;
  constexpr int HQ = LNG_DR_MAX_D / 256;
  float hv[HQ], gv[HQ];
#pragma unroll
  for (int q = 0; q < HQ; ++q) {
    const int c = tid + 256 * q;
    hv[q] = c < d ? hid[static_cast<int64_t>(j) * d + c] : 0.f;
    gv[q] = c < d ? D.out_norm[c] : 0.f;
  }
  const int32_t* lj = lists + static_cast<int64_t>(j) * (cap + 1);
  const int n_sl = min(cap, max(0, lj[0]));
  float ss = 0.f;
#pragma unroll
  for (int q = 0; q < HQ; ++q) ss = fmaf(hv[q], hv[q], ss);
  ss = block_sum256(ss, red_f);
  const float r = 1.0f / sqrtf(ss / static_cast<float>(d) + D.draft_eps);
#pragma unroll
  for (int q = 0; q < HQ; ++q) {
    const int c = tid + 256 * q;
    if (c < d) hn[c] = hv[q] * r * gv[q];
  }
  // an empty list reports tokens 0 .. cap-1 with their logits
  const int nsc = n_sl > 0 ? n_sl : ((sl_out || sll_out) ? min(cap, D.V) : 0);
  for (int i = tid; i < nsc; i += 256) sl[i] = n_sl > 0 ? lj[1 + i] : i;
  __syncthreads();
  const int cpl = ((d >> 3) + 63) >> 6;
  if (cpl <= 1)
    sl_score<TE, 1>(D, sl, nsc, hn, sll);
  else if (cpl <= 2)
    sl_score<TE, 2>(D, sl, nsc, hn, sll);
  else
    sl_score<TE, 4>(D, sl, nsc, hn, sll);
  __syncthreads();
  for (int i = tid; i < cap; i += 256) {
    if (sl_out) sl_out[static_cast<int64_t>(j) * cap + i] = i < nsc ? sl[i] : -1;
    if (sll_out) sll_out[static_cast<int64_t>(j) * cap + i] = i < nsc ? sll[i] : -INFINITY;
  }
  if (tid == 0) need_full[j] = n_sl == 0 ? 1 : 0;
  if (n_sl == 0) return;  // the full-vocabulary kernels write this position's drafts (uniform)
  sl_topk(sl, sll, n_sl, K, sel_id, sel_sc);
  __syncthreads();
  sl_write(D, j, K, C, sel_id, sel_sc, ids, scores);
}

// tokens[dst] = tokens[L - 1] (the root of a draft tree next to its nodes).
__global__ void k_draft_root_copy(lng_drafter D, int32_t dst) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    const int L = *D.length;
    D.tokens[dst] = L > 0 ? D.tokens[L - 1] : -1;
  }
}

// Route tokens of the n-grams ending at each window's last position:
// out[j, r, :] = concat over orders of the table row (zero when invalid).  grid (cdiv(R, 32), P)
template <typename TT>
__global__ __launch_bounds__(256) void k_draft_gather(lng_drafter D, DrWin W, TT* __restrict__ out) {
  __shared__ int32_t slot_rows[DR_MAXN];
  __shared__ int64_t rowsh[32][DR_MAXN];
  const int j = blockIdx.y;
  const int L = *D.length;
  const int r0 = blockIdx.x * 32;
  const int nr = min(32, D.R - r0);
  if (threadIdx.x < DR_MAXN) slot_rows[threadIdx.x] = threadIdx.x < D.maxn ? dr_resolve(W.slot[j][threadIdx.x], L) : -1;
  __syncthreads();
  for (int e = threadIdx.x; e < nr * D.n_orders; e += 256) rowsh[e / D.n_orders][e % D.n_orders] = dr_row(D, slot_rows, e % D.n_orders, r0 + e / D.n_orders);
  __syncthreads();
  const int md = D.mem_dim, Dt = D.dt;
  const TT* const* tabs = reinterpret_cast<const TT* const*>(D.tables);
  for (int e = threadIdx.x; e < nr * Dt; e += 256) {
    const int rr = e / Dt, i = e % Dt, oi = i / md;
    const int64_t row = rowsh[rr][oi];
    out[(static_cast<int64_t>(j) * D.R + r0 + rr) * Dt + i] = row >= 0 ? tabs[oi][row * md + (i % md)] : TT(0.f);
  }
}

// ------------------------------------------------------------------ fast path
// Token-only drafters (no SSM input): router halves, the query-key product and the output
// projection are per-token lookup tables (lng_drafter.lut_*), so one depth of a draft is two
// launches: k_fast_attend (codes of new positions, attention partials per route chunk, online
// matches; the last block of each position merges them into r * o) and k_fast_logits (vocabulary
// scores against lut_out; the last block selects the top-k and writes the children's tokens).
constexpr int FA_RC = 16;     // routes per attention block
constexpr int FA_TB = 64;     // pairs per online block
constexpr int FL_VB = 128;    // vocabulary rows per logits block
constexpr int FL_I = 256;     // q_heads * head_dim handled by the fast logits kernel

struct FastLevel {
  int32_t P;
  int32_t slot[DR_MAXP][DR_MAXN];  // window row specs, oldest first, last = the position itself
  int32_t prev[DR_MAXP];           // row spec of the preceding position (router's previous token)
  int32_t fresh[DR_MAXP];          // != 0: the position's codes are computed (and stored) here
};

__device__ __forceinline__ int dr_lut_code(const lng_drafter& D, int64_t ptok, int64_t tok, int r) {
  if (!dr_tok_ok(D, tok)) return 0;
  const int RB = D.R * D.bits;
  const float* a = dr_tok_ok(D, ptok) ? D.lut_prev + ptok * RB : D.lut_start;
  const float* b = D.lut_cur + tok * RB;
  int code = 0;
  for (int i = 0; i < D.bits; ++i) code |= ((a[r * D.bits + i] + b[r * D.bits + i]) > 0.f ? 1 : 0) << i;
  return code;
}

// Records that one block hands to the last block of its group go through the device-coherent
// level: agent-scope relaxed stores and loads (sc1 on gfx950) bypass the XCD-private L2 copies,
// so the hand-off needs no L2 write-back (buffer_wbl2) per block and no L2 invalidate in the
// reader.  Every block's threads wait until their coherent stores are complete (vmcnt(0)), the
// barrier collects the block, thread 0 counts it in; the last block resets the counter.
__device__ __forceinline__ bool dr_last_block(int32_t* counter, int32_t total, int* flag) {
  __builtin_amdgcn_s_waitcnt(WAITCNT_VM0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const int old = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag = old == total - 1;
    if (*flag) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  return *flag != 0;
}

// Sum over each 16-lane row (DPP row_shr:1,2,4,8 inclusive scan): valid in lanes 15, 31, 47, 63.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_row_shr<0x111>(v, 0.f);
  v += dpp_row_shr<0x112>(v, 0.f);
  v += dpp_row_shr<0x114>(v, 0.f);
  v += dpp_row_shr<0x118>(v, 0.f);
  return v;
}

// sync[] layout (int32, zero between calls)
constexpr int SY_ATT = 0;    // [16] attention-launch block counters, per position
constexpr int SY_LOG = 16;   // logits-launch block counter
constexpr int SY_TOT = 32;   // [16] online weight totals, per position
constexpr int SY_NNZ = 64;   // [16][256] count-bearing tokens per (position, logits block)
constexpr int SY_NNZ_STRIDE = 256;
static_assert(SY_NNZ + DR_MAXP * SY_NNZ_STRIDE == LNG_DR_SYNC_INTS, "sync layout");

// Per-lane top-KM list, sorted by (score desc, id asc); empty slots hold (-inf, INT_MAX).
template <int KM>
struct TopK {
  float v[KM];
  int i[KM];
  __device__ __forceinline__ void clear() {
#pragma unroll
    for (int k = 0; k < KM; ++k) v[k] = -INFINITY, i[k] = INT_MAX;
  }
  __device__ __forceinline__ void insert(float x, int id) {
#pragma unroll
    for (int k = 0; k < KM; ++k) {
      const bool sw = x > v[k] || (x == v[k] && id < i[k]);
      const float tv = v[k];
      const int ti = i[k];
      v[k] = sw ? x : tv;
      i[k] = sw ? id : ti;
      x = sw ? tv : x;
      id = sw ? ti : id;
    }
  }
  __device__ __forceinline__ void pop() {
#pragma unroll
    for (int k = 0; k + 1 < KM; ++k) v[k] = v[k + 1], i[k] = i[k + 1];
    v[KM - 1] = -INFINITY, i[KM - 1] = INT_MAX;
  }
};

__device__ __forceinline__ int wave_min_i(int v) {
  v = min(v, __builtin_amdgcn_update_dpp(INT_MAX, v, 0x111, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(INT_MAX, v, 0x112, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(INT_MAX, v, 0x114, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(INT_MAX, v, 0x118, 0xf, 0xf, false));
  return min(min(__builtin_amdgcn_readlane(v, 15), __builtin_amdgcn_readlane(v, 31)),
             min(__builtin_amdgcn_readlane(v, 47), __builtin_amdgcn_readlane(v, 63)));
}

__device__ __forceinline__ int wave_sum_i(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);
  return (__builtin_amdgcn_readlane(v, 15) + __builtin_amdgcn_readlane(v, 31)) +
         (__builtin_amdgcn_readlane(v, 47) + __builtin_amdgcn_readlane(v, 63));
}

// KM rounds of wave argmax (largest score, then smallest id) over the lanes' lists: sv/si receive
// the wave's top-KM in order, identical in every lane; (-inf, -1) where fewer entries exist.  Ids
// are distinct across the wave.  Call from converged code.
template <int KM>
__device__ __forceinline__ void wave_topk(TopK<KM>& t, float* sv, int* si) {
#pragma unroll
  for (int k = 0; k < KM; ++k) {
    const float m = wave_max(t.v[0]);
    const int id = wave_min_i(t.v[0] == m ? t.i[0] : INT_MAX);
    sv[k] = id == INT_MAX ? -INFINITY : m;
    si[k] = id == INT_MAX ? -1 : id;
    if (t.i[0] == id && id != INT_MAX) t.pop();
  }
}

// The wave's top-KM over every lane's N items, ranked by (value desc, id asc): sv/si receive it in
// order, identical in every lane; (-inf, -1) where fewer items exist.  Per round: the lanes'
// maxima, the wave maximum, the smallest id holding it, the winner's removal -- plain max, min and
// select instructions, independent across items.  Ids are distinct; empty items are
// (-inf, INT_MAX) and every real value is finite.  v/id are consumed.
template <int KM, int N>
__device__ __forceinline__ void wave_topk_items(float (&v)[N], int (&id)[N], float* sv, int* si) {
#pragma unroll
  for (int k = 0; k < KM; ++k) {
    float m = v[0];
#pragma unroll
    for (int a = 1; a < N; ++a) m = fmaxf(m, v[a]);
    const float M = wave_max(m);
    int c = INT_MAX;
#pragma unroll
    for (int a = 0; a < N; ++a) c = min(c, v[a] == M ? id[a] : INT_MAX);
    // no item left (every value -inf, taken ones included): no winner
    const int I = M == -INFINITY ? INT_MAX : wave_min_i(c);
    sv[k] = I == INT_MAX ? -INFINITY : M;
    si[k] = I == INT_MAX ? -1 : I;
#pragma unroll
    for (int a = 0; a < N; ++a) v[a] = id[a] == I ? -INFINITY : v[a];  // a taken item keeps its id
  }
}

// Code of route r for (previous token, token) from the router tables (bits <= 4: one 16-byte load
// per table row).
__device__ __forceinline__ int dr_lut_code4(const lng_drafter& D, int64_t ptok, int64_t tok, int r) {
  if (!dr_tok_ok(D, tok)) return 0;
  const int RB = D.R * D.bits;
  const float* a = dr_tok_ok(D, ptok) ? D.lut_prev + ptok * RB : D.lut_start;
  const float* b = D.lut_cur + tok * RB;
  if (D.bits == 4) {
    const f32x4 x = *reinterpret_cast<const f32x4*>(a + 4 * r);
    const f32x4 y = *reinterpret_cast<const f32x4*>(b + 4 * r);
    return ((x[0] + y[0]) > 0.f ? 1 : 0) | ((x[1] + y[1]) > 0.f ? 2 : 0) | ((x[2] + y[2]) > 0.f ? 4 : 0) |
           ((x[3] + y[3]) > 0.f ? 8 : 0);
  }
  return dr_lut_code(D, ptok, tok, r);
}

// grid (nch + nob, P): blocks [0, nch) attention over route chunks, [nch, nch + nob) online matches.
// Attention block c of position j writes the record part[j, c] = (o_c[QH*hd], m_c[QH], l_c[QH])
// with o_c = Wv (mem_norm . U_c) per query head (linear in U_c, so the last block merges the
// chunks with the softmax weights).  Online blocks add their pairs' match counts to
// counts[j, next token] and to the position's total.  The last block of position j merges o_j,
// applies the Gram matrix y = (W_o^T W_o) o_j and writes ro[j] = r_j * o_j,
// r_j = rsqrt(o_j . y / d + eps) = rsqrt(|W_o o_j|^2 / d + eps).
constexpr int FA_MAXCH = 16;  // attention chunks per position (R <= 256)
constexpr int FA_DW = (((FA_TB + DR_MAXN) * 256 + 8) / 4);

__device__ __host__ __forceinline__ int fa_rec(int QH, int I) { return I + 4 * ((2 * QH + 3) / 4); }

// QH_T, DT_T, HD_T, NO_T, MX_T: q_heads, dt, head_dim, the number of orders and the longest order
// fixed at compile time (0 = read from the drafter), so the per-head, per-feature and per-order
// loops of a common shape unroll without predication
template <int QH_T, int DT_T, int HD_T, int NO_T, int MX_T>
__global__ __launch_bounds__(256) void k_fast_attend(lng_drafter D, FastLevel F, int32_t nch, int32_t nob,
                                                     int32_t online, float* __restrict__ part,
                                                     int32_t* __restrict__ counts, float* __restrict__ ro) {
  __shared__ __attribute__((aligned(16))) float xs[FA_RC][LNG_DR_MAX_DT];
  __shared__ __attribute__((aligned(16))) float qs[LNG_DR_MAX_QH * LNG_DR_MAX_DT];
  __shared__ __attribute__((aligned(16))) float us[LNG_DR_MAX_QH * LNG_DR_MAX_DT];
  __shared__ float sx[FA_RC];
  __shared__ float sc[LNG_DR_MAX_QH][FA_RC];
  __shared__ float pr[LNG_DR_MAX_QH][FA_RC];
  __shared__ float ml[LNG_DR_MAX_QH][2];
  __shared__ int64_t rowsh[FA_RC][DR_MAXN];
  __shared__ uint8_t wc[DR_MAXN][256];      // window codes of the position, per route
  __shared__ int32_t qaddr[4][256];
  __shared__ uint32_t cw[FA_DW];           // staged committed codes (bytes)
  __shared__ int32_t red[4][FA_TB];
  __shared__ int32_t srow[DR_MAXN];
  __shared__ int64_t toks[2];
  __shared__ int last_flag;
  __shared__ float redf[4];
  const int j = blockIdx.y;
  // descriptor fields used in loops, read once (kernel-argument loads otherwise repeat per use)
  const int bits = D.bits, maxn = MX_T ? MX_T : D.maxn, n_ord = NO_T ? NO_T : D.n_orders;
  const int ord0 = D.orders[0], ord1 = D.orders[1], ord2 = D.orders[2], ord3 = D.orders[3];
  const void* const tab0 = D.tables[0];
  const void* const tab1 = D.tables[1];
  const void* const tab2 = D.tables[2];
  const void* const tab3 = D.tables[3];
  auto ord_at = [&](int oi) { return oi == 0 ? ord0 : (oi == 1 ? ord1 : (oi == 2 ? ord2 : ord3)); };
  auto tab_at = [&](int oi) { return oi == 0 ? tab0 : (oi == 1 ? tab1 : (oi == 2 ? tab2 : tab3)); };
  const int L = *D.length;
  const int Dt = DT_T ? DT_T : D.dt, QH = QH_T ? QH_T : D.q_heads, hd = HD_T ? HD_T : D.head_dim;
  const int md = D.mem_dim, R = D.R;
  const int I = QH * hd, QD = QH * Dt, G = QH / D.kv_heads;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int mask = (1 << bits) - 1;
  if (threadIdx.x < DR_MAXN) srow[threadIdx.x] = threadIdx.x < maxn ? dr_resolve(F.slot[j][threadIdx.x], L) : -1;
  if (threadIdx.x == 0) {
    const int32_t cr = dr_resolve(F.slot[j][maxn - 1], L);
    const int32_t pv = dr_resolve(F.prev[j], L);
    toks[0] = cr >= 0 ? D.tokens[cr] : -1;
    toks[1] = pv >= 0 ? D.tokens[pv] : -1;
  }
  __syncthreads();
  const int32_t cur_row = srow[maxn - 1];
  const int64_t tok = toks[0], ptok = toks[1];
  const bool fresh = F.fresh[j] != 0;
  const bool is_attn = static_cast<int>(blockIdx.x) < nch;
  // window codes of the routes this block needs: [r0, r0 + nr) (attention) or all (online)
  const int r0 = is_attn ? blockIdx.x * FA_RC : 0;
  const int nr = is_attn ? min(FA_RC, R - r0) : R;
  // the position's query-key row (attention blocks): in flight with the code lookups below
  const bool tok_ok = dr_tok_ok(D, tok);
  f32x4 qrow[LNG_DR_MAX_QH * LNG_DR_MAX_DT / 1024];
  if (is_attn)
#pragma unroll
    for (int q = 0; q < LNG_DR_MAX_QH * LNG_DR_MAX_DT / 1024; ++q) {
      const int i = 4 * threadIdx.x + 1024 * q;
      qrow[q] = (tok_ok && i < QD) ? *reinterpret_cast<const f32x4*>(D.lut_qk + tok * QD + i) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  // the value weight of the thread's first o_c item (bf16 Wv, attention blocks): it depends on
  // nothing the block computes, so its 32 loads are issued now and land during the codes, gather
  // and scores phases
  const int items_w = QH * (hd / 8) * (Dt / 32);
  const bool wv_pre = is_attn && D.wv_dtype == LNG_BF16 && static_cast<int>(threadIdx.x) < items_w;
  bf16x8 wv8[32];
  if (wv_pre) {
    const int it = threadIdx.x, nob8 = hd / 8, nrb = Dt / 32;
    const int qh = it / (nob8 * nrb), rem = it % (nob8 * nrb), o8 = rem % nob8, rb = rem / nob8;
    const bf16* wt = static_cast<const bf16*>(D.wv_t) + (static_cast<int64_t>(qh / G) * Dt + 32 * rb) * hd + 8 * o8;
#pragma unroll
    for (int q = 0; q < 32; ++q) wv8[q] = *reinterpret_cast<const bf16x8*>(wt + static_cast<int64_t>(q) * hd);
  }
  for (int e = threadIdx.x; e < nr * maxn; e += 256) {
    const int k = e / nr, rr = e % nr, r = r0 + rr;
    const int32_t row = srow[k];
    int c = 0;
    if (k == maxn - 1 && fresh)
      c = dr_lut_code4(D, ptok, tok, r);
    else if (row >= 0)
      c = D.codes[static_cast<int64_t>(row) * R + r] & mask;
    wc[k][rr] = static_cast<uint8_t>(c);
  }
  __syncthreads();
  auto addr_of = [&](int oi, int rr) -> int32_t {  // address of order oi for route r0 + rr, -1 if invalid
    const int n = ord_at(oi);
    int32_t addr = 0;
    for (int k = 0; k < n; ++k) {
      const int slot = maxn - n + k;
      if (srow[slot] < 0) return -1;
      addr |= static_cast<int32_t>(wc[slot][rr]) << (k * bits);
    }
    return addr;
  };
  if (is_attn) {
    // ---------------- attention over routes [r0, r0 + nr)
    if (fresh && cur_row >= 0)
      for (int rr = threadIdx.x; rr < nr; rr += 256) D.codes[static_cast<int64_t>(cur_row) * R + r0 + rr] = wc[maxn - 1][rr];
    for (int e = threadIdx.x; e < nr * n_ord; e += 256) {
      const int rr = e / n_ord, oi = e % n_ord;
      const int32_t a = addr_of(oi, rr);
      rowsh[rr][oi] = a < 0 ? -1 : static_cast<int64_t>(r0 + rr) * (int64_t{1} << (bits * ord_at(oi))) + a;
    }
#pragma unroll
    for (int q = 0; q < LNG_DR_MAX_QH * LNG_DR_MAX_DT / 1024; ++q) {
      const int i = 4 * threadIdx.x + 1024 * q;
      if (i < QD) *reinterpret_cast<f32x4*>(&qs[i]) = qrow[q];
    }
    __syncthreads();
    if (D.table_dtype == LNG_BF16 && md % 8 == 0) {
      const int pieces = md / 8;
      for (int e = threadIdx.x; e < nr * n_ord * pieces; e += 256) {
        const int pc = e % pieces, ro_ = e / pieces, oi = ro_ % n_ord, rr = ro_ / n_ord;
        const int64_t row = rowsh[rr][oi];
        bf16x8 v8 = bf16x8{};
        if (row >= 0) v8 = *reinterpret_cast<const bf16x8*>(static_cast<const bf16*>(tab_at(oi)) + row * md + 8 * pc);
#pragma unroll
        for (int q = 0; q < 8; ++q) xs[rr][oi * md + 8 * pc + q] = static_cast<float>(v8[q]);
      }
    } else {
      for (int e = threadIdx.x; e < nr * Dt; e += 256) {
        const int rr = e / Dt, i = e % Dt, oi = i / md;
        const int64_t row = rowsh[rr][oi];
        xs[rr][i] = row >= 0 ? ld_any(tab_at(oi), D.table_dtype, row * md + (i % md)) : 0.f;
      }
    }
    __syncthreads();
    // scores: 16 lanes per route (lane part p covers features p, p+16, ...), row-level DPP sums
    {
      const int rr = threadIdx.x >> 4, p = threadIdx.x & 15;
      float x[LNG_DR_MAX_DT / 16];
#pragma unroll
      for (int q = 0; q < LNG_DR_MAX_DT / 16; ++q) x[q] = (rr < nr && 16 * q < Dt) ? xs[rr][16 * q + p] : 0.f;
      float ss = 0.f;
#pragma unroll
      for (int q = 0; q < LNG_DR_MAX_DT / 16; ++q) ss = fmaf(x[q], x[q], ss);
      ss = row16_sum(ss);
      const float sv = 1.0f / sqrtf(ss / static_cast<float>(Dt) + D.mem_eps);
      if (p == 15 && rr < nr) sx[rr] = sv;
      for (int qh = 0; qh < QH; ++qh) {
        float a = 0.f;
#pragma unroll
        for (int q = 0; q < LNG_DR_MAX_DT / 16; ++q)
          if (16 * q < Dt) a = fmaf(qs[qh * Dt + 16 * q + p], x[q], a);
        a = row16_sum(a);
        if (p == 15 && rr < nr) sc[qh][rr] = sv * a;
      }
    }
    __syncthreads();
    if (threadIdx.x < QH) {
      const int qh = threadIdx.x;
      float m = -INFINITY;
      for (int rr = 0; rr < nr; ++rr) m = fmaxf(m, sc[qh][rr]);
      float l = 0.f;
      for (int rr = 0; rr < nr; ++rr) {
        const float pp = expf(sc[qh][rr] - m);
        l += pp;
        pr[qh][rr] = pp * sx[rr];
      }
      ml[qh][0] = m;
      ml[qh][1] = l;
    }
    __syncthreads();
    // U[qh] = mem_norm . sum_r p_r s_r x_r (4 features per thread)
    for (int e = 4 * threadIdx.x; e < QD; e += 1024) {
      const int qh = e / Dt, i = e % Dt;
      f32x4 u = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int rr = 0; rr < FA_RC; ++rr)
        if (rr < nr) {
          const f32x4 xv = *reinterpret_cast<const f32x4*>(&xs[rr][i]);
          const float pv = pr[qh][rr];
          u[0] = fmaf(pv, xv[0], u[0]);
          u[1] = fmaf(pv, xv[1], u[1]);
          u[2] = fmaf(pv, xv[2], u[2]);
          u[3] = fmaf(pv, xv[3], u[3]);
        }
      const f32x4 mn = *reinterpret_cast<const f32x4*>(D.mem_norm + i);
      *reinterpret_cast<f32x4*>(&us[e]) = f32x4{u[0] * mn[0], u[1] * mn[1], u[2] * mn[2], u[3] * mn[3]};
    }
    __syncthreads();
    float* rec = part + (static_cast<int64_t>(j) * nch + blockIdx.x) * fa_rec(QH, I);
    // o_c[qh][oe] = sum_i Wv[h][oe][i] U[qh][i]: item (qh, 8 outputs, 32 rows), 16-byte loads of the
    // transposed weight, all in flight; partial sums meet in LDS (xs is free now)
    float* ob = &xs[0][0];  // [QH][Dt/32][hd]
    {
      const int nrb = Dt / 32, nob8 = hd / 8;
      for (int it = threadIdx.x; it < QH * nob8 * nrb; it += 256) {
        const int qh = it / (nob8 * nrb), rem = it % (nob8 * nrb), o8 = rem % nob8, rb = rem / nob8;
        const int h = qh / G;
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (D.wv_dtype == LNG_BF16) {
          const bf16* wt = static_cast<const bf16*>(D.wv_t) + (static_cast<int64_t>(h) * Dt + 32 * rb) * hd + 8 * o8;
          if (it != static_cast<int>(threadIdx.x))  // the first item was loaded at kernel entry
#pragma unroll
            for (int q = 0; q < 32; ++q) wv8[q] = *reinterpret_cast<const bf16x8*>(wt + static_cast<int64_t>(q) * hd);
#pragma unroll
          for (int q = 0; q < 32; ++q) {
            const float uq = us[qh * Dt + 32 * rb + q];
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] = fmaf(static_cast<float>(wv8[q][e]), uq, acc[e]);
          }
        } else {
          const float* wt = static_cast<const float*>(D.wv_t) + (static_cast<int64_t>(h) * Dt + 32 * rb) * hd + 8 * o8;
          for (int q0 = 0; q0 < 32; q0 += 16) {
            f32x4 wa[16], wb[16];
#pragma unroll
            for (int q = 0; q < 16; ++q) {
              wa[q] = *reinterpret_cast<const f32x4*>(wt + static_cast<int64_t>(q0 + q) * hd);
              wb[q] = *reinterpret_cast<const f32x4*>(wt + static_cast<int64_t>(q0 + q) * hd + 4);
            }
#pragma unroll
            for (int q = 0; q < 16; ++q) {
              const float uq = us[qh * Dt + 32 * rb + q0 + q];
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                acc[e] = fmaf(wa[q][e], uq, acc[e]);
                acc[4 + e] = fmaf(wb[q][e], uq, acc[4 + e]);
              }
            }
          }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) ob[(qh * nrb + rb) * hd + 8 * o8 + e] = acc[e];
      }
      __syncthreads();
      for (int e = threadIdx.x; e < I; e += 256) {
        const int qh = e / hd, oe = e % hd;
        float a = 0.f;
        for (int rb = 0; rb < nrb; ++rb) a += ob[(qh * nrb + rb) * hd + oe];
        st_dev(rec + e, a);
        us[e] = a;  // o_c, reused below
      }
    }
    if (threadIdx.x < QH) {
      st_dev(rec + I + threadIdx.x, ml[threadIdx.x][0]);
      st_dev(rec + I + QH + threadIdx.x, ml[threadIdx.x][1]);
    }
  } else {
    // ---------------- online counts over pairs [t0, t0 + FA_TB) (thread = route)
    const int t0 = (blockIdx.x - nch) * FA_TB;
    const int npairs = L - 1;
    const int r = threadIdx.x;
    const bool rv = r < R;
    for (int oi = 0; oi < n_ord; ++oi) qaddr[oi][r] = rv ? addr_of(oi, r) : -1;
    int nt = 0;
    int64_t a_al = 0;
    if (t0 < npairs) {
      // stage the committed codes of positions t0 - maxn + 1 .. t0 + nt - 1 (contiguous bytes)
      const int tb = max(t0 - (maxn - 1), 0);
      const int te = min(t0 + FA_TB, npairs);  // exclusive
      const int64_t a0 = static_cast<int64_t>(tb) * R, a1 = static_cast<int64_t>(te) * R;
      a_al = a0 & ~int64_t{3};
      const int ndw = static_cast<int>((a1 - a_al + 3) / 4);
      const uint32_t* src = reinterpret_cast<const uint32_t*>(D.codes + a_al);
      constexpr int PQ = (FA_DW + 255) / 256;
      uint32_t tmp[PQ];
#pragma unroll
      for (int q = 0; q < PQ; ++q) {
        const int e = threadIdx.x + 256 * q;
        tmp[q] = e < ndw ? src[e] : 0u;
      }
#pragma unroll
      for (int q = 0; q < PQ; ++q) {
        const int e = threadIdx.x + 256 * q;
        if (e < ndw) cw[e] = tmp[q];
      }
      nt = te - t0;
    }
    __syncthreads();
    if (t0 < npairs) {
      const uint8_t* cb = reinterpret_cast<const uint8_t*>(cw);
      // Codes as 8-bit digits (oldest least significant); a position before the sequence start is
      // the digit 0xFF and an unusable query has the digit 0x80, neither of which a code can equal.
      uint32_t pre[DR_MAXN - 1], cur[FA_TB];
#pragma unroll
      for (int k = 0; k < DR_MAXN - 1; ++k) {
        const int t = t0 - (maxn - 1) + k;
        pre[k] = (k < maxn - 1 && t >= 0 && rv) ? (cb[static_cast<int64_t>(t) * R + r - a_al] & mask) : 0xFFu;
      }
#pragma unroll
      for (int tt = 0; tt < FA_TB; ++tt) cur[tt] = cb[static_cast<int64_t>(t0 + tt) * R + r - a_al] & mask;
      uint32_t q8[4], sho[4];
#pragma unroll
      for (int oi = 0; oi < 4; ++oi) {
        const bool used = oi < n_ord;
        const int n = used ? ord_at(oi) : 1;
        const int32_t qa = (rv && used) ? qaddr[oi][r] : -1;
        uint32_t q = 0;
        for (int k = 0; k < n; ++k) q |= ((static_cast<uint32_t>(qa) >> (bits * k)) & mask) << (8 * k);
        q8[oi] = qa >= 0 ? q : 0x80808080u;
        sho[oi] = static_cast<uint32_t>(8 * (maxn - n));
      }
      const int sh = 8 * (maxn - 1);
      // window bytes 0 .. maxn-1 start at the invalid digit; the bytes above the window stay zero so
      // that each shift leaves room for the newest code in byte maxn-1
      uint32_t amax = maxn >= 4 ? 0xFFFFFFFFu : ((1u << (8 * maxn)) - 1u);
#pragma unroll
      for (int k = 0; k < DR_MAXN - 1; ++k)
        if (k < maxn - 1) amax = (amax >> 8) | (pre[k] << sh);
#pragma unroll
      for (int tt = 0; tt < FA_TB; ++tt) {
        amax = (amax >> 8) | (cur[tt] << sh);
        int cnt = 0;
#pragma unroll
        for (int oi = 0; oi < 4; ++oi) cnt += __popcll(__ballot(q8[oi] == (amax >> sho[oi])));
        if (lane == 0) red[w][tt] = cnt;
      }
      __syncthreads();
      int s = 0;
      if (threadIdx.x < nt) {
        const int t = t0 + threadIdx.x;
        s = (red[0][threadIdx.x] + red[1][threadIdx.x]) + (red[2][threadIdx.x] + red[3][threadIdx.x]);
        if (s > 0) {
          // a token's first count also counts it in its logits block (dense candidate offsets)
          const int64_t tok = D.tokens[t + 1];
          if (atomicAdd(&counts[static_cast<int64_t>(j) * D.V + tok], s) == 0)
            atomicAdd(&D.sync[SY_NNZ + j * SY_NNZ_STRIDE + static_cast<int>(tok / FL_VB)], 1);
        }
      }
      // the block's total weight (exact integer) into the position's total
      const float bs = block_sum256(static_cast<float>(s), redf);
      if (threadIdx.x == 0 && bs > 0.f) atomicAdd(&D.sync[SY_TOT + j], static_cast<int32_t>(bs));
    }
  }
  // ---------------- last block of position j: merge, hidden norm
  if (!dr_last_block(&D.sync[SY_ATT + j], nch + nob, &last_flag)) return;
  const float b0 = D.sink_logit;
  const int RS = fa_rec(QH, I);
  const float* rj = part + static_cast<int64_t>(j) * nch * RS;
  const __amdgpu_buffer_rsrc_t rb = dev_buf(rj, static_cast<uint32_t>(nch * RS) * 4u);
  // loads in the order they are needed (the memory counter completes them in order): the chunks'
  // (m, l) pieces, then every chunk's o_c
  const int npc = (2 * QH + 3) / 4;  // 16-byte (m, l) pieces per chunk
  __shared__ __attribute__((aligned(16))) float mlb[FA_MAXCH][2 * LNG_DR_MAX_QH];
  f32x4 mlp = {0.f, 0.f, 0.f, 0.f};
  const bool ml_ld = threadIdx.x < nch * npc;
  if (ml_ld) mlp = ld_dev4(rb, 4u * ((threadIdx.x / npc) * RS + I + 4 * (threadIdx.x % npc)));
  // o_c: thread (c4 = t / 64, e4 = t % 64) loads o_c[4 e4 .. +3] of chunks c4, c4 + 4, ... (I <= 256)
  const int e4 = threadIdx.x & 63, c4 = threadIdx.x >> 6;
  f32x4 ov[FA_MAXCH / 4];
#pragma unroll
  for (int q = 0; q < FA_MAXCH / 4; ++q) {
    const int c = c4 + 4 * q;
    ov[q] = (c < nch && 4 * e4 < I) ? ld_dev4(rb, 4u * (c * RS + 4 * e4)) : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  if (ml_ld) *reinterpret_cast<f32x4*>(&mlb[threadIdx.x / npc][4 * (threadIdx.x % npc)]) = mlp;
  __syncthreads();
  // merge weights per (chunk, head): f = e^{m_c - M} / (e^{b0 - M} + sum_c l_c e^{m_c - M})
  __shared__ float wgt[FA_MAXCH][LNG_DR_MAX_QH];
  __shared__ __attribute__((aligned(16))) float opart[4][LNG_DR_MAX_QH * LNG_DR_MAX_DT / 4];
  // one thread per (chunk, head) takes its exponential, one thread per head then sums l in chunk
  // order, and the weights follow: the exponentials run side by side instead of in one chain
  __shared__ float fex[FA_MAXCH][LNG_DR_MAX_QH];
  __shared__ float hm[LNG_DR_MAX_QH], hl[LNG_DR_MAX_QH];
  for (int t = threadIdx.x; t < FA_MAXCH * QH; t += 256) {
    const int c = t / QH, qh = t % QH;
    float M = b0;
#pragma unroll
    for (int cc = 0; cc < FA_MAXCH; ++cc) M = fmaxf(M, cc < nch ? mlb[cc][qh] : -INFINITY);
    fex[c][qh] = c < nch ? expf(mlb[c][qh] - M) : 0.f;
    if (c == 0) hm[qh] = M;
  }
  __syncthreads();
  if (threadIdx.x < QH) {
    const int qh = threadIdx.x;
    float l = expf(b0 - hm[qh]);
#pragma unroll
    for (int c = 0; c < FA_MAXCH; ++c) l = fmaf(c < nch ? mlb[c][QH + qh] : 0.f, fex[c][qh], l);
    hl[qh] = l;
  }
  __syncthreads();
  for (int t = threadIdx.x; t < FA_MAXCH * QH; t += 256) {
    const int c = t / QH, qh = t % QH;
    wgt[c][qh] = fex[c][qh] / hl[qh];
  }
  __syncthreads();
  // o = sum_c f_{c, qh(e)} o_c: partial sums over the thread's chunks, then over the four groups
  if (4 * e4 < I) {
    const int qh = (4 * e4) / hd;
    f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < FA_MAXCH / 4; ++q) {
      const int c = c4 + 4 * q;
      const float f = c < nch ? wgt[c][qh] : 0.f;
      o[0] = fmaf(f, ov[q][0], o[0]);
      o[1] = fmaf(f, ov[q][1], o[1]);
      o[2] = fmaf(f, ov[q][2], o[2]);
      o[3] = fmaf(f, ov[q][3], o[3]);
    }
    *reinterpret_cast<f32x4*>(&opart[c4][4 * e4]) = o;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < I; e += 256) us[e] = (opart[0][e] + opart[1][e]) + (opart[2][e] + opart[3][e]);
  __syncthreads();
  // o . (Gram o): thread (k4 = e4, quarter c4) sums Gram[e][4 k4 .. +3] o[e] over its quarter of e
  // (Gram is symmetric; one row e is a contiguous kilobyte across the wave), 32 rows per batch
  float acc = 0.f;
  if (4 * e4 < I) {
    const int ne = (I + 3) / 4, eb = c4 * ne, ee = min(I, eb + ne);
    f32x4 y = {0.f, 0.f, 0.f, 0.f};
    for (int e0 = eb; e0 < ee; e0 += 32) {
      f32x4 gv[32];
#pragma unroll
      for (int q = 0; q < 32; ++q)
        gv[q] = e0 + q < ee ? *reinterpret_cast<const f32x4*>(D.gram_out + static_cast<int64_t>(e0 + q) * I + 4 * e4)
                            : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < 32; ++q) {
        const float oe = e0 + q < ee ? us[e0 + q] : 0.f;
        y[0] = fmaf(gv[q][0], oe, y[0]);
        y[1] = fmaf(gv[q][1], oe, y[1]);
        y[2] = fmaf(gv[q][2], oe, y[2]);
        y[3] = fmaf(gv[q][3], oe, y[3]);
      }
    }
    acc = (y[0] * us[4 * e4] + y[1] * us[4 * e4 + 1]) + (y[2] * us[4 * e4 + 2] + y[3] * us[4 * e4 + 3]);
  }
  const float ss = block_sum256(acc, redf);
  const float rn = 1.0f / sqrtf(ss / static_cast<float>(D.d) + D.draft_eps);
  for (int e = threadIdx.x; e < I; e += 256) ro[static_cast<int64_t>(j) * I + e] = rn * us[e];
}

// grid (nblk <= 256): scores of a slice of FL_VB vocabulary rows for every position against lut_out
// (fp32 MFMA).  Per (position, block) the record lpart[j][b] = [max, sum of exponentials, number of
// tokens with online counts, -, top-KM logits, top-KM ids] over the slice's tokens without counts.
// The tokens with counts go to the position's dense list cand[j][0 .. n) as (id, logit bits,
// count, 0), block b from the prefix of the per-block numbers that the attention launch counted
// (sync[SY_NNZ]); their counts are returned to zero here.  The last block selects every
// position's top-K: G = 4 / P waves per position when P <= 2, else one (positions w, w + 4, ...);
// each wave ranks every block's top-KM and its share of the list, by logit or by the
// online-mixed probability (1 - lam) softmax + lam count / total (the log is taken of the
// winners only), then writes the children's tokens.
constexpr int FL_NBL = 4;     // blocks per lane in the selection: nblk <= 256
constexpr int FL_CH = 12;     // count-bearing tokens per lane per load batch
static_assert(FL_NBL * 64 == SY_NNZ_STRIDE, "one counter per logits block");

// Count-bearing tokens of one position in the logits blocks before block b (nnz: that position's
// per-block counters).  Every lane receives it.
__device__ __forceinline__ int fl_prefix(const int32_t* nnz, int b, int lane) {
  int s = 0;
#pragma unroll
  for (int q = 0; q < FL_NBL; ++q) {
    const int bb = FL_NBL * lane + q;
    const int v = nnz[bb];
    s += bb < b ? v : 0;
  }
  return wave_sum_i(s);
}

template <int KM>
__host__ __device__ constexpr int fl_rs() { return 4 + 4 * ((2 * KM + 3) / 4); }  // whole 16-byte pieces

// I_T: q_heads * head_dim fixed at compile time (0 = read from the drafter)
template <int KM, int I_T>
__global__ __launch_bounds__(256) void k_fast_logits(lng_drafter D, int32_t P, int32_t K, int32_t online, float kappa,
                                                     const float* __restrict__ ro, float* __restrict__ logits_out,
                                                     float* __restrict__ lpart, int32_t* __restrict__ counts,
                                                     int4* __restrict__ cand, DrChildren C,
                                                     int64_t* __restrict__ ids, float* __restrict__ scores) {
  constexpr int RS = fl_rs<KM>();
  __shared__ __attribute__((aligned(16))) float rs[DR_MAXP][FL_I];
  __shared__ float lt[DR_MAXP][FL_VB];
  __shared__ int last_flag;
  __shared__ float sel_v[4][KM];
  __shared__ int sel_i[4][KM];
  const int I = I_T ? I_T : D.q_heads * D.head_dim;
  const int64_t V = D.V;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t v0 = static_cast<int64_t>(blockIdx.x) * FL_VB;
  const int64_t va = v0 + lane, vb = v0 + 64 + lane;
  // kernel-argument children (one per lane) and the online total of the position this wave selects
  // for: loaded here, used by the last block
  const int c_row = lane < C.n ? C.row[lane] : 0;
  const int c_par = lane < C.n ? C.parent[lane] : -1;
  const int c_rank = lane < C.n ? C.rank[lane] : 0;
  const int G = P == 1 ? 4 : (P == 2 ? 2 : 1);  // selection waves per position
  const int tot0 = online && w / G < P ? D.sync[SY_TOT + w / G] : 0;
  // count-bearing tokens of this wave's (first) selection position: its per-block counters are
  // final once the attention launch ended, so the selection can size its list loads up front
  const int nc0 = online && w / G < P ? fl_prefix(D.sync + SY_NNZ + (w / G) * SY_NNZ_STRIDE, gridDim.x, lane) : 0;
  // online counts of this wave's first position: in flight during the products
  int ca = 0, cb = 0, pre0 = 0;
  if (online && w < P) {
    const int32_t* cj = counts + static_cast<int64_t>(w) * V;
    ca = va < V ? cj[va] : 0;
    cb = vb < V ? cj[vb] : 0;
    pre0 = fl_prefix(D.sync + SY_NNZ + w * SY_NNZ_STRIDE, blockIdx.x, lane);
  }
  for (int e = threadIdx.x; e < P * I; e += 256) rs[e / I][e % I] = ro[e];
  __syncthreads();
  // fp32 MFMA 16x16x4: D[row][j] += sum_k EO[row][k] ro[j][k].  Lane l feeds A[row l%16][k-slot
  // l/16] and B[k-slot l/16][column l%16]; k-slot l/16 of step (s, q) is feature 16s + 4(l/16) + q
  // (A and B use the same feature order, so the sum is unchanged).  Wave w: tiles 2w, 2w+1.
  const int col = lane & 15, kq = lane >> 4;
  const int nks = I / 16;
  f32x4 bq[FL_I / 16];
#pragma unroll
  for (int st = 0; st < FL_I / 16; ++st)
    bq[st] = (st < nks && col < P) ? *reinterpret_cast<const f32x4*>(&rs[col][16 * st + 4 * kq]) : f32x4{0.f, 0.f, 0.f, 0.f};
  const float* const pk = D.lut_out_pk;
  // both tiles' operands are loaded before either tile's products: one memory round trip per wave
  f32x4 a2[2][FL_I / 16];
#pragma unroll
  for (int t2 = 0; t2 < 2; ++t2) {
    const int tile = 2 * w + t2;
    const int64_t vrow = v0 + tile * 16 + col;
    if (pk) {  // packed tiles: one contiguous kilobyte per load (rows past V are zero)
      const float* tp = pk + (((v0 >> 4) + tile) * nks) * 256 + 4 * lane;
#pragma unroll
      for (int st = 0; st < FL_I / 16; ++st)
        a2[t2][st] = (st < nks && v0 + tile * 16 < V) ? *reinterpret_cast<const f32x4*>(tp + 256 * st)
                                                     : f32x4{0.f, 0.f, 0.f, 0.f};
    } else {
#pragma unroll
      for (int st = 0; st < FL_I / 16; ++st)
        a2[t2][st] = (st < nks && vrow < V) ? *reinterpret_cast<const f32x4*>(D.lut_out + vrow * I + 16 * st + 4 * kq)
                                           : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
#pragma unroll
  for (int t2 = 0; t2 < 2; ++t2) {
    const int tile = 2 * w + t2;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < FL_I / 16; ++st) {
      if (st < nks) {
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a2[t2][st][0], bq[st][0], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a2[t2][st][1], bq[st][1], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a2[t2][st][2], bq[st][2], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a2[t2][st][3], bq[st][3], acc, 0, 0, 0);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int vl = tile * 16 + 4 * kq + r;
      const int64_t v = v0 + vl;
      if (col < P) {
        lt[col][vl] = v < V ? acc[r] : -INFINITY;
        if (logits_out && v < V) logits_out[static_cast<int64_t>(col) * V + v] = acc[r];
      }
    }
  }
  __syncthreads();
  const int nblk = gridDim.x;
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int jj = w; jj < P; jj += 4) {
    float* o = lpart + (static_cast<int64_t>(jj) * nblk + blockIdx.x) * RS;
    const float x0 = lt[jj][lane], x1 = lt[jj][lane + 64];
    if (online && jj != w) {
      const int32_t* cj = counts + static_cast<int64_t>(jj) * V;
      ca = va < V ? cj[va] : 0;
      cb = vb < V ? cj[vb] : 0;
    }
    const float m = wave_max(fmaxf(x0, x1));
    const float s = wave_sum((x0 == -INFINITY ? 0.f : expf(x0 - m)) + (x1 == -INFINITY ? 0.f : expf(x1 - m)));
    int nbk = 0;
    if (online) {
      // tokens with counts: (id, logit bits, count) into the position's list, counts cleared
      int32_t* cj = counts + static_cast<int64_t>(jj) * V;
      // (at most FL_VB per earlier block: stays inside the list whatever the counters hold)
      const int pre = min(jj == w ? pre0 : fl_prefix(D.sync + SY_NNZ + jj * SY_NNZ_STRIDE, blockIdx.x, lane),
                          FL_VB * static_cast<int>(blockIdx.x));
      int4* dst = cand + static_cast<int64_t>(jj) * nblk * FL_VB + pre;
      const uint64_t ma = __ballot(ca > 0), mb = __ballot(cb > 0);
      const int na = __popcll(ma);
      nbk = na + __popcll(mb);
      const __amdgpu_buffer_rsrc_t db = dev_buf(dst, static_cast<uint32_t>(nbk) * 16u);
      if (ca > 0) {
        st_dev4(db, 16u * __popcll(ma & below),
                f32x4{__int_as_float(static_cast<int32_t>(va)), x0, __int_as_float(ca), 0.f});
        cj[va] = 0;
      }
      if (cb > 0) {
        st_dev4(db, 16u * (na + __popcll(mb & below)),
                f32x4{__int_as_float(static_cast<int32_t>(vb)), x1, __int_as_float(cb), 0.f});
        cj[vb] = 0;
      }
    }
    TopK<KM> t;
    t.clear();
    // (-inf, INT_MAX) never enters a list: the inserts need no branch
    const bool oka = x0 != -INFINITY && ca == 0, okb = x1 != -INFINITY && cb == 0;
    t.insert(oka ? x0 : -INFINITY, oka ? static_cast<int>(va) : INT_MAX);
    t.insert(okb ? x1 : -INFINITY, okb ? static_cast<int>(vb) : INT_MAX);
    float sv[KM];
    int si[KM];
    wave_topk(t, sv, si);
    if (lane == 0) {
      float rv[RS];
#pragma unroll
      for (int e = 0; e < RS; ++e) rv[e] = 0.f;
      rv[0] = m;
      rv[1] = s;
      rv[2] = __int_as_float(nbk);
#pragma unroll
      for (int k = 0; k < KM; ++k) {
        rv[4 + k] = sv[k];
        rv[4 + KM + k] = __int_as_float(si[k]);
      }
      const __amdgpu_buffer_rsrc_t ob = dev_buf(o, RS * 4u);
#pragma unroll
      for (int q = 0; q < RS / 4; ++q) st_dev4(ob, 16u * q, f32x4{rv[4 * q], rv[4 * q + 1], rv[4 * q + 2], rv[4 * q + 3]});
    }
  }
  if (!dr_last_block(&D.sync[SY_LOG], nblk, &last_flag)) return;
  // ---------------- selection
  const int g = w % G;
  for (int j = w / G; j < P; j += 4 / G) {
    const float* lp = lpart + static_cast<int64_t>(j) * nblk * RS;
    // the position's count-bearing tokens (the list's first batch, e = 64 (G u + g) + lane, is
    // loaded together with the records: one round trip for both)
    const int nc = online ? (j == w / G ? nc0 : fl_prefix(D.sync + SY_NNZ + j * SY_NNZ_STRIDE, nblk, lane)) : 0;
    const int4* cj = cand + static_cast<int64_t>(j) * nblk * FL_VB;
    const __amdgpu_buffer_rsrc_t cbuf = dev_buf(cj, static_cast<uint32_t>(max(nc, 1)) * 16u);
    f32x4 cr0[FL_CH];
    if (online && nc > 0) {
#pragma unroll
      for (int u = 0; u < FL_CH; ++u) cr0[u] = ld_dev4(cbuf, 16u * min(64 * g + 64 * G * u + lane, nc - 1));
    }
    // records of blocks 4 lane + q (all in flight at once)
    float rm[FL_NBL], rsm[FL_NBL], av[FL_NBL][KM];
    int ai[FL_NBL][KM];
    const __amdgpu_buffer_rsrc_t lbuf = dev_buf(lp, static_cast<uint32_t>(nblk) * RS * 4u);
    f32x4 rq[FL_NBL][RS / 4];
#pragma unroll
    for (int q = 0; q < FL_NBL; ++q)  // unconditional loads (block index clamped into the records)
#pragma unroll
      for (int p4 = 0; p4 < RS / 4; ++p4)
        rq[q][p4] = ld_dev4(lbuf, 4u * (min(FL_NBL * lane + q, nblk - 1) * RS + 4 * p4));
#pragma unroll
    for (int q = 0; q < FL_NBL; ++q) {
      const int b = FL_NBL * lane + q;
      const bool ok = b < nblk;
      float rv[RS];
      __builtin_memcpy(rv, &rq[q][0], sizeof(rv));
      rm[q] = ok ? rv[0] : -INFINITY;
      rsm[q] = ok ? rv[1] : 0.f;
#pragma unroll
      for (int k = 0; k < KM; ++k) {
        const bool mine = ok && q % G == g;
        av[q][k] = mine ? rv[4 + k] : -INFINITY;
        ai[q][k] = mine ? __float_as_int(rv[4 + KM + k]) : -1;
      }
    }
    float m = -INFINITY;
#pragma unroll
    for (int q = 0; q < FL_NBL; ++q) m = fmaxf(m, rm[q]);
    const float M = wave_max(m);
    float s = 0.f;
#pragma unroll
    for (int q = 0; q < FL_NBL; ++q) s += rm[q] == -INFINITY ? 0.f : rsm[q] * expf(rm[q] - M);
    const float S = wave_sum(s);
    const float tj = online ? static_cast<float>(j == w / G ? tot0 : D.sync[SY_TOT + j]) : 0.f;
    const float n_eff = tj / static_cast<float>(D.R * D.n_orders);
    const float lam = tj > 0.f ? n_eff / (n_eff + kappa) : 0.f;
    // online ranking value: (1 - lam) exp(logit - M) / S + lam count / total (log taken at the end)
    const float mix_a = (1.f - lam) / S, mix_b = tj > 0.f ? lam / tj : 0.f;
    // the wave's items: the blocks' top-KM lists and the list's first batch, ranked together
    float sv[KM];
    int si[KM];
    {
      constexpr int NI = FL_NBL * KM + FL_CH;
      float iv[NI];
      int ii[NI];
#pragma unroll
      for (int q = 0; q < FL_NBL; ++q)
#pragma unroll
        for (int k = 0; k < KM; ++k) {
          iv[q * KM + k] = ai[q][k] < 0 ? -INFINITY : online ? mix_a * expf(av[q][k] - M) : av[q][k];
          ii[q * KM + k] = ai[q][k] < 0 ? INT_MAX : ai[q][k];
        }
#pragma unroll
      for (int u = 0; u < FL_CH; ++u) {
        const bool ok = online && 64 * g + 64 * G * u + lane < nc;
        iv[FL_NBL * KM + u] =
            ok ? fmaf(mix_b, static_cast<float>(__float_as_int(cr0[u][2])), mix_a * expf(cr0[u][1] - M)) : -INFINITY;
        ii[FL_NBL * KM + u] = ok ? __float_as_int(cr0[u][0]) : INT_MAX;
      }
      wave_topk_items<KM, NI>(iv, ii, sv, si);
    }
    if (online) {
      if (g == 0)  // every block has read the per-block counters: clear them for the next call
#pragma unroll
        for (int q = 0; q < FL_NBL; ++q) D.sync[SY_NNZ + j * SY_NNZ_STRIDE + FL_NBL * lane + q] = 0;
      // further batches of the list: ranked with the winners so far (lane k holds winner k)
      for (int e0 = 64 * g + 64 * G * FL_CH; e0 < nc; e0 += 64 * G * FL_CH) {
        f32x4 cr[FL_CH];
#pragma unroll
        for (int u = 0; u < FL_CH; ++u) cr[u] = ld_dev4(cbuf, 16u * min(e0 + 64 * G * u + lane, nc - 1));
        constexpr int NB = FL_CH + 1;
        float bv[NB];
        int bi[NB];
        bv[0] = -INFINITY, bi[0] = INT_MAX;
#pragma unroll
        for (int k = 0; k < KM; ++k)
          if (lane == k && si[k] >= 0) bv[0] = sv[k], bi[0] = si[k];
#pragma unroll
        for (int u = 0; u < FL_CH; ++u) {
          const bool ok = e0 + 64 * G * u + lane < nc;
          bv[1 + u] = ok ? fmaf(mix_b, static_cast<float>(__float_as_int(cr[u][2])), mix_a * expf(cr[u][1] - M))
                         : -INFINITY;
          bi[1 + u] = ok ? __float_as_int(cr[u][0]) : INT_MAX;
        }
        wave_topk_items<KM, NB>(bv, bi, sv, si);
      }
    }
    if (G > 1) {
      // merge the group's lists: wave g == 0 ranks the G * KM winners again
      if (lane == 0)
#pragma unroll
        for (int k = 0; k < KM; ++k) sel_v[w][k] = sv[k], sel_i[w][k] = si[k];
      __syncthreads();
      if (g != 0) continue;
      float mv[1];
      int mi[1];
      const bool have = lane < G * KM && sel_i[w + lane / KM][lane % KM] >= 0;
      mv[0] = have ? sel_v[w + lane / KM][lane % KM] : -INFINITY;
      mi[0] = have ? sel_i[w + lane / KM][lane % KM] : INT_MAX;
      wave_topk_items<KM, 1>(mv, mi, sv, si);
      __builtin_amdgcn_wave_barrier();
    }
    if (lane == 0)
#pragma unroll
      for (int k = 0; k < KM; ++k) {
        sel_v[w][k] = online ? (si[k] >= 0 ? logf(sv[k]) : -INFINITY) : sv[k];
        sel_i[w][k] = si[k];
      }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < K) {
      ids[static_cast<int64_t>(j) * K + lane] = sel_i[w][lane];
      scores[static_cast<int64_t>(j) * K + lane] = sel_v[w][lane];
    }
    if (lane == 0 && online) D.sync[SY_TOT + j] = 0;
    if (c_par == j) {
      const int t2 = sel_i[w][c_rank];
      D.tokens[c_row] = t2 >= 0 ? t2 : sel_i[w][0];
    }
  }
}

// Codes of positions (fast path): codes[row_j][r] from the router tables.   grid (cdiv(R, 256), n)
__global__ __launch_bounds__(256) void k_fast_codes(lng_drafter D, DrAdv A) {
  const int j = blockIdx.y;
  const int r = blockIdx.x * 256 + threadIdx.x;
  if (r >= D.R || j >= A.n) return;
  const int L = *D.length;
  const int32_t row = A.range ? A.base + j : dr_resolve(A.row[j], L);
  const int32_t pv = A.range ? (j == 0 ? dr_resolve(A.prev0, L) : A.base + j - 1) : dr_resolve(A.prev[j], L);
  if (row < 0) return;
  const int64_t tok = D.tokens[row];
  const int64_t ptok = pv >= 0 ? D.tokens[pv] : -1;
  D.codes[static_cast<int64_t>(row) * D.R + r] = static_cast<uint8_t>(dr_lut_code(D, ptok, tok, r));
}

// Verification gather of tree nodes (fast path): the codes of fresh nodes come from the router
// tables (and are stored), the rest of each window from the state.     grid (cdiv(R, 32), P)
template <typename TT>
__global__ __launch_bounds__(256) void k_fast_gather(lng_drafter D, FastLevel F, int32_t root_dst, TT* __restrict__ out) {
  __shared__ int32_t srow[DR_MAXN];
  __shared__ int64_t rowsh[32][DR_MAXN];
  __shared__ uint8_t wc[DR_MAXN][32];
  __shared__ int64_t toks[2];
  const int j = blockIdx.y;
  // descriptor fields used in loops, read once (kernel-argument loads otherwise repeat per use)
  const int bits = D.bits, maxn = D.maxn, n_ord = D.n_orders;
  const int ord0 = D.orders[0], ord1 = D.orders[1], ord2 = D.orders[2], ord3 = D.orders[3];
  auto ord_at = [&](int oi) { return oi == 0 ? ord0 : (oi == 1 ? ord1 : (oi == 2 ? ord2 : ord3)); };
  const int L = *D.length;
  const int R = D.R, mask = (1 << bits) - 1;
  if (threadIdx.x < DR_MAXN) srow[threadIdx.x] = threadIdx.x < maxn ? dr_resolve(F.slot[j][threadIdx.x], L) : -1;
  if (threadIdx.x == 0) {
    const int32_t cr = dr_resolve(F.slot[j][maxn - 1], L);
    const int32_t pv = dr_resolve(F.prev[j], L);
    toks[0] = cr >= 0 ? D.tokens[cr] : -1;
    toks[1] = pv >= 0 ? D.tokens[pv] : -1;
  }
  if (root_dst >= 0 && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0)
    D.tokens[root_dst] = L > 0 ? D.tokens[L - 1] : -1;
  __syncthreads();
  const bool fresh = F.fresh[j] != 0;
  const int r0 = blockIdx.x * 32;
  const int nr = min(32, R - r0);
  const int32_t cur_row = srow[maxn - 1];
  if (threadIdx.x < nr * maxn) {
    const int k = threadIdx.x / nr, rr = threadIdx.x % nr, r = r0 + rr;
    int c = 0;
    if (k == maxn - 1 && fresh)
      c = dr_lut_code4(D, toks[1], toks[0], r);
    else if (srow[k] >= 0)
      c = D.codes[static_cast<int64_t>(srow[k]) * R + r] & mask;
    wc[k][rr] = static_cast<uint8_t>(c);
  }
  __syncthreads();
  if (fresh && cur_row >= 0 && threadIdx.x < nr) D.codes[static_cast<int64_t>(cur_row) * R + r0 + threadIdx.x] = wc[maxn - 1][threadIdx.x];
  if (threadIdx.x < nr * n_ord) {
    const int rr = threadIdx.x / n_ord, oi = threadIdx.x % n_ord;
    const int n = ord_at(oi);
    int64_t addr = 0;
    bool ok = true;
    for (int k = 0; k < n; ++k) {
      const int slot = maxn - n + k;
      ok = ok && srow[slot] >= 0;
      addr |= static_cast<int64_t>(wc[slot][rr]) << (k * bits);
    }
    rowsh[rr][oi] = ok ? static_cast<int64_t>(r0 + rr) * (int64_t{1} << (bits * n)) + addr : -1;
  }
  __syncthreads();
  const int md = D.mem_dim, Dt = D.dt;
  const TT* const* tabs = reinterpret_cast<const TT* const*>(D.tables);
  constexpr int VE = 16 / sizeof(TT);  // elements per 16-byte piece
  if (md % VE == 0) {
    typedef uint32_t piece_t __attribute__((ext_vector_type(4)));
    const int pieces = md / VE;
    for (int e = threadIdx.x; e < nr * n_ord * pieces; e += 256) {
      const int pc = e % pieces, ro_ = e / pieces, oi = ro_ % n_ord, rr = ro_ / n_ord;
      const int64_t row = rowsh[rr][oi];
      piece_t v = {0u, 0u, 0u, 0u};
      if (row >= 0) v = *reinterpret_cast<const piece_t*>(tabs[oi] + row * md + VE * pc);
      *reinterpret_cast<piece_t*>(out + (static_cast<int64_t>(j) * R + r0 + rr) * Dt + oi * md + VE * pc) = v;
    }
  } else {
    for (int e = threadIdx.x; e < nr * Dt; e += 256) {
      const int rr = e / Dt, i = e % Dt, oi = i / md;
      const int64_t row = rowsh[rr][oi];
      out[(static_cast<int64_t>(j) * R + r0 + rr) * Dt + i] = row >= 0 ? tabs[oi][row * md + (i % md)] : TT(0.f);
    }
  }
}

// ------------------------------------------------------------------ host side
namespace {

// ------------------------------------------------------------------ small-batch readout and advance
// The per-token launches of a chain draft (at most SM_P positions): one weight row per wave, its
// 16-byte loads issued before the block stages the inputs, so each launch has hundreds of blocks
// with their row loads in flight (the general kernels above amortise rows over 16 positions).
constexpr int SM_P = 4;       // positions
constexpr int SM_RC = 8;      // routes per attention block
constexpr int SM_MAXCH = 32;  // attention blocks per position (R <= 256)

__device__ __forceinline__ const void* dr_table(const lng_drafter& D, int oi) {
  return oi == 0 ? D.tables[0] : (oi == 1 ? D.tables[1] : (oi == 2 ? D.tables[2] : D.tables[3]));
}

// qkw[j, o] = r_j * QK[o] . e_j (+ QKS[o] . s_j); wave w of block b computes row o = 4b + w, wave j
// stages position j's embedding row and RMS factor.              grid (cdiv(QH*Dt, 4))
__global__ __launch_bounds__(256) void k_sm_qkw(lng_drafter D, DrWin W, float* __restrict__ qkw) {
  __shared__ __attribute__((aligned(16))) float es[SM_P][LNG_DR_MAX_D];
  __shared__ __attribute__((aligned(16))) float ss[SM_P][LNG_DR_MAX_N];
  __shared__ float rj[SM_P];
  constexpr int NQ = LNG_DR_MAX_D / 256;
  const int d = D.d, d4 = d >> 2, P = W.n, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int N = D.query_ssm ? D.ssm_dim : 0, QD = D.q_heads * D.dt;
  const int o = blockIdx.x * 4 + w;
  const bool live = o < QD;
  f32x4 wq[NQ];
  const f32x4* qr = reinterpret_cast<const f32x4*>(D.qk + static_cast<int64_t>(live ? o : 0) * d);
#pragma unroll
  for (int q = 0; q < NQ; ++q)
    wq[q] = (live && lane + 64 * q < d4) ? qr[lane + 64 * q] : f32x4{0.f, 0.f, 0.f, 0.f};
  f32x4 wsq = {0.f, 0.f, 0.f, 0.f};
  if (live && lane < (N >> 2)) wsq = reinterpret_cast<const f32x4*>(D.qks + static_cast<int64_t>(o) * N)[lane];
  const int L = *D.length;
  if (w < P) {
    const int32_t row = dr_resolve(W.slot[w][D.maxn - 1], L);
    const int64_t tok = row >= 0 ? D.tokens[row] : -1;
    const bool ok = dr_tok_ok(D, tok);
    float sq = 0.f;
    for (int c4 = lane; c4 < d4; c4 += 64) {
      const f32x4 v = ok ? ld4_any(D.emb, D.emb_dtype, tok * d + 4 * c4) : f32x4{0.f, 0.f, 0.f, 0.f};
      *reinterpret_cast<f32x4*>(&es[w][4 * c4]) = v;
      sq = dot4(v, v, sq);
    }
    sq = wave_sum(sq);
    if (lane == 0) rj[w] = 1.0f / sqrtf(sq / static_cast<float>(d) + D.draft_eps);
    for (int c = lane; c < N; c += 64) ss[w][c] = row >= 0 ? D.ssm[static_cast<int64_t>(row) * D.ssm_dim + c] : 0.f;
  }
  __syncthreads();
  if (!live) return;
  float acc[SM_P] = {0.f, 0.f, 0.f, 0.f}, accs[SM_P] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int c4 = lane + 64 * q;
    if (c4 < d4) {
#pragma unroll
      for (int jj = 0; jj < SM_P; ++jj)
        if (jj < P) acc[jj] = dot4(wq[q], *reinterpret_cast<const f32x4*>(&es[jj][4 * c4]), acc[jj]);
    }
  }
  if (lane < (N >> 2)) {
#pragma unroll
    for (int jj = 0; jj < SM_P; ++jj)
      if (jj < P) accs[jj] = dot4(wsq, *reinterpret_cast<const f32x4*>(&ss[jj][4 * lane]), accs[jj]);
  }
#pragma unroll
  for (int jj = 0; jj < SM_P; ++jj) {
    if (jj >= P) break;
    const float a = wave_sum(acc[jj]);
    const float b = wave_sum(accs[jj]);
    if (lane == 0) qkw[static_cast<int64_t>(jj) * QD + o] = rj[jj] * a + b;
  }
}

// Partial sink-free softmax of position j over SM_RC routes for every query head, then the last
// block of the position merges the chunks with the sink into u[j] [QH * Dt]:
//   part_u [((j * nch + c) * QH + qh) * Dt + i], part_ml [((j * nch + c) * QH + qh) * 2 + {0, 1}] = (m, l)
// (device-coherent hand-off; sync[SY_ATT + j] counts the blocks).       grid (nch (+1), P)
// With LIST, block nch of each position builds its sketch shortlist meanwhile (it needs only the
// window's codes) into lists [P][1 + cap]: the length, then the ids.
template <bool LIST>
__global__ __launch_bounds__(256) void k_sm_attend(lng_drafter D, DrWin W, const float* __restrict__ qkw,
                                                   float* __restrict__ part_u, float* __restrict__ part_ml,
                                                   float* __restrict__ u, SlArgs S, int32_t* __restrict__ lists) {
  if constexpr (LIST) {
    if (blockIdx.x == gridDim.x - 1) {
      __shared__ int32_t sl[SL_MAXCAP];
      const int j = blockIdx.y;
      const int n = sl_build(D, W, S, j, sl);
      int32_t* lj = lists + static_cast<int64_t>(j) * (S.cap + 1);
      if (threadIdx.x == 0) lj[0] = n;
      for (int i = threadIdx.x; i < n; i += 256) lj[1 + i] = sl[i];
      return;
    }
  }
  __shared__ __attribute__((aligned(16))) float xs[SM_RC][LNG_DR_MAX_DT];
  __shared__ __attribute__((aligned(16))) float qs[LNG_DR_MAX_QH * LNG_DR_MAX_DT];
  __shared__ float sxs[SM_RC];
  __shared__ float sc[LNG_DR_MAX_QH][SM_RC];
  __shared__ int64_t rowsh[SM_RC][DR_MAXN];
  __shared__ int32_t slot_rows[DR_MAXN];
  __shared__ float mls[LNG_DR_MAX_QH][SM_MAXCH][2];
  __shared__ float scl[LNG_DR_MAX_QH][SM_MAXCH];
  __shared__ int last_flag;
  const int j = blockIdx.y, c = blockIdx.x, nch = gridDim.x - (LIST ? 1 : 0);
  const int L = *D.length;
  const int Dt = D.dt, D4 = Dt >> 2, QH = D.q_heads, md = D.mem_dim, QD = QH * Dt;
  const int r0 = c * SM_RC, nr = min(SM_RC, D.R - r0);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (threadIdx.x < DR_MAXN) slot_rows[threadIdx.x] = threadIdx.x < D.maxn ? dr_resolve(W.slot[j][threadIdx.x], L) : -1;
  const float* qv = qkw + static_cast<int64_t>(j) * QD;
  for (int e = threadIdx.x; e < (QD >> 2); e += 256)
    reinterpret_cast<f32x4*>(qs)[e] = reinterpret_cast<const f32x4*>(qv)[e];
  __syncthreads();
  if (threadIdx.x < nr * D.n_orders) {
    const int rr = threadIdx.x / D.n_orders, oi = threadIdx.x % D.n_orders;
    rowsh[rr][oi] = dr_row(D, slot_rows, oi, r0 + rr);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < nr * D4; e += 256) {
    const int rr = e / D4, i = 4 * (e % D4), oi = i / md;
    const int64_t row = rowsh[rr][oi];
    *reinterpret_cast<f32x4*>(&xs[rr][i]) =
        row >= 0 ? ld4_any(dr_table(D, oi), D.table_dtype, row * md + (i % md)) : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  __syncthreads();
  for (int rr = w; rr < nr; rr += 4) {
    float ss = 0.f;
    for (int i = lane; i < Dt; i += 64) ss = fmaf(xs[rr][i], xs[rr][i], ss);
    ss = wave_sum(ss);
    const float s = 1.0f / sqrtf(ss / static_cast<float>(Dt) + D.mem_eps);
    if (lane == 0) sxs[rr] = s;
    for (int qh = 0; qh < QH; ++qh) {
      float a = 0.f;
      for (int i = lane; i < Dt; i += 64) a = fmaf(qs[qh * Dt + i], xs[rr][i], a);
      a = wave_sum(a);
      if (lane == 0) sc[qh][rr] = s * a;
    }
  }
  __syncthreads();
  const uint32_t nrec = gridDim.y * static_cast<uint32_t>(nch) * QH;
  const __amdgpu_buffer_rsrc_t ru = dev_buf(part_u, nrec * static_cast<uint32_t>(Dt) * 4u);
  for (int e = threadIdx.x; e < QH * D4; e += 256) {
    const int qh = e / D4, i = 4 * (e % D4);
    float m = -INFINITY;
    for (int rr = 0; rr < nr; ++rr) m = fmaxf(m, sc[qh][rr]);
    float l = 0.f;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int rr = 0; rr < nr; ++rr) {
      const float p = expf(sc[qh][rr] - m);
      l += p;
      const float ps = p * sxs[rr];
      const f32x4 x = *reinterpret_cast<const f32x4*>(&xs[rr][i]);
      acc.x = fmaf(ps, x.x, acc.x);
      acc.y = fmaf(ps, x.y, acc.y);
      acc.z = fmaf(ps, x.z, acc.z);
      acc.w = fmaf(ps, x.w, acc.w);
    }
    const uint32_t rec = (static_cast<uint32_t>(j) * nch + c) * QH + qh;
    st_dev4(ru, 4u * (rec * Dt + i), acc);
    if (i == 0) {
      st_dev(&part_ml[2 * rec], m);
      st_dev(&part_ml[2 * rec + 1], l);
    }
  }
  if (!dr_last_block(&D.sync[SY_ATT + j], nch, &last_flag)) return;
  // merge: per head the sink-seeded normaliser and each chunk's weight
  for (int e = threadIdx.x; e < QH * nch; e += 256) {
    const int qh = e / nch, cc = e % nch;
    const uint32_t rec = (static_cast<uint32_t>(j) * nch + cc) * QH + qh;
    mls[qh][cc][0] = ld_dev(&part_ml[2 * rec]);
    mls[qh][cc][1] = ld_dev(&part_ml[2 * rec + 1]);
  }
  __syncthreads();
  if (threadIdx.x < QH) {
    const int qh = threadIdx.x;
    const float b0 = D.sink_logit;
    float M = b0;
    for (int cc = 0; cc < nch; ++cc) M = fmaxf(M, mls[qh][cc][0]);
    float l = expf(b0 - M);
    for (int cc = 0; cc < nch; ++cc) {
      const float f = expf(mls[qh][cc][0] - M);
      l = fmaf(mls[qh][cc][1], f, l);
      scl[qh][cc] = f;
    }
    for (int cc = 0; cc < nch; ++cc) scl[qh][cc] /= l;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < QH * D4; e += 256) {
    const int qh = e / D4, i = 4 * (e % D4);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int c0 = 0; c0 < nch; c0 += 8) {
      f32x4 v[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const uint32_t rec = (static_cast<uint32_t>(j) * nch + c0 + q) * QH + qh;
        v[q] = c0 + q < nch ? ld_dev4(ru, 4u * (rec * Dt + i)) : f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        if (c0 + q >= nch) break;
        const float f = scl[qh][c0 + q];
        acc.x = fmaf(v[q].x, f, acc.x);
        acc.y = fmaf(v[q].y, f, acc.y);
        acc.z = fmaf(v[q].z, f, acc.z);
        acc.w = fmaf(v[q].w, f, acc.w);
      }
    }
    *reinterpret_cast<f32x4*>(u + static_cast<int64_t>(j) * QD + qh * Dt + i) = acc;
  }
}

// hid[j, o] = OV[o] . u_j, one row per wave.                          grid (cdiv(d, 4))
__global__ __launch_bounds__(256) void k_sm_hidden(lng_drafter D, int32_t P, const float* __restrict__ u,
                                                   float* __restrict__ hid) {
  extern __shared__ __attribute__((aligned(16))) float us[];  // [P][QD]
  constexpr int NQ = LNG_DR_MAX_QH * LNG_DR_MAX_DT / 256;
  const int QD = D.q_heads * D.dt, Q4 = QD >> 2, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int o = blockIdx.x * 4 + w;
  const bool live = o < D.d;
  f32x4 wv[NQ];
  const f32x4* wr = reinterpret_cast<const f32x4*>(D.ov + static_cast<int64_t>(live ? o : 0) * QD);
#pragma unroll
  for (int q = 0; q < NQ; ++q) wv[q] = (live && lane + 64 * q < Q4) ? wr[lane + 64 * q] : f32x4{0.f, 0.f, 0.f, 0.f};
  for (int e = threadIdx.x; e < P * Q4; e += 256) reinterpret_cast<f32x4*>(us)[e] = reinterpret_cast<const f32x4*>(u)[e];
  __syncthreads();
  if (!live) return;
  float acc[SM_P] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int c4 = lane + 64 * q;
    if (c4 < Q4) {
#pragma unroll
      for (int jj = 0; jj < SM_P; ++jj)
        if (jj < P) acc[jj] = dot4(wv[q], reinterpret_cast<const f32x4*>(us)[jj * Q4 + c4], acc[jj]);
    }
  }
#pragma unroll
  for (int jj = 0; jj < SM_P; ++jj) {
    if (jj >= P) break;
    const float a = wave_sum(acc[jj]);
    if (lane == 0) hid[static_cast<int64_t>(jj) * D.d + o] = a;
  }
}

// SSM step of up to SM_P positions in one launch: u_j[n] = W_in[n] . (RMSNorm(E[tok_j]) *
// ssm_norm), then s[row_j][n] = a_n s[prev_j][n] + (1 - a_n) u_j[n] in position order (a chain in
// the batch reads the state the same lane wrote for the earlier position).  One channel per wave.
//                                                                   grid (cdiv(N, 4))
__global__ __launch_bounds__(256) void k_sm_ssm(lng_drafter D, DrAdv A) {
  __shared__ __attribute__((aligned(16))) float xs[SM_P][LNG_DR_MAX_D];
  constexpr int NQ = LNG_DR_MAX_D / 256;
  const int d = D.d, d4 = d >> 2, N = D.ssm_dim, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int n = blockIdx.x * 4 + w;
  const bool live = n < N;
  f32x4 wq[NQ];
  const f32x4* wr = reinterpret_cast<const f32x4*>(D.ssm_w_in + static_cast<int64_t>(live ? n : 0) * d);
#pragma unroll
  for (int q = 0; q < NQ; ++q)
    wq[q] = (live && lane + 64 * q < d4) ? wr[lane + 64 * q] : f32x4{0.f, 0.f, 0.f, 0.f};
  const int L = *D.length;
  if (w < A.n) {
    const int32_t row = A.range ? A.base + w : dr_resolve(A.row[w], L);
    const int64_t tok = row >= 0 ? D.tokens[row] : -1;
    const bool ok = dr_tok_ok(D, tok);
    float sq = 0.f;
    for (int c4 = lane; c4 < d4; c4 += 64) {
      const f32x4 v = ok ? ld4_any(D.emb, D.emb_dtype, tok * d + 4 * c4) : f32x4{0.f, 0.f, 0.f, 0.f};
      *reinterpret_cast<f32x4*>(&xs[w][4 * c4]) = v;
      sq = dot4(v, v, sq);
    }
    sq = wave_sum(sq);
    const float r = 1.0f / sqrtf(sq / static_cast<float>(d) + D.ssm_eps);
    for (int c4 = lane; c4 < d4; c4 += 64) {
      f32x4 v = *reinterpret_cast<const f32x4*>(&xs[w][4 * c4]);
      const f32x4 g = reinterpret_cast<const f32x4*>(D.ssm_norm)[c4];
      v.x = v.x * r * g.x;
      v.y = v.y * r * g.y;
      v.z = v.z * r * g.z;
      v.w = v.w * r * g.w;
      *reinterpret_cast<f32x4*>(&xs[w][4 * c4]) = v;
    }
  }
  __syncthreads();
  if (!live) return;
  float acc[SM_P] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int c4 = lane + 64 * q;
    if (c4 < d4) {
#pragma unroll
      for (int jj = 0; jj < SM_P; ++jj)
        if (jj < A.n) acc[jj] = dot4(wq[q], *reinterpret_cast<const f32x4*>(&xs[jj][4 * c4]), acc[jj]);
    }
  }
  float uj[SM_P];
#pragma unroll
  for (int jj = 0; jj < SM_P; ++jj) uj[jj] = jj < A.n ? wave_sum(acc[jj]) : 0.f;
  if (lane == 0) {
    const float a = D.ssm_decay[n];
#pragma unroll
    for (int jj = 0; jj < SM_P; ++jj) {
      if (jj >= A.n) break;
      const int32_t row = A.range ? A.base + jj : dr_resolve(A.row[jj], L);
      const int32_t pv = A.range ? (jj == 0 ? dr_resolve(A.prev0, L) : A.base + jj - 1) : dr_resolve(A.prev[jj], L);
      if (row < 0) continue;
      const float sp = pv >= 0 ? D.ssm[static_cast<int64_t>(pv) * N + n] : 0.f;
      D.ssm[static_cast<int64_t>(row) * N + n] = a * sp + (1.f - a) * uj[jj];
    }
  }
}

// Router codes of up to SM_P positions, one route per block: wave b < bits computes bit b's logit
// router[r*bits + b] . f_j, f_j = concat(RMSNorm(E[prev_j] or start) * prev_norm,
// RMSNorm(E[tok_j]) * cur_norm [, s[row_j]]) (F = 2d (+N) floats per position in LDS).  grid (R)
template <typename TR>
__global__ __launch_bounds__(256) void k_sm_codes(lng_drafter D, DrAdv A) {
  extern __shared__ __attribute__((aligned(16))) float fs[];  // [n][F]
  __shared__ float lg[SM_P][4];
  __shared__ int32_t rows[SM_P];
  constexpr int NQ = (2 * LNG_DR_MAX_D + LNG_DR_MAX_N + 511) / 512;
  const int d = D.d, d4 = d >> 2, N = D.router_ssm ? D.ssm_dim : 0, F = 2 * d + N, F8 = F >> 3;
  const int r = blockIdx.x, bits = D.bits, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const bool live = w < bits;
  const TR* wrow = static_cast<const TR*>(D.router) + (static_cast<int64_t>(r) * bits + (live ? w : 0)) * F;
  f32x4 wa[NQ], wb[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    if (live && lane + 64 * q < F8) {
      ld8f<TR>(wrow + 8 * (lane + 64 * q), wa[q], wb[q]);
    } else {
      wa[q] = f32x4{0.f, 0.f, 0.f, 0.f};
      wb[q] = wa[q];
    }
  }
  const int L = *D.length;
  if (threadIdx.x < A.n) {
    const int jj = threadIdx.x;
    rows[jj] = A.range ? A.base + jj : dr_resolve(A.row[jj], L);
  }
  for (int t = w; t < 2 * A.n; t += 4) {
    const int jj = t >> 1, half = t & 1;
    const int32_t row = A.range ? A.base + jj : dr_resolve(A.row[jj], L);
    const int32_t pv = A.range ? (jj == 0 ? dr_resolve(A.prev0, L) : A.base + jj - 1) : dr_resolve(A.prev[jj], L);
    if (row < 0) continue;
    const bool use_start = half == 0 && pv < 0;
    const int64_t tk = half == 0 ? (pv >= 0 ? D.tokens[pv] : 0) : D.tokens[row];
    const bool ok = dr_tok_ok(D, tk);
    const float* nw = half == 0 ? D.router_prev_norm : D.router_cur_norm;
    float* f = fs + jj * F + half * d;
    float sq = 0.f;
    for (int c4 = lane; c4 < d4; c4 += 64) {
      const f32x4 v = use_start ? reinterpret_cast<const f32x4*>(D.router_start)[c4]
                                : (ok ? ld4_any(D.emb, D.emb_dtype, tk * d + 4 * c4) : f32x4{0.f, 0.f, 0.f, 0.f});
      *reinterpret_cast<f32x4*>(f + 4 * c4) = v;
      sq = dot4(v, v, sq);
    }
    sq = wave_sum(sq);
    const float rs = 1.0f / sqrtf(sq / static_cast<float>(d) + D.router_eps);
    for (int c4 = lane; c4 < d4; c4 += 64) {
      f32x4 v = *reinterpret_cast<const f32x4*>(f + 4 * c4);
      const f32x4 g = reinterpret_cast<const f32x4*>(nw)[c4];
      v.x = v.x * rs * g.x;
      v.y = v.y * rs * g.y;
      v.z = v.z * rs * g.z;
      v.w = v.w * rs * g.w;
      *reinterpret_cast<f32x4*>(f + 4 * c4) = v;
    }
  }
  for (int e = threadIdx.x; e < A.n * N; e += 256) {
    const int jj = e / N, c = e % N;
    const int32_t row = A.range ? A.base + jj : dr_resolve(A.row[jj], L);
    fs[jj * F + 2 * d + c] = row >= 0 ? D.ssm[static_cast<int64_t>(row) * D.ssm_dim + c] : 0.f;
  }
  __syncthreads();
  if (live) {
    float acc[SM_P] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int c8 = lane + 64 * q;
      if (c8 < F8) {
#pragma unroll
        for (int jj = 0; jj < SM_P; ++jj) {
          if (jj >= A.n) break;
          const float* f = fs + jj * F + 8 * c8;
          acc[jj] = dot4(wb[q], *reinterpret_cast<const f32x4*>(f + 4),
                         dot4(wa[q], *reinterpret_cast<const f32x4*>(f), acc[jj]));
        }
      }
    }
#pragma unroll
    for (int jj = 0; jj < SM_P; ++jj) {
      if (jj >= A.n) break;
      const float s = wave_sum(acc[jj]);
      if (lane == 0) lg[jj][w] = s;
    }
  }
  __syncthreads();
  if (threadIdx.x < A.n && rows[threadIdx.x] >= 0) {
    const int jj = threadIdx.x;
    int code = 0;
    for (int b = 0; b < bits; ++b) code |= (lg[jj][b] > 0.f ? 1 : 0) << b;
    D.codes[static_cast<int64_t>(rows[jj]) * D.R + r] = static_cast<uint8_t>(code);
  }
}

struct DrLayout {
  size_t u, qkw, part, hid, logits, lpart, w, fpart, ro, tot, flpart, cand, smu, smml, smout, need, lists, total;
  int nch, nblk, fnch, fnblk, smch;
};

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

DrLayout dr_layout(const lng_drafter& D, int P, int K, int max_pairs) {
  DrLayout l{};
  l.nch = static_cast<int>(cdiv(D.R, DR_RC));
  l.nblk = static_cast<int>(cdiv(D.V, DR_VB));
  const int QD = D.q_heads * D.dt;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off = align256(off + bytes);
    return o;
  };
  l.u = take(sizeof(float) * static_cast<size_t>(DR_ADV_CHUNK) * std::max(D.ssm_dim, 1));
  l.qkw = take(sizeof(float) * P * QD);
  l.part = take(sizeof(float) * static_cast<size_t>(P) * l.nch * D.q_heads * (D.dt + 2));
  l.hid = take(sizeof(float) * P * D.d);
  l.logits = take(sizeof(float) * static_cast<size_t>(P) * D.V);
  l.lpart = take(sizeof(float) * static_cast<size_t>(P) * l.nblk * (2 + 2 * K));
  l.w = take(sizeof(int32_t) * static_cast<size_t>(P) * std::max(max_pairs, 1));
  l.fnch = static_cast<int>(cdiv(D.R, FA_RC));
  l.fnblk = static_cast<int>(cdiv(D.V, FL_VB));
  const int I = D.q_heads * D.head_dim;
  l.fpart = take(sizeof(float) * static_cast<size_t>(P) * l.fnch * fa_rec(D.q_heads, D.q_heads * D.head_dim));
  l.ro = take(sizeof(float) * P * I);
  l.tot = 0;
  l.flpart = take(sizeof(float) * static_cast<size_t>(P) * l.fnblk * fl_rs<DR_MAXK>());
  l.cand = take(sizeof(int4) * static_cast<size_t>(P) * l.fnblk * FL_VB);
  l.smch = static_cast<int>(cdiv(D.R, SM_RC));
  l.smu = take(sizeof(float) * static_cast<size_t>(std::min(P, SM_P)) * l.smch * QD);
  l.smml = take(sizeof(float) * static_cast<size_t>(std::min(P, SM_P)) * l.smch * D.q_heads * 2);
  l.smout = take(sizeof(float) * static_cast<size_t>(std::min(P, SM_P)) * QD);
  l.need = take(sizeof(int32_t) * DR_MAXP);
  l.lists = take(sizeof(int32_t) * static_cast<size_t>(std::min(P, SM_P)) * (SL_MAXCAP + 1));
  l.total = off;
  return l;
}

// The small-batch kernels apply: at most SM_P positions, 16-byte row loads (d % 8, Dt % 4, mem_dim
// % 4, N % 8), the block counters of sync, and the codes kernel's features within 64 KB of LDS.
bool sm_ok(const lng_drafter& D, int P) {
  return P >= 1 && P <= SM_P && D.sync && D.d % 8 == 0 && D.dt % 4 == 0 && D.mem_dim % 4 == 0 &&
         D.ssm_dim % 8 == 0 && cdiv(D.R, SM_RC) <= SM_MAXCH;
}
bool sm_adv_ok(const lng_drafter& D, int n) {
  const int F = 2 * D.d + (D.router_ssm ? D.ssm_dim : 0);
  return n >= 1 && n <= SM_P && D.d % 8 == 0 && D.ssm_dim % 8 == 0 && D.bits <= 4 &&
         static_cast<size_t>(n) * F * sizeof(float) <= 65536;
}

bool dr_fast(const lng_drafter& D) {
  const int I = D.q_heads * D.head_dim;
  return D.lut_prev && D.lut_cur && D.lut_start && D.lut_qk && D.lut_out && D.gram_out && D.wv_t && D.sync &&
         !D.router_ssm && !D.query_ssm && I <= FL_I && I % 16 == 0 && D.head_dim % 4 == 0 && D.dt % 64 == 0 &&
         cdiv(D.V, FL_VB) <= FL_NBL * 64;
}

int dr_check(const lng_drafter* D, const char* what) {
  if (!D) return fail(LNG_E_ARG, std::string(what) + ": null drafter");
  const lng_drafter& d = *D;
  if (d.d <= 0 || d.d > LNG_DR_MAX_D || d.V <= 0 || d.R <= 0 || d.R > 256 || d.bits <= 0 || d.bits > 4 ||
      d.mem_dim <= 0 || d.n_orders <= 0 || d.n_orders > 4 || d.dt != d.n_orders * d.mem_dim || d.dt > LNG_DR_MAX_DT ||
      d.maxn <= 0 || d.maxn > DR_MAXN || d.q_heads <= 0 || d.q_heads > LNG_DR_MAX_QH || d.kv_heads <= 0 ||
      d.q_heads % d.kv_heads || d.ssm_dim < 0 || d.ssm_dim > LNG_DR_MAX_N || d.rows <= 0)
    return fail(LNG_E_ARG, std::string(what) + ": drafter shape out of range");
  for (int i = 0; i < d.n_orders; ++i)
    if (d.orders[i] < 1 || d.orders[i] > d.maxn || !d.tables[i])
      return fail(LNG_E_ARG, std::string(what) + ": bad n-gram order / table");
  if ((d.router_ssm || d.query_ssm) && (d.ssm_dim <= 0 || !d.ssm))
    return fail(LNG_E_ARG, std::string(what) + ": SSM inputs need ssm_dim > 0 and state rows");
  if (d.query_ssm && !d.qks) return fail(LNG_E_ARG, std::string(what) + ": query_ssm needs qks");
  if (!d.emb || !d.router || !d.qk || !d.ov || !d.tokens || !d.codes || !d.length)
    return fail(LNG_E_ARG, std::string(what) + ": missing pointer");
  for (int dt : {d.emb_dtype, d.table_dtype, d.router_dtype})
    if (dt != LNG_F32 && dt != LNG_BF16 && dt != LNG_F16) return fail(LNG_E_DTYPE, std::string(what) + ": dtype");
  return LNG_OK;
}

bool spec_ok(const lng_drafter& D, int32_t v) { return v == LNG_ROW_NONE || v < 0 || v < D.rows; }

int dr_advance(const lng_drafter& D, const DrAdv& A, int from_router, float* u, hipStream_t s) {
  if (A.n == 0) return LNG_OK;
  if (dr_fast(D)) {
    if (!from_router) return LNG_OK;
    hipLaunchKernelGGL(k_fast_codes, dim3(static_cast<unsigned>(cdiv(D.R, 256)), static_cast<unsigned>(A.n)),
                       dim3(256), 0, s, D, A);
    return check_launch("drafter_advance(fast codes)");
  }
  const bool has_ssm = D.ssm_dim > 0 && D.ssm && D.ssm_w_in;
  if (sm_adv_ok(D, A.n)) {
    if (has_ssm) {
      hipLaunchKernelGGL(k_sm_ssm, dim3(static_cast<unsigned>(cdiv(D.ssm_dim, 4))), dim3(256), 0, s, D, A);
      if (int rc = check_launch("drafter_advance(ssm)")) return rc;
    }
    if (from_router) {
      const size_t lds = sizeof(float) * A.n * (2 * D.d + (D.router_ssm ? D.ssm_dim : 0));
      const dim3 g(static_cast<unsigned>(D.R));
      if (D.router_dtype == LNG_BF16)
        hipLaunchKernelGGL(k_sm_codes<bf16>, g, dim3(256), lds, s, D, A);
      else if (D.router_dtype == LNG_F16)
        hipLaunchKernelGGL(k_sm_codes<_Float16>, g, dim3(256), lds, s, D, A);
      else
        hipLaunchKernelGGL(k_sm_codes<float>, g, dim3(256), lds, s, D, A);
      if (int rc = check_launch("drafter_advance(codes)")) return rc;
    }
    return LNG_OK;
  }
  if (has_ssm) {
    hipLaunchKernelGGL(k_draft_ssm_u, dim3(static_cast<unsigned>(cdiv(D.ssm_dim, 16)), static_cast<unsigned>(cdiv(A.n, 4))),
                       dim3(256), 0, s, D, A, u);
    if (int rc = check_launch("drafter_advance(ssm_u)")) return rc;
    hipLaunchKernelGGL(k_draft_ssm_scan, dim3(static_cast<unsigned>(cdiv(D.ssm_dim, 256))), dim3(256), 0, s, D, A, u);
    if (int rc = check_launch("drafter_advance(ssm_scan)")) return rc;
  }
  if (from_router) {
    hipLaunchKernelGGL(k_draft_codes, dim3(static_cast<unsigned>(cdiv(D.R, 4)), static_cast<unsigned>(cdiv(A.n, 4))),
                       dim3(256), 0, s, D, A);
    if (int rc = check_launch("drafter_advance(codes)")) return rc;
  }
  return LNG_OK;
}

int dr_windows(const lng_drafter& D, const int32_t* windows, int32_t P, DrWin& W) {
  if (P <= 0 || P > DR_MAXP) return fail(LNG_E_ARG, "drafter: 1 <= positions <= 16");
  W = DrWin{};
  W.n = P;
  for (int j = 0; j < P; ++j)
    for (int k = 0; k < D.maxn; ++k) {
      const int32_t v = windows[j * D.maxn + k];
      if (!spec_ok(D, v)) return fail(LNG_E_RANGE, "drafter: window row out of range");
      W.slot[j][k] = v;
    }
  return LNG_OK;
}

int dr_readout_fast(const lng_drafter& D, const FastLevel& F, int K, int online, float kappa, const DrChildren& C,
                    char* work, size_t work_bytes, int32_t* counts, int64_t* ids, float* scores, float* logits_out,
                    hipStream_t s) {
  const int P = F.P;
  const int max_pairs = D.rows;
  const DrLayout l = dr_layout(D, P, K, online ? max_pairs : 1);
  if (work_bytes < l.total) return fail(LNG_E_ARG, "drafter: workspace too small");
  if (online && !counts) return fail(LNG_E_ARG, "drafter: online counts need the counts buffer");
  const int nob = online ? static_cast<int>(cdiv(max_pairs, FA_TB)) : 0;
  {
    const dim3 ga(static_cast<unsigned>(l.fnch + nob), static_cast<unsigned>(P));
    float* fpart = reinterpret_cast<float*>(work + l.fpart);
    float* fro = reinterpret_cast<float*>(work + l.ro);
    if (D.q_heads == 4 && D.dt == 256 && D.head_dim == 64 && D.n_orders == 2 && D.maxn == 3)  // the SD drafters
      hipLaunchKernelGGL((k_fast_attend<4, 256, 64, 2, 3>), ga, dim3(256), 0, s, D, F, l.fnch, nob, online, fpart, counts,
                         fro);
    else
      hipLaunchKernelGGL((k_fast_attend<0, 0, 0, 0, 0>), ga, dim3(256), 0, s, D, F, l.fnch, nob, online, fpart, counts,
                         fro);
  }
  if (int rc = check_launch("drafter_readout(fast attend)")) return rc;
  auto logits = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(l.fnblk)), dim3(256), 0, s, D, P, K, online, kappa,
                       reinterpret_cast<const float*>(work + l.ro), logits_out,
                       reinterpret_cast<float*>(work + l.flpart), counts, reinterpret_cast<int4*>(work + l.cand), C,
                       ids, scores);
  };
  const bool i256 = D.q_heads * D.head_dim == 256;  // the SD drafters' 4 x 64
  switch (K) {
    case 1: i256 ? logits(k_fast_logits<1, 256>) : logits(k_fast_logits<1, 0>); break;
    case 2: i256 ? logits(k_fast_logits<2, 256>) : logits(k_fast_logits<2, 0>); break;
    case 3: i256 ? logits(k_fast_logits<3, 256>) : logits(k_fast_logits<3, 0>); break;
    case 4: i256 ? logits(k_fast_logits<4, 256>) : logits(k_fast_logits<4, 0>); break;
    default: i256 ? logits(k_fast_logits<DR_MAXK, 256>) : logits(k_fast_logits<DR_MAXK, 0>); break;
  }
  return check_launch("drafter_readout(fast logits)");
}

// LDS of the general readout kernels (positions x width) within their 60 KB budget.
bool dr_lds_ok(const lng_drafter& D, int P) {
  const int QD = D.q_heads * D.dt;
  const int Nq = D.query_ssm ? D.ssm_dim : 0;
  const size_t lim = 60 * 1024;
  return sizeof(float) * P * (D.d + Nq) <= lim && sizeof(float) * P * QD <= lim && sizeof(float) * P * D.d <= lim;
}

// The readout of P positions up to the hidden states hid [P, d] (work + l.hid): query-key weights,
// attention over the routes, output projection.  sk (small-batch kernels only): the attention
// launch also builds each position's sketch shortlist into work + l.lists.
int dr_front(const lng_drafter& D, const DrWin& W, const DrLayout& l, char* work, hipStream_t s,
             const SlArgs* sk = nullptr) {
  const int P = W.n, QD = D.q_heads * D.dt;
  const int Nq = D.query_ssm ? D.ssm_dim : 0;
  float* qkw = reinterpret_cast<float*>(work + l.qkw);
  float* hid = reinterpret_cast<float*>(work + l.hid);
  if (sm_ok(D, P)) {
    float* pu = reinterpret_cast<float*>(work + l.smu);
    float* pml = reinterpret_cast<float*>(work + l.smml);
    float* uo = reinterpret_cast<float*>(work + l.smout);
    hipLaunchKernelGGL(k_sm_qkw, dim3(static_cast<unsigned>(cdiv(QD, 4))), dim3(256), 0, s, D, W, qkw);
    if (int rc = check_launch("drafter_readout(qkw)")) return rc;
    if (sk)
      hipLaunchKernelGGL(k_sm_attend<true>, dim3(static_cast<unsigned>(l.smch + 1), static_cast<unsigned>(P)),
                         dim3(256), 0, s, D, W, qkw, pu, pml, uo, *sk, reinterpret_cast<int32_t*>(work + l.lists));
    else
      hipLaunchKernelGGL(k_sm_attend<false>, dim3(static_cast<unsigned>(l.smch), static_cast<unsigned>(P)),
                         dim3(256), 0, s, D, W, qkw, pu, pml, uo, SlArgs{}, nullptr);
    if (int rc = check_launch("drafter_readout(attend)")) return rc;
    hipLaunchKernelGGL(k_sm_hidden, dim3(static_cast<unsigned>(cdiv(D.d, 4))), dim3(256), sizeof(float) * P * QD, s, D,
                       P, uo, hid);
    return check_launch("drafter_readout(hidden)");
  }
  float* part = reinterpret_cast<float*>(work + l.part);
  const size_t lds_q = sizeof(float) * P * (D.d + Nq);
  const size_t lds_h = sizeof(float) * P * QD;
  hipLaunchKernelGGL(k_draft_qkw, dim3(static_cast<unsigned>(cdiv(QD, 32))), dim3(256), lds_q, s, D, W, qkw);
  if (int rc = check_launch("drafter_readout(qkw)")) return rc;
  hipLaunchKernelGGL(k_draft_attend, dim3(static_cast<unsigned>(l.nch), static_cast<unsigned>(P)), dim3(256), 0, s, D,
                     W, qkw, part);
  if (int rc = check_launch("drafter_readout(attend)")) return rc;
  hipLaunchKernelGGL(k_draft_hidden, dim3(static_cast<unsigned>(cdiv(D.d, 16))), dim3(256), lds_h, s, D, P, l.nch, part,
                     hid);
  return check_launch("drafter_readout(hidden)");
}

// Full-vocabulary logits (logits_out, else the workspace) and the top-k of P positions from their
// hidden states; need (optional, [P]): only the positions with need[j] != 0 are drafted.
int dr_vocab(const lng_drafter& D, int P, int K, int online, float kappa, const DrChildren& C, const DrLayout& l,
             char* work, int max_pairs, int32_t* counts, int64_t* ids, float* scores, float* logits_out,
             const int32_t* need, hipStream_t s) {
  const float* hid = reinterpret_cast<const float*>(work + l.hid);
  float* logits = logits_out ? logits_out : reinterpret_cast<float*>(work + l.logits);
  float* lpart = reinterpret_cast<float*>(work + l.lpart);
  const int32_t* wbuf = reinterpret_cast<const int32_t*>(work + l.w);
  const size_t lds_l = sizeof(float) * P * D.d;
  const dim3 g(static_cast<unsigned>(l.nblk));
  auto launch = [&](auto kern) { hipLaunchKernelGGL(kern, g, dim3(256), lds_l, s, D, P, K, hid, logits, lpart, need); };
  const bool small = P <= SM_P;
  if (D.emb_dtype == LNG_BF16)
    small ? launch(k_draft_logits<bf16, SM_P>) : launch(k_draft_logits<bf16, DR_MAXP>);
  else if (D.emb_dtype == LNG_F16)
    small ? launch(k_draft_logits<_Float16, SM_P>) : launch(k_draft_logits<_Float16, DR_MAXP>);
  else
    small ? launch(k_draft_logits<float, SM_P>) : launch(k_draft_logits<float, DR_MAXP>);
  if (int rc = check_launch("drafter_readout(logits)")) return rc;
  hipLaunchKernelGGL(k_draft_select, dim3(static_cast<unsigned>(P)), dim3(256), 0, s, D, K, l.nblk, online, kappa, logits,
                     lpart, wbuf, max_pairs, counts, C, ids, scores, need);
  return check_launch("drafter_readout(select)");
}

int dr_readout(const lng_drafter& D, const DrWin& W, int K, int online, float kappa, const DrChildren& C,
               char* work, size_t work_bytes, int32_t* counts, int64_t* ids, float* scores, float* logits_out,
               hipStream_t s) {
  const int P = W.n;
  if (dr_fast(D)) {
    FastLevel F{};
    F.P = P;
    for (int j = 0; j < P; ++j) {
      for (int k = 0; k < DR_MAXN; ++k) F.slot[j][k] = W.slot[j][k];
      F.prev[j] = LNG_ROW_NONE;
      F.fresh[j] = 0;
    }
    return dr_readout_fast(D, F, K, online, kappa, C, work, work_bytes, counts, ids, scores, logits_out, s);
  }
  const int max_pairs = D.rows;  // the online kernel's grid covers any committed length
  const DrLayout l = dr_layout(D, P, K, online ? max_pairs : 1);
  if (work_bytes < l.total) return fail(LNG_E_ARG, "drafter: workspace too small");
  if (online && !counts) return fail(LNG_E_ARG, "drafter: online counts need the counts buffer");
  if (!dr_lds_ok(D, P)) return fail(LNG_E_ARG, "drafter: too many positions for this width");
  if (int rc = dr_front(D, W, l, work, s)) return rc;
  if (online) {
    int32_t* wbuf = reinterpret_cast<int32_t*>(work + l.w);
    hipLaunchKernelGGL(k_draft_online_match, dim3(static_cast<unsigned>(cdiv(max_pairs, DR_TB)), static_cast<unsigned>(P)),
                       dim3(256), 0, s, D, W, wbuf, counts, max_pairs);
    if (int rc = check_launch("drafter_readout(online)")) return rc;
  }
  return dr_vocab(D, P, K, online, kappa, C, l, work, max_pairs, counts, ids, scores, logits_out, nullptr, s);
}

int dr_gather(const lng_drafter& D, const DrWin& W, void* out, hipStream_t s) {
  const dim3 g(static_cast<unsigned>(cdiv(D.R, 32)), static_cast<unsigned>(W.n));
  if (D.table_dtype == LNG_BF16)
    hipLaunchKernelGGL(k_draft_gather<bf16>, g, dim3(256), 0, s, D, W, static_cast<bf16*>(out));
  else if (D.table_dtype == LNG_F16)
    hipLaunchKernelGGL(k_draft_gather<_Float16>, g, dim3(256), 0, s, D, W, static_cast<_Float16*>(out));
  else
    hipLaunchKernelGGL(k_draft_gather<float>, g, dim3(256), 0, s, D, W, static_cast<float*>(out));
  return check_launch("drafter_gather");
}

// Sketch arguments of the shortlist launches, checked against the drafter's shape.
int sl_args(const lng_drafter& D, const lng_sketch* S, SlArgs& A) {
  if (!S) return fail(LNG_E_ARG, "drafter_shortlist: null sketch");
  if (S->cap < 1 || S->cap > SL_MAXCAP) return fail(LNG_E_ARG, "drafter_shortlist: 1 <= cap <= 256");
  if (S->n_fallback < 0 || S->n_fallback > SL_MAXFB || (S->n_fallback && !S->fallback))
    return fail(LNG_E_ARG, "drafter_shortlist: 0 <= n_fallback <= 1024");
  if (S->k < 1 || D.R > SL_MAXR || static_cast<int64_t>(D.n_orders) * D.R * S->k > SL_SLOTS)
    return fail(LNG_E_ARG, "drafter_shortlist: n_orders * R * k must be <= 8192 (R <= 256)");
  if (D.V > SL_TAKEN) return fail(LNG_E_ARG, "drafter_shortlist: vocabulary must be below 2^30");
  A = SlArgs{};
  for (int o = 0; o < D.n_orders; ++o) {
    if ((S->ids[o] == nullptr) != (S->counts[o] == nullptr))
      return fail(LNG_E_ARG, "drafter_shortlist: an order's ids and counts come together");
    A.ids[o] = S->ids[o];
    A.counts[o] = S->counts[o];
  }
  A.fallback = S->fallback;
  A.K = S->k;
  A.cap = S->cap;
  A.n_fallback = S->n_fallback;
  // hash slots: a power of two >= 2 * slots read (at most 8192, never below the slots read)
  const int64_t M = static_cast<int64_t>(D.n_orders) * D.R * S->k;
  A.tbits = 8;
  while ((int64_t{1} << A.tbits) < 2 * M && (1 << A.tbits) < SL_SLOTS) ++A.tbits;
  return LNG_OK;
}

int dr_shortlist(const lng_drafter& D, const DrWin& W, const SlArgs& A, const float* logits, const int64_t* full_ids,
                 const float* full_sc, int K, const DrChildren& C, int64_t* ids, float* scores, hipStream_t s,
                 int32_t* sl = nullptr, float* sll = nullptr) {
  hipLaunchKernelGGL(k_draft_shortlist, dim3(static_cast<unsigned>(W.n)), dim3(256), 0, s, D, W, A, logits, full_ids,
                     full_sc, K, C, ids, scores, sl, sll);
  return check_launch("drafter_shortlist");
}

// The drafts of P positions scored over the lists the attention launch built (need_full [P]:
// positions left to the full-vocabulary kernels).
int dr_sl_score(const lng_drafter& D, int P, int cap, const int32_t* lists, const float* hid, int K,
                const DrChildren& C, int64_t* ids, float* scores, int32_t* sl, float* sll, int32_t* need_full,
                hipStream_t s) {
  const dim3 g(static_cast<unsigned>(P));
  if (D.emb_dtype == LNG_BF16)
    hipLaunchKernelGGL(k_sl_score<bf16>, g, dim3(256), 0, s, D, cap, lists, hid, K, C, ids, scores, sl, sll, need_full);
  else if (D.emb_dtype == LNG_F16)
    hipLaunchKernelGGL(k_sl_score<_Float16>, g, dim3(256), 0, s, D, cap, lists, hid, K, C, ids, scores, sl, sll,
                       need_full);
  else
    hipLaunchKernelGGL(k_sl_score<float>, g, dim3(256), 0, s, D, cap, lists, hid, K, C, ids, scores, sl, sll, need_full);
  return check_launch("drafter_readout_shortlist(score)");
}

}  // namespace

}  // namespace lng

using namespace lng;

extern "C" {

size_t lng_drafter_size(void) { return sizeof(lng_drafter); }

size_t lng_drafter_workspace_bytes(const lng_drafter* D, int32_t max_positions, int32_t max_k, int32_t max_pairs) {
  if (!D || max_positions <= 0 || max_positions > DR_MAXP || max_k <= 0 || max_k > DR_MAXK) return 0;
  (void)max_pairs;
  return dr_layout(*D, max_positions, max_k, D->rows).total + align256(sizeof(int64_t) * DR_MAXP * max_k) +
         align256(sizeof(float) * DR_MAXP * max_k);
}

int lng_drafter_advance(const lng_drafter* D, const int32_t* rows, const int32_t* prev, int32_t n,
                        int codes_from_router, void* work, size_t work_bytes, void* stream) {
  if (int rc = dr_check(D, "drafter_advance")) return rc;
  if (n < 0 || n > DR_MAXP || (n && (!rows || !prev))) return fail(LNG_E_ARG, "drafter_advance: 0 <= n <= 16");
  if (work_bytes < dr_layout(*D, 1, 1, 1).qkw) return fail(LNG_E_ARG, "drafter_advance: workspace too small");
  DrAdv A{};
  A.n = n;
  for (int j = 0; j < n; ++j) {
    if (rows[j] == LNG_ROW_NONE || !spec_ok(*D, rows[j]) || !spec_ok(*D, prev[j]))
      return fail(LNG_E_RANGE, "drafter_advance: row out of range");
    A.row[j] = rows[j];
    A.prev[j] = prev[j];
  }
  return dr_advance(*D, A, codes_from_router, static_cast<float*>(work), as_stream(stream));
}

int lng_drafter_advance_range(const lng_drafter* D, int32_t base, int32_t prev0, int32_t n, int codes_from_router,
                              void* work, size_t work_bytes, void* stream) {
  if (int rc = dr_check(D, "drafter_advance_range")) return rc;
  if (n < 0 || base < 0 || static_cast<int64_t>(base) + n > D->rows || !spec_ok(*D, prev0))
    return fail(LNG_E_RANGE, "drafter_advance_range: rows out of range");
  if (work_bytes < dr_layout(*D, 1, 1, 1).qkw) return fail(LNG_E_ARG, "drafter_advance_range: workspace too small");
  hipStream_t s = as_stream(stream);
  for (int32_t j0 = 0; j0 < n; j0 += DR_ADV_CHUNK) {
    DrAdv A{};
    A.range = 1;
    A.n = std::min<int32_t>(DR_ADV_CHUNK, n - j0);
    A.base = base + j0;
    A.prev0 = j0 == 0 ? prev0 : base + j0 - 1;
    if (int rc = dr_advance(*D, A, codes_from_router, static_cast<float*>(work), s)) return rc;
  }
  return LNG_OK;
}

int lng_drafter_readout(const lng_drafter* D, const int32_t* windows, int32_t P, int32_t k, int online, float kappa,
                        const int32_t* child_rows, const int32_t* child_parent, const int32_t* child_rank,
                        int32_t n_children, void* work, size_t work_bytes, int32_t* counts, int64_t* ids,
                        float* scores, float* logits, void* stream) {
  if (int rc = dr_check(D, "drafter_readout")) return rc;
  if (k <= 0 || k > DR_MAXK || !ids || !scores || !windows) return fail(LNG_E_ARG, "drafter_readout: 1 <= k <= 8");
  DrWin W;
  if (int rc = dr_windows(*D, windows, P, W)) return rc;
  if (n_children < 0 || n_children > DR_MAXCH) return fail(LNG_E_ARG, "drafter_readout: at most 64 children");
  DrChildren C{};
  C.n = n_children;
  for (int e = 0; e < n_children; ++e) {
    if (child_rows[e] < 0 || child_rows[e] >= D->rows || child_parent[e] < 0 || child_parent[e] >= P ||
        child_rank[e] < 0 || child_rank[e] >= k)
      return fail(LNG_E_RANGE, "drafter_readout: bad child");
    C.row[e] = child_rows[e];
    C.parent[e] = static_cast<int8_t>(child_parent[e]);
    C.rank[e] = static_cast<int8_t>(child_rank[e]);
  }
  return dr_readout(*D, W, k, online, kappa, C, static_cast<char*>(work), work_bytes, counts, ids, scores, logits,
                    as_stream(stream));
}

int lng_drafter_shortlist(const lng_drafter* D, const lng_sketch* S, const int32_t* windows, int32_t P,
                          const float* logits, const int64_t* full_ids, const float* full_scores, int32_t k,
                          const int32_t* child_rows, const int32_t* child_parent, const int32_t* child_rank,
                          int32_t n_children, int64_t* ids, float* scores, int32_t* shortlist,
                          float* shortlist_logits, void* stream) {
  if (int rc = dr_check(D, "drafter_shortlist")) return rc;
  if (!logits || !full_ids || !full_scores || !ids || !scores || !windows)
    return fail(LNG_E_ARG, "drafter_shortlist: null argument");
  if (k <= 0 || k > DR_MAXK) return fail(LNG_E_ARG, "drafter_shortlist: 1 <= k <= 8");
  SlArgs A{};
  if (int rc = sl_args(*D, S, A)) return rc;
  DrWin W;
  if (int rc = dr_windows(*D, windows, P, W)) return rc;
  if (n_children < 0 || n_children > DR_MAXCH) return fail(LNG_E_ARG, "drafter_shortlist: at most 64 children");
  DrChildren C{};
  C.n = n_children;
  for (int e = 0; e < n_children; ++e) {
    if (child_rows[e] < 0 || child_rows[e] >= D->rows || child_parent[e] < 0 || child_parent[e] >= P ||
        child_rank[e] < 0 || child_rank[e] >= k)
      return fail(LNG_E_RANGE, "drafter_shortlist: bad child");
    C.row[e] = child_rows[e];
    C.parent[e] = static_cast<int8_t>(child_parent[e]);
    C.rank[e] = static_cast<int8_t>(child_rank[e]);
  }
  return dr_shortlist(*D, W, A, logits, full_ids, full_scores, k, C, ids, scores, as_stream(stream), shortlist,
                      shortlist_logits);
}

int lng_drafter_readout_shortlist(const lng_drafter* D, const lng_sketch* S, const int32_t* windows, int32_t P,
                                  int32_t k, const int32_t* child_rows, const int32_t* child_parent,
                                  const int32_t* child_rank, int32_t n_children, void* work, size_t work_bytes,
                                  int64_t* ids, float* scores, int32_t* shortlist, float* shortlist_logits,
                                  void* stream) {
  if (int rc = dr_check(D, "drafter_readout_shortlist")) return rc;
  if (k <= 0 || k > DR_MAXK || !ids || !scores || !windows || !work)
    return fail(LNG_E_ARG, "drafter_readout_shortlist: 1 <= k <= 8, non-null windows, ids, scores, work");
  SlArgs A{};
  if (int rc = sl_args(*D, S, A)) return rc;
  DrWin W;
  if (int rc = dr_windows(*D, windows, P, W)) return rc;
  if (n_children < 0 || n_children > DR_MAXCH)
    return fail(LNG_E_ARG, "drafter_readout_shortlist: at most 64 children");
  DrChildren C{};
  C.n = n_children;
  for (int e = 0; e < n_children; ++e) {
    if (child_rows[e] < 0 || child_rows[e] >= D->rows || child_parent[e] < 0 || child_parent[e] >= P ||
        child_rank[e] < 0 || child_rank[e] >= k)
      return fail(LNG_E_RANGE, "drafter_readout_shortlist: bad child");
    C.row[e] = child_rows[e];
    C.parent[e] = static_cast<int8_t>(child_parent[e]);
    C.rank[e] = static_cast<int8_t>(child_rank[e]);
  }
  hipStream_t s = as_stream(stream);
  char* wk = static_cast<char*>(work);
  const DrLayout l = dr_layout(*D, P, k, 1);
  if (!dr_lds_ok(*D, P)) return fail(LNG_E_ARG, "drafter_readout_shortlist: too many positions for this width");
  if (dr_fast(*D) || !sm_ok(*D, P)) {
    // the full-vocabulary logits and top-k in the workspace, then the shortlist reads them
    const size_t o_sc = l.total + align256(sizeof(int64_t) * DR_MAXP * k);
    if (work_bytes < o_sc + align256(sizeof(float) * DR_MAXP * k))
      return fail(LNG_E_ARG, "drafter_readout_shortlist: workspace too small");
    float* lg = reinterpret_cast<float*>(wk + l.logits);
    int64_t* fid = reinterpret_cast<int64_t*>(wk + l.total);
    float* fsc = reinterpret_cast<float*>(wk + o_sc);
    const DrChildren none{};
    if (int rc = dr_readout(*D, W, k, 0, 0.f, none, wk, work_bytes, nullptr, fid, fsc, lg, s)) return rc;
    return dr_shortlist(*D, W, A, lg, fid, fsc, k, C, ids, scores, s, shortlist, shortlist_logits);
  }
  if (work_bytes < l.total) return fail(LNG_E_ARG, "drafter_readout_shortlist: workspace too small");
  if (int rc = dr_front(*D, W, l, wk, s, &A)) return rc;
  int32_t* need = reinterpret_cast<int32_t*>(wk + l.need);
  if (int rc = dr_sl_score(*D, P, A.cap, reinterpret_cast<const int32_t*>(wk + l.lists),
                           reinterpret_cast<const float*>(wk + l.hid), k, C, ids, scores, shortlist, shortlist_logits,
                           need, s))
    return rc;
  return dr_vocab(*D, P, k, 0, 0.f, C, l, wk, 1, nullptr, ids, scores, nullptr, need, s);
}

int lng_drafter_gather(const lng_drafter* D, const int32_t* windows, int32_t P, void* out, void* stream) {
  if (int rc = dr_check(D, "drafter_gather")) return rc;
  if (!out || !windows) return fail(LNG_E_ARG, "drafter_gather: null pointer");
  DrWin W;
  if (int rc = dr_windows(*D, windows, P, W)) return rc;
  return dr_gather(*D, W, out, as_stream(stream));
}

// Draft-tree driver of lng_drafter_tree and lng_drafter_tree_shortlist: with a sketch (sk), each
// depth's readout leaves its full-vocabulary logits in sl_logits and the shortlist kernel picks
// the children's tokens.
static int dr_tree(const lng_drafter* D, const SlArgs* sk, float* sl_logits, const int32_t* parent,
                   const int32_t* rank, int32_t n, int32_t node_row0, int online, float kappa, void* work,
                   size_t work_bytes, int32_t* counts, void* route_tokens, void* stream) {
  if (!parent || !rank || n <= 0 || n > DR_MAXCH || parent[0] != -1)
    return fail(LNG_E_ARG, "drafter_tree: need 1 <= n <= 64 nodes with parent[0] == -1");
  if (node_row0 < 0 || static_cast<int64_t>(node_row0) + n > D->rows)
    return fail(LNG_E_RANGE, "drafter_tree: node rows out of range");
  int K = 1;
  std::vector<int> depth(n, 0), nchild(n, 0);
  for (int i = 1; i < n; ++i) {
    if (parent[i] < 0 || parent[i] >= i) return fail(LNG_E_ARG, "drafter_tree: parent[i] must precede i");
    if (rank[i] < 0 || rank[i] >= DR_MAXK) return fail(LNG_E_ARG, "drafter_tree: rank out of range");
    depth[i] = depth[parent[i]] + 1;
    ++nchild[parent[i]];
    K = std::max(K, rank[i] + 1);
  }
  auto spec = [&](int i) { return i == 0 ? -1 : node_row0 + i; };
  // window of node i: its ancestors, then the committed positions before the root
  auto window = [&](int i, int32_t* out) {
    std::vector<int> path;
    for (int a = i; a >= 0; a = parent[a]) path.push_back(a);  // i, parent, ..., root
    for (int jb = 0; jb < D->maxn; ++jb) {                     // jb steps back from node i
      const int slot = D->maxn - 1 - jb;
      if (jb < static_cast<int>(path.size()))
        out[slot] = spec(path[jb]);
      else
        out[slot] = -1 - (jb - static_cast<int>(path.size()) + 1);
    }
  };
  hipStream_t s = as_stream(stream);
  const bool fast = dr_fast(*D);
  const int maxd = *std::max_element(depth.begin(), depth.end());
  std::vector<char> coded(n, 0);
  coded[0] = 1;
  // scratch for the readout outputs (ids/scores of each level) at the end of the workspace
  const size_t need = dr_layout(*D, DR_MAXP, K, online ? D->rows : 1).total;
  const size_t tail = align256(sizeof(int64_t) * DR_MAXP * K) + align256(sizeof(float) * DR_MAXP * K);
  if (work_bytes < need + tail) return fail(LNG_E_ARG, "drafter_tree: workspace too small");
  int64_t* lvl_ids = reinterpret_cast<int64_t*>(static_cast<char*>(work) + need);
  float* lvl_sc = reinterpret_cast<float*>(static_cast<char*>(work) + need + align256(sizeof(int64_t) * DR_MAXP * K));
  for (int dep = 0; dep <= maxd; ++dep) {
    std::vector<int> parents;
    for (int i = 0; i < n; ++i)
      if (depth[i] == dep && nchild[i] > 0) parents.push_back(i);
    if (parents.empty()) continue;
    for (size_t p0 = 0; p0 < parents.size(); p0 += DR_MAXP) {
      const int P = static_cast<int>(std::min<size_t>(DR_MAXP, parents.size() - p0));
      DrChildren C{};
      for (int i = 1; i < n; ++i)
        for (int j = 0; j < P; ++j)
          if (parent[i] == parents[p0 + j]) {
            C.row[C.n] = node_row0 + i;
            C.parent[C.n] = static_cast<int8_t>(j);
            C.rank[C.n] = static_cast<int8_t>(rank[i]);
            ++C.n;
          }
      if (fast) {
        // the parents' codes are computed inside the attention launch
        FastLevel F{};
        F.P = P;
        std::vector<int32_t> win(D->maxn);
        for (int j = 0; j < P; ++j) {
          const int i = parents[p0 + j];
          window(i, win.data());
          for (int k = 0; k < D->maxn; ++k) F.slot[j][k] = win[k];
          F.prev[j] = i == 0 ? -2 : spec(parent[i]);
          F.fresh[j] = coded[i] ? 0 : 1;
          coded[i] = 1;
        }
        if (int rc = dr_readout_fast(*D, F, K, online, kappa, sk ? DrChildren{} : C, static_cast<char*>(work), need,
                                     counts, lvl_ids, lvl_sc, sk ? sl_logits : nullptr, s))
          return rc;
        if (sk) {
          DrWin W{};
          W.n = P;
          for (int j = 0; j < P; ++j)
            for (int k = 0; k < DR_MAXN; ++k) W.slot[j][k] = F.slot[j][k];
          if (int rc = dr_shortlist(*D, W, *sk, sl_logits, lvl_ids, lvl_sc, K, C, lvl_ids, lvl_sc, s)) return rc;
        }
        continue;
      }
      // codes of the parents of this depth (their tokens were chosen one depth up)
      DrAdv A{};
      for (int j = 0; j < P; ++j) {
        const int i = parents[p0 + j];
        if (coded[i]) continue;
        A.row[A.n] = spec(i);
        A.prev[A.n] = spec(parent[i]);
        ++A.n;
        coded[i] = 1;
      }
      if (int rc = dr_advance(*D, A, 1, static_cast<float*>(work), s)) return rc;
      DrWin W{};
      W.n = P;
      std::vector<int32_t> win(D->maxn);
      for (int j = 0; j < P; ++j) {
        window(parents[p0 + j], win.data());
        for (int k = 0; k < D->maxn; ++k) W.slot[j][k] = win[k];
      }
      if (int rc = dr_readout(*D, W, K, online, kappa, sk ? DrChildren{} : C, static_cast<char*>(work), need, counts,
                              lvl_ids, lvl_sc, sk ? sl_logits : nullptr, s))
        return rc;
      if (sk)
        if (int rc = dr_shortlist(*D, W, *sk, sl_logits, lvl_ids, lvl_sc, K, C, lvl_ids, lvl_sc, s)) return rc;
    }
  }
  if (fast && route_tokens) {
    // leaves' codes, the root token next to the nodes, and the verification gather in one launch each
    const int es = dtype_size(D->table_dtype);
    for (int p0 = 0; p0 < n; p0 += DR_MAXP) {
      FastLevel F{};
      F.P = std::min(DR_MAXP, n - p0);
      std::vector<int32_t> win(D->maxn);
      for (int j = 0; j < F.P; ++j) {
        const int i = p0 + j;
        window(i, win.data());
        for (int k = 0; k < D->maxn; ++k) F.slot[j][k] = win[k];
        F.prev[j] = i == 0 ? -2 : spec(parent[i]);
        F.fresh[j] = coded[i] ? 0 : 1;
      }
      char* out = static_cast<char*>(route_tokens) + static_cast<size_t>(p0) * D->R * D->dt * es;
      const dim3 g(static_cast<unsigned>(cdiv(D->R, 32)), static_cast<unsigned>(F.P));
      const int32_t root_dst = p0 == 0 ? node_row0 : -1;
      if (D->table_dtype == LNG_BF16)
        hipLaunchKernelGGL(k_fast_gather<bf16>, g, dim3(256), 0, s, *D, F, root_dst, reinterpret_cast<bf16*>(out));
      else if (D->table_dtype == LNG_F16)
        hipLaunchKernelGGL(k_fast_gather<_Float16>, g, dim3(256), 0, s, *D, F, root_dst, reinterpret_cast<_Float16*>(out));
      else
        hipLaunchKernelGGL(k_fast_gather<float>, g, dim3(256), 0, s, *D, F, root_dst, reinterpret_cast<float*>(out));
      if (int rc = check_launch("drafter_tree(fast gather)")) return rc;
    }
    return LNG_OK;
  }
  // codes of the nodes that were never a parent (leaves), in index order, 16 at a time
  std::vector<int> rest;
  for (int i = 1; i < n; ++i)
    if (!coded[i]) rest.push_back(i);
  for (size_t p0 = 0; p0 < rest.size(); p0 += DR_MAXP) {
    DrAdv A{};
    for (size_t j = p0; j < std::min(rest.size(), p0 + DR_MAXP); ++j) {
      A.row[A.n] = spec(rest[j]);
      A.prev[A.n] = spec(parent[rest[j]]);
      ++A.n;
    }
    if (int rc = dr_advance(*D, A, 1, static_cast<float*>(work), s)) return rc;
  }
  hipLaunchKernelGGL(k_draft_root_copy, dim3(1), dim3(64), 0, s, *D, node_row0);
  if (int rc = check_launch("drafter_tree(root)")) return rc;
  if (route_tokens) {
    const int es = dtype_size(D->table_dtype);
    for (int p0 = 0; p0 < n; p0 += DR_MAXP) {
      DrWin W{};
      W.n = std::min(DR_MAXP, n - p0);
      std::vector<int32_t> win(D->maxn);
      for (int j = 0; j < W.n; ++j) {
        window(p0 + j, win.data());
        for (int k = 0; k < D->maxn; ++k) W.slot[j][k] = win[k];
      }
      char* out = static_cast<char*>(route_tokens) + static_cast<size_t>(p0) * D->R * D->dt * es;
      if (int rc = dr_gather(*D, W, out, s)) return rc;
    }
  }
  return LNG_OK;
}

int lng_drafter_tree(const lng_drafter* D, const int32_t* parent, const int32_t* rank, int32_t n, int32_t node_row0,
                     int online, float kappa, void* work, size_t work_bytes, int32_t* counts, void* route_tokens,
                     void* stream) {
  if (int rc = dr_check(D, "drafter_tree")) return rc;
  return dr_tree(D, nullptr, nullptr, parent, rank, n, node_row0, online, kappa, work, work_bytes, counts, route_tokens,
                 stream);
}

int lng_drafter_tree_shortlist(const lng_drafter* D, const lng_sketch* S, const int32_t* parent, const int32_t* rank,
                               int32_t n, int32_t node_row0, void* work, size_t work_bytes, float* logits_work,
                               void* route_tokens, void* stream) {
  if (int rc = dr_check(D, "drafter_tree_shortlist")) return rc;
  SlArgs A{};
  if (int rc = sl_args(*D, S, A)) return rc;
  if (!logits_work) return fail(LNG_E_ARG, "drafter_tree_shortlist: logits_work [16, V] needed");
  return dr_tree(D, &A, logits_work, parent, rank, n, node_row0, 0, 0.f, work, work_bytes, nullptr, route_tokens,
                 stream);
}

}  // extern "C"
