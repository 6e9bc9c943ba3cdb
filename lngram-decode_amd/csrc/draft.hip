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
//                                                                   grid (cdiv(V, 64))
template <typename TE>
__global__ __launch_bounds__(256) void k_draft_logits(lng_drafter D, int32_t P, int32_t K,
                                                      const float* __restrict__ hid, float* __restrict__ logits,
                                                      float* __restrict__ lpart) {
  extern __shared__ float hs[];  // [P][d]
  __shared__ float red[4];
  __shared__ float lt[DR_MAXP][DR_VB];
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
  for (int q = 0; q < DR_VB / 4; ++q) {
    const int vl = w * (DR_VB / 4) + q;
    const int64_t v = static_cast<int64_t>(blockIdx.x) * DR_VB + vl;
    if (v >= V) {
      if (lane < DR_MAXP) lt[lane][vl] = -INFINITY;
      continue;
    }
    float acc[DR_MAXP];
#pragma unroll
    for (int j = 0; j < DR_MAXP; ++j) acc[j] = 0.f;
    for (int c = lane; c < d; c += 64) {
      const float ev = to_f32(E[v * d + c]);
#pragma unroll
      for (int j = 0; j < DR_MAXP; ++j)
        if (j < P) acc[j] = fmaf(ev, hs[j * d + c], acc[j]);
    }
#pragma unroll
    for (int j = 0; j < DR_MAXP; ++j) {
      if (j < P) {
        const float a = wave_sum(acc[j]);
        if (lane == 0) {
          lt[j][vl] = a;
          logits[static_cast<int64_t>(j) * V + v] = a;
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
                                                      int64_t* __restrict__ ids, float* __restrict__ scores) {
  __shared__ float redf[4];
  __shared__ float bvs[4];
  __shared__ int bis[4];
  __shared__ int64_t sel_id[DR_MAXK];
  __shared__ float sel_sc[DR_MAXK];
  const int j = blockIdx.x;
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
    a_val[na] = score_of(id, 0.f);
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

// ------------------------------------------------------------------ host side
namespace {

struct DrLayout {
  size_t u, qkw, part, hid, logits, lpart, w, total;
  int nch, nblk;
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
  l.total = off;
  return l;
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
  const bool has_ssm = D.ssm_dim > 0 && D.ssm && D.ssm_w_in;
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

int dr_readout(const lng_drafter& D, const DrWin& W, int K, int online, float kappa, const DrChildren& C,
               char* work, size_t work_bytes, int32_t* counts, int64_t* ids, float* scores, float* logits_out,
               hipStream_t s) {
  const int P = W.n;
  const int max_pairs = D.rows;  // the online kernel's grid covers any committed length
  const DrLayout l = dr_layout(D, P, K, online ? max_pairs : 1);
  if (work_bytes < l.total) return fail(LNG_E_ARG, "drafter: workspace too small");
  if (online && !counts) return fail(LNG_E_ARG, "drafter: online counts need the counts buffer");
  float* qkw = reinterpret_cast<float*>(work + l.qkw);
  float* part = reinterpret_cast<float*>(work + l.part);
  float* hid = reinterpret_cast<float*>(work + l.hid);
  float* logits = logits_out ? logits_out : reinterpret_cast<float*>(work + l.logits);
  float* lpart = reinterpret_cast<float*>(work + l.lpart);
  int32_t* wbuf = reinterpret_cast<int32_t*>(work + l.w);
  const int QD = D.q_heads * D.dt;
  const int Nq = D.query_ssm ? D.ssm_dim : 0;
  const size_t lds_q = sizeof(float) * P * (D.d + Nq);
  const size_t lds_h = sizeof(float) * P * QD;
  const size_t lds_l = sizeof(float) * P * D.d;
  if (lds_q > 60 * 1024 || lds_h > 60 * 1024 || lds_l > 60 * 1024)
    return fail(LNG_E_ARG, "drafter: too many positions for this width");
  hipLaunchKernelGGL(k_draft_qkw, dim3(static_cast<unsigned>(cdiv(QD, 32))), dim3(256), lds_q, s, D, W, qkw);
  if (int rc = check_launch("drafter_readout(qkw)")) return rc;
  if (online) {
    hipLaunchKernelGGL(k_draft_online_match, dim3(static_cast<unsigned>(cdiv(max_pairs, DR_TB)), static_cast<unsigned>(P)),
                       dim3(256), 0, s, D, W, wbuf, counts, max_pairs);
    if (int rc = check_launch("drafter_readout(online)")) return rc;
  }
  hipLaunchKernelGGL(k_draft_attend, dim3(static_cast<unsigned>(l.nch), static_cast<unsigned>(P)), dim3(256), 0, s, D,
                     W, qkw, part);
  if (int rc = check_launch("drafter_readout(attend)")) return rc;
  hipLaunchKernelGGL(k_draft_hidden, dim3(static_cast<unsigned>(cdiv(D.d, 16))), dim3(256), lds_h, s, D, P, l.nch, part,
                     hid);
  if (int rc = check_launch("drafter_readout(hidden)")) return rc;
  if (D.emb_dtype == LNG_BF16)
    hipLaunchKernelGGL(k_draft_logits<bf16>, dim3(static_cast<unsigned>(l.nblk)), dim3(256), lds_l, s, D, P, K, hid,
                       logits, lpart);
  else if (D.emb_dtype == LNG_F16)
    hipLaunchKernelGGL(k_draft_logits<_Float16>, dim3(static_cast<unsigned>(l.nblk)), dim3(256), lds_l, s, D, P, K, hid,
                       logits, lpart);
  else
    hipLaunchKernelGGL(k_draft_logits<float>, dim3(static_cast<unsigned>(l.nblk)), dim3(256), lds_l, s, D, P, K, hid,
                       logits, lpart);
  if (int rc = check_launch("drafter_readout(logits)")) return rc;
  hipLaunchKernelGGL(k_draft_select, dim3(static_cast<unsigned>(P)), dim3(256), 0, s, D, K, l.nblk, online, kappa, logits,
                     lpart, wbuf, max_pairs, counts, C, ids, scores);
  return check_launch("drafter_readout(select)");
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

int lng_drafter_gather(const lng_drafter* D, const int32_t* windows, int32_t P, void* out, void* stream) {
  if (int rc = dr_check(D, "drafter_gather")) return rc;
  if (!out || !windows) return fail(LNG_E_ARG, "drafter_gather: null pointer");
  DrWin W;
  if (int rc = dr_windows(*D, windows, P, W)) return rc;
  return dr_gather(*D, W, out, as_stream(stream));
}

int lng_drafter_tree(const lng_drafter* D, const int32_t* parent, const int32_t* rank, int32_t n, int32_t node_row0,
                     int online, float kappa, void* work, size_t work_bytes, int32_t* counts, void* route_tokens,
                     void* stream) {
  if (int rc = dr_check(D, "drafter_tree")) return rc;
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
      DrChildren C{};
      for (int i = 1; i < n; ++i)
        for (int j = 0; j < P; ++j)
          if (parent[i] == parents[p0 + j]) {
            C.row[C.n] = node_row0 + i;
            C.parent[C.n] = static_cast<int8_t>(j);
            C.rank[C.n] = static_cast<int8_t>(rank[i]);
            ++C.n;
          }
      if (int rc = dr_readout(*D, W, K, online, kappa, C, static_cast<char*>(work), need, counts, lvl_ids, lvl_sc,
                              nullptr, s))
        return rc;
    }
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

}  // extern "C"
