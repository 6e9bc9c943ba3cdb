// Fused route gather + sink readout for the bf16 memory layer (16 query heads x 64,
// 4 KV heads, n-gram orders (2, 3), mem_dim 128): the metric kernel.
//
// Per token t and query head hg = 4h + g (h the KV head), with x_r the 256-wide route
// token (2-gram row | 3-gram row) and s_r = rsqrt(mean(x_r^2) + eps):
//   qkw_hg = scale * w_mem . (Wk[h]^T q_hg)                   (phase A, MFMA)
//   score  = s_r * (qkw_hg . x_r)                              (phase B, MFMA)
//   U_hg   = sum_r p_{hg,r} s_r x_r, online softmax seeded by the sink (m, l) = (b0, 1)
//   o_hg   = Wv[h] (w_mem . U_hg / l_hg)                       (phase C, MFMA)
// which equals the reference's RMSNorm -> KV projection -> sink GQA without ever
// forming keys or values.
//
// Block = TOK waves = TOK tokens (TOK = 4 or 8).  Phases A and C are cooperative: wave w takes
// KV head w & 3 and a TOK/4-th share of that head's weight rows (features in A, head dims in
// C), for TOK/4 MFMA column tiles of 16 = 4 tokens x 4 groups, so every weight row is fetched
// once per block.  The weights come packed in MFMA operand order (lng_memory_readout_pack): one
// weight load is one contiguous kilobyte.  Phase B is one token per wave, routes in chunks of 32.  A chunk is gathered with whole-row loads (16 lanes x 16 B = one
// 256-byte table row per quarter wave), parked in the wave's LDS region in row layout,
// read back as the score MFMA's A operand (ds_read_b128) and, transposed, as the
// B operand of P.X (ds_read_b64_tr_b16).  The next chunk's rows are in flight while a
// chunk is processed.
#include "common.h"

namespace lng {

constexpr int FR_H = 16;           // query heads
constexpr int FR_HD = 64;          // head dim
constexpr int FR_DT = 256;         // route token dim (2 orders x 128)
// LDS row (bf16): 544 B, so row r starts 32 r bytes (mod 256) into the banks.  A 16-lane pass
// of a 16-byte LDS access (lanes 0-7 with 16-23, and so on) covers 256 B of banks; with this skew,
// a chunk row stored by one such pass (the gather's lane map), the score operands (rows 0-7 at
// pieces of opposite parity in the two halves of a pass, fr_col) and the transposed 8-byte reads
// (rows 0-7, 32 B each) all land on distinct bank groups.
constexpr int FR_LD = FR_DT + 16;
constexpr int FR_MAXR = 256;       // max routes (row-index slots per token)
constexpr int FR_RQ = FR_MAXR / 4;
// Token t's 32-row LDS region starts at fr_tok(t) elements: regions 256 B apart beyond their
// size, skewed by 128 (t & 1) + 16 ((t >> 1) & 1) bytes, so the phases that touch several tokens'
// regions in one LDS pass (the query-key products, 8-byte stores of 4 tokens x 4 heads; the value
// operands, 16-byte reads of 2 tokens x 4 heads) spread over distinct bank groups.
constexpr int FR_TS = 32 * (FR_DT + 16) + 128;  // elements per token region (row length 544 B)
__device__ __forceinline__ int fr_tok(int t) { return t * FR_TS + 64 * (t & 1) + 8 * ((t >> 1) & 1); }
// packed KV weight (bf16 elements): keys [h 4][ft 16][ks 2][lane 64][8] = Wk^T[h][16ft + lane%16][32ks + 8(lane/16) ..+8],
// then values [h 4][dt 4][ks 8][lane 64][8] = Wv[h][16dt + lane%16][32ks + 8(lane/16) ..+8]
constexpr int FR_PK_V = 4 * 16 * 2 * 64 * 8;
static_assert(2 * FR_PK_V == LNG_READOUT_PACK_ELEMS, "packed KV weight size");
#ifndef LNG_READOUT_TOK
#define LNG_READOUT_TOK 4
#endif
// Cache policies (measured on the SB-shape forward, 16384 tokens x 184 routes): the 3-gram rows
// (a 193 MB table, each row met ~4 times per pass) load at device scope (sc1), which reads them
// without pushing the 2-gram rows (12 MB, each met ~64 times) out of the XCD's L2; the query and
// raw rows, read once, load non-temporal (nt).  Together 5 us of 244 off the launch; nt on the
// 3-gram rows (which also gives up their reuse in the Infinity Cache) or on the head stores is slower.
constexpr int FR_POL_T3 = CPOL_SC1;
constexpr int FR_POL_STREAM = CPOL_NT;

__device__ __forceinline__ bf16x8 ld16(const bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }
// route-token column of the score operands' 8-feature piece kk of lane group lg: the pieces of lane
// groups 0 and 1 (2 and 3) alternate in parity, so the two halves of an LDS pass never share a
// bank group (the score is a dot product over all 256 features; their grouping is free)
__device__ __forceinline__ int fr_col(int lg, int kk) { return 16 * kk + 8 * (lg & 1) + 128 * (lg >> 1); }
// 16 bytes of a token-major activation (q, raw rows) at element offset e < 2^31, streamed (nt)
__device__ __forceinline__ bf16x8 ldq(const bf16* base, int64_t e) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16*>(base), 0, -1, BUF_DW3);
  return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<uint32_t>(e) * 2u, 0,
                                                                          FR_POL_STREAM));
}
__device__ __forceinline__ bf16x8 zero8() {
  bf16x8 z;
#pragma unroll
  for (int j = 0; j < 8; ++j) z[j] = static_cast<bf16>(0.f);
  return z;
}
__device__ __forceinline__ float sumsq8(const bf16x8 v, float acc) {
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 0, 1), __builtin_shufflevector(v, v, 0, 1), acc,
                                        false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 2, 3), __builtin_shufflevector(v, v, 2, 3), acc,
                                        false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 4, 5), __builtin_shufflevector(v, v, 4, 5), acc,
                                        false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 6, 7), __builtin_shufflevector(v, v, 6, 7), acc,
                                        false);
  return acc;
}

// LDS (TOK = 8: 159,264 B, one block per CU; TOK = 4: 79,888 B, two blocks per CU): per wave a
// 32-row region reused as qkw (rows 0..15, phase A -> B), the route chunk (rows 0..31, phase B)
// and u (rows 0..15, phase B -> C); per wave the token's row indices [order][route parity]
// [route / 2] (-1 = zero row); the memory-norm weight.
template <int FR_TOK>
__global__ __launch_bounds__(64 * FR_TOK, 8 / FR_TOK) void k_readout_fused(const bf16* __restrict__ q,
                                                          const bf16* __restrict__ q_rows, float q_eps,
                                                          const uint8_t* __restrict__ codes,
                                                          int64_t B, int64_t T, int32_t R, int64_t cstride,
                                                          int64_t pos0, const int32_t* __restrict__ pos0_dev,
                                                          const bf16* __restrict__ table2,
                                                          const bf16* __restrict__ table3,
                                                          const bf16* __restrict__ kv_pack,
                                                          const bf16* __restrict__ w_mem, float eps, float scale,
                                                          float sink, bf16* __restrict__ head_out) {
  __shared__ __attribute__((aligned(16))) bf16 xs_lds[FR_TOK * FR_TS];
  __shared__ __attribute__((aligned(16))) int32_t rowsh[FR_TOK][2][4][FR_RQ + 4];  // rows 272 B apart
  // element (row, c) of token t's region (see fr_tok)
  auto XS = [&](int t, int row, int c) -> bf16& { return xs_lds[fr_tok(t) + row * FR_LD + c]; };
  __shared__ __attribute__((aligned(16))) bf16 wms[FR_DT];
  __shared__ float qscale[FR_TOK];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  if (threadIdx.x < FR_DT) wms[threadIdx.x] = w_mem[threadIdx.x];
  // With q_rows, q is the projection of the raw rows with the query RMSNorm's weight folded into
  // it, and each token's query is scaled here by its row's rsqrt(mean(row^2) + q_eps): wave w
  // reduces the row of token w (2 KB, two 16 B pieces per lane)
  const int64_t ntok_all = B * T;
  bf16x8 hq[2];
  const int64_t tq_own = static_cast<int64_t>(blockIdx.x) * FR_TOK + w;
  if (q_rows) {
#pragma unroll
    for (int k = 0; k < 2; ++k)
      hq[k] = tq_own < ntok_all ? ldq(q_rows, tq_own * (FR_H * FR_HD) + 8 * (lane + 64 * k)) : zero8();
  }

  // phase-A operands first (no dependence on the codes), so their latency overlaps stage 0:
  // wave w takes head h = w & 3 and feature tiles ft0 .. ft0 + NFT-1; column tile tt = tokens 4tt .. 4tt+3
  constexpr int NTT = FR_TOK / 4, NFT = 16 / NTT, NDT = 4 / NTT;
  const int a_h = w & 3, a_ft0 = NFT * (w >> 2), a_hg = a_h * 4 + (li & 3);
  bf16x8 bq[NTT][2], wa[NFT][2];
#pragma unroll
  for (int tt = 0; tt < NTT; ++tt) {
    const int64_t tq = static_cast<int64_t>(blockIdx.x) * FR_TOK + 4 * tt + (li >> 2);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      bq[tt][ks] = tq < B * T ? ldq(q, tq * (FR_H * FR_HD) + a_hg * FR_HD + 32 * ks + 8 * lg) : zero8();
  }
#pragma unroll
  for (int ft = 0; ft < NFT; ++ft)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      wa[ft][ks] = ld16(kv_pack + (((a_h * 16 + a_ft0 + ft) * 2 + ks) * 64 + lane) * 8);
  const int64_t ntok = B * T;
  const int64_t tok0 = static_cast<int64_t>(blockIdx.x) * FR_TOK;
  const int64_t tok = tok0 + w;
  const bool tok_ok = tok < ntok;
  // token (b, i) of the B x T outputs sits at position pos0 (+ *pos0_dev) + i of its sequence; its
  // codes at position t are codes[(b * cstride + t) * R ..] (cstride = T, pos0 = 0: a whole
  // sequence; cstride = the cache length, pos0 = L: new positions after a cached prefix)
  const int64_t tb = tok_ok ? tok / T : 0;
  const int64_t tpos = tok_ok ? tok % T + pos0 + (pos0_dev ? static_cast<int64_t>(*pos0_dev) : 0) : 0;
  const int64_t crow = tb * cstride + tpos;  // codes row of the token
  // a position outside [0, cstride) (a device position past the cache) reads no codes
  const bool codes_ok = tok_ok && tpos >= 0 && tpos < cstride;

  // route-token mode (codes == null): table2 / table3 are the caller's route tokens [ntok, R, 256]
  // seen as 128-wide rows, the 2-gram row of (token, route) at 2 (token R + route) of table2 and
  // its 3-gram row at the same index of table3 = table2 + 128 (zeros where the lookup masks)
  const bool rows_mode = codes == nullptr;
  // ---------------- stage 0: row indices of this wave's token (codes at t, t-1, t-2)
  if (rows_mode) {
#pragma unroll
    for (int k = 0; k < FR_MAXR / 64; ++k) {
      const int r = lane + 64 * k;
      const int32_t rr = (tok_ok && r < R) ? static_cast<int32_t>((tok * R + r) * 2) : -1;
      rowsh[w][0][r & 3][r >> 2] = rr;
      rowsh[w][1][r & 3][r >> 2] = rr;
    }
  } else {
    uint8_t cv[3][FR_MAXR / 64];
#pragma unroll
    for (int k = 0; k < FR_MAXR / 64; ++k) {
      const int r = lane + 64 * k;
#pragma unroll
      for (int p = 0; p < 3; ++p)
        cv[p][k] = (codes_ok && r < R && tpos >= p) ? static_cast<uint8_t>(codes[(crow - p) * R + r] & 15) : 0;
    }
#pragma unroll
    for (int k = 0; k < FR_MAXR / 64; ++k) {
      const int r = lane + 64 * k;
      int32_t r2 = -1, r3 = -1;
      if (codes_ok && r < R) {
        if (tpos >= 1) r2 = r * 256 + cv[1][k] + 16 * cv[0][k];
        if (tpos >= 2) r3 = r * 4096 + cv[2][k] + 16 * cv[1][k] + 256 * cv[0][k];
      }
      rowsh[w][0][r & 3][r >> 2] = r2;
      rowsh[w][1][r & 3][r >> 2] = r3;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  __builtin_amdgcn_wave_barrier();

  // chunk gather: instruction m reads order m & 1 for routes c0 + 4 (m >> 1) + g_sub, 16-byte
  // piece g_piece (16 lanes per 256-byte table row); one order per instruction, so that the 3-gram
  // rows take their own cache policy (FR_POL_T3).  Lanes 0-7 and 16-23 (8-15 and 24-31, ...)
  // fetch the two halves of one row, so the LDS pass that stores them writes 256 contiguous bytes.
  const int g_sub = ((lane >> 3) & 1) | ((lane >> 4) & 2), g_piece = (lane & 7) | ((lane >> 1) & 8);
  // every row of a token at t >= 2 exists (both orders), as does every route token: no mask
  const bool all_rows = rows_mode || tpos >= 2;
  // 3-gram rows through a raw buffer descriptor (the table, at most 256 routes x 4096 rows x 256 B,
  // is < 4 GB, so row * 256 fits the 32-bit offset; every row index is in range, the descriptor's
  // size is left at its maximum)
  const __amdgpu_buffer_rsrc_t t3 = __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16*>(table3), 0, -1, BUF_DW3);
  auto row_load = [&](int order, int32_t row) -> u32x4 {
    if (order == 0) return *reinterpret_cast<const u32x4*>(table2 + static_cast<int64_t>(row) * 128 + 8 * g_piece);
    return __builtin_amdgcn_raw_buffer_load_b128(t3, static_cast<uint32_t>(row) * 256u + 16u * g_piece, 0, FR_POL_T3);
  };
  auto gather = [&](int c0, u32x4 (&g)[16]) {
    int32_t rows[2][8];  // [order][j]: route c0 + 4j + g_sub
#pragma unroll
    for (int o = 0; o < 2; ++o) {
      const int32_t* rp = &rowsh[w][o][g_sub][c0 >> 2];
#pragma unroll
      for (int v = 0; v < 2; ++v) {
        const int32_t __attribute__((ext_vector_type(4))) r4 =
            *reinterpret_cast<const int32_t __attribute__((ext_vector_type(4)))*>(rp + 4 * v);
#pragma unroll
        for (int e = 0; e < 4; ++e) rows[o][4 * v + e] = r4[e];
      }
    }
    if (all_rows) {
      // routes past R hold row -1 too: clamp them to row 0 (their scores are masked below)
#pragma unroll
      for (int m = 0; m < 16; ++m) g[m] = row_load(m & 1, max(rows[m & 1][m >> 1], 0));
    } else {
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        const u32x4 z = {0u, 0u, 0u, 0u};
        const int32_t row = rows[m & 1][m >> 1];
        g[m] = row >= 0 ? row_load(m & 1, row) : z;
      }
    }
  };
  auto stash = [&](const u32x4 (&g)[16]) {
#pragma unroll
    for (int m = 0; m < 16; ++m)
      *reinterpret_cast<u32x4*>(&XS(w, 4 * (m >> 1) + g_sub, (m & 1) * 128 + 8 * g_piece)) = g[m];
  };

  u32x4 g[16];
  gather(0, g);  // first chunk in flight during phase A

  if (q_rows) {
    const float ss = wave_sum(sumsq8(hq[1], sumsq8(hq[0], 0.f)));
    if (lane == 0) qscale[w] = __builtin_amdgcn_rsqf(ss * (1.0f / (FR_H * FR_HD)) + q_eps);
  } else if (lane == 0) {
    qscale[w] = 1.0f;
  }

  // ---------------- phase A: qkw[t][4h+g][f] = scale * w_mem[f] * (Wk[h]^T q[t][4h+g])[f]
  __syncthreads();  // wms, qscale
#pragma unroll
  for (int ft = 0; ft < NFT; ++ft) {
    const int f = 16 * (a_ft0 + ft) + 4 * lg;
    const bf16x4 wm4 = *reinterpret_cast<const bf16x4*>(&wms[f]);
#pragma unroll
    for (int tt = 0; tt < NTT; ++tt) {
      f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa[ft][ks], bq[tt][ks], d, 0, 0, 0);
      const float sc_t = scale * qscale[4 * tt + (li >> 2)];
      bf16x4 o;
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = static_cast<bf16>(d[i] * to_f32(wm4[i]) * sc_t);
      *reinterpret_cast<bf16x4*>(&XS(4 * tt + (li >> 2), a_hg, f)) = o;
    }
  }
  __syncthreads();

  // ---------------- phase B: one token per wave
  bf16x8 qb[8];
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) qb[kk] = *reinterpret_cast<const bf16x8*>(&XS(w, li, fr_col(lg, kk)));

  float m_run = sink, l_part = 0.f;
  f32x4 acc[16];
#pragma unroll
  for (int ft = 0; ft < 16; ++ft) acc[ft] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int c0 = 0; c0 < R; c0 += 32) {
    stash(g);
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
    if (c0 + 32 < R) gather(c0 + 32, g);

    // scores: A = route rows (lane: route 16tt + li, features fr_col(lg, kk) ..+8), B = qkw
    float sr[2];
    f32x4 sc[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      bf16x8 x[8];
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) x[kk] = *reinterpret_cast<const bf16x8*>(&XS(w, 16 * tt + li, fr_col(lg, kk)));
      float ss = 0.f;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) ss = sumsq8(x[kk], ss);
      ss += __shfl_xor(ss, 16, 64);
      ss += __shfl_xor(ss, 32, 64);
      sr[tt] = __builtin_amdgcn_rsqf(ss * (1.0f / FR_DT) + eps);  // route c0 + 16tt + li
      sc[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) sc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x[kk], qb[kk], sc[tt], 0, 0, 0);
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
    const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * 1.4426950408889634f);
    m_run = m_new;
    float psum = 0.f;
    bf16x8 pa;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = __builtin_amdgcn_exp2f((s[tt][i] - m_new) * 1.4426950408889634f);
        psum += p;
        pa[4 * tt + i] = static_cast<bf16>(p * sD[tt][i]);
      }
    l_part = l_part * alpha + psum;
    float aD[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) aD[i] = __shfl(alpha, 4 * lg + i, 64);
    // the running max seldom moves past the sink logit: rescale only when some lane's did
    if (__ballot(alpha != 1.f) != 0ull) {
#pragma unroll
      for (int ft = 0; ft < 16; ++ft)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[ft][i] *= aD[i];
    }
    // U += P . X with X transposed out of LDS: ds_read_b64_tr_b16 gives lane i of each
    // 16-lane group element i%4 of the 8-byte chunks addressed by lanes i/4 + 4c
    // (c = 0..3), i.e. X[4g + c][16ft + i] here.  The halves are joined with a shuffle
    // (element-wise bit casts of the returned vector are miscompiled to element 0).
#pragma unroll
    for (int ft = 0; ft < 16; ++ft) {
      const int col = 16 * ft + 4 * (li & 3);
      const bf16x4 b0 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
          (__attribute__((address_space(3))) bf16x4*)(&XS(w, 4 * lg + (li >> 2), col)));
      const bf16x4 b1 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
          (__attribute__((address_space(3))) bf16x4*)(&XS(w, 16 + 4 * lg + (li >> 2), col)));
      const bf16x8 b = __builtin_shufflevector(b0, b1, 0, 1, 2, 3, 4, 5, 6, 7);
      acc[ft] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, b, acc[ft], 0, 0, 0);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
  }

  // phase-C operands (wave w: head h = w & 3, head-dim tiles dt0 .. dt0 + NDT-1), loaded before
  // the block-wide barrier below so that their latency overlaps it
  const int c_h = w & 3, c_dh = NDT * (w >> 2), c_hg = c_h * 4 + (li & 3);
  bf16x8 va[NDT][8];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
      va[dt][ks] = ld16(kv_pack + FR_PK_V + (((c_h * 4 + c_dh + dt) * 8 + ks) * 64 + lane) * 8);

  // normalise and stage u = w_mem . U / l for the value projection
  float lt = l_part + __shfl_xor(l_part, 16, 64);
  lt += __shfl_xor(lt, 32, 64);
  lt += __builtin_amdgcn_exp2f((sink - m_run) * 1.4426950408889634f);
  const float inv = 1.0f / lt;
  float iD[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) iD[i] = __shfl(inv, 4 * lg + i, 64);
#pragma unroll
  for (int ft = 0; ft < 16; ++ft) {
    const int f = 16 * ft + li;
    const float wm = to_f32(wms[f]);
#pragma unroll
    for (int i = 0; i < 4; ++i) XS(w, 4 * lg + i, f) = static_cast<bf16>(acc[ft][i] * iD[i] * wm);
  }
  __syncthreads();

  // ---------------- phase C: o[t][4h+g][d] = Wv[h][d] . u[t][4h+g]; column tile tt = tokens 4tt .. 4tt+3
#pragma unroll
  for (int tt = 0; tt < NTT; ++tt) {
    const int64_t tc = tok0 + 4 * tt + (li >> 2);
    bf16x8 ub[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
      ub[ks] = *reinterpret_cast<const bf16x8*>(&XS(4 * tt + (li >> 2), c_hg, 32 * ks + 8 * lg));
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[dt][ks], ub[ks], d, 0, 0, 0);
      if (tc < ntok) {
        bf16x4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = static_cast<bf16>(d[i]);
        *reinterpret_cast<bf16x4*>(head_out + tc * (FR_H * FR_HD) + c_hg * FR_HD + 16 * (c_dh + dt) + 4 * lg) = o;
      }
    }
  }
}

// kv [512, 256] -> packed operand order (one thread per 16-byte piece, 16384 pieces).
__global__ __launch_bounds__(256) void k_readout_pack(const bf16* __restrict__ kv, bf16* __restrict__ pk) {
  const int p = blockIdx.x * 256 + threadIdx.x;
  if (p >= 2 * FR_PK_V / 8) return;
  bf16x8 v;
  if (p < FR_PK_V / 8) {  // keys: Wk^T[h][f][d] = kv[64h + d][f]
    const int lane = p & 63, ks = (p >> 6) & 1, ft = (p >> 7) & 15, h = p >> 11;
    const int f = 16 * ft + (lane & 15), d0 = 32 * ks + 8 * (lane >> 4);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = kv[(64 * h + d0 + j) * FR_DT + f];
  } else {  // values: Wv[h][d][f] = kv[256 + 64h + d][f]
    const int pv = p - FR_PK_V / 8;
    const int lane = pv & 63, ks = (pv >> 6) & 7, dt = (pv >> 9) & 3, h = pv >> 11;
    const int d = 16 * dt + (lane & 15), f0 = 32 * ks + 8 * (lane >> 4);
    v = ld16(kv + (256 + 64 * h + d) * FR_DT + f0);
  }
  *reinterpret_cast<bf16x8*>(pk + 8 * static_cast<int64_t>(p)) = v;
}

}  // namespace lng

using namespace lng;

static int readout_launch(const void* q, const void* q_rows, float q_eps, const uint8_t* codes, int64_t B, int64_t T,
                          int32_t R, int64_t cstride, int64_t pos0, const int32_t* pos0_dev, const void* table2,
                          const void* table3, const void* kv_pack, const void* w_mem, float eps, float scale,
                          float sink_logit, void* head_out, void* stream) {
  constexpr int FR_TOK = LNG_READOUT_TOK;
  if (B < 0 || T < 0 || R <= 0) return fail(LNG_E_ARG, "memory_readout_fused: bad shape");
  if (R > FR_MAXR) return fail(LNG_E_ARG, "memory_readout_fused: at most 256 routes");
  const int64_t ntok = B * T;
  if (ntok == 0) return LNG_OK;
  const int64_t blocks = cdiv(ntok, FR_TOK);
  if (blocks > 0x7fffffffLL) return fail(LNG_E_ARG, "memory_readout_fused: too many tokens");
  // buffer offsets are 32-bit: the token-major activations (2 KB per token) stay under 4 GB; the
  // 3-gram table (R <= 256 routes x 4096 rows x 256 B) always does
  if (ntok > (int64_t{1} << 21)) return fail(LNG_E_ARG, "memory_readout_fused: more than 2^21 tokens per launch");
  hipLaunchKernelGGL(k_readout_fused<FR_TOK>, dim3(static_cast<unsigned>(blocks)), dim3(64 * FR_TOK), 0,
                     as_stream(stream), static_cast<const bf16*>(q), static_cast<const bf16*>(q_rows), q_eps, codes,
                     B, T, R, cstride, pos0, pos0_dev, static_cast<const bf16*>(table2),
                     static_cast<const bf16*>(table3), static_cast<const bf16*>(kv_pack),
                     static_cast<const bf16*>(w_mem), eps, scale, sink_logit, static_cast<bf16*>(head_out));
  return check_launch("memory_readout_fused");
}

extern "C" int lng_memory_readout_fused(const void* q, const void* q_rows, float q_eps, const uint8_t* codes,
                                        int64_t B, int64_t T, int32_t R,
                                        const void* table2, const void* table3, const void* kv_pack,
                                        const void* w_mem, float eps, float scale, float sink_logit, void* head_out,
                                        void* stream) {
  return readout_launch(q, q_rows, q_eps, codes, B, T, R, T, 0, nullptr, table2, table3, kv_pack, w_mem, eps, scale,
                        sink_logit, head_out, stream);
}

extern "C" int lng_memory_readout_fused_at(const void* q, const void* q_rows, float q_eps, const uint8_t* codes,
                                           int64_t B, int64_t n, int32_t R, int64_t codes_len, int64_t pos0,
                                           const int32_t* pos0_dev, const void* table2, const void* table3,
                                           const void* kv_pack, const void* w_mem, float eps, float scale,
                                           float sink_logit, void* head_out, void* stream) {
  if (codes_len <= 0 || pos0 < 0) return fail(LNG_E_ARG, "memory_readout_fused_at: bad codes length or position");
  if (!pos0_dev && pos0 + n > codes_len)
    return fail(LNG_E_RANGE, "memory_readout_fused_at: positions pos0 .. pos0+n-1 past the codes");
  return readout_launch(q, q_rows, q_eps, codes, B, n, R, codes_len, pos0, pos0_dev, table2, table3, kv_pack, w_mem,
                        eps, scale, sink_logit, head_out, stream);
}

extern "C" int lng_memory_readout_fused_rows(const void* q, const void* q_rows, float q_eps, const void* route_tokens,
                                             int64_t B, int64_t n, int32_t R, const void* kv_pack, const void* w_mem,
                                             float eps, float scale, float sink_logit, void* head_out, void* stream) {
  if (!route_tokens) return fail(LNG_E_ARG, "memory_readout_fused_rows: null route tokens");
  if (B * n * static_cast<int64_t>(R) >= (int64_t{1} << 23))
    return fail(LNG_E_ARG, "memory_readout_fused_rows: route tokens must stay under 4 GB (B * n * R < 2^23)");
  const bf16* tok = static_cast<const bf16*>(route_tokens);
  return readout_launch(q, q_rows, q_eps, nullptr, B, n, R, n, 0, nullptr, tok, tok + 128, kv_pack, w_mem, eps, scale,
                        sink_logit, head_out, stream);
}

extern "C" int lng_memory_readout_pack(const void* kv, void* kv_pack, void* stream) {
  if (!kv || !kv_pack) return fail(LNG_E_ARG, "memory_readout_pack: null pointer");
  hipLaunchKernelGGL(k_readout_pack, dim3(2 * FR_PK_V / 8 / 256), dim3(256), 0, as_stream(stream),
                     static_cast<const bf16*>(kv), static_cast<bf16*>(kv_pack));
  return check_launch("memory_readout_pack");
}
