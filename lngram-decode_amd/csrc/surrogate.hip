// Route-logit gradient of the n-gram lookup's surrogate (training): the backward of
// _LngramSurrogate (ffnmem/memory/lngram_v2.py:328-464) for one n-gram order.
//
// The forward is the identity on the looked-up memory; the backward passes the memory gradient
// through and gives the route logits q [B, T, R, bits] a gradient from counterfactual rows.  With
// window s = 0 .. VL-1 (VL = T - order + 1) ending at position p = s + order - 1, its row
// idx_s = (route_start + r) * A^order + sum_k c[s+k] * A^k (A = 2^bits, oldest code least
// significant), the masked memory gradient g_s = grad[b, p, r, :] * valid[b, p] and the current
// row m_s = hard_memory[b, p, r, :] (with hard_memory null, table[idx_s]: the lookup's hard_memory
// is table[idx_s] * valid, so every window with a gradient reads the same bits from the table,
// out of the route's block that the counterfactual rows come from, instead of a second stream):
//
//   approximate:  G[t, bit] += sign * (table[idx_s ^ (1 << (e*bits + bit))] . g_s - m_s . g_s)
//                 for every e = 0 .. order-1 with t = s + e, sign = +1 if that bit of idx_s is 0
//                 else -1; then G *= scale * temperature * p (1 - p), p = sigmoid(temperature * q)
//   exact:        G[t, bit] += scale * temperature * sum_{code < A} P(code) (bit(code) - p_bit)
//                                                  * (table[idx_s + (code - c[t]) * A^e] . g_s)
//                 P(code) = prod_b (bit_b(code) ? p_b : 1 - p_b) at position t
//
// A block owns one route r of one sequence b and a tile of P = 64 - (order - 1) consecutive
// positions; its 16-lane groups take the 64 windows whose digits fall in the tile (the tile's
// windows plus order - 1 before it), one window at a time: lane l holds elements [l*V, l*V + V)
// of every row (D = 16 V), a dot product is a per-lane sum reduced over the 16 lanes.  A window's
// memory-gradient and looked-up rows are read once (non-temporal: they are streamed), its
// order * bits scores go to LDS, and each output sums its windows' scores in the reference's order
// (e ascending), so the result is a fixed sum with no atomics.  Blocks are numbered so that the
// blocks of one XCD work on one route at a time (the dispatcher deals blocks to the 8 XCDs in
// turn): the route's block of the table (1 MB for order 3, mem_dim 128, bf16) stays in that
// XCD's L2 while every counterfactual row is read from it.  Codes are read under the digit mask
// A - 1, so every row stays inside its route's block of the table.
#include "common.h"

namespace lng {

constexpr int SG_GROUPS = 16;  // 16-lane groups per 256-thread block
constexpr int SG_MAXBITS = 8;
constexpr int SG_MAXORDER = 4;

struct SgArgs {
  const void* grad;       // [B, T, R, D] memory gradient (TM)
  const void* hard;       // [B, T, R, D] looked-up memory (TM)
  const void* q;          // [B, T, R, bits] route logits
  int q_dt;
  const void* codes;      // [B, T, R] codes of these routes
  int codes_dt;
  const void* table;      // [rows, D] (TM)
  const uint8_t* valid;   // [B, T] or null (all valid)
  int64_t B, T;
  int32_t R, route_start, order, bits;
  float temperature, scale, alpha;   // alpha = scale * temperature (rounded as the reference's scalar)
  void* out;              // [B, T, R, bits] in out_dt
  int out_dt;
  int64_t tiles;          // position tiles per sequence
  int32_t nt;             // memory rows within 4 GB of their base: stream them with non-temporal loads
};

// V consecutive elements of a row to fp32 (V * sizeof(TM) bytes, aligned to that size)
template <typename TM, int V>
__device__ __forceinline__ void load_row(const TM* p, float (&v)[V]) {
  if constexpr (sizeof(TM) * V == 16) {
    const u32x4 w = *reinterpret_cast<const u32x4*>(p);
    const TM* e = reinterpret_cast<const TM*>(&w);
#pragma unroll
    for (int j = 0; j < V; ++j) v[j] = to_f32(e[j]);
  } else {
#pragma unroll
    for (int j = 0; j < V; ++j) v[j] = to_f32(p[j]);
  }
}

__device__ __forceinline__ float sum16(float v) {
  // sum over the 16 lanes of this lane's row of the wave (DPP shifts within the row, then the
  // row's last lane broadcast to the row)
  v += dpp_row_shr<0x111>(v, 0.f);
  v += dpp_row_shr<0x112>(v, 0.f);
  v += dpp_row_shr<0x114>(v, 0.f);
  v += dpp_row_shr<0x118>(v, 0.f);
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(((threadIdx.x & 63) | 15) << 2,
                                                                 __builtin_bit_cast(int, v)));
}

__device__ __forceinline__ int64_t sg_code(const void* p, int dt, int64_t i) {
  if (dt == LNG_U8) return static_cast<const uint8_t*>(p)[i];
  if (dt == LNG_I32) return static_cast<const int32_t*>(p)[i];
  return static_cast<const int64_t*>(p)[i];
}

template <typename TM, int V>
__device__ __forceinline__ void load_row_nt(const TM* base, int64_t e, bool nt, float (&v)[V]) {
  // e: element offset from base; nt needs e * sizeof(TM) < 2^32 (checked by the host) and whole
  // 16-byte pieces
  if constexpr ((sizeof(TM) * V) % 16 == 0) {
    if (nt) {
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<TM*>(base), 0, -1, BUF_DW3);
#pragma unroll
      for (int c = 0; c < static_cast<int>(sizeof(TM) * V / 16); ++c) {
        const u32x4 w = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                      rs, static_cast<uint32_t>(e * sizeof(TM)) + 16u * c, 0, CPOL_NT));
        const TM* x = reinterpret_cast<const TM*>(&w);
#pragma unroll
        for (int j = 0; j < static_cast<int>(16 / sizeof(TM)); ++j) v[c * (16 / sizeof(TM)) + j] = to_f32(x[j]);
      }
      return;
    }
  }
  load_row<TM, V>(base + e, v);
}

typedef __bf16 sg_bf16x2 __attribute__((ext_vector_type(2)));

// bf16 rows of 128 (16 bytes per lane) stay packed: a lane's share of a dot product is four
// v_dot2_f32_bf16 (each bf16 product is exact in fp32) instead of eight conversions and FMAs
__device__ __forceinline__ u32x4 ld_raw16(const void* base, int64_t byte_off, bool nt) {
  if (nt) {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, -1, BUF_DW3);
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<uint32_t>(byte_off), 0,
                                                                           CPOL_NT));
  }
  return *reinterpret_cast<const u32x4*>(static_cast<const char*>(base) + byte_off);
}
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(sg_bf16x2, a), __builtin_bit_cast(sg_bf16x2, b), acc,
                                         false);
}
__device__ __forceinline__ float dot8_bf16(u32x4 a, u32x4 b) {
  return dot2_bf16(a.w, b.w, dot2_bf16(a.z, b.z, dot2_bf16(a.y, b.y, dot2_bf16(a.x, b.x, 0.f))));
}

constexpr int SG_WIN = 64;                       // windows per block (16 groups x 4)
constexpr int SG_SC = SG_MAXORDER * SG_MAXBITS;  // scores per window in LDS: [e][bit]

template <typename TM, int V, bool EXACT>
__global__ __launch_bounds__(256) void k_surrogate_grad(SgArgs a) {
  __shared__ float sc[SG_WIN][SG_SC];
  const int grp = threadIdx.x >> 4, l = threadIdx.x & 15;
  // block -> (route, sequence, tile): XCD x = block % 8 keeps to routes r = 8j + x, all of a route's
  // (sequence, tile) blocks in a row
  const int64_t xcd = blockIdx.x & 7;
  const int64_t k8 = blockIdx.x >> 3;
  const int64_t per_route = a.B * a.tiles;
  const int64_t r64 = (k8 / per_route) * 8 + xcd;
  if (r64 >= a.R) return;                        // the whole block: before any barrier
  const int32_t r = static_cast<int32_t>(r64);
  const int64_t rem = k8 % per_route;
  const int64_t b = rem / a.tiles;
  const int bits = a.bits, order = a.order;
  const int P = SG_WIN - (order - 1);
  const int64_t t0 = (rem % a.tiles) * P;
  const int64_t s_lo = t0 - (order - 1);         // the window of local index 0
  const int64_t VL = a.T - order + 1;
  const int64_t A = int64_t(1) << bits;
  const int64_t dmask = A - 1;
  const int64_t D = 16 * V;
  const int64_t RD = static_cast<int64_t>(a.R) * D;
  const TM* grad = static_cast<const TM*>(a.grad);
  const TM* hard = static_cast<const TM*>(a.hard);
  const TM* table = static_cast<const TM*>(a.table);
  const bool nt = a.nt != 0;
  const int64_t block_base = static_cast<int64_t>(a.route_start + r) << (bits * order);
  const bool active = VL > 0 && a.temperature != 0.f && a.scale != 0.f;

  for (int w = grp; w < SG_WIN; w += 16) {
    const int64_t s = s_lo + w;
    float score[SG_MAXORDER][SG_MAXBITS];
#pragma unroll
    for (int e = 0; e < SG_MAXORDER; ++e)
#pragma unroll
      for (int k = 0; k < SG_MAXBITS; ++k) score[e][k] = 0.f;
    // a window whose memory position is masked has a zero gradient row: its scores stay zero
    const bool win = active && s >= 0 && s < VL && (a.valid == nullptr || a.valid[b * a.T + s + order - 1]);
    if (win) {
      const int64_t pos = s + order - 1;
      int64_t addr = 0;
      int64_t digit[SG_MAXORDER];
#pragma unroll
      for (int k = 0; k < SG_MAXORDER; ++k) {
        digit[k] = 0;
        if (k < order) {
          digit[k] = sg_code(a.codes, a.codes_dt, (b * a.T + s + k) * a.R + r) & dmask;
          addr |= digit[k] << (k * bits);
        }
      }
      const int64_t idx = block_base + addr;
      const int64_t mrow = (b * a.T + pos) * RD + static_cast<int64_t>(r) * D + l * V;
      constexpr bool PACKED = sizeof(TM) == 2 && V == 8;
      if constexpr (PACKED && !EXACT) {
        const u32x4 gr = ld_raw16(grad, mrow * 2, nt);
        const u32x4 hr = hard ? ld_raw16(hard, mrow * 2, nt) : ld_raw16(table, (idx * D + l * V) * 2, false);
        const float cd = sum16(dot8_bf16(hr, gr));
#pragma unroll
        for (int e = 0; e < SG_MAXORDER; ++e) {
          if (e < order) {
#pragma unroll
            for (int k0 = 0; k0 < SG_MAXBITS; k0 += 4) {
              if (k0 < bits) {
                u32x4 f[4];
#pragma unroll
                for (int k = 0; k < 4; ++k)
                  if (k0 + k < bits) f[k] = ld_raw16(table, ((idx ^ (int64_t(1) << (e * bits + k0 + k))) * D + l * V) * 2,
                                                     false);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                  if (k0 + k < bits) {
                    const float fd = sum16(dot8_bf16(f[k], gr));
                    score[e][k0 + k] = (fd - cd) * (((idx >> (e * bits + k0 + k)) & 1) ? -1.f : 1.f);
                  }
                }
              }
            }
          }
        }
      } else {
      float g[V];
      load_row_nt<TM, V>(grad, mrow, nt, g);
      if constexpr (!EXACT) {
        float m[V];
        if (hard)
          load_row_nt<TM, V>(hard, mrow, nt, m);
        else
          load_row<TM, V>(table + idx * D + l * V, m);
        float cd = 0.f;
#pragma unroll
        for (int j = 0; j < V; ++j) cd += m[j] * g[j];
        cd = sum16(cd);
#pragma unroll
        for (int e = 0; e < SG_MAXORDER; ++e) {
          if (e < order) {
            // the counterfactual rows of digit e, four at a time, requested before any is reduced
#pragma unroll
            for (int k0 = 0; k0 < SG_MAXBITS; k0 += 4) {
              if (k0 < bits) {
                float f[4][V];
#pragma unroll
                for (int k = 0; k < 4; ++k)
                  if (k0 + k < bits)
                    load_row<TM, V>(table + (idx ^ (int64_t(1) << (e * bits + k0 + k))) * D + l * V, f[k]);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                  if (k0 + k < bits) {
                    float fd = 0.f;
#pragma unroll
                    for (int j = 0; j < V; ++j) fd += f[k][j] * g[j];
                    fd = sum16(fd);
                    score[e][k0 + k] = (fd - cd) * (((idx >> (e * bits + k0 + k)) & 1) ? -1.f : 1.f);
                  }
                }
              }
            }
          }
        }
      } else {
#pragma unroll
        for (int e = 0; e < SG_MAXORDER; ++e) {
          if (e < order) {
            float p[SG_MAXBITS];
#pragma unroll
            for (int k = 0; k < SG_MAXBITS; ++k) {
              p[k] = 0.f;
              if (k < bits) {
                const int64_t qi = ((b * a.T + s + e) * a.R + r) * bits + k;
                const float qv = a.q_dt == LNG_BF16 ? to_f32(static_cast<const bf16*>(a.q)[qi])
                                                    : static_cast<const float*>(a.q)[qi];
                p[k] = 1.f / (1.f + expf(-(a.temperature * qv)));
              }
            }
            const int64_t step = int64_t(1) << (e * bits);
            const int64_t base = idx - digit[e] * step;
#pragma unroll 1
            for (int64_t code = 0; code < A; ++code) {
              float v[V];
              load_row<TM, V>(table + (base + code * step) * D + l * V, v);
              float dot = 0.f;
#pragma unroll
              for (int j = 0; j < V; ++j) dot += v[j] * g[j];
              dot = sum16(dot);
              float cp = 1.f;
#pragma unroll
              for (int k = 0; k < SG_MAXBITS; ++k)
                if (k < bits) cp *= ((code >> k) & 1) ? p[k] : 1.f - p[k];
#pragma unroll
              for (int k = 0; k < SG_MAXBITS; ++k) {
                if (k < bits) {
                  const float local = cp * (static_cast<float>((code >> k) & 1) - p[k]) * dot;
                  score[e][k] = fmaf(a.alpha, local, score[e][k]);
                }
              }
            }
          }
        }
      }
      }
    }
    if (l == 0) {
#pragma unroll
      for (int e = 0; e < SG_MAXORDER; ++e)
#pragma unroll
        for (int k = 0; k < SG_MAXBITS; ++k) sc[w][e * SG_MAXBITS + k] = score[e][k];
    }
  }
  __syncthreads();
  // output (t, bit): the windows t - e, e ascending
  for (int i = threadIdx.x; i < P * bits; i += 256) {
    const int tl = i / bits, k = i - (i / bits) * bits;
    const int64_t t = t0 + tl;
    if (t >= a.T) break;
    float acc = 0.f;
    for (int e = 0; e < order; ++e) acc += sc[tl + order - 1 - e][e * SG_MAXBITS + k];
    const int64_t oi = ((b * a.T + t) * a.R + r) * bits + k;
    if (!EXACT && active) {
      const float qv = a.q_dt == LNG_BF16 ? to_f32(static_cast<const bf16*>(a.q)[oi]) : static_cast<const float*>(a.q)[oi];
      const float p = 1.f / (1.f + expf(-(a.temperature * qv)));
      acc *= a.alpha * p * (1.f - p);
    }
    if (a.out_dt == LNG_BF16)
      static_cast<bf16*>(a.out)[oi] = static_cast<bf16>(acc);
    else
      static_cast<float*>(a.out)[oi] = acc;
  }
}

// The approximate mode for bf16 rows of 128 and 4-bit codes (the SB layer's lookup), orders 2 and
// 3: the same windows, scores and output sums as k_surrogate_grad over blocks of SP_WIN windows
// (SP_WIN / 16 per 16-lane group, fewer blocks and fewer fixed staging and output phases than
// 64-window tiles), with the tile's digits and window validity staged in LDS once per block (one coalesced load each, instead of order
// scattered code loads per window on each window's critical path) and the windows of a 16-lane
// group pipelined two deep: window i + 1's memory-gradient, looked-up and counterfactual rows are
// requested before window i's dot products are reduced.
// SP_WIN windows per block: RG consecutive routes x SP_WIN / RG windows each.
template <int ORDER, int RG, int SP_WIN>
__global__ __launch_bounds__(256) void k_surrogate_grad_pk(SgArgs a) {
  constexpr int BITS = 4, NF = ORDER * BITS, NW = SP_WIN / 16, WR = SP_WIN / RG;
  constexpr int64_t D = 128;
  __shared__ float sc[SP_WIN][SG_SC];                 // window rr * WR + lw
  __shared__ uint8_t cds[RG][WR + SG_MAXORDER];       // digit of route r0 + rr at position s_lo + i
  __shared__ uint8_t vld[WR];                         // window s_lo + lw has a gradient row
  const int grp = threadIdx.x >> 4, l = threadIdx.x & 15;
  // block -> (route group, sequence, tile): XCD x = block % 8 keeps to groups 8j + x, all of a group's
  // (sequence, tile) blocks in a row, so the group's blocks of the table stay in that XCD's L2
  const int64_t xcd = blockIdx.x & 7;
  const int64_t k8 = blockIdx.x >> 3;
  const int64_t per_group = a.B * a.tiles;
  const int64_t g = (k8 / per_group) * 8 + xcd;
  const int64_t r0 = g * RG;
  if (r0 >= a.R) return;                              // the whole block: before any barrier
  const int64_t rem = k8 % per_group;
  const int64_t b = rem / a.tiles;
  constexpr int P = WR - (ORDER - 1);
  const int64_t t0 = (rem % a.tiles) * P;
  const int64_t s_lo = t0 - (ORDER - 1);
  const int64_t VL = a.T - ORDER + 1;
  const int64_t RD = static_cast<int64_t>(a.R) * D;
  const bf16* grad = static_cast<const bf16*>(a.grad);
  const bf16* hard = static_cast<const bf16*>(a.hard);
  const bf16* table = static_cast<const bf16*>(a.table);
  const bool nt = a.nt != 0;
  const bool active = VL > 0 && a.temperature != 0.f && a.scale != 0.f;
  // the codes of RG consecutive routes at one position are consecutive bytes: rr runs fastest
  for (int i = threadIdx.x; i < RG * (WR + ORDER - 1); i += 256) {
    const int rr = i % RG, pi = i / RG;
    const int64_t pos = s_lo + pi;
    cds[rr][pi] = (pos >= 0 && pos < a.T && r0 + rr < a.R)
                      ? static_cast<uint8_t>(sg_code(a.codes, a.codes_dt, (b * a.T + pos) * a.R + r0 + rr) & 15)
                      : 0;
  }
  for (int i = threadIdx.x; i < WR; i += 256) {
    const int64_t sw = s_lo + i;
    vld[i] = active && sw >= 0 && sw < VL && (a.valid == nullptr || a.valid[b * a.T + sw + ORDER - 1]);
  }
  __syncthreads();
  // Window w = rr * WR + lw reads its memory-gradient and looked-up rows (streamed from HBM) and
  // the rows of its route's block of the table (2^(4 ORDER) rows of 256 B) with bit f of its
  // address flipped (mostly L2 hits): offsets (row << 8) | (lane << 4) in a buffer resource over the
  // block, so the row with bit f flipped is the offset with bit f + 8 flipped.  A group's windows
  // are pipelined two deep.
  auto live = [&](int w) { return vld[w % WR] && r0 + w / WR < a.R; };
  auto addr_of = [&](int w) -> uint32_t {
    const int rr = w / WR, lw = w % WR;
    uint32_t addr = 0;
#pragma unroll
    for (int k = 0; k < ORDER; ++k) addr |= static_cast<uint32_t>(cds[rr][lw + k]) << (k * BITS);
    return addr;
  };
  // the window's memory-gradient row, its looked-up row (from hard_memory, or, when that is null,
  // the table row the lookup read: the same bits for every window with a gradient) and the rows of
  // its route's block of the table with bit f of its address flipped
  auto load_rows = [&](int w, uint32_t addr, u32x4 (&gh)[2], u32x4 (&v)[NF]) {
    if (!live(w)) return;
    const int64_t mrow = (b * a.T + s_lo + w % WR + ORDER - 1) * RD + (r0 + w / WR) * D + l * 8;
    gh[0] = ld_raw16(grad, mrow * 2, nt);
    if (hard) gh[1] = ld_raw16(hard, mrow * 2, nt);
    const __amdgpu_buffer_rsrc_t tb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<bf16*>(table + ((static_cast<int64_t>(a.route_start) + r0 + w / WR) << (BITS * ORDER)) * D), 0,
        static_cast<int>((int64_t(1) << (BITS * ORDER)) * D * 2), BUF_DW3);
    const uint32_t off = (addr << 8) | (static_cast<uint32_t>(l) << 4);
    if (!hard) gh[1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(tb, off, 0, 0));
#pragma unroll
    for (int f = 0; f < NF; ++f)
      v[f] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(tb, off ^ (1u << (f + 8)), 0, 0));
  };
  // a dot product's 16-lane partials summed along the row (inclusive prefix by DPP shifts, the order
  // of sum16): the total is in the row's last lane, which alone forms and stores the scores
  auto sum_last = [](float x) {
    x += dpp_row_shr<0x111>(x, 0.f);
    x += dpp_row_shr<0x112>(x, 0.f);
    x += dpp_row_shr<0x114>(x, 0.f);
    x += dpp_row_shr<0x118>(x, 0.f);
    return x;
  };
  auto reduce = [&](int w, uint32_t addr, const u32x4 (&gh)[2], const u32x4 (&cf)[NF]) {
    float score[NF];
#pragma unroll
    for (int f = 0; f < NF; ++f) score[f] = 0.f;
    if (live(w)) {
      const float cd = sum_last(dot8_bf16(gh[1], gh[0]));
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        const float fd = sum_last(dot8_bf16(cf[f], gh[0]));
        score[f] = (fd - cd) * (((addr >> f) & 1) ? -1.f : 1.f);
      }
    }
    if (l == 15) {
#pragma unroll
      for (int e = 0; e < SG_MAXORDER; ++e)
#pragma unroll
        for (int k = 0; k < SG_MAXBITS; ++k)
          sc[w][e * SG_MAXBITS + k] = (e < ORDER && k < BITS) ? score[e * BITS + k] : 0.f;
    }
  };
  // two windows in flight per group: window j + 1's rows are requested before window j is reduced
  u32x4 gh[2][2], cf[2][NF];
  uint32_t ad[2];
  ad[0] = addr_of(grp);
  load_rows(grp, ad[0], gh[0], cf[0]);
#pragma unroll
  for (int j = 0; j < NW; ++j) {
    if (j + 1 < NW) {
      ad[(j + 1) & 1] = addr_of(grp + 16 * (j + 1));
      load_rows(grp + 16 * (j + 1), ad[(j + 1) & 1], gh[(j + 1) & 1], cf[(j + 1) & 1]);
    }
    reduce(grp + 16 * j, ad[j & 1], gh[j & 1], cf[j & 1]);
  }
  __syncthreads();
  // output (t, route, bit), bits then routes fastest (whole lines of the [B, T, R, bits] arrays):
  // the windows t - e, e ascending
  for (int i = threadIdx.x; i < P * RG * BITS; i += 256) {
    const int k = i % BITS, rr = (i / BITS) % RG, tl = i / (BITS * RG);
    const int64_t t = t0 + tl;
    if (t >= a.T) break;
    if (r0 + rr >= a.R) continue;
    float acc = 0.f;
    for (int e = 0; e < ORDER; ++e) acc += sc[rr * WR + tl + ORDER - 1 - e][e * SG_MAXBITS + k];
    const int64_t oi = ((b * a.T + t) * a.R + r0 + rr) * BITS + k;
    if (active) {
      const float qv = a.q_dt == LNG_BF16 ? to_f32(static_cast<const bf16*>(a.q)[oi]) : static_cast<const float*>(a.q)[oi];
      const float p = 1.f / (1.f + expf(-(a.temperature * qv)));
      acc *= a.alpha * p * (1.f - p);
    }
    if (a.out_dt == LNG_BF16)
      static_cast<bf16*>(a.out)[oi] = static_cast<bf16>(acc);
    else
      static_cast<float*>(a.out)[oi] = acc;
  }
}

// Order 2 for bf16 rows of 128 and 4-bit codes, with the route's block of the table (256 rows,
// 64 KB) in LDS: the approximate mode's windows, scores and output sums as k_surrogate_grad_pk
// (HARD: the looked-up rows streamed from hard_memory; else read from the block).  A block owns
// one route of one sequence and 16 * NW windows (NW per 16-lane group); it copies the route's block
// into LDS (straight from L2 by DMA) while the windows' memory-gradient rows are requested from
// HBM, then reads every window's looked-up and eight counterfactual rows from LDS: the rows of one
// route are shared by all its windows, so the gathers leave L2 for LDS.  Lane l of group g holds
// 16-byte piece (l + 8 (g & 1)) & 15 of every row: one LDS pass serves lanes 0-7 with 16-23 (and
// 8-15 with 24-31, ...), which then read opposite halves of their rows, so a pass covers all 64
// banks whatever rows the windows name.  NT threads (NT / 16 groups); two blocks per CU: 512
// threads with 15 windows a group fill the LDS (2 x 81.9 KB) at 4 waves per SIMD.
template <int NW, int NT, bool HARD>
__global__ __launch_bounds__(NT, 2) void k_surrogate_grad_o2lds(SgArgs a) {
  constexpr int NG = NT / 16, W = NG * NW, P = W - 1, NF = 8, NWV = NT / 64;
  static_assert(64 % NWV == 0, "the block copy is whole kilobytes per wave");
  constexpr int64_t D = 128;
  __shared__ __attribute__((aligned(16))) bf16 tab[256 * D];  // the route's block, row-major
  __shared__ float sc[W][NF];                                 // window w's scores [e * 4 + bit]
  __shared__ uint8_t cds[W + 1];                              // code at position s_lo + i
  __shared__ uint8_t vld[W];                                  // window s_lo + w has a gradient row
  const int tid = threadIdx.x, grp = tid >> 4, l = tid & 15, wave = tid >> 6, lane = tid & 63;
  // block -> (route, sequence, tile): XCD x = block % 8 keeps to routes 8j + x, all of a route's
  // (sequence, tile) blocks in a row, so the route's block of the table stays in that XCD's L2
  const int64_t xcd = blockIdx.x & 7, k8 = blockIdx.x >> 3;
  const int64_t per_route = a.B * a.tiles;
  const int64_t r = (k8 / per_route) * 8 + xcd;
  if (r >= a.R) return;  // the whole block: before any barrier
  const int64_t rem = k8 % per_route;
  const int64_t b = rem / a.tiles;
  const int64_t t0 = (rem % a.tiles) * P;
  const int64_t s_lo = t0 - 1;  // window s covers positions s, s + 1
  const int64_t VL = a.T - 1;
  const bool active = VL > 0 && a.temperature != 0.f && a.scale != 0.f;
  // the tile's codes and window validity (small, through registers)
  for (int i = tid; i < W + 1; i += NT) {
    const int64_t pos = s_lo + i;
    cds[i] = (pos >= 0 && pos < a.T) ? static_cast<uint8_t>(sg_code(a.codes, a.codes_dt, (b * a.T + pos) * a.R + r) & 15)
                                     : 0;
  }
  for (int i = tid; i < W; i += NT) {
    const int64_t sw = s_lo + i;
    vld[i] = active && sw >= 0 && sw < VL && (a.valid == nullptr || a.valid[b * a.T + sw + 1]);
  }
  // the route's block into LDS: wave w copies kilobytes NWV i + w (lane: 16 bytes)
  const bf16* blk = static_cast<const bf16*>(a.table) + ((static_cast<int64_t>(a.route_start) + r) << 8) * D;
#pragma unroll
  for (int i = 0; i < 64 / NWV; ++i) {
    const int kb = NWV * i + wave;
    __builtin_amdgcn_global_load_lds(blk + kb * 512 + lane * 8, (__attribute__((address_space(3))) void*)(tab + kb * 512),
                                     16, 0, 0);
  }
  asm volatile("" ::: "memory");
  // the windows' memory-gradient rows: a buffer over sequence b's rows, so a window past the end
  // reads zeros (its scores are not used); position s_lo + w + 1 >= 0 always
  const int pc = (l + 8 * (grp & 1)) & 15;
  const bf16* gseq = static_cast<const bf16*>(a.grad) + b * a.T * a.R * D;
  const __amdgpu_buffer_rsrc_t gr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<bf16*>(gseq), 0, static_cast<int>(a.T * a.R * D * 2), BUF_DW3);
  const __amdgpu_buffer_rsrc_t hr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<bf16*>(static_cast<const bf16*>(HARD ? a.hard : a.grad) + b * a.T * a.R * D), 0,
      static_cast<int>(a.T * a.R * D * 2), BUF_DW3);
  auto ld = [&](__amdgpu_buffer_rsrc_t rs, uint32_t off) {
    return a.nt ? __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(off), 0, CPOL_NT))
                : __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(off), 0, 0));
  };
  u32x4 gv[NW], hv[HARD ? NW : 1];
#pragma unroll
  for (int j = 0; j < NW; ++j) {
    const int64_t pos = s_lo + grp + NG * j + 1;
    const uint32_t off = static_cast<uint32_t>(((pos * a.R + r) * D + pc * 8) * 2);
    gv[j] = ld(gr, off);
    if constexpr (HARD) hv[j] = ld(hr, off);
  }
  // the block copy (issued before the gradient and looked-up row loads) has landed for this wave;
  // the barrier makes it, the codes and the validity visible to all
  if constexpr (HARD)
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * NW) : "memory");
  else
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NW) : "memory");
  __syncthreads();
  auto row = [&](uint32_t rw) { return *reinterpret_cast<const u32x4*>(tab + rw * D + pc * 8); };
  // a dot product's 16-lane partials summed along the row (inclusive DPP prefix): the total lands
  // in the row's last lane, which alone forms and stores the scores
  auto sum_last = [](float x) {
    x += dpp_row_shr<0x111>(x, 0.f);
    x += dpp_row_shr<0x112>(x, 0.f);
    x += dpp_row_shr<0x114>(x, 0.f);
    x += dpp_row_shr<0x118>(x, 0.f);
    return x;
  };
#pragma unroll
  for (int j = 0; j < NW; ++j) {
    const int w = grp + NG * j;
    float score[NF];
#pragma unroll
    for (int f = 0; f < NF; ++f) score[f] = 0.f;
    if (vld[w]) {
      const uint32_t addr = static_cast<uint32_t>(cds[w]) | (static_cast<uint32_t>(cds[w + 1]) << 4);
      u32x4 rv[NF + 1];
      if constexpr (HARD)
        rv[NF] = hv[j];
      else
        rv[NF] = row(addr);
#pragma unroll
      for (int f = 0; f < NF; ++f) rv[f] = row(addr ^ (1u << f));
      const float cd = sum_last(dot8_bf16(rv[NF], gv[j]));
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        const float fd = sum_last(dot8_bf16(rv[f], gv[j]));
        score[f] = (fd - cd) * (((addr >> f) & 1) ? -1.f : 1.f);
      }
    }
    if (l == 15) {
#pragma unroll
      for (int f = 0; f < NF; ++f) sc[w][f] = score[f];
    }
  }
  __syncthreads();
  // output (t, bit) of the route, bits fastest: the windows t (e = 0) and t - 1 (e = 1), e ascending
  for (int i = tid; i < P * 4; i += NT) {
    const int k = i & 3, tl = i >> 2;
    const int64_t t = t0 + tl;
    if (t >= a.T) break;
    float acc = 0.f;
    acc += sc[tl + 1][k];
    acc += sc[tl][4 + k];
    const int64_t oi = ((b * a.T + t) * a.R + r) * 4 + k;
    if (active) {
      const float qv = a.q_dt == LNG_BF16 ? to_f32(static_cast<const bf16*>(a.q)[oi]) : static_cast<const float*>(a.q)[oi];
      const float p = 1.f / (1.f + expf(-(a.temperature * qv)));
      acc *= a.alpha * p * (1.f - p);
    }
    if (a.out_dt == LNG_BF16)
      static_cast<bf16*>(a.out)[oi] = static_cast<bf16>(acc);
    else
      static_cast<float*>(a.out)[oi] = acc;
  }
}

// ---------------------------------------------------------------- order 3 by digit-2 bins
// Order 3 (bf16 rows of 128, 4-bit codes, approximate mode) with a workspace.  A window's looked-up
// row and its eight digit-0 and digit-1 counterfactual rows all lie in the 256-row sub-block of its
// route's table block that its digit 2 (the code at its newest position) selects; only the four
// digit-2 flips lie elsewhere.  A block per (route, bin v) keeps sub-block v of its route in LDS,
// lists the route's windows whose digit 2 is v (from a route-major copy of the codes) and gathers 9
// of each window's 13 rows from LDS (4 from L2), writing the window's 12 scores to the workspace; a
// last kernel sums each output's windows in the reference's order (e ascending) and applies the
// slope.  Windows without a gradient are listed nowhere and contribute 0.
constexpr int SG3_MAXD = 2048;   // windows a block lists in LDS at once
constexpr int SG3_WPT = 32;      // consecutive windows a thread scans
constexpr int SG3_MAXW = 4 * 512 * SG3_WPT;  // windows of a route (B T) this path takes

__host__ __device__ constexpr size_t sg3_al(size_t x) { return (x + 255) & ~size_t{255}; }
struct Sg3Ws {  // byte offsets in the workspace
  size_t codes_t, scores, total, ct_stride;
};
__host__ __device__ inline Sg3Ws sg3_layout(int64_t B, int64_t T, int32_t R) {
  Sg3Ws w{};
  // a route's row holds B T codes rounded up to SG3_WPT, then SG3_WPT readable bytes
  w.ct_stride = sg3_al(static_cast<size_t>((B * T + SG3_WPT - 1) / SG3_WPT + 1) * SG3_WPT);
  w.codes_t = 0;                                                  // uint8 [R][ct_stride]
  w.scores = sg3_al(static_cast<size_t>(R) * w.ct_stride);        // float [3][R][B T][4]
  w.total = sg3_al(w.scores + static_cast<size_t>(B) * T * R * 12 * 4);
  return w;
}

// window (b, s) has a gradient row (its newest position s + 2 is valid); 32-bit indices: this path
// takes B * T * R < 2^28
__device__ __forceinline__ bool sg3_live(const SgArgs& a, int b, int s) {
  const int T = static_cast<int>(a.T);
  return s >= 0 && s < T - 2 && (a.valid == nullptr || a.valid[b * T + s + 2]);
}

// codes [B T, R] (any code dtype) -> codes_t [R][stride] uint8: byte w = the code at flat position w
// (low 4 bits) | 16 when the window starting at w is live; 64 x 64 tiles through LDS
__global__ __launch_bounds__(256) void k_sg3_transpose(SgArgs a, uint8_t* __restrict__ codes_t, int stride) {
  __shared__ uint8_t t[64][65];
  const int T = static_cast<int>(a.T), NWIN = static_cast<int>(a.B) * T, R = a.R;
  const int w0 = blockIdx.x * 64, r0 = blockIdx.y * 64;
  for (int i = threadIdx.x; i < 64 * 64; i += 256) {
    const int wl = i >> 6, rl = i & 63;
    const int w = w0 + wl, r = r0 + rl;
    uint8_t c = 0;
    if (w < NWIN && r < R) {
      const int b = w / T;
      c = static_cast<uint8_t>((sg_code(a.codes, a.codes_dt, static_cast<int64_t>(w) * R + r) & 15) |
                               (sg3_live(a, b, w - b * T) ? 16 : 0));
    }
    t[wl][rl] = c;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 64 * 64; i += 256) {
    const int rl = i >> 6, wl = i & 63;
    const int w = w0 + wl, r = r0 + rl;
    if (w < NWIN && r < R) codes_t[static_cast<int64_t>(r) * stride + w] = t[wl][rl];
  }
}

// A block per (route, bin v): sub-block v of the route's table block in LDS; the route's windows with
// digit 2 == v listed in LDS by one scan of the route's codes, 32 windows a thread (when more than
// SG3_MAXD windows share the bin, the route's windows are listed again in ranges of SG3_MAXD, one list
// at a time); 512 threads at 4 waves per SIMD (two blocks a CU); each 16-lane group takes listed
// windows grp, grp + NG, ...: the memory-gradient row (HBM) and the four digit-2 counterfactual rows
// (L2) of the next window are requested before the current window is reduced; its looked-up row (LDS,
// or the saved row when HARD) and eight digit-0 and digit-1 rows come from LDS.  Lane l of group g
// holds piece (l + 8 (g & 1)) & 15 of every row (the two halves of an LDS pass cover all 64 banks).
// Scores of digit e to plane e: scores[e][r][b T + s][bit].
template <bool HARD>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) void k_sg3_main(
    SgArgs a, const uint8_t* __restrict__ codes_t, int stride, float* __restrict__ scores) {
  constexpr int NT = 512, NG = NT / 16, NWV = NT / 64;
  constexpr int64_t D = 128;
  __shared__ __attribute__((aligned(16))) bf16 tab[256 * D];
  __shared__ uint32_t dl[SG3_MAXD];  // (b T + s) << 12 | address
  __shared__ int nl[2];
  const int tid = threadIdx.x, grp = tid >> 4, l = tid & 15, wave = tid >> 6, lane = tid & 63;
  const int xcd = blockIdx.x & 7, k8 = blockIdx.x >> 3;
  const int r = (k8 >> 4) * 8 + xcd;
  const uint32_t v = static_cast<uint32_t>(k8 & 15);
  if (r >= a.R) return;  // the whole block: before any barrier
  const int T = static_cast<int>(a.T), NWIN = static_cast<int>(a.B) * T;
  const int64_t rbase = (static_cast<int64_t>(a.route_start) + r) << 12;  // the route's first table row
  const bf16* table = static_cast<const bf16*>(a.table);
  const bf16* sub = table + (rbase + (static_cast<int64_t>(v) << 8)) * D;
  const uint8_t* ct = codes_t + static_cast<int64_t>(r) * stride;
  // windows (c NT + tid) SG3_WPT + i, i < SG3_WPT, c < 4, are the thread's; bin_mask says which are
  // live with digit 2 == v (their codes and liveness from three 16-byte loads).  The list is
  // written in the same pass while it has room; a bin of more than SG3_MAXD windows is listed again
  // in ranges below.
  // bit i: window wb + i is live with digit 2 == v (q0, q1, q2 = bytes wb .. wb + 47 of the route's codes)
  auto bin_mask = [&](u32x4 q0, u32x4 q1, u32x4 q2, int wb) {
    const uint32_t wd[9] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w, q2.x};
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < SG3_WPT; ++i) {
      const uint32_t cw = (wd[i >> 2] >> (8 * (i & 3))) & 0xFF;           // position wb + i
      const uint32_t c2 = (wd[(i + 2) >> 2] >> (8 * ((i + 2) & 3))) & 15;  // position wb + i + 2
      m |= ((cw & 16) && c2 == v && wb + i < NWIN) ? (1u << i) : 0u;
    }
    return m;
  };
  {
    u32x4 qv[4][3];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int wb = (c * NT + tid) * SG3_WPT;
#pragma unroll
      for (int k = 0; k < 3; ++k)
        qv[c][k] = wb < NWIN ? *reinterpret_cast<const u32x4*>(ct + wb + 16 * k) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < 64 / NWV; ++i) {  // the sub-block copy, behind the code loads
      const int kb = NWV * i + wave;
      __builtin_amdgcn_global_load_lds(sub + kb * 512 + lane * 8,
                                       (__attribute__((address_space(3))) void*)(tab + kb * 512), 16, 0, 0);
    }
    if (tid == 0) nl[0] = 0;
    __syncthreads();
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int wb = (c * NT + tid) * SG3_WPT;
      const uint32_t wd[9] = {qv[c][0].x, qv[c][0].y, qv[c][0].z, qv[c][0].w, qv[c][1].x,
                              qv[c][1].y, qv[c][1].z, qv[c][1].w, qv[c][2].x};
      uint32_t m = wb < NWIN ? bin_mask(qv[c][0], qv[c][1], qv[c][2], wb) : 0u;
      if (m) {
        int slot = atomicAdd(&nl[0], __builtin_popcount(m));
        for (; m; m &= m - 1, ++slot) {
          const int i = __builtin_ctz(m);  // window wb + i: its codes are bytes i and i + 1 of wd
          uint32_t x0 = wd[0], x1 = wd[0];
#pragma unroll
          for (int q = 1; q < 9; ++q) {
            x0 = (i >> 2) == q ? wd[q] : x0;
            x1 = ((i + 1) >> 2) == q ? wd[q] : x1;
          }
          const uint32_t addr = ((x0 >> (8 * (i & 3))) & 15u) | (((x1 >> (8 * ((i + 1) & 3))) & 15u) << 4) | (v << 8);
          if (slot < SG3_MAXD) dl[slot] = (static_cast<uint32_t>(wb + i) << 12) | addr;
        }
      }
    }
  }
  __syncthreads();
  const int total = nl[0];
  const int span = total <= SG3_MAXD ? NWIN : SG3_MAXD;  // windows per list
  const int pc = (l + 8 * (grp & 1)) & 15;
  const __amdgpu_buffer_rsrc_t trs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<bf16*>(table + rbase * D), 0, static_cast<int>(int64_t{4096} * D * 2), BUF_DW3);
  const bf16* grad = static_cast<const bf16*>(a.grad);
  const bf16* hard = static_cast<const bf16*>(a.hard);
  auto row = [&](uint32_t rw) { return *reinterpret_cast<const u32x4*>(tab + rw * D + pc * 8); };
  auto sum_last = [](float x) {
    x += dpp_row_shr<0x111>(x, 0.f);
    x += dpp_row_shr<0x112>(x, 0.f);
    x += dpp_row_shr<0x114>(x, 0.f);
    x += dpp_row_shr<0x118>(x, 0.f);
    return x;
  };
  const int64_t NW = a.B * a.T * a.R;  // windows per score plane
  struct Win {
    u32x4 g, h, f2[4];
  };
  auto load = [&](uint32_t d, Win& w) {
    const int64_t widx = d >> 12;                              // b T + s
    const int64_t mrow = ((widx + 2) * a.R + r) * D + pc * 8;  // position s + 2 of sequence b
    w.g = ld_raw16(grad, mrow * 2, a.nt != 0);
    if constexpr (HARD) w.h = ld_raw16(hard, mrow * 2, a.nt != 0);
    const uint32_t addr = d & 4095;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      w.f2[k] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                              trs, ((addr ^ (256u << k)) << 8) | (static_cast<uint32_t>(pc) << 4), 0, 0));
  };
  auto score = [&](uint32_t d, const Win& w) {  // the window's 12 scores, digit e to plane e
    const uint32_t addr = d & 4095, loc = addr & 255;
    u32x4 rv[9];
    rv[8] = HARD ? w.h : row(loc);
#pragma unroll
    for (int f = 0; f < 8; ++f) rv[f] = row(loc ^ (1u << f));
    const float cd = sum_last(dot8_bf16(rv[8], w.g));
    float sc[12];
#pragma unroll
    for (int f = 0; f < 8; ++f) sc[f] = (sum_last(dot8_bf16(rv[f], w.g)) - cd) * (((addr >> f) & 1) ? -1.f : 1.f);
#pragma unroll
    for (int k = 0; k < 4; ++k)
      sc[8 + k] = (sum_last(dot8_bf16(w.f2[k], w.g)) - cd) * (((addr >> (8 + k)) & 1) ? -1.f : 1.f);
    if (l == 15) {
      f32x4* o = reinterpret_cast<f32x4*>(scores) + static_cast<int64_t>(r) * NWIN + (d >> 12);
      o[0] = f32x4{sc[0], sc[1], sc[2], sc[3]};
      o[NW] = f32x4{sc[4], sc[5], sc[6], sc[7]};
      o[2 * NW] = f32x4{sc[8], sc[9], sc[10], sc[11]};
    }
  };
  for (int w0 = 0; w0 < NWIN; w0 += span) {
    if (total > SG3_MAXD) {  // list windows [w0, w1) of the bin
      if (tid == 0) nl[1] = 0;
      __syncthreads();
      const int w1 = min(NWIN, w0 + span);
      for (int c = 0; c < 4; ++c) {
        const int wb = (c * NT + tid) * SG3_WPT;
        if (wb >= w1 || wb + SG3_WPT <= w0) continue;
        const u32x4 q0 = *reinterpret_cast<const u32x4*>(ct + wb);
        const u32x4 q1 = *reinterpret_cast<const u32x4*>(ct + wb + 16);
        const u32x4 q2 = *reinterpret_cast<const u32x4*>(ct + wb + 32);
        const int lo = max(w0 - wb, 0), hi = min(w1 - wb, SG3_WPT);  // 0 <= lo < hi <= 32
        uint32_t m = bin_mask(q0, q1, q2, wb) & (hi == 32 ? ~0u : (1u << hi) - 1u) & ~((1u << lo) - 1u);
        if (!m) continue;
        int slot = atomicAdd(&nl[1], __builtin_popcount(m));
        for (; m; m &= m - 1) {
          const int w = wb + __builtin_ctz(m);
          const uint32_t addr = static_cast<uint32_t>(ct[w] & 15) | (static_cast<uint32_t>(ct[w + 1] & 15) << 4) | (v << 8);
          dl[slot++] = (static_cast<uint32_t>(w) << 12) | addr;
        }
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the sub-block copy (first list)
    __syncthreads();
    const int n = total > SG3_MAXD ? nl[1] : total;
    // entries grp, grp + NG, ... of the list, the next window's rows requested before the current one
    // is scored
    if (grp < n) {
      auto at = [&](int j) { return dl[j]; };
      Win cur, nxt;
      load(at(grp), cur);
      for (int j = grp; j < n; j += NG) {
        if (j + NG < n) load(at(j + NG), nxt);
        score(dl[j], cur);
        cur = nxt;
      }
    }
    __syncthreads();  // before the next list overwrites this one
  }
}

// out[b, t, r, k] = slope * (((0 + S0(t)[k]) + S1(t - 1)[k]) + S2(t - 2)[k]) with Se(w) = scores[e][r][w]
// (w = b T + s) and 0 for a window without a gradient row (the reference's sum over e ascending).  A
// block per tile of 64 positions x 16 routes: the scores are read along positions (one route a wave)
// and the sums pass through LDS to be scaled and written along routes.
__global__ __launch_bounds__(256) void k_sg3_out(SgArgs a, const float* __restrict__ scores) {
  __shared__ f32x4 tile[64][17];
  const int T = static_cast<int>(a.T), NWIN = static_cast<int>(a.B) * T, R = a.R;
  const int bt0 = blockIdx.x * 64, r0 = blockIdx.y * 16, tid = threadIdx.x;
  const int64_t NW = static_cast<int64_t>(NWIN) * R;  // windows per score plane
  const bool active = a.T > 2 && a.temperature != 0.f && a.scale != 0.f;
  const f32x4* sp = reinterpret_cast<const f32x4*>(scores);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int p = k * 256 + tid, rl = p >> 6, bl = p & 63;
    const int r = r0 + rl, bt = bt0 + bl;
    f32x4 acc{0.f, 0.f, 0.f, 0.f};
    if (r < R && bt < NWIN) {
      const int b = bt / T, t = bt - b * T;
#pragma unroll
      for (int e = 0; e < 3; ++e) {
        const f32x4 v = active && sg3_live(a, b, t - e) ? sp[e * NW + static_cast<int64_t>(r) * NWIN + (bt - e)]
                                                         : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[q] += v[q];
      }
    }
    tile[bl][rl] = acc;
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int p = k * 256 + tid, bl = p >> 4, rl = p & 15;
    const int r = r0 + rl, bt = bt0 + bl;
    if (r >= R || bt >= NWIN) continue;
    f32x4 acc = tile[bl][rl];
    const int64_t i = static_cast<int64_t>(bt) * R + r;  // (b T + t) R + r
    if (active) {
      f32x4 qv;
      if (a.q_dt == LNG_BF16) {
        const bf16x4 qh = reinterpret_cast<const bf16x4*>(a.q)[i];
#pragma unroll
        for (int q = 0; q < 4; ++q) qv[q] = static_cast<float>(qh[q]);
      } else {
        qv = reinterpret_cast<const f32x4*>(a.q)[i];
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float pr = 1.f / (1.f + expf(-(a.temperature * qv[q])));
        acc[q] *= a.alpha * pr * (1.f - pr);
      }
    }
    if (a.out_dt == LNG_BF16) {
      bf16x4 o;
#pragma unroll
      for (int q = 0; q < 4; ++q) o[q] = static_cast<bf16>(acc[q]);
      reinterpret_cast<bf16x4*>(a.out)[i] = o;
    } else {
      reinterpret_cast<f32x4*>(a.out)[i] = acc;
    }
  }
}

// whether the binned order-3 path serves a call, and its workspace
static bool sg3_ok(int mem_dtype, int exact, int64_t D, int32_t order, int32_t bits, int64_t B, int64_t T, int32_t R) {
  return mem_dtype == LNG_BF16 && !exact && D == 128 && order == 3 && bits == 4 && R <= 256 && T > 2 &&
         B * T <= SG3_MAXW && T * R * D * 2 < (int64_t{1} << 31);
}

static int sg3_launch(const SgArgs& a, uint8_t* ws, hipStream_t s) {
  const Sg3Ws w = sg3_layout(a.B, a.T, a.R);
  uint8_t* codes_t = ws + w.codes_t;
  float* scores = reinterpret_cast<float*>(ws + w.scores);
  const int stride = static_cast<int>(w.ct_stride);
  const dim3 tg(static_cast<unsigned>(cdiv(a.B * a.T, 64)), static_cast<unsigned>(cdiv(a.R, 64)));
  hipLaunchKernelGGL(k_sg3_transpose, tg, dim3(256), 0, s, a, codes_t, stride);
  const unsigned mblocks = static_cast<unsigned>(8 * cdiv(a.R, 8) * 16);
  if (a.hard)
    hipLaunchKernelGGL(k_sg3_main<true>, dim3(mblocks), dim3(512), 0, s, a, codes_t, stride, scores);
  else
    hipLaunchKernelGGL(k_sg3_main<false>, dim3(mblocks), dim3(512), 0, s, a, codes_t, stride, scores);
  hipLaunchKernelGGL(k_sg3_out, dim3(static_cast<unsigned>(cdiv(a.B * a.T, 64)), static_cast<unsigned>(cdiv(a.R, 16))),
                     dim3(256), 0, s, a, scores);
  return check_launch("surrogate_grad (order 3, binned)");
}

// Table gradient of the lookup (the embedding backward behind the surrogate's pass-through,
// lngram_v2.py:1084-1092 and :454): table_grad[row(b, t, r)] += grad[b, t, r, :] * valid[b, t] for
// every position with an order-`order` window.  One 16-lane group per (b, t, r); fp32 atomics, so
// rows met several times sum in an order that varies between calls.
template <typename TM, int V>
__global__ __launch_bounds__(256) void k_table_grad(SgArgs a, float* __restrict__ table_grad) {
  const int grp = threadIdx.x >> 4, l = threadIdx.x & 15;
  const int64_t o = static_cast<int64_t>(blockIdx.x) * SG_GROUPS + grp;
  if (o >= a.B * a.T * a.R) return;
  const int32_t r = static_cast<int32_t>(o % a.R);
  const int64_t bt = o / a.R;
  const int64_t t = bt % a.T, b = bt / a.T;
  const int bits = a.bits, order = a.order;
  if (t < order - 1) return;
  if (a.valid != nullptr && !a.valid[b * a.T + t]) return;
  const int64_t dmask = (int64_t(1) << bits) - 1;
  const int64_t s = t - order + 1;
  int64_t addr = 0;
  for (int k = 0; k < order; ++k)
    addr |= (sg_code(a.codes, a.codes_dt, (b * a.T + s + k) * a.R + r) & dmask) << (k * bits);
  const int64_t row = (static_cast<int64_t>(a.route_start + r) << (bits * order)) + addr;
  const int64_t D = 16 * V;
  float g[V];
  load_row<TM, V>(static_cast<const TM*>(a.grad) + o * D + l * V, g);
  float* dst = table_grad + row * D + l * V;
#pragma unroll
  for (int j = 0; j < V; ++j) atomicAdd(dst + j, g[j]);
}

template <typename TM, bool EXACT>
static int sg_launch_v(const SgArgs& a, int64_t D, hipStream_t s) {
  const int64_t blocks = 8 * cdiv(a.R, 8) * a.B * a.tiles;
  if (blocks > 0x7FFFFFFF) return fail(LNG_E_ARG, "surrogate_grad: too many blocks");
  if constexpr (sizeof(TM) == 2 && !EXACT) {
    if (D == 128 && a.bits == 4 && (a.order == 2 || a.order == 3)) {
      // order 2: 8 routes x 32 windows a block (their table blocks: 512 KB; the logits and gradients
      // of 8 routes fill whole 128 B lines); order 3: one route x 128 windows (its 1 MB block of
      // the table stays in the XCD's L2, where four routes' blocks were evicted by the streams)
      if (a.order == 2 && a.T * a.R * D * 2 < (int64_t{1} << 31)) {
        // the route's block of the table in LDS: 480 windows in 512 threads, or, streaming the
        // saved looked-up rows as well (more registers a lane), 256 windows in 256 threads
        SgArgs al = a;
        const int win = a.hard ? 256 : 480;
        al.tiles = cdiv(a.T, win - 1);
        const int64_t lblocks = 8 * cdiv(a.R, 8) * a.B * al.tiles;
        if (lblocks > 0x7FFFFFFF) return fail(LNG_E_ARG, "surrogate_grad: too many blocks");
        if (a.hard)
          k_surrogate_grad_o2lds<16, 256, true><<<lblocks, 256, 0, s>>>(al);
        else
          k_surrogate_grad_o2lds<15, 512, false><<<lblocks, 512, 0, s>>>(al);
        return check_launch("k_surrogate_grad_o2lds");
      }
      const int rg = a.order == 2 ? 8 : 1, win = a.order == 2 ? 256 : 128;
      SgArgs ap = a;
      ap.tiles = cdiv(a.T, win / rg - (a.order - 1));
      const int64_t pblocks = 8 * cdiv(cdiv(a.R, rg), 8) * a.B * ap.tiles;
      if (pblocks > 0x7FFFFFFF) return fail(LNG_E_ARG, "surrogate_grad: too many blocks");
      if (a.order == 2)
        k_surrogate_grad_pk<2, 8, 256><<<pblocks, 256, 0, s>>>(ap);
      else
        k_surrogate_grad_pk<3, 1, 128><<<pblocks, 256, 0, s>>>(ap);
      return check_launch("k_surrogate_grad_pk");
    }
  }
  switch (D) {
    case 32: k_surrogate_grad<TM, 2, EXACT><<<blocks, 256, 0, s>>>(a); break;
    case 64: k_surrogate_grad<TM, 4, EXACT><<<blocks, 256, 0, s>>>(a); break;
    case 128: k_surrogate_grad<TM, 8, EXACT><<<blocks, 256, 0, s>>>(a); break;
    case 256: k_surrogate_grad<TM, 16, EXACT><<<blocks, 256, 0, s>>>(a); break;
    default: return fail(LNG_E_ARG, "surrogate_grad: mem_dim must be 32, 64, 128 or 256");
  }
  return check_launch("k_surrogate_grad");
}

}  // namespace lng

using namespace lng;

static int surrogate_grad_impl(const void* grad_memory, const void* hard_memory, int mem_dtype, const void* q_logits,
                               int q_dtype, const void* codes, int codes_dtype, const void* table, int64_t table_rows,
                               const uint8_t* valid_mask, int64_t B, int64_t T, int32_t R, int32_t route_start,
                               int32_t mem_dim, int32_t order, int32_t bits, float temperature, float scale, int exact,
                               void* workspace, size_t workspace_bytes, void* grad_q, int out_dtype, void* stream) {
  if (B < 0 || T < 0 || R <= 0 || route_start < 0 || order < 1 || order > SG_MAXORDER || bits < 1 ||
      bits > SG_MAXBITS || bits * order > 40)
    return fail(LNG_E_ARG, "surrogate_grad: bad shape (1 <= order <= 4, 1 <= bits <= 8)");
  if (mem_dtype != LNG_F32 && mem_dtype != LNG_BF16) return fail(LNG_E_DTYPE, "surrogate_grad: memory f32 or bf16");
  if ((q_dtype != LNG_F32 && q_dtype != LNG_BF16) || (out_dtype != LNG_F32 && out_dtype != LNG_BF16))
    return fail(LNG_E_DTYPE, "surrogate_grad: logits and gradient f32 or bf16");
  if (codes_dtype != LNG_U8 && codes_dtype != LNG_I32 && codes_dtype != LNG_I64)
    return fail(LNG_E_DTYPE, "surrogate_grad: codes u8, i32 or i64");
  if (!grad_memory || !q_logits || !codes || !table || !grad_q)
    return fail(LNG_E_ARG, "surrogate_grad: null buffer");
  const int64_t need = (static_cast<int64_t>(route_start) + R) << (bits * order);
  if (table_rows < need) return fail(LNG_E_ARG, "surrogate_grad: table has fewer rows than (route_start + R) * 2^(bits*order)");
  if (B * T == 0) return LNG_OK;
  const int64_t mem_bytes = B * T * R * static_cast<int64_t>(mem_dim) * (mem_dtype == LNG_BF16 ? 2 : 4);
  SgArgs a{grad_memory, hard_memory, q_logits, q_dtype, codes, codes_dtype, table, valid_mask, B, T, R, route_start,
           order, bits, temperature, scale, static_cast<float>(static_cast<double>(scale) * temperature), grad_q,
           out_dtype, cdiv(T, SG_WIN - (order - 1)), mem_bytes < (int64_t(1) << 32) ? 1 : 0};
  hipStream_t s = as_stream(stream);
  const bool active = T - order + 1 > 0 && temperature != 0.f && scale != 0.f;
  // the binned path moves 16-byte vectors (8-byte for bf16 logits and gradient): it serves aligned buffers
  auto al = [](const void* p, uintptr_t n) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & (n - 1)) == 0; };
  const bool aligned = al(workspace, 256) && al(grad_memory, 16) && al(hard_memory, 16) && al(table, 16) &&
                       al(q_logits, q_dtype == LNG_BF16 ? 8 : 16) && al(grad_q, out_dtype == LNG_BF16 ? 8 : 16);
  if (workspace && active && aligned && sg3_ok(mem_dtype, exact, mem_dim, order, bits, B, T, R)) {
    if (workspace_bytes < sg3_layout(B, T, R).total)
      return fail(LNG_E_ARG, "surrogate_grad: workspace smaller than lng_surrogate_workspace_bytes");
    return sg3_launch(a, static_cast<uint8_t*>(workspace), s);
  }
  if (mem_dtype == LNG_BF16)
    return exact ? sg_launch_v<bf16, true>(a, mem_dim, s) : sg_launch_v<bf16, false>(a, mem_dim, s);
  return exact ? sg_launch_v<float, true>(a, mem_dim, s) : sg_launch_v<float, false>(a, mem_dim, s);
}

extern "C" int lng_surrogate_grad(const void* grad_memory, const void* hard_memory, int mem_dtype, const void* q_logits,
                                  int q_dtype, const void* codes, int codes_dtype, const void* table,
                                  int64_t table_rows, const uint8_t* valid_mask, int64_t B, int64_t T, int32_t R,
                                  int32_t route_start, int32_t mem_dim, int32_t order, int32_t bits,
                                  float temperature, float scale, int exact, void* grad_q, int out_dtype,
                                  void* stream) {
  return surrogate_grad_impl(grad_memory, hard_memory, mem_dtype, q_logits, q_dtype, codes, codes_dtype, table,
                             table_rows, valid_mask, B, T, R, route_start, mem_dim, order, bits, temperature, scale,
                             exact, nullptr, 0, grad_q, out_dtype, stream);
}

extern "C" size_t lng_surrogate_workspace_bytes(int64_t B, int64_t T, int32_t R, int32_t mem_dim, int32_t order,
                                                int32_t bits, int mem_dtype, int exact) {
  if (B <= 0 || T <= 0 || R <= 0) return 0;
  return sg3_ok(mem_dtype, exact, mem_dim, order, bits, B, T, R) ? sg3_layout(B, T, R).total : 0;
}

extern "C" int lng_surrogate_grad_ws(const void* grad_memory, const void* hard_memory, int mem_dtype,
                                     const void* q_logits, int q_dtype, const void* codes, int codes_dtype,
                                     const void* table, int64_t table_rows, const uint8_t* valid_mask, int64_t B,
                                     int64_t T, int32_t R, int32_t route_start, int32_t mem_dim, int32_t order,
                                     int32_t bits, float temperature, float scale, int exact, void* workspace,
                                     size_t workspace_bytes, void* grad_q, int out_dtype, void* stream) {
  return surrogate_grad_impl(grad_memory, hard_memory, mem_dtype, q_logits, q_dtype, codes, codes_dtype, table,
                             table_rows, valid_mask, B, T, R, route_start, mem_dim, order, bits, temperature, scale,
                             exact, workspace, workspace_bytes, grad_q, out_dtype, stream);
}

extern "C" int lng_table_grad(const void* grad_memory, int mem_dtype, const void* codes, int codes_dtype,
                              const uint8_t* valid_mask, int64_t B, int64_t T, int32_t R, int32_t route_start,
                              int32_t mem_dim, int32_t order, int32_t bits, int64_t table_rows, float* table_grad,
                              void* stream) {
  if (B < 0 || T < 0 || R <= 0 || route_start < 0 || order < 1 || order > SG_MAXORDER || bits < 1 ||
      bits > SG_MAXBITS || bits * order > 40)
    return fail(LNG_E_ARG, "table_grad: bad shape (1 <= order <= 4, 1 <= bits <= 8)");
  if (mem_dtype != LNG_F32 && mem_dtype != LNG_BF16) return fail(LNG_E_DTYPE, "table_grad: memory f32 or bf16");
  if (codes_dtype != LNG_U8 && codes_dtype != LNG_I32 && codes_dtype != LNG_I64)
    return fail(LNG_E_DTYPE, "table_grad: codes u8, i32 or i64");
  if (!grad_memory || !codes || !table_grad) return fail(LNG_E_ARG, "table_grad: null buffer");
  if (table_rows < ((static_cast<int64_t>(route_start) + R) << (bits * order)))
    return fail(LNG_E_ARG, "table_grad: table has fewer rows than (route_start + R) * 2^(bits*order)");
  if (B * T == 0) return LNG_OK;
  SgArgs a{grad_memory, nullptr, nullptr, LNG_F32, codes, codes_dtype, nullptr, valid_mask, B, T, R, route_start,
           order, bits, 0.f, 0.f, 0.f, nullptr, LNG_F32, 0, 0};
  hipStream_t s = as_stream(stream);
  const int64_t blocks = cdiv(B * T * R, SG_GROUPS);
#define TG_LAUNCH(TM, V) k_table_grad<TM, V><<<blocks, 256, 0, s>>>(a, table_grad)
  const bool bf = mem_dtype == LNG_BF16;
  switch (mem_dim) {
    case 32: if (bf) TG_LAUNCH(bf16, 2); else TG_LAUNCH(float, 2); break;
    case 64: if (bf) TG_LAUNCH(bf16, 4); else TG_LAUNCH(float, 4); break;
    case 128: if (bf) TG_LAUNCH(bf16, 8); else TG_LAUNCH(float, 8); break;
    case 256: if (bf) TG_LAUNCH(bf16, 16); else TG_LAUNCH(float, 16); break;
    default: return fail(LNG_E_ARG, "table_grad: mem_dim must be 32, 64, 128 or 256");
  }
#undef TG_LAUNCH
  return check_launch("k_table_grad");
}
