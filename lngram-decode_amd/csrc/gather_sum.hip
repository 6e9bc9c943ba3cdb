// Random-row gather + sum over an n-gram table grown S = 2^scale_log2 times per route: the
// scaled-table stress of the memory path.  Every (token, route, order) reads one row of its
// route's order block, which holds S copies ("slots") of the 16^n code addresses:
//
//   row(b, t, r, n) = r * S * 16^n + slot(b*T + t, i) * 16^n + addr_n(b, t, r)
//   addr_n          = sum_k c[b, t-n+1+k, r] << (bits k)   c = code & (2^bits - 1), oldest least significant
//   slot(p, i)      = mix32(seed ^ mix32(p * 0x9E3779B1 + i)) & (S - 1),   i = r * n_orders + (order index)
//   mix32           = the MurmurHash3 32-bit finaliser
//   out[b, t, :]    = sum over routes r and orders n with t >= n-1 of table_n[row, :]   (fp32)
//
// With S = 1 the row is the reference's global n-gram row r*16^n + addr (lngram_v2.py:1058,
// :1064-1092) and out is the sum of the route tokens' halves, so the kernel is the gather of
// the memory path with the readout replaced by a plain sum.  Positions t < n-1 read nothing (the
// reference's zero rows).  Table n holds R * S * 16^n rows, so every row read lies inside it.
//
// Layout: one wave per token.  The wave first forms every row index of its token (codes from
// LDS, the slot hash) into an LDS list, so the load loop that follows issues its loads back to
// back with no dependent work in between.  A row of `row_bytes` = mem_dim * elem bytes is read
// as P = row_bytes / 16 pieces by P consecutive lanes, so one wave load moves 64/P whole rows
// (4 rows of 256 B for bf16 x 128).  Each lane keeps the fp32 sums of its piece's elements over
// the rows its lane group reads; the groups are folded with cross-lane permutes at the end.
// Eight loads per lane are in flight before the first is summed.
#include <algorithm>

#include "common.h"

namespace lng {

constexpr int GS_MAXR = 256;   // routes
constexpr int GS_MAXN = 4;     // max order
constexpr int GS_UNROLL = 8;   // loads in flight per lane

__host__ __device__ __forceinline__ uint32_t mix32(uint32_t h) {
  h ^= h >> 16;
  h *= 0x85EBCA6Bu;
  h ^= h >> 13;
  h *= 0xC2B2AE35u;
  h ^= h >> 16;
  return h;
}

struct GsArgs {
  const char* tab[GS_MAXN];
  int32_t order[GS_MAXN];
  int32_t n_orders, maxn, bits, scale_log2, R;
  uint32_t seed;
  int64_t T, n_tok;
};

// grid (cdiv(n_tok, 4)), block 256: wave w owns token 4 * blockIdx.x + w.
// TT = element type (bf16 or float); P = 16-byte pieces per row (divides 64); RT = the type of
// the staged row indices (int32_t when every table has fewer than 2^31 rows, else int64_t).
template <typename TT, int P, typename RT>
__global__ __launch_bounds__(256) void k_gather_sum_scaled(GsArgs A, const uint8_t* __restrict__ codes,
                                                           float* __restrict__ out) {
  constexpr int VE = 16 / sizeof(TT);  // elements per piece
  constexpr int RPI = 64 / P;          // rows per wave load
  __shared__ uint8_t cs[4][GS_MAXN][GS_MAXR];
  __shared__ RT rows_l[4][GS_MAXR * GS_MAXN + 64];  // row index of row i of the token, -1 = masked
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t p = static_cast<int64_t>(blockIdx.x) * 4 + w;
  const bool live = p < A.n_tok;
  const int64_t t = live ? p % A.T : 0;
  const int R = A.R, maxn = A.maxn, n_ord = A.n_orders, bits = A.bits;
  // codes of positions t-maxn+1 .. t of this token's sequence (slot k <-> position t-maxn+1+k)
  for (int e = lane; e < maxn * R; e += 64) {
    const int k = e / R, r = e % R;
    const int64_t tt = t - (maxn - 1) + k;
    cs[w][k][r] = (live && tt >= 0) ? codes[(p - t + tt) * R + r] : 0;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int g = lane / P, pc = lane % P;
  const int nrows = R * n_ord;
  const uint32_t smask = (1u << A.scale_log2) - 1u, cmask = (1u << bits) - 1u;
  const uint32_t pmix = static_cast<uint32_t>(p) * 0x9E3779B1u;
  const int64_t row_bytes = static_cast<int64_t>(P) * 16;
  // row index of row i of this token (i = r * n_orders + oi), -1 where the row is masked
  auto row_of = [&](int i) -> int64_t {
    const int r = i / n_ord, oi = i - r * n_ord;
    const int n = A.order[oi];
    if (!live || t < n - 1) return -1;
    uint32_t addr = 0;
    for (int k = 0; k < n; ++k) addr |= (static_cast<uint32_t>(cs[w][maxn - n + k][r]) & cmask) << (bits * k);
    const uint32_t slot = mix32(A.seed ^ mix32(pmix + static_cast<uint32_t>(i))) & smask;
    const int64_t block = int64_t{1} << (bits * n);
    return (static_cast<int64_t>(r) * (smask + 1) + slot) * block + addr;
  };
  const int steps = (nrows + RPI - 1) / RPI;
  for (int i = lane; i < steps * RPI; i += 64) rows_l[w][i] = i < nrows ? static_cast<RT>(row_of(i)) : RT(-1);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float acc[VE];
#pragma unroll
  for (int e = 0; e < VE; ++e) acc[e] = 0.f;
  for (int s0 = 0; s0 < steps; s0 += GS_UNROLL) {
    u32x4 v[GS_UNROLL];
#pragma unroll
    for (int u = 0; u < GS_UNROLL; ++u) {
      const int i = (s0 + u) * RPI + g;
      const int64_t row = s0 + u < steps ? static_cast<int64_t>(rows_l[w][i]) : -1;
      const int oi = i % n_ord;
      v[u] = row >= 0 ? *reinterpret_cast<const u32x4*>(A.tab[oi] + row * row_bytes + 16 * pc)
                      : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < GS_UNROLL; ++u) {
      if constexpr (sizeof(TT) == 2) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          acc[2 * q] += __uint_as_float(v[u][q] << 16);
          acc[2 * q + 1] += __uint_as_float(v[u][q] & 0xFFFF0000u);
        }
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[q] += __uint_as_float(v[u][q]);
      }
    }
  }
  // fold the RPI lane groups (lanes pc, pc + P, ...) into lanes 0 .. P-1
#pragma unroll
  for (int sh = P; sh < 64; sh <<= 1)
#pragma unroll
    for (int e = 0; e < VE; ++e) acc[e] += __shfl_xor(acc[e], sh);
  if (live && lane < P) {
    float* o = out + p * (P * VE) + VE * pc;
#pragma unroll
    for (int e = 0; e < VE; e += 4) *reinterpret_cast<f32x4*>(o + e) = f32x4{acc[e], acc[e + 1], acc[e + 2], acc[e + 3]};
  }
}

}  // namespace lng

using namespace lng;

extern "C" int lng_gather_sum_scaled(const void* const* tables, int table_dtype, int32_t mem_dim, const uint8_t* codes,
                                     int64_t B, int64_t T, int32_t R, const int32_t* orders, int32_t n_orders,
                                     int32_t bits, int32_t scale_log2, uint32_t seed, float* out, void* stream) {
  if (!tables || !codes || !out || !orders) return fail(LNG_E_ARG, "gather_sum_scaled: null pointer");
  if (B < 0 || T < 0 || R <= 0 || R > GS_MAXR || n_orders <= 0 || n_orders > GS_MAXN || bits <= 0 || bits > 8 ||
      scale_log2 < 0 || scale_log2 > 16)
    return fail(LNG_E_ARG, "gather_sum_scaled: shape out of range (R <= 256, 1..4 orders, bits <= 8, scale_log2 <= 16)");
  if (table_dtype != LNG_BF16 && table_dtype != LNG_F32)
    return fail(LNG_E_DTYPE, "gather_sum_scaled: table dtype must be bf16 or fp32");
  const int es = dtype_size(table_dtype);
  const int64_t row_bytes = static_cast<int64_t>(mem_dim) * es;
  if (mem_dim <= 0 || row_bytes % 16 || 64 % (row_bytes / 16))
    return fail(LNG_E_ARG, "gather_sum_scaled: mem_dim * element size must be 16 B times a divisor of 64");
  GsArgs A{};
  A.maxn = 0;
  bool rows32 = true;  // every table holds fewer than 2^31 rows
  for (int i = 0; i < n_orders; ++i) {
    if (orders[i] < 1 || orders[i] > GS_MAXN || !tables[i])
      return fail(LNG_E_ARG, "gather_sum_scaled: orders must lie in [1, 4] with a table each");
    if (static_cast<int64_t>(bits) * orders[i] + scale_log2 + 8 > 62)
      return fail(LNG_E_ARG, "gather_sum_scaled: table too large to index");
    A.tab[i] = static_cast<const char*>(tables[i]);
    A.order[i] = orders[i];
    A.maxn = std::max(A.maxn, orders[i]);
    rows32 = rows32 && (static_cast<int64_t>(R) << (scale_log2 + bits * orders[i])) <= INT32_MAX;
  }
  A.n_orders = n_orders;
  A.bits = bits;
  A.scale_log2 = scale_log2;
  A.R = R;
  A.seed = seed;
  A.T = T;
  A.n_tok = B * T;
  if (A.n_tok == 0) return LNG_OK;
  const int P = static_cast<int>(row_bytes / 16);
  const dim3 grid(static_cast<unsigned>(cdiv(A.n_tok, 4)));
  hipStream_t s = as_stream(stream);
  auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, dim3(256), 0, s, A, codes, out); };
  auto by_piece = [&](auto tt, auto rt) {
    using TT = decltype(tt);
    using RT = decltype(rt);
    switch (P) {
      case 1: go(k_gather_sum_scaled<TT, 1, RT>); break;
      case 2: go(k_gather_sum_scaled<TT, 2, RT>); break;
      case 4: go(k_gather_sum_scaled<TT, 4, RT>); break;
      case 8: go(k_gather_sum_scaled<TT, 8, RT>); break;
      case 16: go(k_gather_sum_scaled<TT, 16, RT>); break;
      case 32: go(k_gather_sum_scaled<TT, 32, RT>); break;
      default: go(k_gather_sum_scaled<TT, 64, RT>); break;
    }
  };
  if (table_dtype == LNG_BF16) {
    if (rows32) by_piece(bf16{}, int32_t{});
    else by_piece(bf16{}, int64_t{});
  } else {
    if (rows32) by_piece(float{}, int32_t{});
    else by_piece(float{}, int64_t{});
  }
  return check_launch("gather_sum_scaled");
}
