// Token-only router input of SD-B / SD-C (TokenRouterFeatures.forward, ffnmem/memory/router.py:50-59):
//
//   x[p] = concat(RMSNorm_prev(E[x_{t-1}] or start), RMSNorm_cur(E[x_t]) [, s[p] in the feature dtype])
//
// with model.RMSNorm's rounding (model.py:39-48): normalise in fp32, round to the feature dtype,
// multiply by the weight in that dtype.  The rows come either from a token-id array and the
// embedding table (the embedding gather fused in) or from a materialised emb [B*T, d].
//
// One wave per position: the two d-wide rows are read as 16-byte pieces held in registers
// (at most FE_MAXP per lane), both rows' loads issued before either is reduced, squared-summed
// with a wave reduction, scaled and stored.
#include "common.h"

namespace lng {

constexpr int FE_MAXP = 8;  // 16-byte pieces per lane and row: d <= 4096 (bf16) / 2048 (fp32)

struct FeArgs {
  const void* emb;         // [V, d] table (with ids) or [n_tok, d] rows (ids == nullptr)
  const int64_t* ids;      // [n_tok] token ids or nullptr
  int64_t V, T, n_tok;
  const void* start;       // [d]
  const void* prev_w;      // [d]
  const void* cur_w;       // [d]
  const float* ssm;        // [n_tok, N] or nullptr
  int32_t d, N;
  float eps;
};

typedef uint32_t fe_piece_t __attribute__((ext_vector_type(4)));

// The pieces of one d-wide row that lane `lane` holds (pieces lane, lane + 64, ...; PPL of them).
template <typename TT, int PPL>
__device__ __forceinline__ void fe_load_row(const TT* src, int np, int lane, fe_piece_t (&v)[PPL]) {
  constexpr int VE = 16 / sizeof(TT);
#pragma unroll
  for (int i = 0; i < PPL; ++i) {
    const int pc = i * 64 + lane;
    v[i] = (src && pc < np) ? *reinterpret_cast<const fe_piece_t*>(src + pc * VE) : fe_piece_t{0u, 0u, 0u, 0u};
  }
}

// RMSNorm of the row held in v (model.py:39-48 rounding), stored at dst.
template <typename TT, int PPL>
__device__ __forceinline__ void fe_norm_store(const fe_piece_t (&v)[PPL], const TT* w, int d, int np, float eps, TT* dst,
                                              int lane) {
  constexpr int VE = 16 / sizeof(TT);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < PPL; ++i) {
    const TT* e = reinterpret_cast<const TT*>(&v[i]);
#pragma unroll
    for (int j = 0; j < VE; ++j) {
      const float f = to_f32(e[j]);
      ss = fmaf(f, f, ss);
    }
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / static_cast<float>(d) + eps);
#pragma unroll
  for (int i = 0; i < PPL; ++i) {
    const int pc = i * 64 + lane;
    if (pc >= np) continue;
    const fe_piece_t wp = *reinterpret_cast<const fe_piece_t*>(w + pc * VE);
    const TT* e = reinterpret_cast<const TT*>(&v[i]);
    const TT* ww = reinterpret_cast<const TT*>(&wp);
    fe_piece_t o;
    TT* oe = reinterpret_cast<TT*>(&o);
#pragma unroll
    for (int j = 0; j < VE; ++j) oe[j] = from_f32<TT>(round_to<TT>(to_f32(e[j]) * r) * to_f32(ww[j]));
    *reinterpret_cast<fe_piece_t*>(dst + pc * VE) = o;
  }
}

// grid (cdiv(n_tok, 4)), block 256: wave w owns position 4 * blockIdx.x + w.  PPL = 16-byte pieces
// per lane and row (d / (64 VE) rounded up).  The two rows and the SSM state are requested before
// either row is reduced: one memory round trip per position.
template <typename TT, int PPL>
__global__ __launch_bounds__(256) void k_router_features(FeArgs A, TT* __restrict__ out) {
  constexpr int VE = 16 / sizeof(TT);
  constexpr int SQ = 4;  // SSM values per lane held in registers (N <= 256); the rest stream
  const int lane = threadIdx.x & 63;
  const int64_t p = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (p >= A.n_tok) return;
  const int64_t t = p % A.T;
  const TT* emb = static_cast<const TT*>(A.emb);
  const int d = A.d, np = d / VE;
  auto row = [&](int64_t q) -> const TT* {  // embedding row of position q (nullptr: id outside [0, V))
    if (!A.ids) return emb + q * d;
    const int64_t id = A.ids[q];
    return (id >= 0 && id < A.V) ? emb + id * d : nullptr;
  };
  const int64_t od = 2 * static_cast<int64_t>(d) + A.N;
  TT* o = out + p * od;
  const TT* prev = t == 0 ? static_cast<const TT*>(A.start) : row(p - 1);
  const TT* cur = row(p);
  fe_piece_t vp[PPL], vc[PPL];
  fe_load_row<TT, PPL>(prev, np, lane, vp);
  fe_load_row<TT, PPL>(cur, np, lane, vc);
  float sq[SQ];
  if (A.ssm) {
#pragma unroll
    for (int k = 0; k < SQ; ++k) sq[k] = lane + 64 * k < A.N ? A.ssm[p * A.N + lane + 64 * k] : 0.f;
  }
  fe_norm_store<TT, PPL>(vp, static_cast<const TT*>(A.prev_w), d, np, A.eps, o, lane);
  fe_norm_store<TT, PPL>(vc, static_cast<const TT*>(A.cur_w), d, np, A.eps, o + d, lane);
  if (A.ssm) {
#pragma unroll
    for (int k = 0; k < SQ; ++k)
      if (lane + 64 * k < A.N) o[2 * d + lane + 64 * k] = from_f32<TT>(sq[k]);
    for (int i = lane + 64 * SQ; i < A.N; i += 64) o[2 * d + i] = from_f32<TT>(A.ssm[p * A.N + i]);
  }
}

// The router's normalised embedding tables (bf16): fprev [V+2, d] = RMSNorm_prev of E's rows,
// then of `start` (row V), then a zero row (V+1); fcur [V+1, d] = RMSNorm_cur of E's rows, then a
// zero row (V).  Rows are normalised exactly as k_router_features normalises a gathered row, so a
// feature row assembled from the tables equals the one that kernel writes.  One wave per row index.
template <int PPL>
__global__ __launch_bounds__(256) void k_router_feature_tables(const bf16* __restrict__ E, int64_t V,
                                                               const bf16* __restrict__ start,
                                                               const bf16* __restrict__ prev_w,
                                                               const bf16* __restrict__ cur_w, int32_t d, float eps,
                                                               bf16* __restrict__ fprev, bf16* __restrict__ fcur) {
  const int lane = threadIdx.x & 63;
  const int64_t v = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (v > V + 1) return;
  const int np = d / 8;
  const bf16* row = v < V ? E + v * d : nullptr;
  fe_piece_t vp[PPL], vc[PPL];
  fe_load_row<bf16, PPL>(v < V ? row : (v == V ? start : nullptr), np, lane, vp);
  fe_load_row<bf16, PPL>(row, np, lane, vc);
  fe_norm_store<bf16, PPL>(vp, prev_w, d, np, eps, fprev + v * d, lane);
  if (v <= V) fe_norm_store<bf16, PPL>(vc, cur_w, d, np, eps, fcur + v * d, lane);
}

}  // namespace lng

using namespace lng;

extern "C" int lng_router_feature_tables(const void* emb, int64_t vocab, int32_t d, const void* start,
                                         const void* prev_w, const void* cur_w, float eps, void* fprev, void* fcur,
                                         void* stream) {
  if (!emb || !start || !prev_w || !cur_w || !fprev || !fcur) return fail(LNG_E_ARG, "router_feature_tables: null pointer");
  if (vocab <= 0 || vocab > (int64_t{1} << 30) || d <= 0 || d % 8 || d / 8 > FE_MAXP * 64)
    return fail(LNG_E_ARG, "router_feature_tables: bf16 rows of d % 8 == 0, d <= 4096, 0 < vocab <= 2^30");
  const dim3 grid(static_cast<unsigned>(cdiv(vocab + 2, 4)));
  hipStream_t s = as_stream(stream);
  const bf16 *e = static_cast<const bf16*>(emb), *st = static_cast<const bf16*>(start);
  const bf16 *pw = static_cast<const bf16*>(prev_w), *cw = static_cast<const bf16*>(cur_w);
  bf16 *fp = static_cast<bf16*>(fprev), *fc = static_cast<bf16*>(fcur);
  switch (static_cast<int>(cdiv(d / 8, 64))) {
    case 1: hipLaunchKernelGGL((k_router_feature_tables<1>), grid, dim3(256), 0, s, e, vocab, st, pw, cw, d, eps, fp, fc); break;
    case 2: hipLaunchKernelGGL((k_router_feature_tables<2>), grid, dim3(256), 0, s, e, vocab, st, pw, cw, d, eps, fp, fc); break;
    case 3:
    case 4: hipLaunchKernelGGL((k_router_feature_tables<4>), grid, dim3(256), 0, s, e, vocab, st, pw, cw, d, eps, fp, fc); break;
    default:
      hipLaunchKernelGGL((k_router_feature_tables<FE_MAXP>), grid, dim3(256), 0, s, e, vocab, st, pw, cw, d, eps, fp, fc);
      break;
  }
  return check_launch("router_feature_tables");
}

extern "C" int lng_router_features(const void* emb, int dtype, const int64_t* token_ids, int64_t vocab, int64_t B,
                                   int64_t T, int32_t d, const void* start, const void* prev_w, const void* cur_w,
                                   float eps, const float* ssm_state, int32_t N, void* out, void* stream) {
  if (!emb || !start || !prev_w || !cur_w || !out) return fail(LNG_E_ARG, "router_features: null pointer");
  if (dtype != LNG_BF16 && dtype != LNG_F32) return fail(LNG_E_DTYPE, "router_features: dtype must be bf16 or fp32");
  if (B < 0 || T < 0 || N < 0 || (N > 0) != (ssm_state != nullptr))
    return fail(LNG_E_ARG, "router_features: bad shape (ssm_state and N > 0 go together)");
  if (token_ids && vocab <= 0) return fail(LNG_E_ARG, "router_features: vocab must be positive with token ids");
  const int es = dtype_size(dtype), ve = 16 / es;
  if (d <= 0 || d % ve || d / ve > FE_MAXP * 64 || ((2 * static_cast<int64_t>(d) + N) * es) % 16)
    return fail(LNG_E_ARG, "router_features: d must be a multiple of 16 bytes (at most 8 KB) and the feature row "
                           "(2 d + N elements) a multiple of 16 bytes");
  FeArgs A{emb, token_ids, vocab, T, B * T, start, prev_w, cur_w, ssm_state, d, N, eps};
  if (A.n_tok == 0) return LNG_OK;
  const dim3 grid(static_cast<unsigned>(cdiv(A.n_tok, 4)));
  hipStream_t s = as_stream(stream);
  const int ppl = static_cast<int>(cdiv(d / ve, 64));  // pieces per lane and row
  auto go = [&](auto tt) {
    using TT = decltype(tt);
    TT* o = static_cast<TT*>(out);
    switch (ppl) {
      case 1: hipLaunchKernelGGL((k_router_features<TT, 1>), grid, dim3(256), 0, s, A, o); break;
      case 2: hipLaunchKernelGGL((k_router_features<TT, 2>), grid, dim3(256), 0, s, A, o); break;
      case 3:
      case 4: hipLaunchKernelGGL((k_router_features<TT, 4>), grid, dim3(256), 0, s, A, o); break;
      default: hipLaunchKernelGGL((k_router_features<TT, FE_MAXP>), grid, dim3(256), 0, s, A, o); break;
    }
  };
  if (dtype == LNG_BF16)
    go(bf16{});
  else
    go(float{});
  return check_launch("router_features");
}
