// Status plumbing and the integer kernels of the hot path: route-code packing,
// n-gram addresses, global rows, the route-token gather and tree acceptance.
#include "common.h"

namespace lng {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(LNG_E_HIP, std::string(what) + ": " + hipGetErrorString(e));
  return LNG_OK;
}

// ------------------------------------------------------------------ code access
// Route codes are stored as uint8 (decode caches), int32 (quantize output) or int64.
struct CodeView {
  const void* p;
  int dt;
  __device__ __forceinline__ int64_t at(int64_t i) const {
    if (dt == LNG_U8) return static_cast<const uint8_t*>(p)[i];
    if (dt == LNG_I32) return static_cast<const int32_t*>(p)[i];
    return static_cast<const int64_t*>(p)[i];
  }
};

static bool code_dtype_ok(int dt) { return dt == LNG_U8 || dt == LNG_I32 || dt == LNG_I64; }

// Global row of the order-`order` n-gram of route r ending at position t, or -1
// where the reference masks the row to zero (t < order-1, a segment change inside
// the window, or an invalid last token).  Oldest code least significant.
// `digit_mask` = -1 keeps the codes as given (pure index arithmetic); the gather passes
// 2^bits - 1 so that an out-of-range code can never address outside its route's block.
__device__ __forceinline__ int64_t ngram_row(const CodeView& codes, int64_t T, int32_t R, int64_t b, int64_t t,
                                             int32_t r, int32_t order, int32_t bits, const int32_t* seg,
                                             const uint8_t* valid, int64_t digit_mask = -1) {
  if (t < order - 1) return -1;
  const int64_t t0 = t - order + 1;
  if (seg && seg[b * T + t0] != seg[b * T + t]) return -1;
  if (valid && !valid[b * T + t]) return -1;
  int64_t addr = 0;
  for (int k = 0; k < order; ++k) addr |= (codes.at((b * T + t0 + k) * R + r) & digit_mask) << (k * bits);
  return static_cast<int64_t>(r) * (int64_t(1) << (bits * order)) + addr;
}

// ------------------------------------------------------------------ kernels
__global__ void k_pack_codes(const float* __restrict__ logits, int64_t M, int64_t routes, int32_t bits,
                             void* __restrict__ codes, int codes_dt) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= M * routes) return;
  const float* q = logits + i * bits;
  int v = 0;
  for (int k = 0; k < bits; ++k) v |= (q[k] > 0.f ? 1 : 0) << k;
  if (codes_dt == LNG_U8)
    static_cast<uint8_t*>(codes)[i] = static_cast<uint8_t>(v);
  else
    static_cast<int32_t*>(codes)[i] = v;
}

__global__ void k_ngram_address(CodeView codes, int64_t B, int64_t T, int32_t R, int32_t order, int32_t bits,
                                void* __restrict__ out, int out_dt) {
  const int64_t tv = T - order + 1;
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= B * tv * R) return;
  const int32_t r = static_cast<int32_t>(i % R);
  const int64_t t = (i / R) % tv;
  const int64_t b = i / (R * tv);
  int64_t addr = 0;
  for (int k = 0; k < order; ++k) addr |= codes.at((b * T + t + k) * R + r) << (k * bits);
  if (out_dt == LNG_I32)
    static_cast<int32_t*>(out)[i] = static_cast<int32_t>(addr);
  else
    static_cast<int64_t*>(out)[i] = addr;
}

struct OrderList {
  int32_t n;
  int32_t v[8];
};

template <typename RowT>
__global__ void k_ngram_rows(CodeView codes, int64_t B, int64_t T, int32_t R, int32_t rs, int32_t re, OrderList ords,
                             int32_t bits, const int32_t* seg, const uint8_t* valid, RowT* __restrict__ rows) {
  const int32_t rw = re - rs;
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= B * T * rw * ords.n) return;
  const int32_t oi = static_cast<int32_t>(i % ords.n);
  const int32_t r = rs + static_cast<int32_t>((i / ords.n) % rw);
  const int64_t bt = i / (static_cast<int64_t>(ords.n) * rw);
  const int64_t t = bt % T, b = bt / T;
  rows[i] = static_cast<RowT>(ngram_row(codes, T, R, b, t, r, ords.v[oi], bits, seg, valid));
}

// One thread copies one `vec`-byte piece of an output route token.  Output
// [B, T_out, rw, n_orders * mem_dim]; segment = (b, t, r, order), mem_dim*esize bytes.
template <typename V>
__global__ void k_route_tokens(CodeView codes, int64_t B, int64_t T, int64_t t_first, int64_t T_out, int32_t R,
                               int32_t rs, int32_t rw, OrderList ords, int32_t bits, const void* t0, const void* t1,
                               const void* t2, const void* t3, int32_t seg_bytes, const int32_t* seg,
                               const uint8_t* valid, V* __restrict__ out) {
  const int32_t per_seg = seg_bytes / static_cast<int32_t>(sizeof(V));
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  const int64_t total = B * T_out * rw * ords.n * static_cast<int64_t>(per_seg);
  if (i >= total) return;
  const int32_t piece = static_cast<int32_t>(i % per_seg);
  const int64_t s = i / per_seg;
  const int32_t oi = static_cast<int32_t>(s % ords.n);
  const int32_t r = rs + static_cast<int32_t>((s / ords.n) % rw);
  const int64_t bt = s / (static_cast<int64_t>(ords.n) * rw);
  const int64_t t = t_first + bt % T_out, b = bt / T_out;
  const int64_t row = ngram_row(codes, T, R, b, t, r, ords.v[oi], bits, seg, valid, (int64_t(1) << bits) - 1);
  V val;
  if (row < 0) {
    val = V{};
  } else {
    const void* tab = oi == 0 ? t0 : oi == 1 ? t1 : oi == 2 ? t2 : t3;
    val = reinterpret_cast<const V*>(static_cast<const char*>(tab) + row * seg_bytes)[piece];
  }
  out[i] = val;
}

__global__ void k_tree_accept(const int32_t* parent, const int64_t* node_tokens, const int64_t* argmax, int32_t n,
                              int32_t* path, int32_t* path_len, int64_t* new_tokens) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  int32_t cur = 0, len = 1;
  path[0] = 0;
  for (;;) {
    int32_t nxt = -1;
    for (int32_t c = cur + 1; c < n; ++c) {  // parent[c] < c: children of cur come after it
      if (parent[c] == cur && node_tokens[c] == argmax[cur]) {
        nxt = c;
        break;
      }
    }
    if (nxt < 0) break;
    path[len++] = nxt;
    cur = nxt;
  }
  for (int32_t i = 1; i < len; ++i) new_tokens[i - 1] = node_tokens[path[i]];
  new_tokens[len - 1] = argmax[cur];
  *path_len = len;
}

// The n-gram windows of a draft tree's nodes for the memory block of tree verification
// (tree_ngram_codes / tree_route_tokens, drafting/tree.py:114-136 and :179-196), over a history of
// `hist` cached codes, in one launch: idx [n][hist + 1] names each window slot in cat(history,
// nodes); win[(b n + i)][j][r] is that slot's code (0 where the slot is not real: a history
// position before 0), seg and val its reality (the lookup's segment ids and valid tokens); the
// nodes' codes go into the cache at L .. L + n - 1 (disjoint from the history read) and the conv
// slots are rel + L.  L = L0 + *L_dev (L_dev may be null).  One grid-stride pass over the four parts.
__global__ __launch_bounds__(256) void k_tree_windows(const void* __restrict__ node_codes, int nc_dt,
                                                      uint8_t* __restrict__ cache, int64_t stride, int32_t R,
                                                      int64_t B, int32_t n, int32_t hist,
                                                      const int32_t* __restrict__ idx, int64_t L0,
                                                      const int32_t* __restrict__ L_dev,
                                                      const int32_t* __restrict__ rel, int32_t nrel,
                                                      uint8_t* __restrict__ win, int32_t* __restrict__ seg,
                                                      uint8_t* __restrict__ val, int32_t* __restrict__ slots) {
  const int64_t L = L0 + (L_dev ? static_cast<int64_t>(*L_dev) : 0);
  const int64_t H = hist + 1;
  const int64_t e_win = B * n * H * R, e_seg = B * n * H, e_cache = B * n * R, e_slot = static_cast<int64_t>(n) * nrel;
  auto code = [&](int64_t i) -> uint8_t {  // node code i of [B, n, R], cast as the cache's dtype
    switch (nc_dt) {
      case LNG_U8: return static_cast<const uint8_t*>(node_codes)[i];
      case LNG_I32: return static_cast<uint8_t>(static_cast<const int32_t*>(node_codes)[i]);
      default: return static_cast<uint8_t>(static_cast<const int64_t*>(node_codes)[i]);
    }
  };
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < e_win + e_seg + e_cache + e_slot;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    if (e < e_win) {
      const int64_t r = e % R, bij = e / R, j = bij % H, bi = bij / H, i = bi % n, b = bi / n;
      const int q = idx[i * H + j];
      uint8_t c = 0;
      if (q >= hist) {
        c = code((b * n + (q - hist)) * R + r);
      } else {
        const int64_t pos = L - hist + q;
        if (pos >= 0) c = cache[(b * stride + pos) * R + r];
      }
      win[e] = c;
    } else if (e < e_win + e_seg) {
      const int64_t k = e - e_win, j = k % H, i = (k / H) % n;
      const int q = idx[i * H + j];
      const bool real = q >= hist || L - hist + q >= 0;
      seg[k] = real ? 1 : 0;
      val[k] = real ? 1 : 0;
    } else if (e < e_win + e_seg + e_cache) {
      const int64_t k = e - e_win - e_seg, r = k % R, bi = k / R, i = bi % n, b = bi / n;
      cache[(b * stride + L + i) * R + r] = code(k);
    } else {
      const int64_t k = e - e_win - e_seg - e_cache;
      slots[k] = static_cast<int32_t>(rel[k] + L);
    }
  }
}

}  // namespace lng

using namespace lng;

extern "C" {

int lng_tree_windows(const void* node_codes, int node_codes_dtype, uint8_t* cache, int64_t B, int64_t max_len,
                     int32_t R, int32_t n, int32_t hist, const int32_t* idx, int64_t L0, const int32_t* L_dev,
                     const int32_t* rel, int32_t n_rel, uint8_t* win, int32_t* seg, uint8_t* val, int32_t* slots,
                     void* stream) {
  if (B <= 0 || max_len <= 0 || R <= 0 || n <= 0 || hist < 0 || n_rel < 0 || L0 < 0)
    return fail(LNG_E_ARG, "tree_windows: bad shape");
  if (node_codes_dtype != LNG_U8 && node_codes_dtype != LNG_I32 && node_codes_dtype != LNG_I64)
    return fail(LNG_E_DTYPE, "tree_windows: node codes u8, i32 or i64");
  if (!node_codes || !cache || !idx || !win || !seg || !val || (n_rel && (!rel || !slots)))
    return fail(LNG_E_ARG, "tree_windows: null buffer");
  if (!L_dev && L0 + n > max_len) return fail(LNG_E_ARG, "tree_windows: cache full");
  const int64_t total = B * n * (hist + 1) * (R + 1) + B * n * R + static_cast<int64_t>(n) * n_rel;
  const unsigned grid = static_cast<unsigned>(cdiv(total, 256) < 1024 ? cdiv(total, 256) : 1024);
  hipLaunchKernelGGL(k_tree_windows, dim3(grid), dim3(256), 0, as_stream(stream), node_codes, node_codes_dtype,
                     cache, max_len, R, B, n, hist, idx, L0, L_dev, rel, n_rel, win, seg, val, slots);
  return check_launch("tree_windows");
}

int lng_abi_version(void) { return 2; }

const char* lng_last_error(void) { return g_last_error.c_str(); }

int lng_pack_route_codes(const float* logits, int64_t M, int64_t C, int32_t bits, void* codes, int codes_dtype,
                         void* stream) {
  if (M < 0 || C <= 0 || bits <= 0 || bits > 8 || C % bits) return fail(LNG_E_ARG, "pack_route_codes: bad shape");
  if (codes_dtype != LNG_U8 && codes_dtype != LNG_I32) return fail(LNG_E_DTYPE, "pack_route_codes: codes u8/i32");
  const int64_t n = M * (C / bits);
  if (n == 0) return LNG_OK;
  hipLaunchKernelGGL(k_pack_codes, dim3(cdiv(n, 256)), dim3(256), 0, as_stream(stream), logits, M, C / bits, bits,
                     codes, codes_dtype);
  return check_launch("pack_route_codes");
}

int lng_ngram_address(const void* codes, int codes_dtype, int64_t B, int64_t T, int32_t R, int32_t order,
                      int32_t bits, void* out, int out_dtype, void* stream) {
  if (!code_dtype_ok(codes_dtype)) return fail(LNG_E_DTYPE, "ngram_address: codes dtype");
  if (out_dtype != LNG_I32 && out_dtype != LNG_I64) return fail(LNG_E_DTYPE, "ngram_address: out i32/i64");
  if (B < 0 || T < 0 || R <= 0 || order <= 0 || bits <= 0 || bits * order > 62)
    return fail(LNG_E_ARG, "ngram_address: bad shape");
  const int64_t tv = T - order + 1;
  if (tv <= 0 || B == 0) return LNG_OK;
  const int64_t n = B * tv * R;
  hipLaunchKernelGGL(k_ngram_address, dim3(cdiv(n, 256)), dim3(256), 0, as_stream(stream),
                     CodeView{codes, codes_dtype}, B, T, R, order, bits, out, out_dtype);
  return check_launch("ngram_address");
}

static int make_orders(const int32_t* orders, int32_t n_orders, int32_t bits, OrderList* ol) {
  if (n_orders <= 0 || n_orders > 4) return fail(LNG_E_ARG, "n_orders must be in [1, 4]");
  ol->n = n_orders;
  for (int i = 0; i < n_orders; ++i) {
    if (orders[i] <= 0 || orders[i] * bits > 30) return fail(LNG_E_ARG, "n-gram order out of range");
    ol->v[i] = orders[i];
  }
  return LNG_OK;
}

int lng_ngram_rows(const void* codes, int codes_dtype, int64_t B, int64_t T, int32_t R, int32_t route_start,
                   int32_t route_end, const int32_t* orders, int32_t n_orders, int32_t bits,
                   const int32_t* segment_ids, const uint8_t* valid_tokens, void* rows, int rows_dtype,
                   void* stream) {
  if (!code_dtype_ok(codes_dtype)) return fail(LNG_E_DTYPE, "ngram_rows: codes dtype");
  if (rows_dtype != LNG_I32 && rows_dtype != LNG_I64) return fail(LNG_E_DTYPE, "ngram_rows: rows i32/i64");
  if (B < 0 || T < 0 || R <= 0 || route_start < 0 || route_end > R || route_start > route_end || bits <= 0)
    return fail(LNG_E_ARG, "ngram_rows: bad shape");
  OrderList ol;
  if (int rc = make_orders(orders, n_orders, bits, &ol)) return rc;
  // the largest row is R * 2^(bits * n) - 1 (lngram_v2.py:951-959 switches to int64 past int32)
  if (rows_dtype == LNG_I32)
    for (int i = 0; i < n_orders; ++i)
      if ((static_cast<int64_t>(R) << (bits * orders[i])) - 1 > INT32_MAX)
        return fail(LNG_E_RANGE, "ngram_rows: rows exceed int32 at this route count and order; ask for int64 rows");
  const int64_t n = B * T * (route_end - route_start) * n_orders;
  if (n == 0) return LNG_OK;
  if (rows_dtype == LNG_I32)
    hipLaunchKernelGGL(k_ngram_rows<int32_t>, dim3(cdiv(n, 256)), dim3(256), 0, as_stream(stream),
                       CodeView{codes, codes_dtype}, B, T, R, route_start, route_end, ol, bits, segment_ids,
                       valid_tokens, static_cast<int32_t*>(rows));
  else
    hipLaunchKernelGGL(k_ngram_rows<int64_t>, dim3(cdiv(n, 256)), dim3(256), 0, as_stream(stream),
                       CodeView{codes, codes_dtype}, B, T, R, route_start, route_end, ol, bits, segment_ids,
                       valid_tokens, static_cast<int64_t*>(rows));
  return check_launch("ngram_rows");
}

int lng_route_tokens(const void* codes, int codes_dtype, int64_t B, int64_t T, int32_t R, int32_t route_start,
                     int32_t route_end, const int32_t* orders, int32_t n_orders, int32_t bits,
                     const void* const* tables, int table_dtype, int32_t mem_dim, const int32_t* segment_ids,
                     const uint8_t* valid_tokens, int32_t target_length, void* out, void* stream) {
  if (!code_dtype_ok(codes_dtype)) return fail(LNG_E_DTYPE, "route_tokens: codes dtype");
  const int es = dtype_size(table_dtype);
  if (table_dtype != LNG_F32 && table_dtype != LNG_BF16 && table_dtype != LNG_F16)
    return fail(LNG_E_DTYPE, "route_tokens: tables f32/bf16/f16");
  if (B < 0 || T < 0 || R <= 0 || route_start < 0 || route_end > R || route_start > route_end || mem_dim <= 0)
    return fail(LNG_E_ARG, "route_tokens: bad shape");
  if (target_length < 0 || target_length > T) return fail(LNG_E_ARG, "route_tokens: target_length out of range");
  OrderList ol;
  if (int rc = make_orders(orders, n_orders, bits, &ol)) return rc;
  const int64_t t_out = target_length > 0 ? target_length : T;
  const int32_t rw = route_end - route_start;
  const int32_t seg_bytes = mem_dim * es;
  const int64_t segs = B * t_out * rw * n_orders;
  if (segs == 0) return LNG_OK;
  const void* tp[4] = {tables[0], n_orders > 1 ? tables[1] : nullptr, n_orders > 2 ? tables[2] : nullptr,
                       n_orders > 3 ? tables[3] : nullptr};
  CodeView cv{codes, codes_dtype};
  hipStream_t s = as_stream(stream);
  if (seg_bytes % 16 == 0) {
    const int64_t n = segs * (seg_bytes / 16);
    hipLaunchKernelGGL(k_route_tokens<u32x4>, dim3(cdiv(n, 256)), dim3(256), 0, s, cv, B, T, T - t_out, t_out, R,
                       route_start, rw, ol, bits, tp[0], tp[1], tp[2], tp[3], seg_bytes, segment_ids, valid_tokens,
                       static_cast<u32x4*>(out));
  } else if (seg_bytes % 4 == 0) {
    const int64_t n = segs * (seg_bytes / 4);
    hipLaunchKernelGGL(k_route_tokens<uint32_t>, dim3(cdiv(n, 256)), dim3(256), 0, s, cv, B, T, T - t_out, t_out, R,
                       route_start, rw, ol, bits, tp[0], tp[1], tp[2], tp[3], seg_bytes, segment_ids, valid_tokens,
                       static_cast<uint32_t*>(out));
  } else {
    const int64_t n = segs * (seg_bytes / 2);
    hipLaunchKernelGGL(k_route_tokens<uint16_t>, dim3(cdiv(n, 256)), dim3(256), 0, s, cv, B, T, T - t_out, t_out, R,
                       route_start, rw, ol, bits, tp[0], tp[1], tp[2], tp[3], seg_bytes, segment_ids, valid_tokens,
                       static_cast<uint16_t*>(out));
  }
  return check_launch("route_tokens");
}

int lng_tree_accept(const int32_t* parent, const int64_t* node_tokens, const int64_t* argmax, int32_t n,
                    int32_t* path, int32_t* path_len, int64_t* new_tokens, void* stream) {
  if (n <= 0) return fail(LNG_E_ARG, "tree_accept: need at least the root");
  hipLaunchKernelGGL(k_tree_accept, dim3(1), dim3(64), 0, as_stream(stream), parent, node_tokens, argmax, n, path,
                     path_len, new_tokens);
  return check_launch("tree_accept");
}

}  // extern "C"
