// Serving layout of the n-gram tables and the row movers of host-RAM serving
// (serving/layout.py:26-116, serving/prefetch.py).
//
// Serving layout: inside each route's block of A^n rows (A = 2^bits) the row of address
// sum_m c[t-m] A^m (the CURRENT code least significant) holds the v2 row of the reversed digits,
// so the A rows that step t+1 may read form one contiguous block.  The permutation reverses the n
// base-A digits of the in-block index: an involution, so the same kernel maps either way.
//
// Every mover reads its table through a plain pointer: device memory, or pinned host memory
// mapped into the device's address space (lng_host_device_pointer), in which case the loads
// cross the host link and nothing else changes (the zero-copy transfer of the reference's
// ZeroCopyGather).  A row is D elements of 2 or 4 bytes, D * elem a multiple of 16 bytes: one
// 16-lane group moves one row, 16 bytes per lane per step.
#include "common.h"

namespace lng {

constexpr int SV_MAXO = 4;

struct SvOrders {
  int32_t n;
  int32_t order[SV_MAXO];
  const char* table[SV_MAXO];     // row 0 of the order's serving table (device-visible address)
};

// copy one row of `rb` bytes (a multiple of 16) with the 16 lanes of a group
__device__ __forceinline__ void copy_row(const char* src, char* dst, int rb, int l) {
  for (int o = l * 16; o < rb; o += 256)
    *reinterpret_cast<u32x4*>(dst + o) = *reinterpret_cast<const u32x4*>(src + o);
}
__device__ __forceinline__ void zero_row(char* dst, int rb, int l) {
  for (int o = l * 16; o < rb; o += 256) *reinterpret_cast<u32x4*>(dst + o) = u32x4{0u, 0u, 0u, 0u};
}

__device__ __forceinline__ int64_t sv_code(const void* p, int dt, int64_t i) {
  if (dt == LNG_U8) return static_cast<const uint8_t*>(p)[i];
  if (dt == LNG_I32) return static_cast<const int32_t*>(p)[i];
  return static_cast<const int64_t*>(p)[i];
}

// dst row (r, j) = src row (r, rev(j)), rev reversing the `order` base-2^bits digits of j
__global__ __launch_bounds__(256) void k_permute_table(const char* __restrict__ src, char* __restrict__ dst,
                                                       int64_t rows, int32_t order, int32_t bits, int rb) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 16 + (threadIdx.x >> 4);
  if (row >= rows) return;
  const int64_t block = int64_t(1) << (bits * order);
  const int64_t j = row & (block - 1);
  const int64_t amask = (int64_t(1) << bits) - 1;
  int64_t rj = 0;
  for (int m = 0; m < order; ++m) rj |= ((j >> (m * bits)) & amask) << ((order - 1 - m) * bits);
  copy_row(src + (row - j + rj) * rb, dst + row * rb, rb, threadIdx.x & 15);
}

// out[b, t', r] = sum_m codes[b, t'+order-1-m, r] << (m*bits): the current code least significant
__global__ void k_serving_address(const void* codes, int cdt, int64_t B, int64_t T, int32_t R, int32_t order,
                                  int32_t bits, int64_t* __restrict__ out) {
  const int64_t tv = T - order + 1;
  const int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (i >= B * tv * R) return;
  const int32_t r = static_cast<int32_t>(i % R);
  const int64_t t = (i / R) % tv, b = i / (R * tv);
  int64_t a = 0;
  for (int m = 0; m < order; ++m) a |= sv_code(codes, cdt, (b * T + t + order - 1 - m) * R + r) << (m * bits);
  out[i] = a;
}

// Exact rows of n new positions: ctx [B, h + n, R] holds h history codes, then the new ones, the
// first new position being absolute position `start`.  out [B, n, R, n_orders * D]: the row of
// order o at position p = start + j (zeros when p < o - 1, as the v2 lookup reads there).
__global__ __launch_bounds__(256) void k_serving_gather(SvOrders ord, const void* ctx, int cdt, int64_t B, int64_t h,
                                                        int64_t n, int32_t R, int64_t start, int32_t bits, int rb,
                                                        char* __restrict__ out) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * 16 + (threadIdx.x >> 4);
  const int64_t total = B * n * R * ord.n;
  if (g >= total) return;
  const int l = threadIdx.x & 15;
  const int k = static_cast<int>(g % ord.n);
  const int64_t brj = g / ord.n;                 // (b, j, r)
  const int32_t r = static_cast<int32_t>(brj % R);
  const int64_t bj = brj / R;
  const int64_t j = bj % n, b = bj / n;
  const int o = ord.order[k];
  char* dst = out + g * rb;                      // [B, n, R, n_orders, D] = [B, n, R, n_orders * D]
  const int64_t i = h + j;                       // index of position start + j in ctx
  if (start + j < o - 1 || i - (o - 1) < 0) {
    zero_row(dst, rb, l);
    return;
  }
  const int64_t tc = h + n;
  const int64_t amask = (int64_t(1) << bits) - 1;
  int64_t a = 0;
  for (int m = 0; m < o; ++m) a |= (sv_code(ctx, cdt, (b * tc + i - m) * R + r) & amask) << (m * bits);
  const int64_t row = (static_cast<int64_t>(r) << (bits * o)) + a;
  copy_row(ord.table[k] + row * rb, dst, rb, l);
}

// Candidate blocks for position `position`: hist [B, h, R] are the codes ending at position - 1.
// out [M = B, R, n_orders, A, D]: rows base .. base + A - 1 of order o, base = r A^o +
// A * sum_{m=1}^{o-1} c[position - m] A^(m-1); zeros when the n-gram does not fit (position < o - 1).
__global__ __launch_bounds__(256) void k_serving_candidates(SvOrders ord, const void* hist, int cdt, int64_t B,
                                                            int64_t h, int32_t R, int64_t position, int32_t bits,
                                                            int rb, char* __restrict__ out) {
  const int A = 1 << bits;
  const int64_t g = static_cast<int64_t>(blockIdx.x) * 16 + (threadIdx.x >> 4);
  const int64_t total = B * R * ord.n * A;
  if (g >= total) return;
  const int l = threadIdx.x & 15;
  const int c = static_cast<int>(g % A);
  const int64_t brk = g / A;
  const int k = static_cast<int>(brk % ord.n);
  const int64_t br = brk / ord.n;
  const int32_t r = static_cast<int32_t>(br % R);
  const int64_t b = br / R;
  const int o = ord.order[k];
  char* dst = out + g * rb;
  if (position < o - 1 || h < o - 1) {
    zero_row(dst, rb, l);
    return;
  }
  const int64_t amask = A - 1;
  int64_t a = c;
  for (int m = 1; m < o; ++m) a |= (sv_code(hist, cdt, (b * h + h - m) * R + r) & amask) << (m * bits);
  const int64_t row = (static_cast<int64_t>(r) << (bits * o)) + a;
  copy_row(ord.table[k] + row * rb, dst, rb, l);
}

// out[m, r, k*D ..] = cand[m, r, k, codes[m, r], :]
__global__ __launch_bounds__(256) void k_select_candidates(const char* __restrict__ cand, const void* codes, int cdt,
                                                           int64_t M, int32_t R, int32_t n_orders, int32_t bits,
                                                           int rb, char* __restrict__ out) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * 16 + (threadIdx.x >> 4);
  if (g >= M * R * n_orders) return;
  const int A = 1 << bits;
  const int64_t mr = g / n_orders;
  const int64_t c = sv_code(codes, cdt, mr) & (A - 1);
  copy_row(cand + (g * A + c) * rb, out + g * rb, rb, threadIdx.x & 15);
}

// out[i] = table[idx[i]] (an index outside the table reads as a zero row)
__global__ __launch_bounds__(256) void k_gather_rows(const char* __restrict__ table, int64_t table_rows,
                                                     const int64_t* __restrict__ idx, int64_t N, int rb,
                                                     char* __restrict__ out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 16 + (threadIdx.x >> 4);
  if (i >= N) return;
  const int64_t row = idx[i];
  if (row < 0 || row >= table_rows)
    zero_row(out + i * rb, rb, threadIdx.x & 15);
  else
    copy_row(table + row * rb, out + i * rb, rb, threadIdx.x & 15);
}

static int orders_arg(const int32_t* orders, int32_t n_orders, const void* const* tables, int32_t bits, int32_t R,
                      const int64_t* table_rows, SvOrders& o) {
  if (n_orders < 1 || n_orders > SV_MAXO) return fail(LNG_E_ARG, "serving: 1..4 orders");
  o.n = n_orders;
  for (int k = 0; k < n_orders; ++k) {
    if (orders[k] < 1 || orders[k] * bits > 40) return fail(LNG_E_ARG, "serving: bad order");
    if (!tables[k] || !table_rows) return fail(LNG_E_ARG, "serving: null table or row counts");
    if (table_rows[k] < (static_cast<int64_t>(R) << (bits * orders[k])))
      return fail(LNG_E_ARG, "serving: a table has fewer rows than R * 2^(bits*order)");
    o.order[k] = orders[k];
    o.table[k] = static_cast<const char*>(tables[k]);
  }
  return LNG_OK;
}

static int row_bytes(int dtype, int32_t D, int& rb) {
  const int es = dtype_size(dtype);
  if (es != 2 && es != 4) return fail(LNG_E_DTYPE, "serving: table dtype f32, bf16 or f16");
  rb = es * D;
  if (D <= 0 || rb % 16) return fail(LNG_E_ARG, "serving: a row must be a multiple of 16 bytes");
  return LNG_OK;
}

static bool codes_dt_ok(int dt) { return dt == LNG_U8 || dt == LNG_I32 || dt == LNG_I64; }

}  // namespace lng

using namespace lng;

extern "C" int lng_host_device_pointer(const void* host_ptr, void** dev_ptr) {
  if (!host_ptr || !dev_ptr) return fail(LNG_E_ARG, "host_device_pointer: null pointer");
  void* d = nullptr;
  const hipError_t e = hipHostGetDevicePointer(&d, const_cast<void*>(host_ptr), 0);
  if (e != hipSuccess || d == nullptr) {
    (void)hipGetLastError();
    return fail(LNG_E_HIP, std::string("host_device_pointer: not pinned, mapped host memory (") +
                               hipGetErrorString(e) + ")");
  }
  *dev_ptr = d;
  return LNG_OK;
}

extern "C" int lng_permute_table(const void* src, void* dst, int dtype, int32_t routes, int32_t order, int32_t bits,
                                 int32_t mem_dim, void* stream) {
  int rb = 0;
  if (int rc = row_bytes(dtype, mem_dim, rb)) return rc;
  if (!src || !dst || src == dst) return fail(LNG_E_ARG, "permute_table: distinct, non-null buffers");
  if (routes <= 0 || order < 1 || bits < 1 || bits * order > 40) return fail(LNG_E_ARG, "permute_table: bad shape");
  const int64_t rows = static_cast<int64_t>(routes) << (bits * order);
  k_permute_table<<<cdiv(rows, 16), 256, 0, as_stream(stream)>>>(static_cast<const char*>(src),
                                                                 static_cast<char*>(dst), rows, order, bits, rb);
  return check_launch("k_permute_table");
}

extern "C" int lng_serving_address(const void* codes, int codes_dtype, int64_t B, int64_t T, int32_t R, int32_t order,
                                   int32_t bits, int64_t* out, void* stream) {
  if (!codes_dt_ok(codes_dtype)) return fail(LNG_E_DTYPE, "serving_address: codes u8, i32 or i64");
  if (B < 0 || T < 0 || R <= 0 || order < 1 || bits < 1 || bits * order > 62)
    return fail(LNG_E_ARG, "serving_address: bad shape");
  const int64_t n = B * std::max<int64_t>(0, T - order + 1) * R;
  if (n == 0) return LNG_OK;
  k_serving_address<<<cdiv(n, 256), 256, 0, as_stream(stream)>>>(codes, codes_dtype, B, T, R, order, bits, out);
  return check_launch("k_serving_address");
}

extern "C" int lng_serving_gather(const void* const* tables, const int64_t* table_rows, int table_dtype,
                                  int32_t mem_dim, const int32_t* orders, int32_t n_orders, int32_t bits,
                                  const void* ctx, int codes_dtype, int64_t B, int64_t h, int64_t n, int32_t R,
                                  int64_t start, void* out, void* stream) {
  SvOrders o{};
  int rb = 0;
  if (int rc = row_bytes(table_dtype, mem_dim, rb)) return rc;
  if (int rc = orders_arg(orders, n_orders, tables, bits, R, table_rows, o)) return rc;
  if (!codes_dt_ok(codes_dtype)) return fail(LNG_E_DTYPE, "serving_gather: codes u8, i32 or i64");
  if (B < 0 || h < 0 || n < 0 || R <= 0 || start < 0 || h > start) return fail(LNG_E_ARG, "serving_gather: bad shape");
  const int64_t groups = B * n * R * n_orders;
  if (groups == 0) return LNG_OK;
  k_serving_gather<<<cdiv(groups, 16), 256, 0, as_stream(stream)>>>(o, ctx, codes_dtype, B, h, n, R, start, bits, rb,
                                                                    static_cast<char*>(out));
  return check_launch("k_serving_gather");
}

extern "C" int lng_serving_candidates(const void* const* tables, const int64_t* table_rows, int table_dtype,
                                      int32_t mem_dim, const int32_t* orders, int32_t n_orders, int32_t bits,
                                      const void* hist, int codes_dtype, int64_t B, int64_t h, int32_t R,
                                      int64_t position, void* out, void* stream) {
  SvOrders o{};
  int rb = 0;
  if (int rc = row_bytes(table_dtype, mem_dim, rb)) return rc;
  if (int rc = orders_arg(orders, n_orders, tables, bits, R, table_rows, o)) return rc;
  if (!codes_dt_ok(codes_dtype)) return fail(LNG_E_DTYPE, "serving_candidates: codes u8, i32 or i64");
  if (B < 0 || h < 0 || R <= 0 || position < 0 || h > position || bits > 8)
    return fail(LNG_E_ARG, "serving_candidates: bad shape");
  const int64_t groups = B * R * n_orders * (int64_t(1) << bits);
  if (groups == 0) return LNG_OK;
  k_serving_candidates<<<cdiv(groups, 16), 256, 0, as_stream(stream)>>>(o, hist, codes_dtype, B, h, R, position, bits,
                                                                        rb, static_cast<char*>(out));
  return check_launch("k_serving_candidates");
}

extern "C" int lng_select_candidates(const void* cand, int dtype, int32_t mem_dim, const void* codes, int codes_dtype,
                                     int64_t M, int32_t R, int32_t n_orders, int32_t bits, void* out, void* stream) {
  int rb = 0;
  if (int rc = row_bytes(dtype, mem_dim, rb)) return rc;
  if (!codes_dt_ok(codes_dtype)) return fail(LNG_E_DTYPE, "select_candidates: codes u8, i32 or i64");
  if (M < 0 || R <= 0 || n_orders < 1 || n_orders > SV_MAXO || bits < 1 || bits > 8)
    return fail(LNG_E_ARG, "select_candidates: bad shape");
  const int64_t groups = M * R * n_orders;
  if (groups == 0) return LNG_OK;
  k_select_candidates<<<cdiv(groups, 16), 256, 0, as_stream(stream)>>>(static_cast<const char*>(cand), codes,
                                                                       codes_dtype, M, R, n_orders, bits, rb,
                                                                       static_cast<char*>(out));
  return check_launch("k_select_candidates");
}

extern "C" int lng_gather_rows(const void* table, int64_t table_rows, int dtype, int32_t mem_dim, const int64_t* idx,
                               int64_t N, void* out, void* stream) {
  int rb = 0;
  if (int rc = row_bytes(dtype, mem_dim, rb)) return rc;
  if (!table || (N > 0 && (!idx || !out)) || N < 0 || table_rows < 0) return fail(LNG_E_ARG, "gather_rows: bad arguments");
  if (N == 0) return LNG_OK;
  k_gather_rows<<<cdiv(N, 16), 256, 0, as_stream(stream)>>>(static_cast<const char*>(table), table_rows, idx, N, rb,
                                                            static_cast<char*>(out));
  return check_launch("k_gather_rows");
}
