// Draft tree of a token-only drafter in one launch (drafting/tree.py:243-257 draft_tree over the
// readout of drafting/cpu_drafter.py:208-270 and the online counts of drafters.py:117-142; the
// verification gather of tree.py:96-136).
//
// The grid is one resident block per CU; each block keeps one role for the whole tree:
//   A blocks (16): head qh of parent slot p of every depth (block a: p = a % 4, qh = a / 4).  At
//       depth l the node is the rank-th pick of its own parent's top-K, which the block selects
//       itself from depth l-1's vocabulary records; its codes come from the router tables; the
//       window's n-gram rows are gathered into LDS, and the sink attention of head qh over the routes
//       gives o_qh = w * Wv (mem_norm . U) (w the softmax weight of the routes against the sink) and
//       Y_qh = Gram[:, qh] o_qh.  Head 0 also publishes the window codes (the online counts' query),
//       stores the node's token and codes, and writes its verification route tokens.  The value
//       weight and Gram rows of the block's head are loaded once.
//   V blocks (one per slice of TL_VS vocabulary rows): the slice's lut_out rows stay in registers for
//       the whole tree, and the committed pairs whose next token lies in the slice are listed once.
//       Per depth: once the window codes arrive, each listed pair's matches are added to the slice's
//       counts; once the A records arrive, r = rsqrt(o . sum_qh Y_qh / d + eps), the slice's logits
//       r lut_out o for every parent, and one record per (parent, slice): max, sum of exponentials,
//       online total, top-KM of the tokens without counts, and the count-bearing tokens; then the
//       slice's ready word.
//   G blocks (the rest): leaves of each depth: selection, codes, verification gather.
// Every hand-off goes through the device-coherent level (sc1 loads and stores, past the XCD-private
// L2s) into buffers of its own depth.  A -> V: self-validating (value, tag) pairs written and read
// with single 64-bit accesses (the tag holds the call's epoch and the depth), so a reader needs no
// flag and a writer no completion wait.  V -> next depth: the records, then (after the block's
// stores are complete) a ready word holding the tag.  Waits are bounded (TL_SPIN_TICKS of the 100 MHz
// constant clock; a timeout sets the error word and the grid drains); the host launches the grid
// only when every block can be resident at once.  The last block to finish advances the epoch.
#include <algorithm>
#include <atomic>
#include <climits>
#include <vector>

#include "common.h"

namespace lng {
namespace {

constexpr int TL_THREADS = 512, TL_WAVES = TL_THREADS / 64;
constexpr int TL_QH = 4, TL_DT = 256, TL_HD = 64, TL_I = TL_QH * TL_HD;  // heads, route-token features, head dim
constexpr int TL_MD = TL_DT / 2;  // mem_dim (two orders: 2 and 3)
constexpr int TL_MAXR = 192;      // routes
constexpr int TL_CR = TL_MAXR + 1;  // pairs of a window record: the codes of each route, then the token
constexpr int TL_MAXP = 4;        // parents per depth
constexpr int TL_NA = TL_MAXP * TL_QH;  // A blocks
constexpr int TL_MAXN = 32;       // tree nodes
constexpr int TL_MAXL = 8;        // depths with parents
constexpr int TL_NLB = TL_MAXL + 1;  // depth buffers
constexpr int TL_VS = 160;        // vocabulary rows per V block (64-row MFMA groups: 64, 64, 32)
constexpr int TL_VG = 3;          // 64-row groups of a V block
constexpr int TL_VK = TL_I / TL_WAVES;  // features per wave in the vocabulary product
constexpr int TL_MAXVB = 224;     // V blocks: V <= 224 * 160
constexpr int TL_MINGB = 8;       // G blocks at least
constexpr int TL_MAXGRID = 256;
constexpr int TL_KM = 4;          // top-k kept per record (K <= 4)
constexpr int TL_NI = 16;         // count-bearing tokens inline in a record
constexpr int TL_RW = 64;         // words per record
constexpr int TL_AP = TL_DT + TL_HD;  // pairs per A record: Y[256], then o[64]
constexpr int TL_PL = 4096;       // listed pairs of a V block (more: re-listed per depth in rounds)
constexpr int TL_KL = 48;         // listed pairs whose match keys a V block keeps in LDS
constexpr long long TL_SPIN_TICKS = 2000000;  // 20 ms
constexpr int TL_NST = 16;        // phase stamps per block and depth

struct TlPlan {
  int32_t n, node_row0, K, online, nlev, nvb, ngb;
  float kappa;
  int8_t parent[TL_MAXN], rank[TL_MAXN], pslot[TL_MAXN];
  int8_t lev_np[TL_NLB];
  int8_t lev_par[TL_NLB][TL_MAXP];
  int8_t lev_nleaf[TL_NLB];
  int8_t lev_leaf[TL_NLB][TL_MAXN];
};

struct TlWork {
  uint32_t* hdr;      // [0] epoch, [1] error word, [2] stamps on, [3] blocks finished
  uint64_t* crec;     // [TL_NLB][TL_MAXP][TL_CR] (value, tag): each parent's window codes and token
  uint64_t* arec;     // [TL_NLB][TL_MAXP][TL_QH][TL_AP] (value, tag)
  uint32_t* vrec;     // [TL_NLB][TL_MAXP][TL_MAXVB][TL_RW] vocabulary records
  uint32_t* rdy;      // [TL_NLB][TL_MAXVB] ready words of the records
  uint32_t* spill;    // [TL_NLB][TL_MAXP][TL_MAXVB][TL_VS][3] count-bearing tokens past the inline ones
  long long* stamps;  // [TL_NLB][TL_MAXGRID][TL_NST] phase times (100 MHz clock) when hdr[2] != 0
  void* route_tokens; // [n, R, Dt] bf16 or null
};

struct TlLayout {
  size_t hdr, crec, arec, vrec, rdy, spill, stamps, total;
};

constexpr size_t tl_al(size_t x) { return (x + 255) & ~size_t{255}; }

TlLayout tl_layout() {
  TlLayout l{};
  size_t o = 0;
  l.hdr = o, o += 256;
  l.crec = o, o += tl_al(sizeof(uint64_t) * TL_NLB * TL_MAXP * TL_CR);
  l.arec = o, o += tl_al(sizeof(uint64_t) * TL_NLB * TL_MAXP * TL_QH * TL_AP);
  l.vrec = o, o += tl_al(sizeof(uint32_t) * TL_NLB * TL_MAXP * TL_MAXVB * TL_RW);
  l.rdy = o, o += tl_al(sizeof(uint32_t) * TL_NLB * TL_MAXVB);
  l.spill = o, o += tl_al(sizeof(uint32_t) * TL_NLB * TL_MAXP * TL_MAXVB * TL_VS * 3);
  l.stamps = o, o += tl_al(sizeof(long long) * TL_NLB * TL_MAXGRID * TL_NST);
  l.total = o;
  return l;
}

// ------------------------------------------------------------------ small helpers
__device__ __forceinline__ uint32_t tl_tag(uint32_t epoch, int lev) { return ((epoch + 1u) << 4) | static_cast<uint32_t>(lev); }

__device__ __forceinline__ void tl_st_pair(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t v, uint32_t tag) {
  const uint64_t w = (static_cast<uint64_t>(tag) << 32) | v;
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(__attribute__((ext_vector_type(2))) unsigned int, w), r, off,
                                        0, CPOL_SC1);
}
__device__ __forceinline__ uint64_t tl_ld_pair(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, CPOL_SC1));
}
__device__ __forceinline__ void tl_st_w(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t v) {
  __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, CPOL_SC1);
}
__device__ __forceinline__ uint32_t tl_ld_w(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, CPOL_SC1);
}

__device__ __forceinline__ float tl_row16_sum(float v) {
  v += dpp_row_shr<0x111>(v, 0.f);
  v += dpp_row_shr<0x112>(v, 0.f);
  v += dpp_row_shr<0x114>(v, 0.f);
  v += dpp_row_shr<0x118>(v, 0.f);
  return v;  // valid in lanes 15, 31, 47, 63
}

__device__ __forceinline__ int tl_wave_min_i(int v) {
  v = min(v, __builtin_amdgcn_update_dpp(INT_MAX, v, 0x111, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(INT_MAX, v, 0x112, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(INT_MAX, v, 0x114, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(INT_MAX, v, 0x118, 0xf, 0xf, false));
  return min(min(__builtin_amdgcn_readlane(v, 15), __builtin_amdgcn_readlane(v, 31)),
             min(__builtin_amdgcn_readlane(v, 47), __builtin_amdgcn_readlane(v, 63)));
}

__device__ __forceinline__ int tl_wave_sum_i(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);
  return (__builtin_amdgcn_readlane(v, 15) + __builtin_amdgcn_readlane(v, 31)) +
         (__builtin_amdgcn_readlane(v, 47) + __builtin_amdgcn_readlane(v, 63));
}

// Ranking key of a candidate (value desc, then id asc): the value's bits in an order-preserving
// unsigned form (-0 taken as +0, so equal values compare equal) above 2^31 - 1 - id.  A larger key
// ranks first; 0 is below every candidate's key.
__device__ __forceinline__ uint64_t tl_key(float v, int id) {
  uint32_t b = __float_as_uint(v + 0.0f);
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return (static_cast<uint64_t>(b) << 32) | static_cast<uint32_t>(0x7FFFFFFF - id);
}
__device__ __forceinline__ int tl_key_id(uint64_t k) { return 0x7FFFFFFF - static_cast<int>(static_cast<uint32_t>(k)); }
__device__ __forceinline__ float tl_key_value(uint64_t k) {
  uint32_t b = static_cast<uint32_t>(k >> 32);
  b = (b & 0x80000000u) ? (b & 0x7FFFFFFFu) : ~b;
  return __uint_as_float(b);
}

// The wave's largest 64-bit key (row maxima by DPP row_shr, then the four rows), in every lane.
template <int CTRL>
__device__ __forceinline__ uint64_t tl_dpp_u64(uint64_t k) {
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(k >> 32), CTRL, 0xf, 0xf, false));
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(k)), CTRL, 0xf, 0xf, false));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}
__device__ __forceinline__ uint64_t tl_wave_max_u64(uint64_t k) {
  uint64_t o;
  o = tl_dpp_u64<0x111>(k), k = o > k ? o : k;
  o = tl_dpp_u64<0x112>(k), k = o > k ? o : k;
  o = tl_dpp_u64<0x114>(k), k = o > k ? o : k;
  o = tl_dpp_u64<0x118>(k), k = o > k ? o : k;
  uint64_t m = 0;
#pragma unroll
  for (int r = 15; r < 64; r += 16) {
    const uint64_t x = (static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(k >> 32), r))) << 32) |
                       static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(k)), r));
    m = x > m ? x : m;
  }
  return m;
}

// Block-wide sum / max of one value per thread through red[TL_WAVES] (every thread receives it).
// Block barrier that orders the block's LDS accesses only: global stores still in flight are not
// waited for (a hand-off to other blocks is tagged, so no block reads its own global stores back)
__device__ __forceinline__ void tl_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ float tl_block_sum(float v, float* red) {
  v = wave_sum(v);
  tl_sync();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  tl_sync();
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < TL_WAVES; ++k) s += red[k];
  return s;
}
__device__ __forceinline__ float tl_block_max(float v, float* red) {
  v = wave_max(v);
  tl_sync();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  tl_sync();
  float m = red[0];
#pragma unroll
  for (int k = 1; k < TL_WAVES; ++k) m = fmaxf(m, red[k]);
  return m;
}

// Per-thread top-KM list by (value desc, id asc); empty slots (-inf, INT_MAX).
struct TlTop {
  float v[TL_KM];
  int i[TL_KM];
  __device__ __forceinline__ void clear() {
#pragma unroll
    for (int k = 0; k < TL_KM; ++k) v[k] = -INFINITY, i[k] = INT_MAX;
  }
  __device__ __forceinline__ void insert(float x, int id) {
#pragma unroll
    for (int k = 0; k < TL_KM; ++k) {
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
    for (int k = 0; k + 1 < TL_KM; ++k) v[k] = v[k + 1], i[k] = i[k + 1];
    v[TL_KM - 1] = -INFINITY, i[TL_KM - 1] = INT_MAX;
  }
};

__device__ __forceinline__ bool tl_tok_ok(const lng_drafter& D, int64_t tok) { return tok >= 0 && tok < D.V; }

// Code of route r for (previous token, token) from the router tables (bits 4: one 16-byte load per row).
__device__ __forceinline__ int tl_lut_code(const lng_drafter& D, int64_t ptok, int64_t tok, int r) {
  if (!tl_tok_ok(D, tok)) return 0;
  const int RB = D.R * 4;
  const float* a = tl_tok_ok(D, ptok) ? D.lut_prev + ptok * RB : D.lut_start;
  const float* b = D.lut_cur + tok * RB;
  const f32x4 x = *reinterpret_cast<const f32x4*>(a + 4 * r);
  const f32x4 y = *reinterpret_cast<const f32x4*>(b + 4 * r);
  return ((x[0] + y[0]) > 0.f ? 1 : 0) | ((x[1] + y[1]) > 0.f ? 2 : 0) | ((x[2] + y[2]) > 0.f ? 4 : 0) |
         ((x[3] + y[3]) > 0.f ? 8 : 0);
}

// Row of tree node a (the root is the last committed row).
__device__ __forceinline__ int32_t tl_nrow(const TlPlan& T, int a, int32_t L) { return a == 0 ? L - 1 : T.node_row0 + a; }

// Rows of the window of node i, oldest first (slot 2 = i itself); -1 before the sequence start.
__device__ __forceinline__ void tl_window(const TlPlan& T, int i, int32_t L, int32_t (&row)[3]) {
  int a = i;
  int32_t back = 0;  // committed rows stepped back past the root
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    if (a >= 0) {
      row[2 - k] = tl_nrow(T, a, L);
      a = a == 0 ? -1 : T.parent[a];
      if (a < 0) back = 1;
    } else {
      row[2 - k] = L - 1 - back;
      ++back;
    }
    if (row[2 - k] < 0) row[2 - k] = -1;
  }
}

// ------------------------------------------------------------------ selection
struct TlSelLds {
  float rv[TL_WAVES];
  float rs[TL_WAVES];
  int rt[TL_WAVES];
  uint64_t wk[TL_WAVES * TL_KM];  // each wave's top-KM ranking keys
  int sel[TL_KM];
};

// Bounded wait until every V block's ready word of depth `lev` holds `tag` (whole block; returns
// false after a timeout).
__device__ __forceinline__ bool tl_wait_ready(int nvb, const uint32_t* rdy, int lev, uint32_t tag) {
  const __amdgpu_buffer_rsrc_t rb = dev_buf(rdy + static_cast<size_t>(lev) * TL_MAXVB, TL_MAXVB * 4u);
  const int t = threadIdx.x;
  const long long t0 = wall_clock64();
  for (;;) {
    const bool ok = t >= nvb || tl_ld_w(rb, 4u * t) == tag;
    if (__syncthreads_and(ok ? 1 : 0)) return true;
    if (__syncthreads_or(wall_clock64() - t0 > TL_SPIN_TICKS ? 1 : 0)) return false;
    __builtin_amdgcn_s_sleep(1);
  }
}

// Top-K (K <= KM) of parent `slot` of depth `lev` from the V records, ranked as k_fast_logits'
// selection ranks them: logits, or the online mixture (1 - lam) softmax + lam count / total.  Whole
// block; ids land in S.sel (-1 past the candidates).  Two threads per V block's record: the even one
// takes the record's header, its top-KM of the tokens without counts and the even count-bearing
// entries, the odd one the odd entries; each wave ranks its candidates' keys, then the block ranks the
// waves' lists.
__device__ __forceinline__ void tl_select(const TlPlan& T, const uint32_t* vrec, const uint32_t* spill, float denom, int lev,
                          int slot, TlSelLds& S, long long* stp = nullptr) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int rec = t >> 1, h = t & 1;
  const bool ok = rec < T.nvb;
  const bool online = T.online != 0;
  // one descriptor for the slot's records (a buffer descriptor is taken from the first lane), the
  // record at a per-lane offset; the count-bearing entries only with online counts
  const size_t r0 = (static_cast<size_t>(lev) * TL_MAXP + slot) * TL_MAXVB;
  const __amdgpu_buffer_rsrc_t rb = dev_buf(vrec + r0 * TL_RW, TL_MAXVB * TL_RW * 4u);
  const __amdgpu_buffer_rsrc_t sb = dev_buf(spill + r0 * (TL_VS * 3), TL_MAXVB * TL_VS * 12u);
  const uint32_t roff = 4u * TL_RW * static_cast<uint32_t>(ok ? rec : 0);
  u32x4 q[TL_RW / 4];
#pragma unroll
  for (int k = 0; k < TL_RW / 4; ++k)
    q[k] = (ok && (k < 3 || online)) ? __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, roff + 16u * k, 0, CPOL_SC1))
                                     : u32x4{0u, 0u, 0u, 0u};
  auto word = [&](int k) { return q[k >> 2][k & 3]; };  // constant k: a register
  // max, sum of exponentials and online total over the records (even lanes), merged per wave and
  // then across the waves in a fixed order
  const bool head = ok && h == 0;
  const float m = head ? __uint_as_float(word(0)) : -INFINITY;
  const float mw = wave_max(m);
  const float sw = wave_sum(m == -INFINITY ? 0.f : __uint_as_float(word(1)) * expf(m - mw));
  const int totw = tl_wave_sum_i(head ? static_cast<int>(word(2)) : 0);
  if (lane == 0) S.rv[w] = mw, S.rs[w] = sw, S.rt[w] = totw;
  __syncthreads();
  if (stp && t == 0) stp[8] = wall_clock64();
  float M = S.rv[0];
  int totb = S.rt[0];
#pragma unroll
  for (int k = 1; k < TL_WAVES; ++k) M = fmaxf(M, S.rv[k]), totb += S.rt[k];
  float Ssum = 0.f;
#pragma unroll
  for (int k = 0; k < TL_WAVES; ++k) Ssum += S.rv[k] == -INFINITY ? 0.f : S.rs[k] * expf(S.rv[k] - M);
  const float tj = online ? static_cast<float>(totb) : 0.f;
  const float n_eff = tj / denom;
  const float lam = tj > 0.f ? n_eff / (n_eff + T.kappa) : 0.f;
  const float mix_a = (1.f - lam) / Ssum, mix_b = tj > 0.f ? lam / tj : 0.f;
  // the thread's candidates as ranking keys: slots 0-3 the record's top-KM (even thread), 4-11 its
  // inline count-bearing entries (this lane's parity, as far as the wave's largest share reaches),
  // 12-15 the best four of its spill entries; key 0: none
  uint64_t ck[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) ck[k] = 0;
  if (head)
#pragma unroll
    for (int k = 0; k < TL_KM; ++k) {
      const int id = static_cast<int>(word(4 + TL_KM + k));
      if (id >= 0)
        ck[k] = tl_key(online ? mix_a * expf(__uint_as_float(word(4 + k)) - M) : __uint_as_float(word(4 + k)), id);
    }
  const int nc = ok && online ? min(static_cast<int>(word(3)), TL_VS) : 0;
  const int mine = (min(nc, TL_NI) + 1 - h) >> 1;  // entries h, h + 2, ... below min(nc, NI)
  const int mw_n = online ? static_cast<int>(wave_max(static_cast<float>(mine))) : 0;
#pragma unroll
  for (int u = 0; u < TL_NI / 2; ++u) {
    if (u < mw_n && u < mine) {
      const uint32_t id = h ? word(15 + 6 * u) : word(12 + 6 * u);
      const uint32_t lb = h ? word(16 + 6 * u) : word(13 + 6 * u);
      const uint32_t c = h ? word(17 + 6 * u) : word(14 + 6 * u);
      ck[4 + u] = tl_key(fmaf(mix_b, static_cast<float>(static_cast<int>(c)), mix_a * expf(__uint_as_float(lb) - M)),
                         static_cast<int>(id));
    }
  }
  if (nc > TL_NI + h) {
    TlTop tk;
    tk.clear();
    const uint32_t soff = 12u * TL_VS * static_cast<uint32_t>(ok ? rec : 0);
    for (int e = TL_NI + h; e < nc; e += 2) {
      const int id = static_cast<int>(tl_ld_w(sb, soff + 12u * e));
      const float l = __uint_as_float(tl_ld_w(sb, soff + 12u * e + 4u));
      const int c = static_cast<int>(tl_ld_w(sb, soff + 12u * e + 8u));
      tk.insert(fmaf(mix_b, static_cast<float>(c), mix_a * expf(l - M)), id);
    }
#pragma unroll
    for (int k = 0; k < TL_KM; ++k)
      if (tk.i[k] != INT_MAX) ck[12 + k] = tl_key(tk.v[k], tk.i[k]);
  }
  if (stp && t == 0) stp[9] = wall_clock64();
  // each wave's top-K by K rounds of (the wave's largest key, taken out of its thread: ids are unique
  // among the candidates), then the block's top-K of the waves' lists by counting, for each listed
  // key, the keys above it
  uint64_t bk;
  int bs;
  auto best = [&]() {  // a 4-level tree of pairwise maxima (short dependency chain)
    uint64_t m[8];
    int ms[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const bool bt = ck[2 * q + 1] > ck[2 * q];
      m[q] = bt ? ck[2 * q + 1] : ck[2 * q];
      ms[q] = bt ? 2 * q + 1 : 2 * q;
    }
#pragma unroll
    for (int n = 4; n >= 1; n >>= 1)
#pragma unroll
      for (int q = 0; q < n; ++q) {
        const bool bt = m[q + n] > m[q];
        m[q] = bt ? m[q + n] : m[q];
        ms[q] = bt ? ms[q + n] : ms[q];
      }
    bk = m[0], bs = ms[0];
  };
  best();
  uint64_t wl = 0;  // lane k < KM: the wave's k-th key
#pragma unroll
  for (int k = 0; k < TL_KM; ++k) {
    if (k >= T.K) break;  // (K is block-uniform)
    const uint64_t wk = tl_wave_max_u64(bk);
    if (lane == k) wl = wk;
    if (wk != 0 && bk == wk) {
#pragma unroll
      for (int q = 0; q < 16; ++q) ck[q] = q == bs ? 0 : ck[q];
      best();
    }
  }
  if (lane < TL_KM) S.wk[w * TL_KM + lane] = wl;
  if (t < TL_KM) S.sel[t] = -1;
  tl_sync();
  if (t < TL_WAVES * TL_KM) {
    const uint64_t kj = S.wk[t];
    int above = 0;
#pragma unroll
    for (int q = 0; q < TL_WAVES * TL_KM; ++q) above += S.wk[q] > kj ? 1 : 0;
    if (kj != 0 && above < T.K) S.sel[above] = tl_key_id(kj);
  }
  tl_sync();
}

// ------------------------------------------------------------------ LDS of the three roles
struct TlALds {
  alignas(16) float gram[TL_HD][TL_I];  // Gram rows qh*64 .. qh*64 + 63 of the block's head
  alignas(16) uint16_t wv[TL_HD][TL_DT + 8];  // the head's value weight Wv[h] (bf16 bits, padded rows)
  float qk[TL_DT];
  float sc[TL_MAXR], sx[TL_MAXR], wr[TL_MAXR];
  float red[TL_THREADS / 16][TL_DT];  // U partials per route row; then Y partials per eighth of o
  float opart[TL_WAVES][TL_HD];  // o' partials per input run
  float un[TL_DT];
  float o[TL_HD];
  uint8_t wc[3][TL_MAXR];
  float stat[TL_WAVES];
  TlSelLds S;
  int64_t ptok;
  uint32_t vfl;
};
struct TlVLds {
  float ro[TL_MAXP][TL_DT];
  float lt[TL_MAXP][TL_VS];
  f32x4 lpart[TL_WAVES][TL_VG * 64];  // per wave: (row, 4 parents) partial logits over its features
  int32_t sc[TL_MAXP][TL_VS];
  uint32_t qry[TL_MAXP][TL_MAXR];
  uint16_t keys[TL_KL][TL_MAXR];  // match keys of the first listed pairs: 12-bit order-3 key, bit 12 order 2
                                  // usable (pair >= 1), bit 13 order 3 usable (pair >= 2)
  uint8_t knt[TL_KL];             // their next tokens, relative to the slice
  int32_t list[TL_PL];
  int32_t nmatch;
  int32_t tot[TL_MAXP][TL_WAVES];
  float part[TL_MAXP][TL_WAVES];
};
struct TlGLds {
  uint8_t wc[3][TL_MAXR];
  TlSelLds S;
  int64_t ptok;
  uint32_t vfl;
};
union TlLds {
  TlALds a;
  TlVLds v;
  TlGLds g;
};

// Window of the root into wc (slots 0..2, oldest first: the committed rows L-3, L-2, L-1) and its
// validity bits (bit 0: slot 2 inside the sequence, bit 1: slots 1-2, bit 2: slots 0-2).  Whole block.
__device__ __forceinline__ uint32_t tl_root_window(const lng_drafter& D, const TlPlan& T, int32_t L, uint8_t (*wc)[TL_MAXR]) {
  int32_t row[3];
  tl_window(T, 0, L, row);
  const int R = D.R;
  for (int e = threadIdx.x; e < 3 * R; e += TL_THREADS) {
    const int k = e / R, r = e % R;
    wc[k][r] = static_cast<uint8_t>(row[k] >= 0 ? D.codes[static_cast<int64_t>(row[k]) * R + r] & 15 : 0);
  }
  const uint32_t v1 = row[2] >= 0, v2 = v1 && row[1] >= 0, v3 = v2 && row[0] >= 0;
  return v1 | (v2 << 1) | (v3 << 2);
}

// Slots 0 and 1 of node i's window from its parent's published window (depth lev - 1: the parent's
// slots 1 and 2) into wc, the parent's token into *ptok and node i's validity bits into *vfl
// (LDS).  Whole block; false after a timeout.
__device__ __forceinline__ bool tl_parent_window(int R, const TlPlan& T, const uint64_t* crec, uint32_t epoch, int lev, int i,
                                 uint8_t (*wc)[TL_MAXR], int64_t* ptok, uint32_t* vfl) {
  const int pp = T.parent[i], ps = T.pslot[pp];
  const uint32_t tag = tl_tag(epoch, lev - 1);
  const __amdgpu_buffer_rsrc_t cb =
      dev_buf(crec + (static_cast<size_t>(lev - 1) * TL_MAXP + ps) * TL_CR, TL_CR * 8u);
  const int t = threadIdx.x;
  const bool mine = t < R || t == TL_THREADS - 1;
  const uint32_t off = 8u * (t < R ? t : TL_MAXR);
  const long long t0 = wall_clock64();
  uint64_t x = mine ? tl_ld_pair(cb, off) : 0;
  for (;;) {
    const bool ok = !mine || static_cast<uint32_t>(x >> 32) == tag;
    if (__syncthreads_and(ok ? 1 : 0)) break;
    if (__syncthreads_or(wall_clock64() - t0 > TL_SPIN_TICKS ? 1 : 0)) return false;
    __builtin_amdgcn_s_sleep(1);
    if (!ok) x = tl_ld_pair(cb, off);
  }
  const uint32_t q = static_cast<uint32_t>(x);
  if (t < R) {
    wc[0][t] = static_cast<uint8_t>((q >> 4) & 15u);
    wc[1][t] = static_cast<uint8_t>((q >> 8) & 15u);
  }
  // node i itself is inside the sequence; its slot 1 is the parent (the parent's slot 2), its
  // slot 0 the parent's slot 1
  if (t == 0) *vfl = 1u | (((q >> 14) & 1u) << 1) | (((q >> 12) & 1u) << 2);
  if (t == TL_THREADS - 1) *ptok = static_cast<int32_t>(q);
  return true;
}

// Slot 2 of a window from the router tables: the codes of (previous token, token).  Whole block.
__device__ __forceinline__ void tl_fresh_codes(const lng_drafter& D, int64_t ptok, int64_t tok, uint8_t (*wc)[TL_MAXR]) {
  for (int r = threadIdx.x; r < D.R; r += TL_THREADS) wc[2][r] = static_cast<uint8_t>(tl_lut_code(D, ptok, tok, r));
}

// ------------------------------------------------------------------ the tree kernel
__global__ __launch_bounds__(TL_THREADS) void k_tree_step(lng_drafter D, TlPlan T_arg, TlWork W) {
  __shared__ __attribute__((aligned(16))) TlLds lds;
  // the plan in LDS: its arrays are indexed by block-varying values (a kernel-argument array indexed
  // that way is copied to scratch memory first)
  __shared__ __attribute__((aligned(16))) TlPlan T_l;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  static_assert(sizeof(TlPlan) % 4 == 0 && sizeof(TlPlan) / 4 <= TL_THREADS, "plan copy");
  if (t < static_cast<int>(sizeof(TlPlan) / 4))
    reinterpret_cast<uint32_t*>(&T_l)[t] = reinterpret_cast<const uint32_t*>(&T_arg)[t];
  __syncthreads();
  const TlPlan& T = T_l;
  const bf16* const tab2 = static_cast<const bf16*>(D.tables[0]);  // orders 2 and 3
  const bf16* const tab3 = static_cast<const bf16*>(D.tables[1]);
  const int32_t L = *D.length;
  const uint32_t epoch = W.hdr[0];
  const bool stamps_on = W.hdr[2] != 0u;
  const int b = blockIdx.x;
  const int R = D.R;
  const int nvb = T.nvb;
  const float denom = static_cast<float>(D.R * D.n_orders);  // online counts: n_eff = total / (R * n_orders)
  const int64_t* const toks_d = D.tokens;
  const uint8_t* const codes_d = D.codes;
  bf16* const rt_out = static_cast<bf16*>(W.route_tokens);
  auto stamp = [&](int lev, int k) {
    if (stamps_on && t == 0) W.stamps[(static_cast<size_t>(lev) * TL_MAXGRID + b) * TL_NST + k] = wall_clock64();
  };
  bool failed = false;

  if (b < TL_NA) {
    // =============================================================== A: parent slot, head qh
    TlALds& A = lds.a;
    const int slot = b % TL_MAXP, qh = b / TL_MAXP;
    const int h = qh / (TL_QH / D.kv_heads);
    // the head's value weight (bf16 Wv[h], rows oc) and Gram rows (qh*64 ..) into LDS, once for every
    // depth; the o' product's thread takes output oc and inputs 32 iq .., the Gram product's
    // features 4 eq .. and rows 8 cq ..
    const int oc = t & 63, iq = t >> 6, eq = t & 63, cq = t >> 6;
    {
      const uint16_t* wsrc = static_cast<const uint16_t*>(D.wv_t) + static_cast<int64_t>(h) * TL_DT * TL_HD;
      for (int e = t; e < TL_DT * TL_HD; e += TL_THREADS) A.wv[e % TL_HD][e / TL_HD] = wsrc[e];
    }
    for (int e = t; e < TL_HD * TL_I / 4; e += TL_THREADS)
      reinterpret_cast<f32x4*>(&A.gram[0][0])[e] =
          reinterpret_cast<const f32x4*>(D.gram_out + static_cast<int64_t>(qh * TL_HD) * TL_I)[e];
    const float mnorm = t < TL_DT ? D.mem_norm[t] : 0.f;
    for (int lev = 0; lev < T.nlev; ++lev) {
      const int P = T.lev_np[lev];
      if (slot >= P) continue;
      stamp(lev, 0);
      const uint32_t tag = tl_tag(epoch, lev);
      const int j = T.lev_par[lev][slot];
      // the node's token, its window codes and their validity
      int64_t tok;
      if (lev == 0) {
        tok = L >= 1 ? D.tokens[L - 1] : -1;
        const uint32_t v = tl_root_window(D, T, L, A.wc);
        if (t == 0) A.vfl = v;
      } else {
        // the parent's window (published at the start of its own readout), then the pick
        failed |= !tl_parent_window(R, T, W.crec, epoch, lev, j, A.wc, &A.ptok, &A.vfl);
        failed |= !tl_wait_ready(nvb, W.rdy, lev - 1, tl_tag(epoch, lev - 1));
        stamp(lev, 1);
        long long* stp = stamps_on ? W.stamps + (static_cast<size_t>(lev) * TL_MAXGRID + b) * TL_NST : nullptr;
        tl_select(T, W.vrec, W.spill, denom, lev - 1, T.pslot[T.parent[j]], A.S, stp);
        stamp(lev, 10);
        const int a = A.S.sel[T.rank[j]];
        tok = a >= 0 ? a : A.S.sel[0];
        tl_fresh_codes(D, A.ptok, tok, A.wc);
      }
      // the query-key row of head qh, by the last wave (idle in the codes above: R <= 192), so its load
      // overlaps the code lookups
      if (t >= TL_THREADS - TL_DT / 4) {
        const int q = t - (TL_THREADS - TL_DT / 4);
        const f32x4 v = tl_tok_ok(D, tok)
                            ? *reinterpret_cast<const f32x4*>(D.lut_qk + tok * (TL_QH * TL_DT) + qh * TL_DT + 4 * q)
                            : f32x4{0.f, 0.f, 0.f, 0.f};
        *reinterpret_cast<f32x4*>(&A.qk[4 * q]) = v;
      }
      stamp(lev, 2);
      __syncthreads();
      const uint32_t vfl = A.vfl;
      if (qh == 0) {
        // the window codes (the V blocks' online query, the children's windows) and the token;
        // the node's token and codes into its row
        const __amdgpu_buffer_rsrc_t cb =
            dev_buf(W.crec + (static_cast<size_t>(lev) * TL_MAXP + slot) * TL_CR, TL_CR * 8u);
        const uint32_t vb3 = ((vfl >> 1) & 1u) << 12 | ((vfl >> 2) & 1u) << 13 | (vfl & 1u) << 14;
        for (int r = t; r < R; r += TL_THREADS) tl_st_pair(cb, 8u * r, A.wc[0][r] | (A.wc[1][r] << 4) | (A.wc[2][r] << 8) | vb3, tag);
        if (t == TL_THREADS - 1) tl_st_pair(cb, 8u * TL_MAXR, static_cast<uint32_t>(tok), tag);
        if (lev > 0) {
          const int32_t nr = tl_nrow(T, j, L);
          for (int r = t; r < R; r += TL_THREADS) D.codes[static_cast<int64_t>(nr) * R + r] = A.wc[2][r];
          if (t == 0) D.tokens[nr] = tok;
        }
      }
      stamp(lev, 3);
      // the window's rows straight into registers: thread t holds features fo .. fo + 15 (fo = 128 oi +
      // 16 pc: order oi, 16-byte pieces 2 pc and 2 pc + 1) of routes rs + 32 u (R <= 192: 6 routes),
      // so the 16 lanes of a DPP row hold one route
      const int pc = t & 7, oi = (t >> 3) & 1, rs = t >> 4;
      const int fo = oi * TL_MD + 16 * pc;
      // the thread's routes rs + 32 u < R are u < nu; per-route LDS entries at constant offsets from
      // one address (no per-route address registers)
      const int nu = R > rs ? (R - rs + 31) >> 5 : 0;
      const uint8_t* const wc0 = &A.wc[0][rs];
      const uint8_t* const wc1 = &A.wc[1][rs];
      const uint8_t* const wc2 = &A.wc[2][rs];
      const bool vo2 = (vfl >> 1) & 1u, vo3 = (vfl >> 2) & 1u;
      float* const sxp = &A.sx[rs];
      float* const scp = &A.sc[rs];
      const float* const wrp = &A.wr[rs];
      u32x4 pv[6][2];
#pragma unroll
      for (int u = 0; u < 6; ++u) {
        // the route's row of order oi (order 2: 256 r + the two newest codes, order 3: 4096 r + all
        // three), -1 when a window slot is outside the sequence
        const int r = rs + 32 * u;
        const int32_t c0 = wc0[32 * u], c1 = wc1[32 * u], c2 = wc2[32 * u];
        const int32_t rw = u >= nu ? -1
                           : oi  ? (vo3 ? r * 4096 + (c0 | (c1 << 4) | (c2 << 8)) : -1)
                                 : (vo2 ? r * 256 + (c1 | (c2 << 4)) : -1);
        const bf16* src = (oi ? tab3 : tab2) + static_cast<int64_t>(rw < 0 ? 0 : rw) * TL_MD + 16 * pc;
#pragma unroll
        for (int k = 0; k < 2; ++k)
          pv[u][k] = rw >= 0 ? *reinterpret_cast<const u32x4*>(src + 8 * k) : u32x4{0u, 0u, 0u, 0u};
      }
      stamp(lev, 4);
      // scores: each route's sum of squares and query-key dot, summed over its DPP row
      {
        float qv[16];
#pragma unroll
        for (int k = 0; k < 16; k += 4) {
          const f32x4 v = *reinterpret_cast<const f32x4*>(&A.qk[fo + k]);
          qv[k] = v[0], qv[k + 1] = v[1], qv[k + 2] = v[2], qv[k + 3] = v[3];
        }
        float s2[6], d2[6];
#pragma unroll
        for (int u = 0; u < 6; ++u) {
          float sa = 0.f, da = 0.f;
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            const uint32_t wd = pv[u][k >> 2][k & 3];
            const float x0 = __uint_as_float(wd << 16), x1 = __uint_as_float(wd & 0xffff0000u);
            sa = fmaf(x0, x0, sa);
            sa = fmaf(x1, x1, sa);
            da = fmaf(qv[2 * k], x0, da);
            da = fmaf(qv[2 * k + 1], x1, da);
          }
          s2[u] = sa, d2[u] = da;
          __builtin_amdgcn_sched_barrier(0);  // one route at a time: the unpacked words stay few
        }
#pragma unroll
        for (int u = 0; u < 6; ++u) s2[u] = tl_row16_sum(s2[u]), d2[u] = tl_row16_sum(d2[u]);
        if ((t & 15) == 15) {
#pragma unroll
          for (int u = 0; u < 6; ++u) {
            if (u < nu) {
              const float sv = 1.0f / sqrtf(s2[u] / static_cast<float>(TL_DT) + D.mem_eps);
              sxp[32 * u] = sv;
              scp[32 * u] = sv * d2[u];
            }
          }
        }
      }
      tl_sync();
      stamp(lev, 5);
      // softmax over the routes (the sink enters through the weight below)
      const float scv = t < R ? A.sc[t] : -INFINITY;
      const float m = tl_block_max(scv, A.stat);
      const float pe = t < R ? expf(scv - m) : 0.f;
      if (t < R) A.wr[t] = pe * A.sx[t];
      const float l = tl_block_sum(pe, A.stat);
      const float b0 = D.sink_logit;
      const float Mx = fmaxf(b0, m);
      const float fex = expf(m - Mx);
      const float wgt = fex / fmaf(l, fex, expf(b0 - Mx));
      // U[i] = sum_r wr[r] x_r[i]: the thread's routes, then the 32 route rows of the block
      {
        float ua[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) ua[k] = 0.f;
#pragma unroll
        for (int u = 0; u < 6; ++u) {
          const float wv = u < nu ? wrp[32 * u] : 0.f;
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            const uint32_t wd = pv[u][k >> 2][k & 3];
            ua[2 * k] = fmaf(wv, __uint_as_float(wd << 16), ua[2 * k]);
            ua[2 * k + 1] = fmaf(wv, __uint_as_float(wd & 0xffff0000u), ua[2 * k + 1]);
          }
        }
#pragma unroll
        for (int k = 0; k < 16; k += 4)
          *reinterpret_cast<f32x4*>(&A.red[rs][fo + k]) = f32x4{ua[k], ua[k + 1], ua[k + 2], ua[k + 3]};
      }
      tl_sync();
      if (t < TL_DT) {
        float u = 0.f;
#pragma unroll
        for (int k = 0; k < TL_THREADS / 16; ++k) u += A.red[k][t];
        A.un[t] = u * mnorm;  // mem_norm . U
      }
      tl_sync();
      stamp(lev, 6);
      // o'[c] = sum_i Wv[h][c][i] un[i]: thread (output oc, inputs 32 iq .. 32 iq + 31), then the
      // eight input runs
      {
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < 32; k += 8) {
          const u32x4 wq = *reinterpret_cast<const u32x4*>(&A.wv[oc][32 * iq + k]);
          const f32x4 ua = *reinterpret_cast<const f32x4*>(&A.un[32 * iq + k]);
          const f32x4 ub = *reinterpret_cast<const f32x4*>(&A.un[32 * iq + k + 4]);
          const float uq[8] = {ua[0], ua[1], ua[2], ua[3], ub[0], ub[1], ub[2], ub[3]};
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const uint32_t pr = wq[e >> 1];
            const float wf = (e & 1) ? __uint_as_float(pr & 0xffff0000u) : __uint_as_float(pr << 16);
            acc = fmaf(wf, uq[e], acc);
          }
        }
        A.opart[iq][oc] = acc;
      }
      tl_sync();
      if (t < TL_HD) {
        float a = 0.f;
#pragma unroll
        for (int g = 0; g < TL_WAVES; ++g) a += A.opart[g][t];
        A.o[t] = wgt * a;
      }
      tl_sync();
      // Y[e] = sum_c Gram[qh*64 + c][e] o[c]: thread (features 4 eq .., rows 8 cq ..)
      {
        f32x4 y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const float ov = A.o[8 * cq + q];
          const f32x4 gq = *reinterpret_cast<const f32x4*>(&A.gram[8 * cq + q][4 * eq]);
          y[0] = fmaf(gq[0], ov, y[0]);
          y[1] = fmaf(gq[1], ov, y[1]);
          y[2] = fmaf(gq[2], ov, y[2]);
          y[3] = fmaf(gq[3], ov, y[3]);
        }
        *reinterpret_cast<f32x4*>(&A.red[cq][4 * eq]) = y;
      }
      tl_sync();
      {
        const __amdgpu_buffer_rsrc_t ab =
            dev_buf(W.arec + ((static_cast<size_t>(lev) * TL_MAXP + slot) * TL_QH + qh) * TL_AP, TL_AP * 8u);
        if (t < TL_DT) {
          float yv = 0.f;
#pragma unroll
          for (int k = 0; k < TL_WAVES; ++k) yv += A.red[k][t];
          tl_st_pair(ab, 8u * t, __float_as_uint(yv), tag);
        } else if (t < TL_DT + TL_HD) {
          tl_st_pair(ab, 8u * t, __float_as_uint(A.o[t - TL_DT]), tag);
        }
      }
      stamp(lev, 7);
      // head 0: the node's verification route tokens, from the registers (after the record: the
      // barriers wait for the block's global stores)
      if (qh == 0 && rt_out) {
        // the node's [R, 256] block at a uniform base; route step 32 u as the constant offset
        const __amdgpu_buffer_rsrc_t ob = dev_buf(rt_out + static_cast<int64_t>(j) * R * TL_DT, 2u * R * TL_DT);
        const uint32_t vo = 2u * static_cast<uint32_t>(rs * TL_DT + fo);
#pragma unroll
        for (int u = 0; u < 6; ++u)
          if (u < nu)
#pragma unroll
            for (int k = 0; k < 2; ++k) __builtin_amdgcn_raw_buffer_store_b128(pv[u][k], ob, vo + 16u * k, 2 * 32 * TL_DT * u, 0);
      }
      __syncthreads();  // LDS is reused by the next depth
    }
  } else if (b < TL_NA + nvb) {
    // =============================================================== V: vocabulary slice
    TlVLds& S = lds.v;
    const int vb = b - TL_NA;
    const int64_t v0 = static_cast<int64_t>(vb) * TL_VS;
    const int64_t V = D.V;
    // lut_out rows v0 + 64 g + lane (g < 3), features TL_VK w .. + TL_VK: the A operands of the
    // wave's 4x4x1 MFMAs (lane 4b + i holds row 4b + i of block b), held for every depth
    f32x4 av[TL_VG][TL_VK / 4];
#pragma unroll
    for (int g = 0; g < TL_VG; ++g) {
      const int i = 64 * g + lane;
      const int64_t v = v0 + i;
#pragma unroll
      for (int q = 0; q < TL_VK / 4; ++q)
        av[g][q] = (i < TL_VS && v < V) ? *reinterpret_cast<const f32x4*>(D.lut_out + v * TL_I + TL_VK * w + 4 * q)
                                       : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const bool online = T.online != 0;
    const int npairs = L - 1;
    // the committed pairs q (0 <= q < L - 1, next token tokens[q + 1]) whose next token lies in the slice
    auto list_pairs = [&](int base, int span) {
      for (int e = t; e < span; e += TL_THREADS) {
        const int q = base + e;
        if (q < npairs) {
          const int64_t nt = toks_d[q + 1];
          if (nt >= v0 && nt < v0 + TL_VS) {
            const int at = atomicAdd(&S.nmatch, 1);
            if (at < TL_PL) S.list[at] = q;
          }
        }
      }
    };
    if (t == 0) S.nmatch = 0;
    __syncthreads();
    if (online && npairs > 0) list_pairs(0, npairs);
    __syncthreads();
    const bool overflow = S.nmatch > TL_PL;
    const int nlist = min(S.nmatch, TL_PL);
    const int nkey = min(nlist, TL_KL);
    // match keys of the first listed pairs, formed once for every depth (committed codes only)
    for (int e = t; e < nkey * R; e += TL_THREADS) {
      const int li = e / R, r = e % R;
      const int q = S.list[li];
      const int c0 = codes_d[static_cast<int64_t>(q) * R + r] & 15;
      const int c1 = q >= 1 ? codes_d[static_cast<int64_t>(q - 1) * R + r] & 15 : 0;
      const int c2 = q >= 2 ? codes_d[static_cast<int64_t>(q - 2) * R + r] & 15 : 0;
      S.keys[li][r] = static_cast<uint16_t>(c2 | (c1 << 4) | (c0 << 8) | (q >= 1 ? 1 << 12 : 0) | (q >= 2 ? 1 << 13 : 0));
    }
    for (int li = t; li < nkey; li += TL_THREADS) S.knt[li] = static_cast<uint8_t>(toks_d[S.list[li] + 1] - v0);
    __syncthreads();
    const __amdgpu_buffer_rsrc_t rdb = dev_buf(W.rdy, TL_NLB * TL_MAXVB * 4u);
    for (int lev = 0; lev < T.nlev; ++lev) {
      const int P = T.lev_np[lev];
      const uint32_t tag = tl_tag(epoch, lev);
      stamp(lev, 0);
      for (int e = t; e < TL_MAXP * TL_VS; e += TL_THREADS) (&S.sc[0][0])[e] = 0;
      int tot_p[TL_MAXP] = {0, 0, 0, 0};
      if (online) {
        // window codes of every parent (self-validating pairs; re-read what is still stale)
        const __amdgpu_buffer_rsrc_t cb =
            dev_buf(W.crec + static_cast<size_t>(lev) * TL_MAXP * TL_CR, TL_MAXP * TL_CR * 8u);
        const long long t0 = wall_clock64();
        while (!failed) {
          bool okq = true;
          for (int e = t; e < P * R; e += TL_THREADS) {
            const int p = e / R, r = e % R;
            const uint64_t x = tl_ld_pair(cb, 8u * (p * TL_CR + r));
            if (static_cast<uint32_t>(x >> 32) == tag)
              S.qry[p][r] = static_cast<uint32_t>(x);
            else
              okq = false;
          }
          if (__syncthreads_and(okq ? 1 : 0)) break;
          failed = __syncthreads_or(wall_clock64() - t0 > TL_SPIN_TICKS ? 1 : 0) != 0;
          __builtin_amdgcn_s_sleep(2);
        }
        __syncthreads();
        stamp(lev, 1);
        // matches of the listed pairs: item (listed pair, route r); the keys of the window ending at pair q
        // items (listed pair, route); pairs li < k0 take their keys from LDS
        auto count = [&](int nl, int k0) {
          for (int e = t; e < nl * R; e += TL_THREADS) {
            const int li = e / R, r = e % R;
            uint32_t k3, nt;
            if (li < k0) {
              k3 = S.keys[li][r];
              nt = S.knt[li];
            } else {
              const int q = S.list[li];
              const int c0 = codes_d[static_cast<int64_t>(q) * R + r] & 15;
              const int c1 = q >= 1 ? codes_d[static_cast<int64_t>(q - 1) * R + r] & 15 : 0;
              const int c2 = q >= 2 ? codes_d[static_cast<int64_t>(q - 2) * R + r] & 15 : 0;
              k3 = static_cast<uint32_t>(c2 | (c1 << 4) | (c0 << 8) | (q >= 1 ? 1 << 12 : 0) | (q >= 2 ? 1 << 13 : 0));
              nt = static_cast<uint32_t>(toks_d[q + 1] - v0);
            }
#pragma unroll
            for (int p = 0; p < TL_MAXP; ++p) {
              if (p >= P) break;
              const uint32_t qv = S.qry[p][r];
              // order 2: key (t - 1, t) against query slots (1, 2); order 3: all three
              const int mt = ((qv & k3 & (1u << 12)) && ((k3 >> 4) & 0xffu) == ((qv >> 4) & 0xffu) ? 1 : 0) +
                             ((qv & k3 & (1u << 13)) && (k3 & 0xfffu) == (qv & 0xfffu) ? 1 : 0);
              if (mt) {
                atomicAdd(&S.sc[p][nt], mt);
                tot_p[p] += mt;
              }
            }
          }
        };
        if (!overflow) {
          count(nlist, nkey);
        } else {
          // more listed pairs than the list holds: list and count them in rounds
          for (int base = 0; base < npairs; base += TL_PL) {
            __syncthreads();
            if (t == 0) S.nmatch = 0;
            __syncthreads();
            list_pairs(base, TL_PL);
            __syncthreads();
            count(min(S.nmatch, TL_PL), 0);
          }
        }
      }
      stamp(lev, 2);
      // A records of every (parent, head); re-read what is still stale
      const __amdgpu_buffer_rsrc_t ab =
          dev_buf(W.arec + static_cast<size_t>(lev) * TL_MAXP * TL_QH * TL_AP, TL_MAXP * TL_QH * TL_AP * 8u);
      // a light probe first (one pair per record: the last value its head's block writes), then the
      // bulk read of every (parent, head) record
      if (w == 0 && !failed) {
        const long long t0 = wall_clock64();
        for (;;) {
          const bool okp =
              lane >= TL_QH * P || static_cast<uint32_t>(tl_ld_pair(ab, 8u * (lane * TL_AP + TL_AP - 1)) >> 32) == tag;
          if (__ballot(!okp) == 0 || wall_clock64() - t0 > TL_SPIN_TICKS) break;
          __builtin_amdgcn_s_sleep(1);
        }
      }
      __syncthreads();
      // thread t < 256 = feature e: o[e] (head e / 64) and Y[e] of every head, per parent
      float ov[TL_MAXP], yv[TL_MAXP];
      {
        const int e = t & (TL_DT - 1);
        const bool mine = t < TL_DT;
        uint64_t xo[TL_MAXP], xy[TL_MAXP][TL_QH];
#pragma unroll
        for (int p = 0; p < TL_MAXP; ++p) {
          xo[p] = 0;
          if (mine && p < P) xo[p] = tl_ld_pair(ab, 8u * ((p * TL_QH + e / TL_HD) * TL_AP + TL_DT + e % TL_HD));
#pragma unroll
          for (int qq = 0; qq < TL_QH; ++qq) {
            xy[p][qq] = 0;
            if (mine && p < P) xy[p][qq] = tl_ld_pair(ab, 8u * ((p * TL_QH + qq) * TL_AP + e));
          }
        }
        const long long t0 = wall_clock64();
        while (!failed) {
          bool okr = true;
          if (mine) {
#pragma unroll
            for (int p = 0; p < TL_MAXP; ++p) {
              if (p < P && static_cast<uint32_t>(xo[p] >> 32) != tag) {
                okr = false;
                xo[p] = tl_ld_pair(ab, 8u * ((p * TL_QH + e / TL_HD) * TL_AP + TL_DT + e % TL_HD));
              }
#pragma unroll
              for (int qq = 0; qq < TL_QH; ++qq)
                if (p < P && static_cast<uint32_t>(xy[p][qq] >> 32) != tag) {
                  okr = false;
                  xy[p][qq] = tl_ld_pair(ab, 8u * ((p * TL_QH + qq) * TL_AP + e));
                }
            }
          }
          if (__syncthreads_and(okr ? 1 : 0)) break;
          failed = __syncthreads_or(wall_clock64() - t0 > TL_SPIN_TICKS ? 1 : 0) != 0;
          __builtin_amdgcn_s_sleep(1);
        }
#pragma unroll
        for (int p = 0; p < TL_MAXP; ++p) {
          ov[p] = __uint_as_float(static_cast<uint32_t>(xo[p]));
          yv[p] = (__uint_as_float(static_cast<uint32_t>(xy[p][0])) + __uint_as_float(static_cast<uint32_t>(xy[p][1]))) +
                  (__uint_as_float(static_cast<uint32_t>(xy[p][2])) + __uint_as_float(static_cast<uint32_t>(xy[p][3])));
        }
      }
      stamp(lev, 3);
      // hidden-state scale per parent: r = rsqrt(o . (Gram o) / d + eps); the waves' partial dots and
      // o itself through LDS, then every lane forms the four scales (the same sums in the same order)
#pragma unroll
      for (int p = 0; p < TL_MAXP; ++p) {
        const float sp = wave_sum(t < TL_DT ? ov[p] * yv[p] : 0.f);
        const int tp = tl_wave_sum_i(tot_p[p]);
        if (lane == 0) S.part[p][w] = sp, S.tot[p][w] = tp;
      }
      if (t < TL_DT)
#pragma unroll
        for (int p = 0; p < TL_MAXP; ++p) S.ro[p][t] = ov[p];
      tl_sync();
      float rl;  // the scale of parent lane % 4, the column of the MFMAs' B operand (0 past the parents)
      {
        const int pl = lane & 3;
        float ss = 0.f;
#pragma unroll
        for (int k = 0; k < TL_WAVES; ++k) ss += S.part[pl][k];
        rl = pl < P ? 1.0f / sqrtf(ss / static_cast<float>(D.d) + D.draft_eps) : 0.f;
      }
      // logits: D[row][parent] over the wave's features with 4x4x1 MFMAs (16 blocks of 4 rows x 4
      // parents; B = r o[lane % 4][k]), then the waves' partials summed in wave order
      {
        f32x4 acc[TL_VG];
#pragma unroll
        for (int g = 0; g < TL_VG; ++g) acc[g] = f32x4{0.f, 0.f, 0.f, 0.f};
        const float* rop = &S.ro[lane & 3][TL_VK * w];
#pragma unroll
        for (int q = 0; q < TL_VK / 4; ++q) {
          const f32x4 bq = *reinterpret_cast<const f32x4*>(rop + 4 * q);
#pragma unroll
          for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int g = 0; g < TL_VG; ++g) acc[g] = __builtin_amdgcn_mfma_f32_4x4x1f32(av[g][q][e], rl * bq[e], acc[g], 0, 0, 0);
        }
        // lane 4b + n, register i: row 64 g + 4b + i, parent n
#pragma unroll
        for (int g = 0; g < TL_VG; ++g) S.lpart[w][64 * g + lane] = acc[g];
      }
      __syncthreads();
      for (int e = t; e < TL_MAXP * TL_VS; e += TL_THREADS) {
        const int p = e / TL_VS, i = e % TL_VS;
        const int blk = i >> 2, ii = i & 3;  // row i = 64 g + 4 b + ii sits in lane 4 b + p of group g
        const int g = blk >> 4, bb = blk & 15;
        float a = 0.f;
#pragma unroll
        for (int ww = 0; ww < TL_WAVES; ++ww) a += S.lpart[ww][64 * g + 4 * bb + p][ii];
        S.lt[p][i] = a;
      }
      __syncthreads();
      stamp(lev, 4);
      // records: wave p takes parent p (tokens lane, lane + 64, lane + 128 of the slice)
      if (w < P) {
        const int p = w;
        float x[3];
        int c[3];
        int64_t id[3];
#pragma unroll
        for (int u = 0; u < 3; ++u) {
          const int i = lane + 64 * u;
          id[u] = v0 + i;
          const bool in = i < TL_VS && id[u] < V;
          x[u] = in ? S.lt[p][min(i, TL_VS - 1)] : -INFINITY;
          c[u] = in && online ? S.sc[p][min(i, TL_VS - 1)] : 0;
        }
        const float m = wave_max(fmaxf(fmaxf(x[0], x[1]), x[2]));
        float se = 0.f;
#pragma unroll
        for (int u = 0; u < 3; ++u) se += x[u] == -INFINITY ? 0.f : expf(x[u] - m);
        const float s = wave_sum(se);
        // top-KM of the tokens without counts: KM rounds of the wave's largest ranking key (value
        // desc, id asc), each taken out of its lane
        uint64_t ck[3];
#pragma unroll
        for (int u = 0; u < 3; ++u) ck[u] = (x[u] != -INFINITY && c[u] == 0) ? tl_key(x[u], static_cast<int>(id[u])) : 0;
        float sv[TL_KM];
        int si[TL_KM];
#pragma unroll
        for (int k = 0; k < TL_KM; ++k) {
          const uint64_t b01 = ck[1] > ck[0] ? ck[1] : ck[0];
          const uint64_t wk = tl_wave_max_u64(ck[2] > b01 ? ck[2] : b01);
          sv[k] = wk == 0 ? -INFINITY : tl_key_value(wk);
          si[k] = wk == 0 ? -1 : tl_key_id(wk);
#pragma unroll
          for (int u = 0; u < 3; ++u) ck[u] = (wk != 0 && ck[u] == wk) ? 0 : ck[u];
        }
        const size_t ri = (static_cast<size_t>(lev) * TL_MAXP + p) * TL_MAXVB + vb;
        const __amdgpu_buffer_rsrc_t rb = dev_buf(W.vrec + ri * TL_RW, TL_RW * 4u);
        const __amdgpu_buffer_rsrc_t sb = dev_buf(W.spill + ri * (TL_VS * 3), TL_VS * 12u);
        // count-bearing tokens, compacted in slice order
        int nc = 0;
#pragma unroll
        for (int u = 0; u < 3; ++u) {
          const uint64_t mk = __ballot(c[u] > 0);
          const int at = nc + __popcll(mk & ((lane == 0) ? 0ull : (~0ull >> (64 - lane))));
          if (c[u] > 0) {
            if (at < TL_NI) {
              tl_st_w(rb, 4u * (12 + 3 * at), static_cast<uint32_t>(id[u]));
              tl_st_w(rb, 4u * (13 + 3 * at), __float_as_uint(x[u]));
              tl_st_w(rb, 4u * (14 + 3 * at), static_cast<uint32_t>(c[u]));
            } else {
              tl_st_w(sb, 12u * at, static_cast<uint32_t>(id[u]));
              tl_st_w(sb, 12u * at + 4u, __float_as_uint(x[u]));
              tl_st_w(sb, 12u * at + 8u, static_cast<uint32_t>(c[u]));
            }
          }
          nc += __popcll(mk);
        }
        if (lane == 0) {
          int tp = 0;
#pragma unroll
          for (int k = 0; k < TL_WAVES; ++k) tp += S.tot[p][k];
          const u32x4 h0 = {__float_as_uint(m), __float_as_uint(s), static_cast<uint32_t>(tp), static_cast<uint32_t>(nc)};
          u32x4 h1, h2;
#pragma unroll
          for (int k = 0; k < TL_KM; ++k) h1[k] = __float_as_uint(sv[k]), h2[k] = static_cast<uint32_t>(si[k]);
          __builtin_amdgcn_raw_buffer_store_b128(h0, rb, 0u, 0, CPOL_SC1);
          __builtin_amdgcn_raw_buffer_store_b128(h1, rb, 16u, 0, CPOL_SC1);
          __builtin_amdgcn_raw_buffer_store_b128(h2, rb, 32u, 0, CPOL_SC1);
        }
      }
      // the slice's ready word, once every store of the block is complete
      __builtin_amdgcn_s_waitcnt(WAITCNT_VM0);
      __syncthreads();
      if (t == 0) tl_st_w(rdb, 4u * (lev * TL_MAXVB + vb), tag);
      stamp(lev, 5);
    }
  } else {
    // =============================================================== G: leaves of every depth
    TlGLds& G = lds.g;
    const int gi = b - TL_NA - nvb;
    if (gi == 0 && t == 0) D.tokens[T.node_row0] = L > 0 ? D.tokens[L - 1] : -1;
    for (int lev = 0; lev <= T.nlev; ++lev) {
      for (int g = gi; g < T.lev_nleaf[lev]; g += T.ngb) {
        const int i = T.lev_leaf[lev][g];
        int64_t tok;
        if (i == 0) {
          tok = L >= 1 ? D.tokens[L - 1] : -1;
          const uint32_t v = tl_root_window(D, T, L, G.wc);
          if (t == 0) G.vfl = v;
        } else {
          failed |= !tl_parent_window(R, T, W.crec, epoch, lev, i, G.wc, &G.ptok, &G.vfl);
          failed |= !tl_wait_ready(nvb, W.rdy, lev - 1, tl_tag(epoch, lev - 1));
          tl_select(T, W.vrec, W.spill, denom, lev - 1, T.pslot[T.parent[i]], G.S);
          const int a = G.S.sel[T.rank[i]];
          tok = a >= 0 ? a : G.S.sel[0];
          tl_fresh_codes(D, G.ptok, tok, G.wc);
        }
        __syncthreads();
        if (i != 0) {
          const int32_t nr = tl_nrow(T, i, L);
          for (int r = t; r < R; r += TL_THREADS) D.codes[static_cast<int64_t>(nr) * R + r] = G.wc[2][r];
          if (t == 0) D.tokens[nr] = tok;
        }
        if (rt_out) {
          // the leaf's route tokens: every row load in flight before the stores (thread t: features
          // fo .. fo + 15 of routes rs + 32 u, row indices formed from the window codes)
          const uint32_t vfl = G.vfl;
          const bool vo2 = (vfl >> 1) & 1u, vo3 = (vfl >> 2) & 1u;
          const int pc = t & 7, oi = (t >> 3) & 1, rs = t >> 4;
          const int fo = oi * TL_MD + 16 * pc;
          const int nu = R > rs ? (R - rs + 31) >> 5 : 0;
          u32x4 pv[6][2];
#pragma unroll
          for (int u = 0; u < 6; ++u) {
            const int r = rs + 32 * u;
            const int32_t c0 = u < nu ? G.wc[0][r] : 0, c1 = u < nu ? G.wc[1][r] : 0, c2 = u < nu ? G.wc[2][r] : 0;
            const int32_t rw = u >= nu ? -1
                               : oi  ? (vo3 ? r * 4096 + (c0 | (c1 << 4) | (c2 << 8)) : -1)
                                     : (vo2 ? r * 256 + (c1 | (c2 << 4)) : -1);
            const bf16* src = (oi ? tab3 : tab2) + static_cast<int64_t>(rw < 0 ? 0 : rw) * TL_MD + 16 * pc;
#pragma unroll
            for (int k = 0; k < 2; ++k)
              pv[u][k] = rw >= 0 ? *reinterpret_cast<const u32x4*>(src + 8 * k) : u32x4{0u, 0u, 0u, 0u};
          }
          const __amdgpu_buffer_rsrc_t ob = dev_buf(rt_out + static_cast<int64_t>(i) * R * TL_DT, 2u * R * TL_DT);
          const uint32_t vo = 2u * static_cast<uint32_t>(rs * TL_DT + fo);
#pragma unroll
          for (int u = 0; u < 6; ++u)
            if (u < nu)
#pragma unroll
              for (int k = 0; k < 2; ++k) __builtin_amdgcn_raw_buffer_store_b128(pv[u][k], ob, vo + 16u * k, 2 * 32 * TL_DT * u, 0);
        }
        __syncthreads();  // LDS is reused by the next leaf
      }
    }
  }
  // error word; the last block to finish advances the epoch (every block read it at entry)
  if (failed && t == 0) __hip_atomic_fetch_or(reinterpret_cast<int32_t*>(W.hdr + 1), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (t == 0) {
    const uint32_t done = __hip_atomic_fetch_add(W.hdr + 3, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (done == gridDim.x - 1) {
      __hip_atomic_store(W.hdr + 3, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(W.hdr + 0, epoch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ------------------------------------------------------------------ host side
// A token-only drafter with the per-token tables at the shape the kernel is written for.
bool tl_drafter_ok(const lng_drafter& D) {
  return D.lut_prev && D.lut_cur && D.lut_start && D.lut_qk && D.lut_out && D.gram_out && D.wv_t && D.mem_norm &&
         D.tokens && D.codes && D.length && D.tables[0] && D.tables[1] && !D.router_ssm && !D.query_ssm &&
         D.V > 0 && D.rows > 0 && D.R > 0 && D.q_heads == TL_QH && D.head_dim == TL_HD && D.dt == TL_DT &&
         D.mem_dim == TL_MD && D.n_orders == 2 && D.orders[0] == 2 && D.orders[1] == 3 && D.maxn == 3 &&
         D.bits == 4 && D.R <= TL_MAXR && D.table_dtype == LNG_BF16 && D.wv_dtype == LNG_BF16 &&
         D.kv_heads > 0 && TL_QH % D.kv_heads == 0 && cdiv(D.V, TL_VS) <= TL_MAXVB;
}

// Blocks that can be resident at once on the current device (one per CU at this kernel's LDS),
// cached per device.
int tl_resident() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int nb = cache[dev].load(std::memory_order_relaxed);
  if (nb > 0) return nb;
  int cus = 0, per = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, reinterpret_cast<const void*>(&k_tree_step), TL_THREADS, 0) !=
      hipSuccess)
    return 0;
  nb = std::min(TL_MAXGRID, cus * std::max(per, 0));
  cache[dev].store(nb, std::memory_order_relaxed);
  return nb;
}

int tl_plan(const lng_drafter& D, const int32_t* parent, const int32_t* rank, int32_t n, int32_t node_row0, int online,
            float kappa, int grid, TlPlan& T) {
  if (!parent || !rank || n <= 0 || n > TL_MAXN || parent[0] != -1)
    return fail(LNG_E_ARG, "drafter_tree_levels: need 1 <= n <= 32 nodes with parent[0] == -1");
  if (node_row0 < 0 || static_cast<int64_t>(node_row0) + n > D.rows)
    return fail(LNG_E_RANGE, "drafter_tree_levels: node rows out of range");
  T = TlPlan{};
  T.n = n, T.node_row0 = node_row0, T.online = online ? 1 : 0, T.kappa = kappa;
  T.nvb = static_cast<int32_t>(cdiv(D.V, TL_VS));
  T.ngb = grid - TL_NA - T.nvb;
  if (T.ngb < TL_MINGB) return fail(LNG_E_ARG, "drafter_tree_levels: too few resident blocks for the vocabulary");
  std::vector<int> depth(n, 0), nchild(n, 0);
  int K = 1;
  for (int i = 1; i < n; ++i) {
    if (parent[i] < 0 || parent[i] >= i) return fail(LNG_E_ARG, "drafter_tree_levels: parent[i] must precede i");
    if (rank[i] < 0 || rank[i] >= TL_KM) return fail(LNG_E_ARG, "drafter_tree_levels: rank out of range");
    depth[i] = depth[parent[i]] + 1;
    ++nchild[parent[i]];
    K = std::max(K, rank[i] + 1);
  }
  const int maxd = *std::max_element(depth.begin(), depth.end());
  // depths 0 .. maxd - 1 have parents; depth maxd holds leaves only
  if (maxd > TL_MAXL) return fail(LNG_E_ARG, "drafter_tree_levels: tree deeper than 8");
  T.K = K;
  T.nlev = maxd;
  for (int i = 0; i < n; ++i) {
    T.parent[i] = static_cast<int8_t>(parent[i]);
    T.rank[i] = static_cast<int8_t>(i ? rank[i] : 0);
    T.pslot[i] = -1;
    const int d = depth[i];
    if (nchild[i] > 0) {
      if (T.lev_np[d] >= TL_MAXP) return fail(LNG_E_ARG, "drafter_tree_levels: more than 4 parents at one depth");
      T.pslot[i] = T.lev_np[d];
      T.lev_par[d][T.lev_np[d]++] = static_cast<int8_t>(i);
    } else {
      T.lev_leaf[d][T.lev_nleaf[d]++] = static_cast<int8_t>(i);
    }
  }
  return LNG_OK;
}

}  // namespace
}  // namespace lng

using namespace lng;

extern "C" {

size_t lng_drafter_tree_levels_workspace(const lng_drafter* D) {
  if (!D || !tl_drafter_ok(*D)) return 0;
  const int grid = tl_resident();
  return grid - TL_NA - cdiv(D->V, TL_VS) >= TL_MINGB ? tl_layout().total : 0;
}

int lng_drafter_tree_levels(const lng_drafter* D, const int32_t* parent, const int32_t* rank, int32_t n,
                            int32_t node_row0, int online, float kappa, void* work, size_t work_bytes,
                            void* route_tokens, void* stream) {
  if (!D || !tl_drafter_ok(*D)) return fail(LNG_E_ARG, "drafter_tree_levels: drafter outside the kernel's shape");
  if (!work) return fail(LNG_E_ARG, "drafter_tree_levels: null workspace");
  const TlLayout l = tl_layout();
  if (work_bytes < l.total) return fail(LNG_E_ARG, "drafter_tree_levels: workspace too small");
  const int grid = tl_resident();
  TlPlan T;
  if (int rc = tl_plan(*D, parent, rank, n, node_row0, online, kappa, grid, T)) return rc;
  char* w = static_cast<char*>(work);
  TlWork Wk{reinterpret_cast<uint32_t*>(w + l.hdr),   reinterpret_cast<uint64_t*>(w + l.crec),
            reinterpret_cast<uint64_t*>(w + l.arec),  reinterpret_cast<uint32_t*>(w + l.vrec),
            reinterpret_cast<uint32_t*>(w + l.rdy),   reinterpret_cast<uint32_t*>(w + l.spill),
            reinterpret_cast<long long*>(w + l.stamps), route_tokens};
  hipLaunchKernelGGL(k_tree_step, dim3(static_cast<unsigned>(grid)), dim3(TL_THREADS), 0, as_stream(stream), *D, T, Wk);
  return check_launch("drafter_tree_levels");
}

}  // extern "C"
