// Diagonal SSM scan: s_t = a * s_{t-1} + (1 - a) * u_t, s_{-1} = s0 (or 0)
// (ffnmem/memory/ssm.py:37-91; the carried-state continuation of ffnmem/infer.py:125-137).
//
// One pass: every element of u is read once and every state written once.  A block owns one tile,
// (batch b, 256-channel group g, span of SSM_WAVES * SSM_LW consecutive steps); each wave takes
// SSM_LW steps of it and each lane 4 channels, so one step of a wave is one coalesced 1 KB access.
//   1. a wave loads its inputs into registers and scans them from a zero state (end e_w);
//   2. wave 0 folds the waves' ends into the tile's aggregate (its end state from a zero start;
//      the first tile of a sequence starts from s0 instead, so its aggregate is its end state)
//      and publishes it;
//   3. the carry into the tile is the fold of the aggregates of the SSM_WIN tiles before it
//      (tile k back weighted by the decay a^(k * span)), plus, past that window, the
//      published end state of the tile just before it; the 8 waves fetch those records at once;
//   4. the tile publishes its end state; every wave re-scans its registers from its carry in and
//      writes s.
// Records are self-validating: every element is a 64-bit (value, tag) pair written and read with
// single 64-bit accesses at the device-coherent level, the tag holding the call's epoch and the
// record kind, so a reader needs no separate flag and a writer no completion wait.  The epoch lives
// in the workspace header: every tile reads it at entry and the last tile to finish advances it, so
// consecutive launches (a replayed HIP graph included) never accept each other's records.  A tile
// waits only on tiles with smaller block indices (tiles run in span-major order), which the in-order
// dispatcher has started before it and which publish their aggregate before they wait on anything.
// Waits are bounded all the same: a tile whose wait runs out forms its carry directly from u
// (a sequential scan of the steps before it: slow, exact), and sets bit 0 of the header's status
// word, so the result is right either way.
#include "common.h"

#include <mutex>

namespace lng {

constexpr int SSM_WAVES = 8;          // waves per block
constexpr int SSM_GC = 256;           // channels per group (64 lanes x 4)
#ifndef LNG_SSM_LW
#define LNG_SSM_LW 16
#endif
constexpr int SSM_LW = LNG_SSM_LW;    // steps per wave
constexpr int SSM_SPAN = SSM_WAVES * SSM_LW;
constexpr int SSM_WIN = 32;           // aggregates folded per look-back; the record before comes inclusive
constexpr int SSM_PER_WAVE = (SSM_WIN + 1 + SSM_WAVES - 1) / SSM_WAVES;
// workspace: a 256-byte header (int32 words: 0 status bits, 1 epoch, 2 finished tiles of the
// running launch), then one record per tile: its aggregate and its end state, 256 (value, tag)
// pairs each
constexpr size_t SSM_HDR = 256;
constexpr size_t SSM_REC = 2 * SSM_GC * sizeof(uint64_t);
constexpr uint32_t SSM_AGG = 1u, SSM_INC = 2u;
constexpr int SSM_SPIN_LIMIT = 1 << 22;  // sleeps of ~64 cycles: well past any real wait

// (value, tag) pairs move as single 64-bit buffer accesses with the cache policy CPOL; sc1 puts
// them at the device-coherent level, past the XCD-private L2s, where every XCD reads the same copy
// (which XCD runs a block is up to the dispatcher: records through one XCD's L2 (sc0) were seen
// stale by blocks on another)
template <int CPOL>
__device__ __forceinline__ void st_pair(__amdgpu_buffer_rsrc_t r, uint32_t off, float v, uint32_t tag) {
  const uint64_t w = (static_cast<uint64_t>(tag) << 32) | __float_as_uint(v);
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(__attribute__((ext_vector_type(2))) unsigned int, w), r,
                                        off, 0, CPOL);
}
template <int CPOL>
__device__ __forceinline__ uint64_t ld_pair(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, CPOL));
}

template <bool VEC>
__device__ __forceinline__ void load4(const float* p, int c, int N, float (&v)[4]) {
  if (VEC) {
    const f32x4 q = c < N ? *reinterpret_cast<const f32x4*>(p + c) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = q[j];
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = c + j < N ? p[c + j] : 0.f;
  }
}

template <bool VEC>
__device__ __forceinline__ void store4(float* p, int c, int N, const float (&v)[4]) {
  if (VEC) {
    if (c < N) *reinterpret_cast<f32x4*>(p + c) = f32x4{v[0], v[1], v[2], v[3]};
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (c + j < N) p[c + j] = v[j];
  }
}

__device__ __forceinline__ float pow_f(float x, int n) {
  float r = 1.0f;
  while (n > 0) {
    if (n & 1) r *= x;
    x *= x;
    n >>= 1;
  }
  return r;
}

template <bool VEC, int CPOL>
__global__ __launch_bounds__(512) void k_ssm_scan(const float* __restrict__ a, const float* __restrict__ u,
                                                  const float* __restrict__ s0, int32_t T, int32_t N, int32_t G,
                                                  int32_t chains, uint8_t* __restrict__ ws, uint32_t ws_bytes,
                                                  int32_t spin_limit, float* __restrict__ s_out,
                                                  bf16* __restrict__ sb_out) {
  __shared__ float s_end[SSM_WAVES][SSM_GC];   // wave ends from a zero start
  __shared__ float s_term[SSM_WAVES][SSM_GC];  // the waves' terms of the tile's aggregate
  __shared__ float s_part[SSM_WAVES][SSM_GC];  // the waves' shares of the carry
  __shared__ int s_direct;                     // some wave's look-back wait ran out
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int32_t* hdr = reinterpret_cast<int32_t*>(ws);
  const uint32_t epoch =
      static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(ld_dev(hdr + 1))) & 0x3FFFFFFFu;
  if (tid == 0) s_direct = 0;
  // span-major tile order: every tile's predecessors have smaller block indices
  const int tile = static_cast<int>(blockIdx.x);
  const int span = tile / chains, chain = tile % chains;
  const int g = chain % G, b = chain / G;
  const int c = g * SSM_GC + lane * 4;
  const int ts = span * SSM_SPAN;              // first step of the tile
  const int t0 = ts + wave * SSM_LW;           // first step of this wave
  const int nw = max(0, min(SSM_LW, T - t0));  // steps of this wave
  float av[4], bv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    av[j] = c + j < N ? a[c + j] : 0.f;
    bv[j] = 1.0f - av[j];
  }
  const float* ub = u + static_cast<int64_t>(b) * T * N;
  float x[SSM_LW][4];
#pragma unroll
  for (int i = 0; i < SSM_LW; ++i) {
    if (i < nw) {
      load4<VEC>(ub + static_cast<int64_t>(t0 + i) * N, c, N, x[i]);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) x[i][j] = 0.f;
    }
  }
  float e[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < SSM_LW; ++i)
    if (i < nw) {
#pragma unroll
      for (int j = 0; j < 4; ++j) e[j] = fmaf(av[j], e[j], bv[j] * x[i][j]);
    }
  // decays: a^SSM_LW per wave, at = a^SSM_SPAN per full tile, A = a^(steps of this tile); the
  // wave's term of the aggregate e_w a^(steps after it); the carry weights at^k of its records
  const int n_tile = max(0, min(SSM_SPAN, T - ts));
  const int after = max(0, n_tile - (wave * SSM_LW + nw));
  const int m = min(span, SSM_WIN);            // aggregates folded into the carry
  const bool past = span > SSM_WIN;            // ... then the end state of the tile before them
  float pw[4], A[4], coef[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    pw[j] = pow_f(av[j], SSM_LW);
    A[j] = pow_f(av[j], n_tile);
    coef[j] = pow_f(pow_f(pw[j], SSM_WAVES), wave);
    s_end[wave][lane * 4 + j] = e[j];
    s_term[wave][lane * 4 + j] = e[j] * pow_f(av[j], after);
  }
  __syncthreads();

  // record of tile k (byte offsets): aggregate at REC*k, end state at REC*k + 8*SSM_GC; lane owns 4 pairs
  const __amdgpu_buffer_rsrc_t wsb = dev_buf(ws, ws_bytes);
  auto rec_off = [&](int k, bool end_state) {
    return static_cast<uint32_t>(SSM_HDR + static_cast<size_t>(k) * SSM_REC) + (end_state ? 8u * SSM_GC : 0u);
  };
  const uint32_t tag_agg = (epoch << 2) | SSM_AGG, tag_inc = (epoch << 2) | SSM_INC;
  float E[4] = {0.f, 0.f, 0.f, 0.f};  // the tile's end state from a zero start
#pragma unroll
  for (int j = 0; j < 4; ++j)
    for (int w = 0; w < SSM_WAVES; ++w) E[j] += s_term[w][lane * 4 + j];
  if (wave == 0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // the first tile of a chain starts from s0: its aggregate is its end state
      const float agg = (span == 0 && s0 && c + j < N) ? fmaf(A[j], s0[static_cast<int64_t>(b) * N + c + j], E[j])
                                                        : E[j];
      st_pair<CPOL>(wsb, rec_off(tile, false) + 32u * lane + 8u * j, agg, tag_agg);
    }
  }
  // carry = sum_{k < m} at^k agg[k back] (+ at^m end state [m back]); this wave takes k = wave,
  // wave + 8, ...  First a light probe, one load per record of the last pair its writer stores (lane i
  // of the wave probes the wave's record i); then every lane reads its pairs and checks their tags,
  // re-reading what is still missing.  (Polling with whole records from every wave of every tile
  // slowed the whole grid down.)
  {
    const int k = wave + SSM_WAVES * lane;
    const bool mine = lane < SSM_PER_WAVE && (k < m || (past && k == m));
    const uint32_t poff = mine ? rec_off(tile - (k + 1) * chains, k >= m) + 8u * (SSM_GC - 1) : 0u;
    const uint32_t pwant = k < m ? tag_agg : tag_inc;
    for (int spins = 0; spins < spin_limit; ++spins) {
      const bool ok = !mine || static_cast<uint32_t>(ld_pair<CPOL>(wsb, poff) >> 32) == pwant;
      if (__ballot(!ok) == 0) break;
      __builtin_amdgcn_s_sleep(4);
    }
  }
  uint32_t off[SSM_PER_WAVE], want[SSM_PER_WAVE];
  bool need[SSM_PER_WAVE];
  uint64_t q[SSM_PER_WAVE][4];
#pragma unroll
  for (int i = 0; i < SSM_PER_WAVE; ++i) {
    const int k = wave + SSM_WAVES * i;
    need[i] = k < m || (past && k == m);
    want[i] = k < m ? tag_agg : tag_inc;
    off[i] = need[i] ? rec_off(tile - (k + 1) * chains, k >= m) + 32u * lane : 0u;
    if (need[i]) {
#pragma unroll
      for (int j = 0; j < 4; ++j) q[i][j] = ld_pair<CPOL>(wsb, off[i] + 8u * j);
    }
  }
  for (int spins = 0;; ++spins) {
    bool again = false;
#pragma unroll
    for (int i = 0; i < SSM_PER_WAVE; ++i) {
      if (!need[i]) continue;
      const bool ok = static_cast<uint32_t>(q[i][0] >> 32) == want[i] && static_cast<uint32_t>(q[i][1] >> 32) == want[i] &&
                      static_cast<uint32_t>(q[i][2] >> 32) == want[i] && static_cast<uint32_t>(q[i][3] >> 32) == want[i];
      need[i] = __ballot(!ok) != 0;  // still missing somewhere in the wave
      again |= need[i];
    }
    if (!again) break;
    if (spins >= spin_limit) {
      if (lane == 0) {
        __hip_atomic_fetch_or(hdr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_direct = 1;
      }
      break;  // the tile forms its carry directly from u below
    }
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int i = 0; i < SSM_PER_WAVE; ++i)
      if (need[i]) {
#pragma unroll
        for (int j = 0; j < 4; ++j) q[i][j] = ld_pair<CPOL>(wsb, off[i] + 8u * j);
      }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float at8 = pow_f(pw[j], SSM_WAVES * SSM_WAVES);  // at^8
    float part = 0.f, cf = coef[j];
#pragma unroll
    for (int i = 0; i < SSM_PER_WAVE; ++i) {
      const int k = wave + SSM_WAVES * i;
      if (k < m || (past && k == m)) part = fmaf(cf, __uint_as_float(static_cast<uint32_t>(q[i][j])), part);
      cf *= at8;
    }
    s_part[wave][lane * 4 + j] = part;
  }
  __syncthreads();
  // a wait ran out: wave 0 forms the carry into the tile directly, a sequential scan of the steps
  // before it from s0 (or 0), and puts it where the shares were
  const bool direct = s_direct != 0 && span > 0;
  if (direct) {
    if (wave == 0) {
      float sd[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) sd[j] = (s0 && c + j < N) ? s0[static_cast<int64_t>(b) * N + c + j] : 0.f;
      for (int t = 0; t < ts; ++t) {
        float xv[4];
        load4<VEC>(ub + static_cast<int64_t>(t) * N, c, N, xv);
#pragma unroll
        for (int j = 0; j < 4; ++j) sd[j] = fmaf(av[j], sd[j], bv[j] * xv[j]);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) s_part[0][lane * 4 + j] = sd[j];
    }
    __syncthreads();
  }
  // every wave sums the shares (same order in every wave), wave 0 publishes the tile's end state,
  // and each wave carries the tile's carry through the waves before it
  float st[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float carry = 0.f;
    if (direct) {
      carry = s_part[0][lane * 4 + j];
    } else {
      for (int w = 0; w < SSM_WAVES; ++w) carry += s_part[w][lane * 4 + j];
    }
    if (span == 0) carry = (s0 && c + j < N) ? s0[static_cast<int64_t>(b) * N + c + j] : 0.f;
    if (wave == 0) st_pair<CPOL>(wsb, rec_off(tile, true) + 32u * lane + 8u * j, fmaf(A[j], carry, E[j]), tag_inc);
    for (int w = 0; w < wave; ++w) carry = fmaf(pw[j], carry, s_end[w][lane * 4 + j]);
    st[j] = carry;
  }
  if (nw > 0) {
    float* sb = s_out + static_cast<int64_t>(b) * T * N;
#pragma unroll
    for (int i = 0; i < SSM_LW; ++i) {
      if (i < nw) {
#pragma unroll
        for (int j = 0; j < 4; ++j) st[j] = fmaf(av[j], st[j], bv[j] * x[i][j]);
        store4<VEC>(sb + static_cast<int64_t>(t0 + i) * N, c, N, st);
        if (sb_out) {
          // the states rounded to bf16 as well (the token router's feature columns): one 8-byte
          // store a lane when rows are whole groups of 4
          bf16* q = sb_out + static_cast<int64_t>(b) * T * N + static_cast<int64_t>(t0 + i) * N;
          if (VEC) {
            if (c < N)
              *reinterpret_cast<bf16x4*>(q + c) = bf16x4{static_cast<bf16>(st[0]), static_cast<bf16>(st[1]),
                                                         static_cast<bf16>(st[2]), static_cast<bf16>(st[3])};
          } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
              if (c + j < N) q[c + j] = static_cast<bf16>(st[j]);
          }
        }
      }
    }
  }
  // the last tile to finish advances the epoch for the next launch (every tile of this one read it
  // at entry, and the next launch on the stream starts after this one has ended)
  if (tid == 0) {
    const int32_t done = __hip_atomic_fetch_add(hdr + 2, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (done == static_cast<int32_t>(gridDim.x) - 1) {
      st_dev(hdr + 2, 0);
      st_dev(hdr + 1, static_cast<int32_t>((epoch + 1) & 0x3FFFFFFFu));
    }
  }
}

int64_t ssm_tiles(int64_t B, int64_t T, int32_t N) { return B * cdiv(N, SSM_GC) * cdiv(T, SSM_SPAN); }

size_t ssm_workspace_bytes(int64_t B, int64_t T, int32_t N) {
  return SSM_HDR + static_cast<size_t>(ssm_tiles(B, T, N)) * SSM_REC;
}

int ssm_scan_launch(const float* a, const float* u, const float* s0, int64_t B, int64_t T, int32_t N, uint8_t* ws,
                    size_t ws_bytes, int32_t spin_limit, float* s, hipStream_t st, bf16* sb = nullptr) {
  if (B < 0 || T < 0 || N <= 0) return fail(LNG_E_ARG, "ssm_scan: bad shape");
  if (B == 0 || T == 0) return LNG_OK;
  if (T > INT32_MAX / 2 || static_cast<int64_t>(N) * T > (int64_t{1} << 40))
    return fail(LNG_E_ARG, "ssm_scan: sequence too long");
  const int64_t tiles = ssm_tiles(B, T, N);
  if (tiles > INT32_MAX || ssm_workspace_bytes(B, T, N) > UINT32_MAX) return fail(LNG_E_ARG, "ssm_scan: too many tiles");
  if (!ws || ws_bytes < ssm_workspace_bytes(B, T, N))
    return fail(LNG_E_ARG, "ssm_scan: workspace too small (lng_ssm_workspace_bytes)");
  const int32_t G = static_cast<int32_t>(cdiv(N, SSM_GC));
  const int32_t chains = static_cast<int32_t>(B * G);
  const int32_t Ti = static_cast<int32_t>(T);
  if (spin_limit < 0) return fail(LNG_E_ARG, "ssm_scan: negative spin limit");
  const uint32_t wsb = static_cast<uint32_t>(ssm_workspace_bytes(B, T, N));
  const dim3 grid(static_cast<unsigned>(tiles)), blk(512);
  if (N % 4 == 0)
    hipLaunchKernelGGL((k_ssm_scan<true, CPOL_SC1>), grid, blk, 0, st, a, u, s0, Ti, N, G, chains, ws, wsb,
                       spin_limit, s, sb);
  else
    hipLaunchKernelGGL((k_ssm_scan<false, CPOL_SC1>), grid, blk, 0, st, a, u, s0, Ti, N, G, chains, ws, wsb,
                       spin_limit, s, sb);
  return check_launch("ssm_scan");
}

// ------------------------------------------------------------------ the allocation-free entry point
// Hand-off records in a file-scope device array (zeroed when the library's code object is loaded),
// sized for SSM_STATIC_TILES tiles.  Host code reaches it only through the address that
// hipGetSymbolAddress returns for the current device, looked up on the first call on each device.
constexpr int64_t SSM_STATIC_TILES = 2048;
constexpr size_t SSM_STATIC_BYTES = SSM_HDR + SSM_STATIC_TILES * SSM_REC;  // 8.4 MB per device
static __device__ __align__(256) uint8_t scratch[SSM_STATIC_BYTES];

constexpr int SSM_MAX_DEVICES = 64;
static std::mutex g_scratch_mu;
static uint8_t* g_scratch_ptr[SSM_MAX_DEVICES];

static int scratch_of_current_device(uint8_t** ptr, int* dev) {
  if (hipGetDevice(dev) != hipSuccess || *dev < 0 || *dev >= SSM_MAX_DEVICES)
    return fail(LNG_E_HIP, "ssm_scan_static: no current HIP device");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[*dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(LNG_E_HIP, std::string("ssm_scan_static: hipGetSymbolAddress: ") + hipGetErrorString(e));
    g_scratch_ptr[*dev] = static_cast<uint8_t*>(p);
  }
  *ptr = g_scratch_ptr[*dev];
  return LNG_OK;
}

// The states of a draft tree's nodes (drafting/tree.py:153-161): node i continues from its parent's
// state, s[b, i] = a * s[b, parent[i]] + (1 - a) * u[b, i] with k_ssm_scan's step (one fmaf over
// a and (1 - a) * u), so a node's state equals the scan's along its root path.  A parent outside
// [0, i) (the root's -1) continues from s_root[b] (the state before the tree), or from zero when
// s_root is null.  One thread per (sequence, channel); the nodes run in index order, each reading
// back the parent state it wrote itself.
__global__ __launch_bounds__(256) void k_ssm_tree(const float* __restrict__ a, const float* __restrict__ u,
                                                  const float* __restrict__ s_root, const int32_t* __restrict__ parent,
                                                  int64_t B, int32_t n, int32_t N, float* __restrict__ s) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= B * N) return;
  const int64_t b = g / N;
  const int c = static_cast<int>(g - b * N);
  const float av = a[c], bv = 1.0f - av;
  const float s0 = s_root ? s_root[b * N + c] : 0.f;
  const float* ub = u + b * n * N + c;
  float* sb = s + b * n * N + c;
  for (int32_t i = 0; i < n; ++i) {
    const int32_t p = parent[i];
    const float sp = (p >= 0 && p < i) ? sb[static_cast<int64_t>(p) * N] : s0;
    sb[static_cast<int64_t>(i) * N] = fmaf(av, sp, bv * ub[static_cast<int64_t>(i) * N]);
  }
}

}  // namespace lng

using namespace lng;

extern "C" {

int lng_ssm_tree(const float* a, const float* u, const float* s_root, const int32_t* parent, int64_t B, int32_t n,
                 int32_t N, float* s, void* stream) {
  if (B < 0 || n < 0 || N <= 0) return fail(LNG_E_ARG, "ssm_tree: bad shape");
  if (B * n == 0) return LNG_OK;
  if (!a || !u || !parent || !s) return fail(LNG_E_ARG, "ssm_tree: null pointer");
  if (s == u) return fail(LNG_E_ARG, "ssm_tree: s must not alias u");
  const int64_t threads = B * N;
  hipLaunchKernelGGL(k_ssm_tree, dim3(static_cast<unsigned>(cdiv(threads, 256))), dim3(256), 0, as_stream(stream), a,
                     u, s_root, parent, B, n, N, s);
  return check_launch("ssm_tree");
}

int lng_ssm_scan_static(const float* a, const float* u, const float* s0, int64_t B, int64_t T, int32_t N, float* s,
                        void* stream) {
  if (B < 0 || T < 0 || N <= 0) return fail(LNG_E_ARG, "ssm_scan_static: bad shape");
  if (B == 0 || T == 0) return LNG_OK;
  if (ssm_tiles(B, T, N) > SSM_STATIC_TILES)
    return fail(LNG_E_ARG, "ssm_scan_static: B * ceil(N/256) * ceil(T/128) exceeds the 2048 tiles of its static "
                           "scratch; use lng_ssm_scan with a workspace");
  uint8_t* ws = nullptr;
  int dev = 0;
  if (int rc = scratch_of_current_device(&ws, &dev)) return rc;
  return ssm_scan_launch(a, u, s0, B, T, N, ws, SSM_STATIC_BYTES, SSM_SPIN_LIMIT, s, as_stream(stream));
}

int lng_ssm_scan_static_status(int32_t* status) {
  if (!status) return fail(LNG_E_ARG, "ssm_scan_static_status: null status");
  uint8_t* ws = nullptr;
  int dev = 0;
  if (int rc = scratch_of_current_device(&ws, &dev)) return rc;
  // stream-ordered behind every call on the null stream and synchronous: read, then clear, word 0
  int32_t v = 0;
  hipError_t e = hipMemcpy(&v, ws, sizeof(v), hipMemcpyDeviceToHost);
  if (e == hipSuccess && v) e = hipMemset(ws, 0, sizeof(v));
  if (e != hipSuccess) return fail(LNG_E_HIP, std::string("ssm_scan_static_status: ") + hipGetErrorString(e));
  *status = v;
  return LNG_OK;
}

size_t lng_ssm_workspace_bytes(int64_t B, int64_t T, int32_t N) {
  if (B < 0 || T < 0 || N <= 0) return 0;
  return ssm_workspace_bytes(B, T, N);
}

int lng_ssm_scan(const float* a, const float* u, const float* s0, int64_t B, int64_t T, int32_t N, void* workspace,
                 size_t workspace_bytes, float* s, void* stream) {
  return ssm_scan_launch(a, u, s0, B, T, N, static_cast<uint8_t*>(workspace), workspace_bytes, SSM_SPIN_LIMIT, s,
                         as_stream(stream));
}

int lng_ssm_scan_with_bf16(const float* a, const float* u, const float* s0, int64_t B, int64_t T, int32_t N,
                           void* workspace, size_t workspace_bytes, float* s, void* s_bf16, void* stream) {
  if (!s_bf16) return fail(LNG_E_ARG, "ssm_scan_with_bf16: null bf16 output");
  return ssm_scan_launch(a, u, s0, B, T, N, static_cast<uint8_t*>(workspace), workspace_bytes, SSM_SPIN_LIMIT, s,
                         as_stream(stream), static_cast<bf16*>(s_bf16));
}

int lng_ssm_scan_bounded(const float* a, const float* u, const float* s0, int64_t B, int64_t T, int32_t N,
                         void* workspace, size_t workspace_bytes, int32_t spin_limit, float* s, void* stream) {
  return ssm_scan_launch(a, u, s0, B, T, N, static_cast<uint8_t*>(workspace), workspace_bytes, spin_limit, s,
                         as_stream(stream));
}

}  // extern "C"
