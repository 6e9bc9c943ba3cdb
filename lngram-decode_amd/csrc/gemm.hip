// Dense projections: y[M,N] = x[M,K] . w[N,K]^T (nn.Linear without bias).
//
// bf16 runs on MFMA (v_mfma_f32_16x16x32_bf16, fp32 accumulation): a 256-thread
// block computes a 128 (w rows) x 128 (x rows) tile, each wave a 64x64 quarter
// as 4x4 MFMA tiles, with K staged through double-buffered LDS in steps of 64.
// The MFMA "A" operand is the weight, so each lane ends up holding 4
// consecutive output channels of one token: a packed store for plain outputs,
// and exactly one route's 4 sign bits for the router epilogue.
// fp32 runs on a VALU tile kernel (the tiny fp32 layer and fp32 routers).
#include "common.h"

namespace lng {

enum { EPI_BF16 = 0, EPI_F32 = 1, EPI_ROUTER = 2 };

constexpr int GB = 128;     // block tile (both operands)
constexpr int GK = 64;      // K step per LDS stage
constexpr int GLD = GK + 8; // padded LDS row (bf16): 144 B stride, conflict-free b128 reads

template <int EPI>
__global__ __launch_bounds__(256) void k_gemm_nt_bf16(const bf16* __restrict__ W, const bf16* __restrict__ X,
                                                      int64_t N, int64_t M, int64_t K, void* __restrict__ out,
                                                      float* __restrict__ logits, void* __restrict__ codes,
                                                      int codes_dt, int64_t routes) {
  __shared__ __attribute__((aligned(16))) bf16 Ws[2][GB * GLD];
  __shared__ __attribute__((aligned(16))) bf16 Xs[2][GB * GLD];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wr = wave >> 1, wc = wave & 1;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * GB;  // weight rows (output channels)
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * GB;  // x rows (tokens)
  const int nk = static_cast<int>((K + GK - 1) / GK);

  // global -> register staging: 128 rows x 8 chunks of 16 B per operand, 4 chunks per thread
  u32x4 rw[4], rx[4];
  auto gload = [&](int kt) {
    const int64_t kb = static_cast<int64_t>(kt) * GK;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int idx = tid + c * 256;
      const int row = idx >> 3, kc = idx & 7;
      const int64_t k = kb + kc * 8;
      u32x4 z = {0u, 0u, 0u, 0u};
      rw[c] = (n0 + row < N && k < K) ? *reinterpret_cast<const u32x4*>(W + (n0 + row) * K + k) : z;
      rx[c] = (m0 + row < M && k < K) ? *reinterpret_cast<const u32x4*>(X + (m0 + row) * K + k) : z;
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int idx = tid + c * 256;
      const int row = idx >> 3, kc = idx & 7;
      *reinterpret_cast<u32x4*>(&Ws[buf][row * GLD + kc * 8]) = rw[c];
      *reinterpret_cast<u32x4*>(&Xs[buf][row * GLD + kc * 8]) = rx[c];
    }
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) gload(kt + 1);
#pragma unroll
    for (int ks = 0; ks < GK / 32; ++ks) {
      bf16x8 a[4], b[4];
      const int kof = ks * 32 + 8 * (lane >> 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[i] = *reinterpret_cast<const bf16x8*>(&Ws[cur][(wr * 64 + i * 16 + (lane & 15)) * GLD + kof]);
        b[i] = *reinterpret_cast<const bf16x8*>(&Xs[cur][(wc * 64 + i * 16 + (lane & 15)) * GLD + kof]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) sstore(cur ^ 1);
    __syncthreads();
  }

  // epilogue: lane holds out[m][n .. n+3] for n = n0 + wr*64 + i*16 + 4*(lane>>4), m = m0 + wc*64 + j*16 + lane%16
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t n = n0 + wr * 64 + i * 16 + 4 * (lane >> 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t m = m0 + wc * 64 + j * 16 + (lane & 15);
      if (m >= M) continue;
      const f32x4 v = acc[i][j];
      if (EPI == EPI_BF16) {
        bf16* o = static_cast<bf16*>(out) + m * N + n;
        if (n + 3 < N && (N & 3) == 0) {
          bf16x4 pk = {static_cast<bf16>(v[0]), static_cast<bf16>(v[1]), static_cast<bf16>(v[2]),
                       static_cast<bf16>(v[3])};
          *reinterpret_cast<bf16x4*>(o) = pk;
        } else {
          for (int e = 0; e < 4; ++e)
            if (n + e < N) o[e] = static_cast<bf16>(v[e]);
        }
      } else if (EPI == EPI_F32) {
        float* o = static_cast<float*>(out) + m * N + n;
        if (n + 3 < N && (N & 3) == 0) {
          *reinterpret_cast<f32x4*>(o) = v;
        } else {
          for (int e = 0; e < 4; ++e)
            if (n + e < N) o[e] = v[e];
        }
      } else {  // router: 4 bits per route, n is a multiple of 4
        if (n >= N) continue;
        if (logits) *reinterpret_cast<f32x4*>(logits + m * N + n) = v;
        const int code = (v[0] > 0.f ? 1 : 0) | (v[1] > 0.f ? 2 : 0) | (v[2] > 0.f ? 4 : 0) | (v[3] > 0.f ? 8 : 0);
        const int64_t r = n >> 2;
        if (codes_dt == LNG_U8)
          static_cast<uint8_t*>(codes)[m * routes + r] = static_cast<uint8_t>(code);
        else
          static_cast<int32_t*>(codes)[m * routes + r] = code;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// DMA-pipelined bf16 GEMM (K % 32 == 0): global_load_lds_dwordx4 writes each 1 KB piece of a
// tile straight into LDS (no register staging); a ring of 4 K-stages (32 wide) keeps three
// stages in flight while one is consumed.  Tile rows are 64 B (4 x 16 B pieces); piece p of
// row r is stored at slot p ^ ((r >> 2) & 3), which makes the MFMA operand reads
// (16 B per lane, 16 rows per instruction) bank-conflict free.  The DMA lane that fills a
// slot fetches the matching swizzled piece from global memory.
constexpr int DK = 32;              // K per stage
constexpr int DSLOTS = 4;           // ring depth
constexpr int DTILE = GB * DK;      // bf16 per operand tile (128 x 32)

__device__ __forceinline__ int dswz(int row, int piece) { return piece ^ ((row >> 2) & 3); }

template <int EPI>
__global__ __launch_bounds__(256, 2) void k_gemm_dma_bf16(const bf16* __restrict__ W, const bf16* __restrict__ X,
                                                          int64_t N, int64_t M, int64_t K, void* __restrict__ out,
                                                          float* __restrict__ logits, void* __restrict__ codes,
                                                          int codes_dt, int64_t routes) {
  __shared__ __attribute__((aligned(16))) bf16 ring[DSLOTS][2][DTILE];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wr = wave >> 1, wc = wave & 1;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * GB;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * GB;
  const int nk = static_cast<int>(K / DK);

  // DMA assignment: each wave fills 2 x 1 KB of each operand tile per stage (16 rows x 64 B
  // per instruction); lane -> (row, slot) and the global piece that belongs in that slot.
  const int d_row0 = wave * 32 + (lane >> 2);  // rows d_row0 and d_row0 + 16
  const int d_slot = lane & 3;
  const int64_t wrow0 = n0 + d_row0 < N ? n0 + d_row0 : N - 1;
  const int64_t wrow1 = n0 + d_row0 + 16 < N ? n0 + d_row0 + 16 : N - 1;
  const int64_t xrow0 = m0 + d_row0 < M ? m0 + d_row0 : M - 1;
  const int64_t xrow1 = m0 + d_row0 + 16 < M ? m0 + d_row0 + 16 : M - 1;
  const int p0 = dswz(d_row0, d_slot), p1 = dswz(d_row0 + 16, d_slot);
  const bf16* w0 = W + wrow0 * K + 8 * p0;
  const bf16* w1 = W + wrow1 * K + 8 * p1;
  const bf16* x0 = X + xrow0 * K + 8 * p0;
  const bf16* x1 = X + xrow1 * K + 8 * p1;
  auto issue = [&](int kt) {
    const int s = kt % DSLOTS;
    const int64_t kb = static_cast<int64_t>(kt) * DK;
    bf16* wt = &ring[s][0][wave * 32 * DK];
    bf16* xt = &ring[s][1][wave * 32 * DK];
    __builtin_amdgcn_global_load_lds(w0 + kb, (__attribute__((address_space(3))) void*)wt, 16, 0, 0);
    __builtin_amdgcn_global_load_lds(w1 + kb, (__attribute__((address_space(3))) void*)(wt + 16 * DK), 16, 0, 0);
    __builtin_amdgcn_global_load_lds(x0 + kb, (__attribute__((address_space(3))) void*)xt, 16, 0, 0);
    __builtin_amdgcn_global_load_lds(x1 + kb, (__attribute__((address_space(3))) void*)(xt + 16 * DK), 16, 0, 0);
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int s = 0; s < DSLOTS - 1 && s < nk; ++s) issue(s);
  const int rsel = lane & 15, psel = lane >> 4;
  for (int kt = 0; kt < nk; ++kt) {
    // stage kt landed: later stages may still be in flight (4 DMA ops each)
    const int ahead = nk - 1 - kt;
    if (ahead >= 2)
      asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    else if (ahead == 1)
      asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    // every wave's DMA for stage kt has landed and every wave is done reading slot
    // (kt - 1) % DSLOTS; a plain barrier (no release fence: that would wait for the
    // stages still in flight)
    __builtin_amdgcn_s_barrier();
    if (kt + DSLOTS - 1 < nk) issue(kt + DSLOTS - 1);
    const int s = kt % DSLOTS;
    bf16x8 a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ra = wr * 64 + i * 16 + rsel, rb = wc * 64 + i * 16 + rsel;
      a[i] = *reinterpret_cast<const bf16x8*>(&ring[s][0][ra * DK + 8 * dswz(ra, psel)]);
      b[i] = *reinterpret_cast<const bf16x8*>(&ring[s][1][rb * DK + 8 * dswz(rb, psel)]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
  }

#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t n = n0 + wr * 64 + i * 16 + 4 * (lane >> 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t m = m0 + wc * 64 + j * 16 + (lane & 15);
      if (m >= M) continue;
      const f32x4 v = acc[i][j];
      if (EPI == EPI_BF16) {
        bf16* o = static_cast<bf16*>(out) + m * N + n;
        if (n + 3 < N && (N & 3) == 0) {
          bf16x4 pk = {static_cast<bf16>(v[0]), static_cast<bf16>(v[1]), static_cast<bf16>(v[2]),
                       static_cast<bf16>(v[3])};
          *reinterpret_cast<bf16x4*>(o) = pk;
        } else {
          for (int e = 0; e < 4; ++e)
            if (n + e < N) o[e] = static_cast<bf16>(v[e]);
        }
      } else if (EPI == EPI_F32) {
        float* o = static_cast<float*>(out) + m * N + n;
        if (n + 3 < N && (N & 3) == 0) {
          *reinterpret_cast<f32x4*>(o) = v;
        } else {
          for (int e = 0; e < 4; ++e)
            if (n + e < N) o[e] = v[e];
        }
      } else {
        if (n >= N) continue;
        if (logits) *reinterpret_cast<f32x4*>(logits + m * N + n) = v;
        const int code = (v[0] > 0.f ? 1 : 0) | (v[1] > 0.f ? 2 : 0) | (v[2] > 0.f ? 4 : 0) | (v[3] > 0.f ? 8 : 0);
        const int64_t r = n >> 2;
        if (codes_dt == LNG_U8)
          static_cast<uint8_t*>(codes)[m * routes + r] = static_cast<uint8_t>(code);
        else
          static_cast<int32_t*>(codes)[m * routes + r] = code;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// Large-M variant: 256 (W rows) x 256 (X rows) tile, 8 waves (2 x 4, each 128 x 64), same
// DMA ring (4 stages of K = 32, 128 KB LDS, one block per CU).  Twice the MFMA work per
// stage and half the L2 traffic of the 128-tile kernel, so three stages in flight cover the
// load latency.
constexpr int GB2 = 256;
constexpr int DTILE2 = GB2 * DK;

template <int EPI>
__global__ __launch_bounds__(512, 1) void k_gemm_dma256_bf16(const bf16* __restrict__ W, const bf16* __restrict__ X,
                                                             int64_t N, int64_t M, int64_t K, void* __restrict__ out,
                                                             float* __restrict__ logits, void* __restrict__ codes,
                                                             int codes_dt, int64_t routes,
                                                             float* __restrict__ rowsq) {
  __shared__ __attribute__((aligned(16))) bf16 ring[DSLOTS][2][DTILE2];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wr = wave >> 2, wc = wave & 3;  // wave tile: W rows wr*128 .. +128, X rows wc*64 .. +64
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * GB2;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * GB2;
  const int nk = static_cast<int>(K / DK);

  // DMA: each wave fills rows wave*32 .. +32 of both tiles (2 instructions per tile per stage)
  const int d_row0 = wave * 32 + (lane >> 2);
  const int d_slot = lane & 3;
  const int p0 = dswz(d_row0, d_slot), p1 = dswz(d_row0 + 16, d_slot);
  const int64_t wrow0 = n0 + d_row0 < N ? n0 + d_row0 : N - 1;
  const int64_t wrow1 = n0 + d_row0 + 16 < N ? n0 + d_row0 + 16 : N - 1;
  const int64_t xrow0 = m0 + d_row0 < M ? m0 + d_row0 : M - 1;
  const int64_t xrow1 = m0 + d_row0 + 16 < M ? m0 + d_row0 + 16 : M - 1;
  const bf16* w0 = W + wrow0 * K + 8 * p0;
  const bf16* w1 = W + wrow1 * K + 8 * p1;
  const bf16* x0 = X + xrow0 * K + 8 * p0;
  const bf16* x1 = X + xrow1 * K + 8 * p1;
  auto issue = [&](int kt) {
    const int s = kt % DSLOTS;
    const int64_t kb = static_cast<int64_t>(kt) * DK;
    bf16* wt = &ring[s][0][wave * 32 * DK];
    bf16* xt = &ring[s][1][wave * 32 * DK];
    __builtin_amdgcn_global_load_lds(w0 + kb, (__attribute__((address_space(3))) void*)wt, 16, 0, 0);
    __builtin_amdgcn_global_load_lds(w1 + kb, (__attribute__((address_space(3))) void*)(wt + 16 * DK), 16, 0, 0);
    __builtin_amdgcn_global_load_lds(x0 + kb, (__attribute__((address_space(3))) void*)xt, 16, 0, 0);
    __builtin_amdgcn_global_load_lds(x1 + kb, (__attribute__((address_space(3))) void*)(xt + 16 * DK), 16, 0, 0);
  };

  f32x4 acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int s = 0; s < DSLOTS - 1 && s < nk; ++s) issue(s);
  const int rsel = lane & 15, psel = lane >> 4;
  for (int kt = 0; kt < nk; ++kt) {
    const int ahead = nk - 1 - kt;
    if (ahead >= 2)
      asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    else if (ahead == 1)
      asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    if (kt + DSLOTS - 1 < nk) issue(kt + DSLOTS - 1);
    const int s = kt % DSLOTS;
    bf16x8 a[8], b[4];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int ra = wr * 128 + i * 16 + rsel;
      a[i] = *reinterpret_cast<const bf16x8*>(&ring[s][0][ra * DK + 8 * dswz(ra, psel)]);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int rb = wc * 64 + j * 16 + rsel;
      b[j] = *reinterpret_cast<const bf16x8*>(&ring[s][1][rb * DK + 8 * dswz(rb, psel)]);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
  }

#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int64_t n = n0 + wr * 128 + i * 16 + 4 * (lane >> 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t m = m0 + wc * 64 + j * 16 + (lane & 15);
      if (m >= M) continue;
      const f32x4 v = acc[i][j];
      if (EPI == EPI_BF16) {
        bf16* o = static_cast<bf16*>(out) + m * N + n;
        if (n + 3 < N && (N & 3) == 0) {
          bf16x4 pk = {static_cast<bf16>(v[0]), static_cast<bf16>(v[1]), static_cast<bf16>(v[2]),
                       static_cast<bf16>(v[3])};
          *reinterpret_cast<bf16x4*>(o) = pk;
        } else {
          for (int e = 0; e < 4; ++e)
            if (n + e < N) o[e] = static_cast<bf16>(v[e]);
        }
      } else if (EPI == EPI_F32) {
        float* o = static_cast<float*>(out) + m * N + n;
        if (n + 3 < N && (N & 3) == 0) {
          *reinterpret_cast<f32x4*>(o) = v;
        } else {
          for (int e = 0; e < 4; ++e)
            if (n + e < N) o[e] = v[e];
        }
      } else {
        if (n >= N) continue;
        if (logits) *reinterpret_cast<f32x4*>(logits + m * N + n) = v;
        const int code = (v[0] > 0.f ? 1 : 0) | (v[1] > 0.f ? 2 : 0) | (v[2] > 0.f ? 4 : 0) | (v[3] > 0.f ? 8 : 0);
        const int64_t r = n >> 2;
        if (codes_dt == LNG_U8)
          static_cast<uint8_t*>(codes)[m * routes + r] = static_cast<uint8_t>(code);
        else
          static_cast<int32_t*>(codes)[m * routes + r] = code;
      }
    }
  }
  // partial sums of squares of the bf16-rounded output rows (RMSNorm statistics for a
  // following row norm): one partial per (256-wide N tile, wave row half), fixed order
  if (EPI == EPI_BF16 && rowsq) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float ps = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int64_t n = n0 + wr * 128 + i * 16 + 4 * (lane >> 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float r = static_cast<float>(static_cast<bf16>(acc[i][j][e]));
          ps = (n + e < N) ? fmaf(r, r, ps) : ps;
        }
      }
      ps += __shfl_xor(ps, 16, 64);
      ps += __shfl_xor(ps, 32, 64);
      const int64_t m = m0 + wc * 64 + j * 16 + (lane & 15);
      if (lane < 16 && m < M) rowsq[(static_cast<int64_t>(blockIdx.x) * 2 + wr) * M + m] = ps;
    }
  }
}

// ---------------------------------------------------------------------------------------
// Wide-N variant for large M and N of a few hundred (the route routers, N = 724 .. 736):
// 384 (W rows) x 128 (X rows) tile, 8 waves (4 x 2, each 96 x 64 of 16x16x32 MFMAs).  N = 736
// splits into two tiles, so 16384 tokens make 256 blocks, one per CU, where the 256 x 256 tile
// leaves a quarter of the CUs idle.  K advances 64 per stage: every row of a stage is one whole
// 128 B line, fetched by one DMA lane group (8 lanes x 16 B), in a 2-slot ring (2 x 64 KB of
// LDS): stage k + 1 is in flight while stage k is multiplied.  Piece p of row r sits at slot
// p ^ (r & 7), so the 8 rows that 8 consecutive lanes read land in 8 distinct 16 B bank groups.
// Epilogues: fp32 outputs (optional for the router) and the router's sign codes.
constexpr int WT_N = 384, WT_M = 128, WT_WN = 4, WT_WM = 2, WT_K = 64;
constexpr int WT_ROWS = WT_N + WT_M;
constexpr int WT_DPW = WT_ROWS / 8 / (WT_WN * WT_WM);  // DMA instructions (8 rows each) per wave per stage

__device__ __forceinline__ int wswz(int row, int piece) { return piece ^ (row & 7); }

// Gathered X rows (the token router of SD-B / SD-C): row m of X is
//   concat(fprev[id(m - 1), or `start` at a sequence start], fcur[id(m)], xs[m])
// over K = 2 dm + ns columns, with fprev / fcur the tabled RMSNorms of the embedding rows
// (lng_router_feature_tables: row vocab of fprev is `start`, the last row of each table is zero
// and takes every id outside [0, vocab)) and xs the bf16 SSM states [M, ns] (ns = 0: none).
// dm and ns are multiples of the 64-column K stage, so every stage reads one source.
struct XGather {
  const bf16* fprev;
  const bf16* fcur;
  const int64_t* ids;  // [M] token ids, sequences of T
  int64_t T, vocab;
  int32_t dm, ns;
};

template <int EPI, bool GATHER>
__global__ __launch_bounds__(512, 1) void k_gemm_wide_bf16(const bf16* __restrict__ W, const bf16* __restrict__ X,
                                                           int64_t N, int64_t M, int64_t K, int n_tiles,
                                                           int xcd_local, float* __restrict__ y, void* __restrict__ codes,
                                                           int codes_dt, int64_t routes, XGather xg) {
  static_assert(EPI == EPI_F32 || EPI == EPI_ROUTER, "fp32 outputs and router codes only");
  constexpr int TN = WT_N / WT_WN, TM = WT_M / WT_WM, FI = TN / 16, FJ = TM / 16;
  __shared__ __attribute__((aligned(16))) bf16 ring[2][WT_ROWS * WT_K];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wn = wave % WT_WN, wm = wave / WT_WN;
  // block -> tiles: with xcd_local, the n_tiles blocks of one X tile are dispatched to the same XCD
  // (blocks go to XCDs round-robin, block b to XCD b % 8), so the X tile comes from HBM into one L2
  const int b = static_cast<int>(blockIdx.x);
  const int slot = xcd_local ? b >> 3 : b;
  const int64_t n0 = static_cast<int64_t>(slot % n_tiles) * WT_N;
  const int64_t m0 = (static_cast<int64_t>(xcd_local ? (b & 7) * xcd_local : 0) + slot / n_tiles) * WT_M;
  const int nk = static_cast<int>(K / WT_K);
  // DMA: tile rows 0 .. WT_N-1 are W rows, the rest X rows; wave w fills rows
  // 8 * (w * WT_DPW + d) .. +8, 8 lanes (16 B pieces) per row
  // src[d]: address of the lane's piece at column 0 of its row's current source (a gathered X row:
  // of the source's first column, less that column's K offset), as an integer
  uint64_t src[WT_DPW];
  int32_t idp[WT_DPW], idc[WT_DPW];  // GATHER: table rows of the previous and the current token
  const bool x_wave = wave * WT_DPW * 8 >= WT_N;  // waves that fill X rows (uniform per wave)
#pragma unroll
  for (int d = 0; d < WT_DPW; ++d) {
    const int row = (wave * WT_DPW + d) * 8 + (lane >> 3);
    const int piece = wswz(row, lane & 7);
    if (row < WT_N) {
      const int64_t r = n0 + row < N ? n0 + row : N - 1;
      src[d] = reinterpret_cast<uint64_t>(W + r * K + 8 * piece);
    } else {
      const int64_t r = m0 + row - WT_N < M ? m0 + row - WT_N : M - 1;
      if constexpr (GATHER) {
        // a sequence start reads `start` (fprev row vocab); an id outside [0, vocab) the zero row
        const bool seq_start = r % xg.T == 0;
        const int64_t cur = xg.ids[r], prev = seq_start ? 0 : xg.ids[r - 1];
        idc[d] = static_cast<int32_t>(cur >= 0 && cur < xg.vocab ? cur : xg.vocab);
        idp[d] = static_cast<int32_t>(seq_start ? xg.vocab : (prev >= 0 && prev < xg.vocab ? prev : xg.vocab + 1));
        src[d] = reinterpret_cast<uint64_t>(xg.fprev + static_cast<int64_t>(idp[d]) * xg.dm + 8 * piece);
      } else {
        src[d] = reinterpret_cast<uint64_t>(X + r * K + 8 * piece);
      }
    }
  }
  // GATHER: at the first stage of the fcur and of the state columns, X rows switch source
  auto x_section = [&](int kt) {
    if constexpr (GATHER) {
      const int64_t kb = static_cast<int64_t>(kt) * WT_K;
      if (!x_wave || (kb != xg.dm && kb != 2 * static_cast<int64_t>(xg.dm))) return;
#pragma unroll
      for (int d = 0; d < WT_DPW; ++d) {
        const int row = (wave * WT_DPW + d) * 8 + (lane >> 3);
        const int piece = wswz(row, lane & 7);
        const int64_t r = m0 + row - WT_N < M ? m0 + row - WT_N : M - 1;
        const bf16* p = kb == xg.dm ? xg.fcur + static_cast<int64_t>(idc[d]) * xg.dm + 8 * piece
                                    : X + r * xg.ns + 8 * piece;
        src[d] = reinterpret_cast<uint64_t>(p) - static_cast<uint64_t>(kb) * sizeof(bf16);
      }
    }
  };
  auto issue = [&](int kt) {
    bf16* base = &ring[kt & 1][wave * WT_DPW * 8 * WT_K];
    const uint64_t kb = static_cast<uint64_t>(kt) * WT_K * sizeof(bf16);
#pragma unroll
    for (int d = 0; d < WT_DPW; ++d) {
      bf16* dst = base + d * 8 * WT_K;
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const bf16*>(src[d] + kb),
                                       (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
    }
  };

  f32x4 acc[FI][FJ];
#pragma unroll
  for (int i = 0; i < FI; ++i)
#pragma unroll
    for (int j = 0; j < FJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  issue(0);
  const int rsel = lane & 15, psel = lane >> 4;
  for (int kt = 0; kt < nk; ++kt) {
    // stage kt (the only one in flight) landed for this wave; the barrier makes it landed for all
    // and every wave done with slot (kt + 1) & 1, which stage kt + 1 then refills
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (kt + 1 < nk) {
      x_section(kt + 1);
      issue(kt + 1);
    }
    const bf16* st = &ring[kt & 1][0];
#pragma unroll
    for (int kk = 0; kk < WT_K / 32; ++kk) {
      bf16x8 a[FI], bv[FJ];
#pragma unroll
      for (int i = 0; i < FI; ++i) {
        const int ra = wn * TN + i * 16 + rsel;
        a[i] = *reinterpret_cast<const bf16x8*>(st + ra * WT_K + 8 * wswz(ra, 4 * kk + psel));
      }
#pragma unroll
      for (int j = 0; j < FJ; ++j) {
        const int rb = WT_N + wm * TM + j * 16 + rsel;
        bv[j] = *reinterpret_cast<const bf16x8*>(st + rb * WT_K + 8 * wswz(rb, 4 * kk + psel));
      }
#pragma unroll
      for (int i = 0; i < FI; ++i)
#pragma unroll
        for (int j = 0; j < FJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], bv[j], acc[i][j], 0, 0, 0);
    }
  }

#pragma unroll
  for (int i = 0; i < FI; ++i) {
    const int64_t n = n0 + wn * TN + i * 16 + 4 * (lane >> 4);
#pragma unroll
    for (int j = 0; j < FJ; ++j) {
      const int64_t m = m0 + wm * TM + j * 16 + (lane & 15);
      if (m >= M || n >= N) continue;
      const f32x4 v = acc[i][j];
      if (EPI == EPI_F32 || y) *reinterpret_cast<f32x4*>(y + m * N + n) = v;  // N % 4 == 0
      if (EPI == EPI_ROUTER) {
        const int code = (v[0] > 0.f ? 1 : 0) | (v[1] > 0.f ? 2 : 0) | (v[2] > 0.f ? 4 : 0) | (v[3] > 0.f ? 8 : 0);
        const int64_t r = n >> 2;
        if (codes_dt == LNG_U8)
          static_cast<uint8_t*>(codes)[m * routes + r] = static_cast<uint8_t>(code);
        else
          static_cast<int32_t*>(codes)[m * routes + r] = code;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// Projection GEMM for large M (the memory readout's query and output projections, 16384 x 1024 x
// 1024 at SB): 256 (W rows) x 256 (X rows) tiles, 8 waves in a 2 x 4 grid, each 128 x 64 of
// v_mfma_f32_32x32x16_bf16 (a lane holds 4 consecutive channels of one token per 4 registers).
//
// - K advances 64 per stage, so every tile row of a stage is one whole 128 B line; a 2-slot ring
//   (2 x 64 KB of LDS) holds stage k + 1 in flight while stage k is multiplied.  The loads are raw
//   buffer loads straight into LDS over the tile's rows (rows past N or M lie outside the buffer
//   and read as zero, so ragged edges need no clamping); piece p of row r sits at slot pswz(r, p).
// - A stage is four k16 slices; the fragments of slice s + 1 are read from LDS under the MFMAs of
//   slice s (two register sets), and the scheduling hints interleave one LDS read (or two buffer
//   loads) with each MFMA.
// - Epilogue: the accumulators go through LDS (the ring, free once every wave has left the K
//   loop) as each wave's [64 tokens][128 channels] bf16 tile, so every store instruction writes
//   four whole 256 B row pieces instead of 32 scattered 8 B pieces.  Optionally the same pass forms
//   each token's sum of squares of its bf16-rounded outputs over the wave's 128 channels: partial
//   p = 2 * (column tile) + (wave column) of row m lands at rowsq[p * M + m] (a following RMSNorm's
//   statistics, summed in that fixed order by its consumer).
// - Blocks go to the 8 XCDs round-robin; with the M tiles a multiple of 8, the N tiles of one M
//   tile run on one XCD, so that token slice is fetched into one L2.
// - XRMS (the query projection of the memory readout): every block streams its X rows over the
//   whole of K, so it also forms each row's sum of squares from the B fragments it reads
//   (v_dot2_f32_bf16 beside the MFMAs) and scales the row's outputs by rsqrt(mean(x^2) + x_eps)
//   before rounding: y = (x . w^T) / rms(x), a row RMSNorm (its weight folded into w) applied
//   without a pass over x of its own.
constexpr int PT = 256, PK = 64, P_ROWS = 2 * PT, P_STAGE = P_ROWS * PK;
constexpr int P_FN = 4, P_FM = 2;      // 32 x 32 fragments per wave: 4 (W rows) x 2 (X rows)
constexpr int P_DPW = P_ROWS / 8 / 8;  // buffer loads (8 rows each) per wave per stage
// Piece p of tile row r sits at 16 B slot p ^ (r & 7) ^ (bit 4 of r).  A ds_read_b128 is served
// in passes of 16 lanes, lanes 0-7 with 16-23 (and so on), over 256 B of banks; the 32 x 32
// fragment puts rows r and r + 16 in one pass at the same piece, which the r & 7 term alone maps to
// the same bank group (rocprofv3: 3.46 M bank-conflict cycles per launch at 16384 x 1024 x 1024,
// 0.26 M with the bit-4 term).
__device__ __forceinline__ int pswz(int r, int p) { return p ^ (r & 7) ^ ((r >> 4) & 1); }

template <bool XRMS>
__global__ __launch_bounds__(512, 1) void k_gemm_proj_bf16(const bf16* __restrict__ W, const bf16* __restrict__ X,
                                                           int64_t N, int64_t M, int64_t K, int n_tiles,
                                                           int xcd_local, bf16* __restrict__ out,
                                                           float* __restrict__ rowsq, float x_eps) {
  __shared__ __attribute__((aligned(16))) bf16 ring[2 * P_STAGE];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave & 1, wm = wave >> 1;  // wave tile: W rows wn*128 .. +128, X rows wm*64 .. +64
  const int b = static_cast<int>(blockIdx.x);
  const int slot = xcd_local ? b >> 3 : b;
  const int nt = slot % n_tiles;
  const int64_t n0 = static_cast<int64_t>(nt) * PT;
  const int64_t m0 = (static_cast<int64_t>(xcd_local ? (b & 7) * xcd_local : 0) + slot / n_tiles) * PT;
  const int nk = static_cast<int>(K / PK);

  // loads: waves 0-3 fill the W rows of a stage, waves 4-7 the X rows, 8 rows per instruction
  const bool is_w = wave < 4;
  const int row0 = (wave & 3) * P_DPW * 8 + (lane >> 3);
  const int64_t rows_left = is_w ? N - n0 : M - m0;
  const uint64_t bytes = static_cast<uint64_t>(rows_left) * K * 2;
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<bf16*>(is_w ? W + n0 * K : X + m0 * K), 0,
      static_cast<int>(bytes < 0x7fffffffull ? bytes : 0x7fffffffull), BUF_DW3);
  // instruction d covers rows row0 + 8 d (row bit 4 changes with d, so the swizzle does too)
  uint32_t voff[P_DPW];
#pragma unroll
  for (int d = 0; d < P_DPW; ++d) {
    const int r = row0 + 8 * d;
    voff[d] = static_cast<uint32_t>((r * K + 8 * pswz(r, lane & 7)) * 2);
  }
  auto issue = [&](int stage, int c) {
    bf16* dst = ring + c * P_STAGE + wave * P_DPW * 8 * PK;
#pragma unroll
    for (int d = 0; d < P_DPW; ++d)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)(dst + d * 8 * PK), 16,
                                               voff[d] + static_cast<uint32_t>(stage) * PK * 2, 0, 0, 0);
  };
  // fragment of 32 rows x 16 k: lane (r31, hi) reads row r31 at k piece 2 ks + hi (rows of one
  // fragment differ from r31 by multiples of 32, so their swizzle is r31's)
  const int r31 = lane & 31, hi = lane >> 5;
  const int a_base = (wn * 128 + r31) * PK, b_base = (PT + wm * 64 + r31) * PK;
  auto frags = [&](bf16x8* a, bf16x8* bb, int c, int ks) {
    const int off = c * P_STAGE + 8 * pswz(r31, 2 * ks + hi);
#pragma unroll
    for (int i = 0; i < P_FN; ++i) a[i] = *reinterpret_cast<const bf16x8*>(&ring[off + a_base + i * 32 * PK]);
#pragma unroll
    for (int j = 0; j < P_FM; ++j) bb[j] = *reinterpret_cast<const bf16x8*>(&ring[off + b_base + j * 32 * PK]);
  };
  f32x16 acc[P_FN][P_FM];
#pragma unroll
  for (int i = 0; i < P_FN; ++i)
#pragma unroll
    for (int j = 0; j < P_FM; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
  float xss[P_FM] = {0.f, 0.f};  // XRMS: sum of squares of this lane's k pieces of X row 32 j + r31
  auto mm = [&](const bf16x8* a, const bf16x8* bb) {
#pragma unroll
    for (int i = 0; i < P_FN; ++i)
#pragma unroll
      for (int j = 0; j < P_FM; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], bb[j], acc[i][j], 0, 0, 0);
    if (XRMS) {
#pragma unroll
      for (int j = 0; j < P_FM; ++j) {
        const bf16x2 p0 = __builtin_shufflevector(bb[j], bb[j], 0, 1), p1 = __builtin_shufflevector(bb[j], bb[j], 2, 3);
        const bf16x2 p2 = __builtin_shufflevector(bb[j], bb[j], 4, 5), p3 = __builtin_shufflevector(bb[j], bb[j], 6, 7);
        xss[j] = __builtin_amdgcn_fdot2_f32_bf16(p0, p0, xss[j], false);
        xss[j] = __builtin_amdgcn_fdot2_f32_bf16(p1, p1, xss[j], false);
        xss[j] = __builtin_amdgcn_fdot2_f32_bf16(p2, p2, xss[j], false);
        xss[j] = __builtin_amdgcn_fdot2_f32_bf16(p3, p3, xss[j], false);
      }
    }
  };
  constexpr int NR = P_FN + P_FM, NMF = P_FN * P_FM;
  auto interleave_reads = [&]() {  // one LDS read after each of the first NR MFMAs
#pragma unroll
    for (int q = 0; q < NR; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, NMF - NR, 0);
  };
  bf16x8 a0[P_FN], b0[P_FM], a1[P_FN], b1[P_FM];
  issue(0, 0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  issue(nk > 1 ? 1 : 0, 1);
  frags(a0, b0, 0, 0);
  for (int kt = 0; kt < nk; ++kt) {
    const int c = kt & 1;
    frags(a1, b1, c, 1);
    mm(a0, b0);
    interleave_reads();
    frags(a0, b0, c, 2);
    mm(a1, b1);
    interleave_reads();
    frags(a1, b1, c, 3);
    mm(a0, b0);
    interleave_reads();
    // every wave's reads of slot c are complete and stage kt + 1 has landed in slot c ^ 1
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    // stage kt + 2 into the freed slot (past the end: a reload of the last stage, never read)
    issue(kt + 2 < nk ? kt + 2 : nk - 1, c);
    frags(a0, b0, c ^ 1, 0);
    mm(a1, b1);
#pragma unroll
    for (int q = 0; q < P_DPW; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();  // every wave has left the ring

  // lane (r31, hi) holds token t = 32 j + r31 of the wave's 64 and channels 32 i + 8 g + 4 hi + e of
  // its 128; the wave's tile goes to LDS as [64][128] bf16 rows, 16 B unit u of row t at u ^ (t & 15)
  bf16* tl = ring + wave * 64 * 128;
  if (XRMS) {
#pragma unroll
    for (int j = 0; j < P_FM; ++j) {
      const float ss = xss[j] + __shfl_xor(xss[j], 32, 64);  // the other half of the row's k pieces
      const float rs = __builtin_amdgcn_rsqf(ss / static_cast<float>(K) + x_eps);
#pragma unroll
      for (int i = 0; i < P_FN; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] *= rs;
    }
  }
  float ps[P_FM] = {0.f, 0.f};
#pragma unroll
  for (int i = 0; i < P_FN; ++i)
#pragma unroll
    for (int j = 0; j < P_FM; ++j) {
      const int t = j * 32 + r31;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const bf16x4 pk = {static_cast<bf16>(acc[i][j][4 * g]), static_cast<bf16>(acc[i][j][4 * g + 1]),
                           static_cast<bf16>(acc[i][j][4 * g + 2]), static_cast<bf16>(acc[i][j][4 * g + 3])};
        if (rowsq) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float r = static_cast<float>(pk[e]);
            ps[j] = fmaf(r, r, ps[j]);
          }
        }
        const int u = (i * 4 + g) ^ (t & 15);
        *reinterpret_cast<bf16x4*>(tl + t * 128 + u * 8 + 4 * hi) = pk;
      }
    }
  if (rowsq) {
#pragma unroll
    for (int j = 0; j < P_FM; ++j) {
      const float v = ps[j] + __shfl_xor(ps[j], 32, 64);
      const int64_t m = m0 + wm * 64 + j * 32 + r31;
      if (hi == 0 && m < M) rowsq[(static_cast<int64_t>(nt) * 2 + wn) * M + m] = v;
    }
  }
  const int u = lane & 15;
  const int64_t n = n0 + wn * 128 + 8 * u;
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int t = 4 * q + (lane >> 4);
    const bf16x8 v = *reinterpret_cast<const bf16x8*>(tl + t * 128 + 8 * (u ^ (t & 15)));
    const int64_t m = m0 + wm * 64 + t;
    if (m < M && n < N) *reinterpret_cast<bf16x8*>(out + m * N + n) = v;  // N % 8 == 0
  }
}

// fp32 VALU tile GEMM: 64x64 tile per 256-thread block, 4x4 outputs per thread,
// K staged through LDS 16 at a time.  A/B element types may be float or bf16.
template <typename TA, typename TB, typename TO>
__global__ __launch_bounds__(256) void k_gemm_nt_f32(const TA* __restrict__ X, const TB* __restrict__ W, int64_t M,
                                                     int64_t N, int64_t K, TO* __restrict__ Y) {
  __shared__ float xs[16][64 + 1];
  __shared__ float ws[16][64 + 1];
  const int tid = threadIdx.x;
  const int tx = tid & 15, ty = tid >> 4;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * 64, n0 = static_cast<int64_t>(blockIdx.x) * 64;
  float acc[4][4] = {};
  for (int64_t k0 = 0; k0 < K; k0 += 16) {
    for (int e = tid; e < 16 * 64; e += 256) {
      const int r = e >> 4, kk = e & 15;
      const int64_t k = k0 + kk;
      xs[kk][r] = (m0 + r < M && k < K) ? to_f32(X[(m0 + r) * K + k]) : 0.f;
      ws[kk][r] = (n0 + r < N && k < K) ? to_f32(W[(n0 + r) * K + k]) : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      float xv[4], wv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        xv[i] = xs[kk][ty * 4 + i];
        wv[i] = ws[kk][tx * 4 + i];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(xv[i], wv[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t m = m0 + ty * 4 + i;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t n = n0 + tx * 4 + j;
      if (n < N) Y[m * N + n] = from_f32<TO>(acc[i][j]);
    }
  }
}

// ---------------------------------------------------------------------------------------
// Skinny GEMM for a few rows of X (decode steps, M <= 64): one wave per (16 columns of W, 16 rows
// of X).  K is streamed in order in rounds of SK_CH MFMA steps whose operands go straight from
// memory into registers (a 16-column tile of W at K = 1024 is 32 KB: one round trip), each step a
// 16x16x32 MFMA accumulating in K order -- per output the same instruction sequence as the tiled
// kernels above, so the results equal theirs.  The tiled kernels would run M = 8 rows on a handful
// of 128-wide blocks.  Output rows may be scattered into a cache: row(m) = (m / group) * stride +
// p0 + m % group, p0 = pos0 (+ *pos0_dev); the identity is group = M, stride = 0, p0 = 0.
constexpr int SK_CH = 32;  // MFMA steps (32 K each) per load round
constexpr int SK_MAXM = 64;

struct RowMap {
  int64_t group, stride, pos0;
  const int32_t* pos0_dev;
};

template <int EPI>
__global__ __launch_bounds__(64, 1) void k_gemm_skinny(const bf16* __restrict__ W, const bf16* __restrict__ X,
                                                       int64_t N, int64_t M, int64_t K, RowMap map,
                                                       void* __restrict__ out, float* __restrict__ logits,
                                                       void* __restrict__ codes, int codes_dt, int64_t routes) {
  const int lane = threadIdx.x;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 16, m0 = static_cast<int64_t>(blockIdx.y) * 16;
  const int rsel = lane & 15, psel = lane >> 4;
  const int64_t wr = n0 + rsel < N ? n0 + rsel : N - 1;
  const int64_t xr = m0 + rsel < M ? m0 + rsel : M - 1;
  const bf16* wp = W + wr * K + 8 * psel;
  const bf16* xp = X + xr * K + 8 * psel;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  const int nk = static_cast<int>(K / 32);
  for (int k0 = 0; k0 < nk; k0 += SK_CH) {
    const int cnt = nk - k0 < SK_CH ? nk - k0 : SK_CH;
    bf16x8 a[SK_CH], b[SK_CH];
#pragma unroll
    for (int q = 0; q < SK_CH; ++q)
      if (q < cnt) {
        a[q] = *reinterpret_cast<const bf16x8*>(wp + static_cast<int64_t>(k0 + q) * 32);
        b[q] = *reinterpret_cast<const bf16x8*>(xp + static_cast<int64_t>(k0 + q) * 32);
      }
#pragma unroll
    for (int q = 0; q < SK_CH; ++q)
      if (q < cnt) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[q], b[q], acc, 0, 0, 0);
  }
  const int64_t n = n0 + 4 * psel, m = m0 + rsel;
  if (m >= M || n >= N) return;
  const int64_t p0 = map.pos0 + (map.pos0_dev ? static_cast<int64_t>(*map.pos0_dev) : 0);
  const int64_t row = (m / map.group) * map.stride + p0 + m % map.group;
  if (EPI == EPI_BF16) {
    bf16* o = static_cast<bf16*>(out) + row * N + n;
    const bf16x4 pk = {static_cast<bf16>(acc[0]), static_cast<bf16>(acc[1]), static_cast<bf16>(acc[2]),
                       static_cast<bf16>(acc[3])};
    *reinterpret_cast<bf16x4*>(o) = pk;  // N % 16 == 0
  } else if (EPI == EPI_F32) {
    *reinterpret_cast<f32x4*>(static_cast<float*>(out) + row * N + n) = acc;
  } else {
    if (logits) *reinterpret_cast<f32x4*>(logits + m * N + n) = acc;
    const int code = (acc[0] > 0.f ? 1 : 0) | (acc[1] > 0.f ? 2 : 0) | (acc[2] > 0.f ? 4 : 0) | (acc[3] > 0.f ? 8 : 0);
    const int64_t r = n >> 2;
    if (codes_dt == LNG_U8)
      static_cast<uint8_t*>(codes)[row * routes + r] = static_cast<uint8_t>(code);
    else
      static_cast<int32_t*>(codes)[row * routes + r] = code;
  }
}

template <int EPI>
static int launch_skinny(const bf16* w, const bf16* x, int64_t N, int64_t M, int64_t K, const RowMap& map, void* out,
                         float* logits, void* codes, int codes_dt, int64_t routes, hipStream_t s) {
  const dim3 g(static_cast<unsigned>(cdiv(N, 16)), static_cast<unsigned>(cdiv(M, 16)));
  hipLaunchKernelGGL(k_gemm_skinny<EPI>, g, dim3(64), 0, s, w, x, N, M, K, map, out, logits, codes, codes_dt, routes);
  return check_launch("gemm_bf16_skinny");
}

template <int EPI>
static int launch_mfma(const bf16* w, const bf16* x, int64_t N, int64_t M, int64_t K, void* out, float* logits,
                       void* codes, int codes_dt, int64_t routes, hipStream_t s, float* rowsq = nullptr) {
  if (!rowsq && M <= SK_MAXM && K % 32 == 0 && N % 16 == 0 && (EPI != EPI_ROUTER || N % 4 == 0))
    return launch_skinny<EPI>(w, x, N, M, K, RowMap{M, 0, 0, nullptr}, out ? out : logits, logits, codes, codes_dt,
                              routes, s);
  if constexpr (EPI != EPI_BF16) {
    if (K % WT_K == 0 && M >= 4096 && N > GB2 && N <= 2 * WT_N && (N & 3) == 0) {
      const int n_tiles = static_cast<int>(cdiv(N, WT_N));
      const int64_t m_tiles = cdiv(M, WT_M);
      // X tiles per XCD when the grid divides evenly over the 8 XCDs, else 0 (plain order)
      const int xcd_local = m_tiles % 8 == 0 ? static_cast<int>(m_tiles / 8) : 0;
      const dim3 g(static_cast<unsigned>(n_tiles * m_tiles));
      hipLaunchKernelGGL((k_gemm_wide_bf16<EPI, false>), g, dim3(512), 0, s, w, x, N, M, K, n_tiles, xcd_local,
                         logits ? logits : static_cast<float*>(out), codes, codes_dt, routes, XGather{});
      return check_launch("gemm_bf16_wide");
    }
  }
  if (K % DK == 0 && (M >= 4096 || rowsq)) {
    dim3 g2(static_cast<unsigned>(cdiv(N, GB2)), static_cast<unsigned>(cdiv(M, GB2)));
    hipLaunchKernelGGL(k_gemm_dma256_bf16<EPI>, g2, dim3(512), 0, s, w, x, N, M, K, out, logits, codes, codes_dt,
                       routes, rowsq);
    return check_launch("gemm_bf16_256");
  }
  dim3 grid(static_cast<unsigned>(cdiv(N, GB)), static_cast<unsigned>(cdiv(M, GB)));
  if (K % DK == 0)
    hipLaunchKernelGGL(k_gemm_dma_bf16<EPI>, grid, dim3(256), 0, s, w, x, N, M, K, out, logits, codes, codes_dt,
                       routes);
  else
    hipLaunchKernelGGL(k_gemm_nt_bf16<EPI>, grid, dim3(256), 0, s, w, x, N, M, K, out, logits, codes, codes_dt,
                       routes);
  return check_launch("gemm_bf16");
}

// The projection kernel takes M >= 1024 (at least 4 tiles of rows), K % 64 == 0 and N % 8 == 0.
static bool proj_shape(int64_t N, int64_t M, int64_t K) { return M >= 1024 && N >= 64 && K % PK == 0 && N % 8 == 0; }

static int launch_proj(const bf16* w, const bf16* x, int64_t N, int64_t M, int64_t K, bf16* out, float* rowsq,
                       hipStream_t s, bool x_rms = false, float x_eps = 0.f) {
  const int n_tiles = static_cast<int>(cdiv(N, PT));
  const int64_t m_tiles = cdiv(M, PT);
  const int xcd_local = m_tiles % 8 == 0 ? static_cast<int>(m_tiles / 8) : 0;
  const dim3 grid(static_cast<unsigned>(n_tiles * m_tiles));
  if (x_rms)
    hipLaunchKernelGGL(k_gemm_proj_bf16<true>, grid, dim3(512), 0, s, w, x, N, M, K, n_tiles, xcd_local, out, rowsq,
                       x_eps);
  else
    hipLaunchKernelGGL(k_gemm_proj_bf16<false>, grid, dim3(512), 0, s, w, x, N, M, K, n_tiles, xcd_local, out, rowsq,
                       x_eps);
  return check_launch("gemm_bf16_proj");
}

template <typename TA, typename TB, typename TO>
static int launch_f32(const void* x, const void* w, int64_t M, int64_t N, int64_t K, void* y, hipStream_t s) {
  dim3 grid(static_cast<unsigned>(cdiv(N, 64)), static_cast<unsigned>(cdiv(M, 64)));
  hipLaunchKernelGGL((k_gemm_nt_f32<TA, TB, TO>), grid, dim3(256), 0, s, static_cast<const TA*>(x),
                     static_cast<const TB*>(w), M, N, K, static_cast<TO*>(y));
  return check_launch("gemm_f32");
}

// out[n, k] = bf16(w[n, k] * s[k]): a row RMSNorm's weight folded into the projection after it
__global__ void k_fold_columns(const bf16* __restrict__ w, const bf16* __restrict__ s, int64_t N, int64_t K,
                               bf16* __restrict__ out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= N * K) return;
  out[i] = static_cast<bf16>(static_cast<float>(w[i]) * static_cast<float>(s[i % K]));
}

// Shared entry for bf16 MFMA linears (used by other translation units).
int linear_bf16(const void* x, const void* w, int64_t M, int64_t N, int64_t K, void* y, hipStream_t s) {
  if (proj_shape(N, M, K))
    return launch_proj(static_cast<const bf16*>(w), static_cast<const bf16*>(x), N, M, K, static_cast<bf16*>(y),
                       nullptr, s);
  return launch_mfma<EPI_BF16>(static_cast<const bf16*>(w), static_cast<const bf16*>(x), N, M, K, y, nullptr,
                               nullptr, 0, 0, s);
}

}  // namespace lng

using namespace lng;

extern "C" {

int lng_fold_columns(const void* w, const void* s, int64_t N, int64_t K, void* out, void* stream) {
  if (N <= 0 || K <= 0) return fail(LNG_E_ARG, "fold_columns: bad shape");
  const int64_t n = N * K;
  hipLaunchKernelGGL(k_fold_columns, dim3(static_cast<unsigned>(cdiv(n, 256))), dim3(256), 0, as_stream(stream),
                     static_cast<const bf16*>(w), static_cast<const bf16*>(s), N, K, static_cast<bf16*>(out));
  return check_launch("fold_columns");
}

int32_t lng_linear_rowsq_partials(int64_t N) { return static_cast<int32_t>(2 * cdiv(N, GB2)); }

int lng_linear_rowsq(const void* x, const void* w, int64_t M, int64_t N, int64_t K, void* y, float* rowsq,
                     void* stream) {
  if (M < 0 || N <= 0 || K <= 0) return fail(LNG_E_ARG, "linear_rowsq: bad shape");
  if (K % DK) return fail(LNG_E_ARG, "linear_rowsq: needs K % 32 == 0");
  if (!rowsq) return fail(LNG_E_ARG, "linear_rowsq: rowsq buffer required");
  if (M == 0) return LNG_OK;
  if (proj_shape(N, M, K))
    return launch_proj(static_cast<const bf16*>(w), static_cast<const bf16*>(x), N, M, K, static_cast<bf16*>(y),
                       rowsq, as_stream(stream));
  return launch_mfma<EPI_BF16>(static_cast<const bf16*>(w), static_cast<const bf16*>(x), N, M, K, y, nullptr,
                               nullptr, 0, 0, as_stream(stream), rowsq);
}

int32_t lng_linear_rowscale_ok(int64_t M, int64_t N, int64_t K) { return proj_shape(N, M, K) ? 1 : 0; }

int lng_linear_rowscale(const void* x, const void* w, int64_t M, int64_t N, int64_t K, float eps, void* y,
                        void* stream) {
  if (M < 0 || N <= 0 || K <= 0) return fail(LNG_E_ARG, "linear_rowscale: bad shape");
  if (M == 0) return LNG_OK;
  if (!proj_shape(N, M, K))
    return fail(LNG_E_ARG, "linear_rowscale: needs M >= 1024, N >= 64, N % 8 == 0 and K % 64 == 0");
  return launch_proj(static_cast<const bf16*>(w), static_cast<const bf16*>(x), N, M, K, static_cast<bf16*>(y), nullptr,
                     as_stream(stream), true, eps);
}

int lng_linear(const void* x, const void* w, int dtype, int64_t M, int64_t N, int64_t K, void* y, void* stream) {
  if (M < 0 || N <= 0 || K <= 0) return fail(LNG_E_ARG, "linear: bad shape");
  if (M == 0) return LNG_OK;
  hipStream_t s = as_stream(stream);
  if (dtype == LNG_BF16) {
    if (K % 8) return fail(LNG_E_ARG, "linear: bf16 needs K % 8 == 0");
    return linear_bf16(x, w, M, N, K, y, s);
  }
  if (dtype == LNG_F32) return launch_f32<float, float, float>(x, w, M, N, K, y, s);
  return fail(LNG_E_DTYPE, "linear: dtype must be f32 or bf16");
}

int lng_router_codes(const void* x, int x_dtype, const void* w, int w_dtype, int64_t M, int64_t K, int64_t N,
                     int32_t bits, float* logits, void* codes, int codes_dtype, void* stream) {
  if (M < 0 || K <= 0 || N <= 0 || bits <= 0 || bits > 8 || N % bits)
    return fail(LNG_E_ARG, "router_codes: bad shape");
  if (codes && codes_dtype != LNG_U8 && codes_dtype != LNG_I32) return fail(LNG_E_DTYPE, "router_codes: codes u8/i32");
  if (!codes && !logits) return fail(LNG_E_ARG, "router_codes: nothing to write");
  if (M == 0) return LNG_OK;
  hipStream_t s = as_stream(stream);
  const int64_t routes = N / bits;
  if (x_dtype == LNG_BF16 && w_dtype == LNG_BF16 && K % 8 == 0) {
    if (codes && bits == 4)
      return launch_mfma<EPI_ROUTER>(static_cast<const bf16*>(w), static_cast<const bf16*>(x), N, M, K, nullptr,
                                     logits, codes, codes_dtype, routes, s);
    if (!logits) return fail(LNG_E_ARG, "router_codes: bits != 4 needs a logits buffer");
    if (int rc = launch_mfma<EPI_F32>(static_cast<const bf16*>(w), static_cast<const bf16*>(x), N, M, K, logits,
                                      nullptr, nullptr, 0, 0, s))
      return rc;
  } else {
    if (!logits) return fail(LNG_E_ARG, "router_codes: fp32 router needs a logits buffer");
    int rc;
    if (x_dtype == LNG_F32 && w_dtype == LNG_F32)
      rc = launch_f32<float, float, float>(x, w, M, N, K, logits, s);
    else if (x_dtype == LNG_BF16 && w_dtype == LNG_F32)
      rc = launch_f32<bf16, float, float>(x, w, M, N, K, logits, s);
    else if (x_dtype == LNG_F32 && w_dtype == LNG_BF16)
      rc = launch_f32<float, bf16, float>(x, w, M, N, K, logits, s);
    else if (x_dtype == LNG_BF16 && w_dtype == LNG_BF16)
      rc = launch_f32<bf16, bf16, float>(x, w, M, N, K, logits, s);
    else
      return fail(LNG_E_DTYPE, "router_codes: x/w must be f32 or bf16");
    if (rc) return rc;
  }
  if (!codes) return LNG_OK;
  return lng_pack_route_codes(logits, M, N, bits, codes, codes_dtype, stream);
}

int32_t lng_router_codes_ids_ok(int64_t M, int32_t d, int32_t N, int64_t n_out) {
  const int64_t K = 2 * static_cast<int64_t>(d) + N;
  return M >= 4096 && d > 0 && d % WT_K == 0 && N >= 0 && N % WT_K == 0 && n_out > GB2 && n_out <= 2 * WT_N &&
                 n_out % 4 == 0 && K <= (int64_t{1} << 20)
             ? 1
             : 0;
}

int lng_router_codes_ids(const int64_t* token_ids, int64_t vocab, int64_t B, int64_t T, const void* fprev,
                         const void* fcur, int32_t d, const void* ssm_bf16, int32_t N, const void* w, int64_t n_out,
                         float* logits, uint8_t* codes, void* stream) {
  if (!token_ids || !fprev || !fcur || !w || !codes || (N > 0) != (ssm_bf16 != nullptr))
    return fail(LNG_E_ARG, "router_codes_ids: null pointer (ssm_bf16 and N > 0 go together)");
  if (B < 0 || T <= 0 || vocab <= 0 || vocab > (int64_t{1} << 30)) return fail(LNG_E_ARG, "router_codes_ids: bad shape");
  const int64_t M = B * T;
  if (M == 0) return LNG_OK;
  if (!lng_router_codes_ids_ok(M, d, N, n_out))
    return fail(LNG_E_ARG, "router_codes_ids: needs B*T >= 4096, d and N multiples of 64, 256 < n_out <= 768, "
                           "n_out % 4 == 0 (lng_router_codes_ids_ok)");
  const int64_t K = 2 * static_cast<int64_t>(d) + N;
  const int n_tiles = static_cast<int>(cdiv(n_out, WT_N));
  const int64_t m_tiles = cdiv(M, WT_M);
  const int xcd_local = m_tiles % 8 == 0 ? static_cast<int>(m_tiles / 8) : 0;
  const dim3 g(static_cast<unsigned>(n_tiles * m_tiles));
  const XGather xg{static_cast<const bf16*>(fprev), static_cast<const bf16*>(fcur), token_ids, T, vocab, d, N};
  hipLaunchKernelGGL((k_gemm_wide_bf16<EPI_ROUTER, true>), g, dim3(512), 0, as_stream(stream),
                     static_cast<const bf16*>(w), static_cast<const bf16*>(ssm_bf16), n_out, M, K, n_tiles, xcd_local,
                     logits, codes, LNG_U8, n_out / 4, xg);
  return check_launch("router_codes_ids");
}

int lng_linear_at(const void* x, const void* w, int64_t M, int64_t N, int64_t K, int64_t group, int64_t stride,
                  int64_t pos0, const int32_t* pos0_dev, void* y, void* stream) {
  if (M < 0 || M > SK_MAXM || N <= 0 || N % 16 || K <= 0 || K % 32 || group <= 0 || M % group || pos0 < 0 ||
      stride < 0)
    return fail(LNG_E_ARG, "linear_at: bf16, M <= 64 (a multiple of group), N % 16 == 0, K % 32 == 0");
  if (M == 0) return LNG_OK;
  return launch_skinny<EPI_BF16>(static_cast<const bf16*>(w), static_cast<const bf16*>(x), N, M, K,
                                 RowMap{group, stride, pos0, pos0_dev}, y, nullptr, nullptr, 0, 0, as_stream(stream));
}

int lng_router_codes_at(const void* x, const void* w, int64_t M, int64_t K, int64_t N, int64_t group,
                        int64_t stride, int64_t pos0, const int32_t* pos0_dev, uint8_t* codes, void* stream) {
  if (M < 0 || M > SK_MAXM || N <= 0 || N % 16 || K <= 0 || K % 32 || group <= 0 || M % group || pos0 < 0 ||
      stride < 0 || !codes)
    return fail(LNG_E_ARG, "router_codes_at: bf16, 4-bit codes, M <= 64 (a multiple of group), N % 16 == 0, "
                           "K % 32 == 0");
  if (M == 0) return LNG_OK;
  return launch_skinny<EPI_ROUTER>(static_cast<const bf16*>(w), static_cast<const bf16*>(x), N, M, K,
                                   RowMap{group, stride, pos0, pos0_dev}, nullptr, nullptr, codes, LNG_U8, N / 4,
                                   as_stream(stream));
}

}  // extern "C"
