// Shared helpers of the gfx950 kernels: status plumbing, dtype codes, bf16 and
// MFMA vector types, wave-level reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/lngram_hip.h"

namespace lng {

// ------------------------------------------------------------------ status
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
// Check the launch status of the kernel just enqueued.
int check_launch(const char* what);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ------------------------------------------------------------------ types
typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16 x) { return static_cast<float>(x); }
__device__ __forceinline__ float to_f32(_Float16 x) { return static_cast<float>(x); }

template <typename T>
__device__ __forceinline__ T from_f32(float x);
template <>
__device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float x) { return static_cast<bf16>(x); }
template <>
__device__ __forceinline__ _Float16 from_f32<_Float16>(float x) { return static_cast<_Float16>(x); }

// Round a float to the storage type and back (the reference's intermediate rounding).
template <typename T>
__device__ __forceinline__ float round_to(float x) { return to_f32(from_f32<T>(x)); }

// ------------------------------------------------------------------ wave reductions (wave64)
// Inclusive scans inside each 16-lane row with DPP row_shr:1,2,4,8 (VALU data movement, no LDS
// round trip), then the four row totals (lanes 15, 31, 47, 63) read as scalars.  Every lane
// receives the result.  Call from converged code: inactive lanes would contribute stale values.
template <int CTRL>
__device__ __forceinline__ float dpp_row_shr(float x, float identity) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, identity),
                                                                __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float lane_f(float x, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), lane));
}
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_row_shr<0x111>(v, 0.f);
  v += dpp_row_shr<0x112>(v, 0.f);
  v += dpp_row_shr<0x114>(v, 0.f);
  v += dpp_row_shr<0x118>(v, 0.f);
  return (lane_f(v, 15) + lane_f(v, 31)) + (lane_f(v, 47) + lane_f(v, 63));
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_row_shr<0x111>(v, -INFINITY));
  v = fmaxf(v, dpp_row_shr<0x112>(v, -INFINITY));
  v = fmaxf(v, dpp_row_shr<0x114>(v, -INFINITY));
  v = fmaxf(v, dpp_row_shr<0x118>(v, -INFINITY));
  return fmaxf(fmaxf(lane_f(v, 15), lane_f(v, 31)), fmaxf(lane_f(v, 47), lane_f(v, 63)));
}

// ------------------------------------------------------------------ device-coherent hand-off
// Data one block hands to another goes through the device-coherent level: agent-scope relaxed
// stores and loads (sc1 on gfx950) bypass the XCD-private L2 copies, so a hand-off needs no L2
// write-back (buffer_wbl2) in the writer and no L2 invalidate in the reader.  A writer waits until
// its coherent stores are complete (vmcnt(0)) before it publishes the flag that releases them.
__device__ __forceinline__ void st_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(int32_t* p, int32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int32_t ld_dev(const int32_t* p) {
  return __hip_atomic_load(const_cast<int32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
constexpr int WAITCNT_VM0 = 0x0F70;  // s_waitcnt vmcnt(0), expcnt and lgkmcnt left open

// 16-byte device-coherent hand-off through raw buffer operations with the sc1 cache policy (the
// policy the agent-scope relaxed loads and stores above use), one instruction per 16 bytes.
constexpr int BUF_DW3 = 0x00020000;  // raw buffer descriptor word 3 (gfx9 family)
constexpr int CPOL_NT = 2;           // cache policy bit nt (non-temporal)
constexpr int CPOL_SC1 = 16;         // cache policy bit sc1
// base and bytes must be the same in every active lane: they are taken from the first one, so the
// descriptor lives in scalar registers (a per-lane descriptor would serialise every access).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t dev_buf(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a >> 32));
  const int n = static_cast<int>(__builtin_amdgcn_readfirstlane(bytes));
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>((static_cast<uint64_t>(hi) << 32) | lo), 0, n,
                                           BUF_DW3);
}
__device__ __forceinline__ f32x4 ld_dev4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, CPOL_SC1));
}
__device__ __forceinline__ void st_dev4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, f32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, byte_off, 0, CPOL_SC1);
}


inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline int dtype_size(int dt) {
  switch (dt) {
    case LNG_F32: return 4;
    case LNG_BF16: return 2;
    case LNG_F16: return 2;
    case LNG_U8: return 1;
    case LNG_I32: return 4;
    case LNG_I64: return 8;
    default: return 0;
  }
}

}  // namespace lng
