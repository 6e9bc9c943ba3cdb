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
