// Internal helpers shared by the HIP translation units of libturboquant_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include <string>

#include "tq_c_api.h"

namespace tq {

// ---- host-side error plumbing ----------------------------------------------
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

#define TQ_CHECK_ARG(cond, ...)          \
  do {                                   \
    if (!(cond)) {                       \
      ::tq::set_error(__VA_ARGS__);      \
      return TQ_ERR_INVALID;             \
    }                                    \
  } while (0)

#define TQ_CHECK_HIP(expr)                                                     \
  do {                                                                         \
    hipError_t e_ = (expr);                                                    \
    if (e_ != hipSuccess) {                                                    \
      ::tq::set_error("%s failed: %s", #expr, hipGetErrorString(e_));         \
      return TQ_ERR_HIP;                                                       \
    }                                                                          \
  } while (0)

// Launch-error check after a <<<>>> launch.
#define TQ_CHECK_LAUNCH(name)                                                  \
  do {                                                                         \
    hipError_t e_ = hipGetLastError();                                         \
    if (e_ != hipSuccess) {                                                    \
      ::tq::set_error("launch of %s failed: %s", name, hipGetErrorString(e_)); \
      return TQ_ERR_HIP;                                                       \
    }                                                                          \
  } while (0)

inline bool valid_dtype(int d) { return d == TQ_F32 || d == TQ_F16 || d == TQ_BF16; }
inline size_t dtype_size(int d) { return d == TQ_F32 ? 4 : 2; }

// ---- device-side helpers ---------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Element load of a q/x tensor whose dtype is only known at run time.
__device__ __forceinline__ float load_any(const void* p, int dtype, int64_t i) {
  if (dtype == TQ_F32) return static_cast<const float*>(p)[i];
  if (dtype == TQ_F16) return __half2float(static_cast<const __half*>(p)[i]);
  return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
}

template <typename SB>
__device__ __forceinline__ float sb_to_f32(SB v);
template <>
__device__ __forceinline__ float sb_to_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ float sb_to_f32<__half>(__half v) { return __half2float(v); }

template <typename SB>
__device__ __forceinline__ SB f32_to_sb(float v);
template <>
__device__ __forceinline__ float f32_to_sb<float>(float v) { return v; }
template <>
__device__ __forceinline__ __half f32_to_sb<__half>(float v) { return __float2half_rn(v); }

// Cross-lane xor exchange inside a wave64.  Offsets < 64 only.
__device__ __forceinline__ float shfl_xor_f(float v, int off) { return __shfl_xor(v, off, 64); }
__device__ __forceinline__ uint32_t shfl_xor_u(uint32_t v, int off) {
  return static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), off, 64));
}

// v combined with its value in lane l ^ 16 or l ^ 32, in VALU: gfx950's
// v_permlane16_swap / v_permlane32_swap of v with itself leave the pair
// {v[l], v[l ^ 16]} (resp. {v[l], v[l ^ 32]}) in the two results of every
// lane (lane layout checked on hardware), with no LDS round trip.
__device__ __forceinline__ float xor16_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ int xor16_sum(int v) {
  const auto r = __builtin_amdgcn_permlane16_swap(static_cast<unsigned>(v), static_cast<unsigned>(v), false, false);
  return static_cast<int>(r[0] + r[1]);
}
__device__ __forceinline__ int xor32_sum(int v) {
  const auto r = __builtin_amdgcn_permlane32_swap(static_cast<unsigned>(v), static_cast<unsigned>(v), false, false);
  return static_cast<int>(r[0] + r[1]);
}

// Butterfly sum over aligned groups of N consecutive lanes (N <= 64), every
// lane of the group receiving the total.  Within a row of 16 lanes this uses
// DPP (quad_perm xor-1 / xor-2, half-row mirror, row mirror), which is exact
// for a butterfly because after the first two steps all lanes of a quad hold
// the same value; beyond 16 lanes it uses the permlane swaps above.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(N == 1 || N == 2 || N == 4 || N == 8 || N == 16 || N == 32 || N == 64, "N");
  if constexpr (N >= 2)
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
  if constexpr (N >= 4)
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
  if constexpr (N >= 8)
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
  if constexpr (N >= 16)
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));
  if constexpr (N >= 32) v = xor16_sum(v);
  if constexpr (N >= 64) v = xor32_sum(v);
  return v;
}

// v of lane l ^ 8 within each row of 16 lanes (DPP row_ror:8).  Every lane
// reads a lane of its own row, so no old value is needed (mov_dpp: no
// register initialised for lanes without a source).
__device__ __forceinline__ float ror8(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xF, 0xF, true));
}

// The same butterfly as a max over aligned groups of 16 lanes.
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false)));
  return fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false)));
}

// Max over aligned groups of N consecutive lanes (N = 16, 32 or 64), every
// lane of the group receiving it.
template <int N>
__device__ __forceinline__ float group_max(float v) {
  static_assert(N == 16 || N == 32 || N == 64, "N");
  v = row16_max(v);
  if constexpr (N >= 32) v = xor16_max(v);
  if constexpr (N >= 64) v = xor32_max(v);
  return v;
}

// Exact int32 sum over aligned groups of N consecutive lanes (N <= 16), the
// butterfly of group_sum.
template <int N>
__device__ __forceinline__ int group_sum_i(int v) {
  static_assert(N == 2 || N == 4 || N == 8 || N == 16, "N");
  if constexpr (N >= 2) v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
  if constexpr (N >= 4) v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
  if constexpr (N >= 8) v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);
  if constexpr (N >= 16) v += __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false);
  return v;
}

// The same butterfly over all 64 lanes for a max, and for an exact int32
// sum: four DPP steps inside each row of 16 lanes, then the two cross-row
// permlane swaps.
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false)));
  return xor32_max(xor16_max(v));
}
__device__ __forceinline__ int wave_sum_dpp(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false);
  return xor32_sum(xor16_sum(v));
}

// exp2 with -inf handled (v_exp_f32 returns 0 for -inf already; kept explicit).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

}  // namespace tq
