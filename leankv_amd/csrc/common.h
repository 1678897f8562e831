// Shared helpers for the leankv_amd HIP kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "../../include/leankv_amd.h"

namespace lkv {

constexpr int kWave = 64;

// ---------------------------------------------------------------- errors
void set_error(const char* fmt, ...);

#define LKV_REQUIRE(cond, ...)                 \
  do {                                         \
    if (!(cond)) {                             \
      ::lkv::set_error(__VA_ARGS__);           \
      return LKV_ERR_INVALID;                  \
    }                                          \
  } while (0)

#define LKV_LAUNCH_CHECK(what)                                                 \
  do {                                                                         \
    hipError_t e_ = hipGetLastError();                                         \
    if (e_ != hipSuccess) {                                                    \
      ::lkv::set_error("%s: launch failed: %s", what, hipGetErrorString(e_)); \
      return LKV_ERR_HIP;                                                      \
    }                                                                          \
  } while (0)

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }

// Number of compute units of the current device (cached per device id).
int device_cu_count();

// ---------------------------------------------------------------- device helpers
__device__ __forceinline__ float h2f(uint16_t h) {
  return __half2float(__ushort_as_half(h));
}
__device__ __forceinline__ uint16_t f2h(float f) {
  return __half_as_ushort(__float2half_rn(f));
}

// Lane prefix count of set bits below this lane in a 64-bit wave mask.
__device__ __forceinline__ int lane_prefix(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0));
}

__device__ __forceinline__ uint64_t wave_ballot(bool p) {
  return __ballot(p);
}

// Every split-K workspace starts with a reserved area of kTicketBytes at
// offset 0 (no kernel reads or writes it; the partial sums and records start
// after it), so the workspace layouts and sizes stay those the C ABI reports.
constexpr size_t kTicketBytes = 64 * 1024;

// Cross-lane reductions on DPP (VALU lane permutes, no LDS round trip).
// Within a 16-lane row: xor 1, xor 2 (quad_perm), then the half-row and row
// mirrors, which pair each quad with the opposite one -- the addition tree of
// an xor-1/2/4/8 butterfly, so every lane of the row ends with the same value.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_f<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_f<0x141>(v));  // row_half_mirror
  v = fmaxf(v, dpp_f<0x140>(v));  // row_mirror
  return v;
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x141>(v);
  v += dpp_f<0x140>(v);
  return v;
}
__device__ __forceinline__ float lane_f(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
// Across the wave: the four row results combined as ((r0 + r1) + (r2 + r3)).
__device__ __forceinline__ float wave_max(float v) {
  v = row16_max(v);
  return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

}  // namespace lkv
