// Shared device helpers and host-side error plumbing for the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cmath>
#include <string>

#include "../../include/flashloop_amd.h"

namespace fl {

constexpr int kDim = FL_HEAD_DIM;   // channels per head
constexpr int kGroup = FL_GROUP;    // tokens per K group, channels per V group
constexpr int kRowBytes = kDim / 2; // packed bytes per token row (K or V)
constexpr int kCodeStride = FL_CODE_STRIDE;  // bytes between code rows: [K row | V row]
constexpr int kWave = 64;

// ---------------------------------------------------------------- host errors
void set_error(const std::string& msg);
void clear_error();

#define FL_REQUIRE(cond, msg)                  \
  do {                                         \
    if (!(cond)) {                             \
      ::fl::set_error(msg);                    \
      return FL_E_INVALID;                     \
    }                                          \
  } while (0)

#define FL_LAUNCH_CHECK(what)                                                   \
  do {                                                                          \
    hipError_t _e = hipGetLastError();                                          \
    if (_e != hipSuccess) {                                                     \
      ::fl::set_error(std::string(what) + ": " + hipGetErrorString(_e));       \
      return FL_E_LAUNCH;                                                       \
    }                                                                           \
  } while (0)

// ---------------------------------------------------------------- bf16
// bf16 is carried as its 16-bit pattern.  Widening is exact; narrowing rounds to
// nearest even (the rounding of torch's .to(torch.bfloat16)).
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}
__device__ __forceinline__ float bf16lo_to_f32(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi_to_f32(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t rne = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
  const uint32_t qnan = (u >> 16) | 0x0040u;  // quiet NaN, payload kept
  const bool is_nan = (u & 0x7FFFFFFFu) > 0x7F800000u;
  return static_cast<uint16_t>(is_nan ? qnan : rne);  // a select, not a branch per value
}
__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16_rne(f)); }

// fp16 bits: narrowing rounds to nearest even, with fp16 subnormals, and finite values
// beyond the fp16 range become +-inf (torch's .to(torch.float16)); widening is exact.
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// ---------------------------------------------------------------- wave reductions
// Lane exchanges use DPP (a VALU operand modifier, no LDS round trip): quad_perm for
// xor 1 / xor 2 inside a quad, row_half_mirror / row_mirror to fold 8 and 16 lanes, then
// readlane for the four 16-lane rows of the wave.
template <typename T>
__device__ __forceinline__ T shfl_xor(T v, int mask) {
  return __shfl_xor(v, mask, kWave);
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7-i within 8
constexpr int kDppMirror = 0x140;     // lane i <-> 15-i within 16

// sum over the 4 lanes of a quad, result in every lane of the quad
__device__ __forceinline__ float quad_sum(float v) {
  v += dpp<kDppXor1>(v);
  v += dpp<kDppXor2>(v);
  return v;
}
__device__ __forceinline__ float quad_min(float v) {
  v = fminf(v, dpp<kDppXor1>(v));
  return fminf(v, dpp<kDppXor2>(v));
}
__device__ __forceinline__ float quad_max(float v) {
  v = fmaxf(v, dpp<kDppXor1>(v));
  return fmaxf(v, dpp<kDppXor2>(v));
}
__device__ __forceinline__ int quad_sum_i(int v) {
  v += dpp_i<kDppXor1>(v);
  return v + dpp_i<kDppXor2>(v);
}
__device__ __forceinline__ float pair_min(float v) { return fminf(v, dpp<kDppXor1>(v)); }
__device__ __forceinline__ float pair_max(float v) { return fmaxf(v, dpp<kDppXor1>(v)); }

__device__ __forceinline__ float row_lane(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// sum / max over the whole wave, result (uniform) in every lane
__device__ __forceinline__ float wave_sum(float v) {
  v = quad_sum(v);
  v += dpp<kDppHalfMirror>(v);
  v += dpp<kDppMirror>(v);
  return (row_lane(v, 0) + row_lane(v, 16)) + (row_lane(v, 32) + row_lane(v, 48));
}
__device__ __forceinline__ float wave_max(float v) {
  v = quad_max(v);
  v = fmaxf(v, dpp<kDppHalfMirror>(v));
  v = fmaxf(v, dpp<kDppMirror>(v));
  return fmaxf(fmaxf(row_lane(v, 0), row_lane(v, 16)), fmaxf(row_lane(v, 32), row_lane(v, 48)));
}

// Workgroup barrier that orders LDS only: global loads still in flight stay in flight
// (__syncthreads also fences global memory, which drains every outstanding load).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// exp2 of a finite-or--inf argument (v_exp_f32); exp(x) = exp2(x*log2e)
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
constexpr float kLog2e = 1.4426950408889634f;


}  // namespace fl
