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
constexpr int kRowBytes = kDim / 2; // packed bytes per token row
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
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) {
    return static_cast<uint16_t>((u >> 16) | 0x0040u);  // quiet NaN
  }
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}
__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16_rne(f)); }

// ---------------------------------------------------------------- wave reductions
template <typename T>
__device__ __forceinline__ T shfl_xor(T v, int mask) {
  return __shfl_xor(v, mask, kWave);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += shfl_xor(v, m);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, shfl_xor(v, m));
  return v;
}

// exp2 of a finite-or--inf argument (v_exp_f32); exp(x) = exp2(x*log2e)
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
constexpr float kLog2e = 1.4426950408889634f;


}  // namespace fl
