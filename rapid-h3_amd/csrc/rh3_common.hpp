// Shared helpers of librh3: error reporting for the C ABI, bf16 bit handling, wavefront reductions.
// gfx950 only (64-lane wavefronts). Built with -ffp-contract=off so every fp32 multiply and add
// rounds on its own; fused multiply-adds are written out as fmaf where the arithmetic calls for one.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstdio>
#include <cstdarg>
#include <string>

#include "../../include/rh3.h"

namespace rh3 {

// ---------------------------------------------------------------- host: errors
void set_error(const char* fmt, ...);
void clear_error();

#define RH3_REQUIRE(cond, ...)            \
  do {                                    \
    if (!(cond)) {                        \
      ::rh3::set_error(__VA_ARGS__);      \
      return RH3_EINVAL;                  \
    }                                     \
  } while (0)

// after a launch: any HIP error becomes RH3_ELAUNCH with its name
int launch_status(const char* what);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// ---------------------------------------------------------------- device: number formats
__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }

// fp32 -> bf16 bits, round to nearest even (inputs here are finite or +-inf; NaN maps to a quiet NaN)
__device__ __forceinline__ uint16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}
__device__ __forceinline__ float round_bf(float f) { return bf2f(f2bf(f)); }

__device__ __forceinline__ uint32_t pack_bf2(float a, float b) {
  return static_cast<uint32_t>(f2bf(a)) | (static_cast<uint32_t>(f2bf(b)) << 16);
}

// 8 bf16 in a uint4 -> 8 floats
__device__ __forceinline__ void unpack8(const uint4 r, float* v) {
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(w[i] << 16);
    v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

// round-half-even to the nearest integer of x / s as torch computes it: fp32(x / s) (IEEE division),
// then rint. The product x * inv (inv = 1/s) is within 2 ulp of the true quotient, so rint of it
// can only differ when the quotient lies within a few ulp of a half-integer; those lanes take the
// IEEE division. |x / s| <= 2^8 here, where 2^-12 is far above the error bound.
__device__ __forceinline__ float rint_div(float x, float s, float inv) {
  const float t = x * inv;
  const float n = rintf(t);
  if (fabsf(t - n) > 0.5f - 0x1p-12f) return rintf(x / s);
  return n;
}

// ---------------------------------------------------------------- device: wavefront reductions
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum_tree(float v) {  // lane distances 32, 16, ..., 1 (fixed order)
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = v + __shfl_xor(v, o, 64);
  return v;
}

}  // namespace rh3
