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

// compute units of the current device (0 if the query fails), cached per device
int device_cus();

// ---------------------------------------------------------------- device: number formats
__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }

// fp32 -> bf16 bits, round to nearest even, by the hardware conversion (v_cvt_pk_bf16_f32); the same bits as
// adding 0x7fff + lsb to the fp32 pattern for every finite value and +-inf (overflow rounds to inf); NaN maps
// to a quiet NaN
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f)); }
__device__ __forceinline__ float round_bf(float f) { return bf2f(f2bf(f)); }

__device__ __forceinline__ uint32_t pack_bf2(float a, float b) {
  const bf16x2_t v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}

// Streaming global accesses (the nontemporal hint): for data a kernel touches exactly once, so that it
// does not displace reused lines in L2 / MALL
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 ld_stream16(const void* p) {
  const u32x4_t t = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(t[0], t[1], t[2], t[3]);
}
__device__ __forceinline__ void st_stream8(void* p, uint2 v) {
  const u32x2_t t = {v.x, v.y};
  __builtin_nontemporal_store(t, reinterpret_cast<u32x2_t*>(p));
}

// Buffer-resource accesses: word 3 of a raw (stride 0) gfx9 buffer descriptor (32-bit data format), and the
// nontemporal cache policy bit. A load whose byte offset (lane offset + immediate) lies at or past the
// descriptor's size returns 0 and such a store is dropped, so a row's tail needs no branch.
constexpr int BUF_RSRC_WORD3 = 0x00020000;
constexpr int BUF_NT = 2;

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
// Butterflies over lane distances 32, 16, ..., 1: at distance d every lane combines its value with lane l ^ d's.
// The partners come from VALU lane moves, not the LDS crossbar: v_permlane32_swap / v_permlane16_swap (the two
// halves of the result are a lane's own value and its partner's), DPP row_ror:8 (l ^ 8 within a 16-lane row),
// row_half_mirror then quad_perm [3,2,1,0] (l ^ 7, then ^ 3: l ^ 4), quad_perm [2,3,0,1] (l ^ 2) and
// [1,0,3,2] (l ^ 1). The additions pair the same lanes as the shuffle butterfly, so the sums keep its bits.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, true));
}
// max(a, b) and max(m, |a|, |b|) as single instructions: fmaxf in the kernels' IEEE mode first quiets each operand
// (an extra v_max per operand), which finite values do not need
__device__ __forceinline__ float fmax_nc(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float max3_abs(float m, float a, float b) {
  float r;
  asm("v_max3_f32 %0, %1, |%2|, |%3|" : "=v"(r) : "v"(m), "v"(a), "v"(b));
  return r;
}

// Four integer-valued floats n in [-128, 127] -> their int8 codes packed in a word, low byte first. The float
// n + 1.5 * 2^23 holds n's two's-complement byte in its low 8 bits (exact for |n| < 2^22); the SDWA form of that add
// writes the low byte of its result straight into byte k of the word (dst_sel BYTE_k: the first pads the rest with
// zeros, the others keep what is there), so the packing costs no permutes.
__device__ __forceinline__ uint32_t pack4_codes(const float* n) {
  const float magic = 12582912.0f;
  uint32_t w;
  asm("v_add_f32_sdwa %0, %1, %2 dst_sel:BYTE_0 dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:DWORD"
      : "=v"(w) : "v"(n[0]), "s"(magic));
  asm("v_add_f32_sdwa %0, %1, %2 dst_sel:BYTE_1 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD"
      : "+v"(w) : "v"(n[1]), "s"(magic));
  asm("v_add_f32_sdwa %0, %1, %2 dst_sel:BYTE_2 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD"
      : "+v"(w) : "v"(n[2]), "s"(magic));
  asm("v_add_f32_sdwa %0, %1, %2 dst_sel:BYTE_3 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD"
      : "+v"(w) : "v"(n[3]), "s"(magic));
  return w;
}

// 8 int8 codes rint(x[e] / s) packed little-endian into two words. The callers' scales are max(amax / 127, floor)
// with amax = max|x|, so |x / s| <= 127 (1 + 2^-23) < 128: every code lies in [-127, 127] without a clamp. The
// product t = x * inv (inv = 1/s) is within 2^-16 of the quotient x / s and the IEEE quotient within 2^-17 of it, so
// rint(t) equals rint(fp32(x / s)) unless t lies within 2^-15 of a half-integer: one wave-wide vote per 8 values (on
// the largest |t - rint(t)|, flagged past 0.5 - 2^-14) sends only those lanes through the IEEE division, which makes
// the codes bit-identical to rint_div element by element; pack4_codes packs them.
__device__ __forceinline__ uint2 quant8_i8(const float* x, float s, float inv) {
  constexpr float NEAR_TIE = 0.5f - 0x1p-14f;
  float n[8], d = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    const float t0 = x[e] * inv, t1 = x[e + 1] * inv;
    n[e] = rintf(t0);
    n[e + 1] = rintf(t1);
    d = max3_abs(d, t0 - n[e], t1 - n[e + 1]);
  }
  if (__builtin_amdgcn_ballot_w64(d > NEAR_TIE) != 0) {
    // s passes through an empty asm here so that the division's divisor-only steps stay on this rare path
    // instead of being hoisted into the common one
    float so = s;
    asm volatile("" : "+v"(so));
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float t = x[e] * inv;
      if (fabsf(t - n[e]) > NEAR_TIE) n[e] = rintf(x[e] / so);
    }
  }
  return make_uint2(pack4_codes(n), pack4_codes(n + 4));
}

// running max of |x| over 8 bf16 held as raw words: the magnitude bits (sign cleared) order like the values, so
// two 16-bit integer maxima per word track both halves (m2 holds two bf16 magnitudes); amax_of_pair gives the float
__device__ __forceinline__ uint32_t absmax8_bf16(uint32_t m2, const uint4 r) {
  typedef short v2s __attribute__((ext_vector_type(2)));
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int i = 0; i < 4; ++i)
    m2 = __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(v2s, m2), __builtin_bit_cast(v2s, w[i] & 0x7fff7fffu)));
  return m2;
}
__device__ __forceinline__ float amax_of_pair(uint32_t m2) {
  return __uint_as_float((m2 > (m2 << 16) ? m2 : m2 << 16) & 0xffff0000u);
}

template <typename Op>
__device__ __forceinline__ float wave_butterfly(float v, Op op) {
  {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
    v = op(__int_as_float(r[0]), __int_as_float(r[1]));
  }
  {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_int(v), __float_as_int(v), false, false);
    v = op(__int_as_float(r[0]), __int_as_float(r[1]));
  }
  v = op(v, dpp_mov<0x128>(v));                   // row_ror:8
  v = op(v, dpp_mov<0x1B>(dpp_mov<0x141>(v)));    // row_half_mirror, quad_perm [3,2,1,0]
  v = op(v, dpp_mov<0x4E>(v));                    // quad_perm [2,3,0,1]
  v = op(v, dpp_mov<0xB1>(v));                    // quad_perm [1,0,3,2]
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
  return wave_butterfly(v, [](float a, float b) { return fmax_nc(a, b); });
}
__device__ __forceinline__ float wave_sum_tree(float v) {  // lane distances 32, 16, ..., 1 (fixed pairing)
  return wave_butterfly(v, [](float a, float b) { return a + b; });
}

// ---------------------------------------------------------------- device: global -> LDS copies
// Global -> LDS copy of 16 bytes per lane: lane l of the wave writes LDS byte offset lds_base + 16*l
// (M0 holds the wave-uniform base). Issued from inline assembly so that the compiler adds no wait of
// its own for it: the calling kernel accounts for these loads itself (s_waitcnt vmcnt). M0 is a reserved
// register, so the statement restores the value it found; gfx9 requires one wait state between writing M0
// and an LDS DMA that reads it.
__device__ __forceinline__ void lds_dma16(const void* gptr, uint32_t lds_base) {
  uint32_t saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off\n\t"
               "s_nop 0\n\ts_mov_b32 m0, %0"
               : "=&s"(saved)
               : "v"(gptr), "s"(lds_base)
               : "memory");
}

// The same copy addressed as a wave-uniform 64-bit base in SGPRs plus a 32-bit per-lane byte offset (the
// saddr form): a kernel that walks a tile sequence advances the base with scalar adds and keeps the lane
// offsets fixed, so the per-step address arithmetic costs no vector instructions.
__device__ __forceinline__ void lds_dma16_s(const void* sbase, uint32_t voff, uint32_t lds_base) {
  uint32_t saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2\n\t"
               "s_nop 0\n\ts_mov_b32 m0, %0"
               : "=&s"(saved)
               : "v"(voff), "s"(sbase), "s"(lds_base)
               : "memory");
}

}  // namespace rh3
