// Device helpers of the attention pre-pass that other kernels reuse (the qkv GEMM epilogue): one 128-channel
// row held by 16 lanes (8 channels each, lane l16 owns channels 8*l16..8*l16+7), the per-head RMSNorm + RoPE
// prologue and the normalized 128-point Walsh-Hadamard transform.
#pragma once

#include <type_traits>

#include "rh3_common.hpp"

namespace rh3 {
namespace attn {

struct RR {
  const uint16_t* tab;  // [S][rot/2][2][2] bf16, nullptr = no RMSNorm/RoPE
  const uint16_t* w;    // [128] bf16
  float eps;
  int rot;
};

__device__ __forceinline__ void load8(const uint16_t* p, float* v) {
  unpack8(*reinterpret_cast<const uint4*>(p), v);
}

// The value of lane l ^ M (M = 1, 2, 4, 8) of the 16-lane row group, by DPP lane moves instead of the LDS crossbar:
// row_ror:8 (l ^ 8 in a 16-lane row), row_half_mirror then quad_perm [3,2,1,0] (l ^ 7, then ^ 3: l ^ 4),
// quad_perm [2,3,0,1] (l ^ 2) and [1,0,3,2] (l ^ 1)
template <int M>
__device__ __forceinline__ float xor16(float v) {
  static_assert(M == 1 || M == 2 || M == 4 || M == 8, "lane distance");
  if constexpr (M == 8) return dpp_mov<0x128>(v);
  else if constexpr (M == 4) return dpp_mov<0x1B>(dpp_mov<0x141>(v));
  else if constexpr (M == 2) return dpp_mov<0x4E>(v);
  else return dpp_mov<0xB1>(v);
}
// sum over the 16 lanes of a row group, in the butterfly order of lane distances 8, 4, 2, 1 (each lane adds its
// partner's value to its own, as x + shfl_xor(x, m) does: the same bits)
__device__ __forceinline__ float row_sum16(float v) {
  v = v + xor16<8>(v);
  v = v + xor16<4>(v);
  v = v + xor16<2>(v);
  v = v + xor16<1>(v);
  return v;
}
// integer sum over the 16 lanes of a row group (exact in any order), on the same lane moves
__device__ __forceinline__ int row_sum16_i(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x128, 0xf, 0xf, true);
  v += __builtin_amdgcn_update_dpp(0, __builtin_amdgcn_update_dpp(0, v, 0x141, 0xf, 0xf, true), 0x1B, 0xf, 0xf, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xf, 0xf, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xf, 0xf, true);
  return v;
}
// the RoPE partner of every lane's 8 channels: lane l16 + step for the first rot/2 channels, l16 - step for the next
// rot/2, the lane itself past rot (step = rot/16 lanes); rot = 128 is one DPP move (l ^ 8), other widths go through
// the LDS crossbar
__device__ __forceinline__ void rope_partner8(const float* y, float* py, int lane, int rot) {
  if (rot == 128) {
#pragma unroll
    for (int e = 0; e < 8; ++e) py[e] = xor16<8>(y[e]);
    return;
  }
  const int l16 = lane & 15, hr = rot >> 1, step = hr >> 3, c0 = 8 * l16;
  const int src = c0 < hr ? l16 + step : (c0 < rot ? l16 - step : l16);
#pragma unroll
  for (int e = 0; e < 8; ++e) py[e] = __shfl(y[e], (lane & ~15) + src, 64);
}

// Per-head RMSNorm + split-half RoPE of one 128-channel row held by 16 lanes (8 channels each,
// lane l16 owns channels 8*l16..8*l16+7). Fixed order: per-lane x*x sum over e, then xor 8,4,2,1.
__device__ __forceinline__ void rms_rope8(float* x, int lane, const RR& rr, int64_t s) {
  const int l16 = lane & 15;
  // x is a bf16 value, so x * x is exact in fp32 and fma(x, x, ss) rounds exactly as ss + x * x
  float ss = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss = fmaf(x[e], x[e], ss);
  ss = row_sum16(ss);
  const float r = 1.0f / sqrtf(ss / 128.0f + rr.eps);
  float w[8];
  load8(rr.w + 8 * l16, w);
  float y[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = round_bf((r * x[e]) * w[e]);
  const int hr = rr.rot >> 1;
  const int c0 = 8 * l16;
  float py[8];
  rope_partner8(y, py, lane, rr.rot);
  if (c0 < rr.rot) {
    const bool first = c0 < hr;
    const int i0 = first ? c0 : c0 - hr;  // rotary pair index of channel e is i0 + e
    const uint16_t* t = rr.tab + (s * hr + i0) * 4;
    float tv[32];
#pragma unroll
    for (int q = 0; q < 4; ++q) load8(t + 8 * q, tv + 8 * q);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float a = first ? y[e] : py[e];
      const float b = first ? py[e] : y[e];
      // a, b and the table are bf16 values: a * t is exact in fp32, so fma(a, t0, b * t1) rounds exactly as
      // (a * t0) + (b * t1)
      x[e] = first ? round_bf(fmaf(a, tv[4 * e + 0], b * tv[4 * e + 1]))
                   : round_bf(fmaf(a, tv[4 * e + 2], b * tv[4 * e + 3]));
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = y[e];
  }
}

// The two halves of rms_rope8 for callers that issue the loads of several rows before computing: the rope-table
// values of the lane's 8 channels for token s (lanes past rot load nothing), and the arithmetic with the norm
// weights w and those table values already in registers (the same operations in the same order).
__device__ __forceinline__ void rope_tab8(const RR& rr, int l16, int64_t s, float* tv) {
  const int hr = rr.rot >> 1, c0 = 8 * l16;
  if (c0 < rr.rot) {
    const int i0 = c0 < hr ? c0 : c0 - hr;
    const uint16_t* t = rr.tab + (s * hr + i0) * 4;
#pragma unroll
    for (int q = 0; q < 4; ++q) load8(t + 8 * q, tv + 8 * q);
  }
}

// rope_tab8 with no lane-dependent branch (lanes past rot load pair 0 of the row and ignore it), as raw bf16
// words, so that a kernel can issue the row and table loads of several tokens before any arithmetic
__device__ __forceinline__ void rope_tab8_raw(const RR& rr, int l16, int64_t s, uint4* raw) {
  const int hr = rr.rot >> 1, c0 = 8 * l16;
  const int i0 = c0 < hr ? c0 : (c0 < rr.rot ? c0 - hr : 0);
  const uint16_t* t = rr.tab + (s * hr + i0) * 4;
#pragma unroll
  for (int q = 0; q < 4; ++q) raw[q] = *reinterpret_cast<const uint4*>(t + 8 * q);
}

__device__ __forceinline__ void rms_rope8_pre(float* x, int lane, const RR& rr, const float* w, const float* tv) {
  const int l16 = lane & 15;
  // x is a bf16 value, so x * x is exact in fp32 and fma(x, x, ss) rounds exactly as ss + x * x
  float ss = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss = fmaf(x[e], x[e], ss);
  ss = row_sum16(ss);
  const float r = 1.0f / sqrtf(ss / 128.0f + rr.eps);
  float y[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = round_bf((r * x[e]) * w[e]);
  const int hr = rr.rot >> 1;
  const int c0 = 8 * l16;
  float py[8];
  rope_partner8(y, py, lane, rr.rot);
  if (c0 < rr.rot) {
    const bool first = c0 < hr;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float a = first ? y[e] : py[e];
      const float b = first ? py[e] : y[e];
      // a, b and the table are bf16 values: a * t is exact in fp32, so fma(a, t0, b * t1) rounds exactly as
      // (a * t0) + (b * t1)
      x[e] = first ? round_bf(fmaf(a, tv[4 * e + 0], b * tv[4 * e + 1]))
                   : round_bf(fmaf(a, tv[4 * e + 2], b * tv[4 * e + 3]));
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = y[e];
  }
}

// rms_rope8_pre on the raw table words of rope_tab8_raw, with no lane-dependent branch. With a, b the pair of the
// reference's formula, a first-half lane computes round_bf(a t00 + b t01) = round_bf(fma(y, t00, py t01)) and a
// second-half lane round_bf(a t10 + b t11) = round_bf(fma(y, t11, py t10)) (a = py, b = y there): every product of
// bf16 values is exact in fp32, so both forms round alike. Each lane therefore needs one coefficient pair (A, B):
// (t00, t01) from the pair's first word, (t11, t10) from its second word, (1, 0) past rot; v_perm_b32 with
// per-lane selectors moves the right bf16 halves into place, one instruction per coefficient.
__device__ __forceinline__ void rms_rope8_raw(float* x, int lane, const RR& rr, const float* w, const uint4* rt) {
  const int l16 = lane & 15;
  float ss = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss = fmaf(x[e], x[e], ss);
  ss = row_sum16(ss);
  const float r = 1.0f / sqrtf(ss / 128.0f + rr.eps);
  float y[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = round_bf((r * x[e]) * w[e]);
  const int hr = rr.rot >> 1;
  const int c0 = 8 * l16;
  const bool first = c0 < hr, rotl = c0 < rr.rot;
  float py[8];
  rope_partner8(y, py, lane, rr.rot);
  // v_perm_b32(hi, lo, sel): selector bytes 0-3 take lo's bytes, 4-7 hi's, 0x0c gives 0x00
  const uint32_t sela = first || !rotl ? 0x01000c0cu : 0x07060c0cu;  // A: lo16(word 0) or hi16(word 1)
  const uint32_t selb = first || !rotl ? 0x03020c0cu : 0x05040c0cu;  // B: hi16(word 0) or lo16(word 1)
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint4 q = rt[e >> 1];
    const uint32_t w0 = rotl ? ((e & 1) ? q.z : q.x) : 0x00003f80u;  // (1.0, 0) past rot
    const uint32_t w1 = (e & 1) ? q.w : q.y;
    const float A = __uint_as_float(__builtin_amdgcn_perm(w1, w0, sela));
    const float B = __uint_as_float(__builtin_amdgcn_perm(w1, w0, selb));
    x[e] = round_bf(fmaf(y[e], A, py[e] * B));
  }
}

// Normalized Walsh-Hadamard transform of the 16-lane row (attn_int8.cu:113-128): stages at channel strides 1,
// 2, 4 inside the lane, then 8, 16, 32, 64 (lane distances 1, 2, 4, 8), (lo, hi) -> (lo + hi, lo - hi), each
// rounded to fp32 (the reference's order), then * fp32(1 / sqrt(128)).
__device__ __forceinline__ void wht128_row(float* v, int l16) {
#pragma unroll
  for (int st = 1; st < 8; st <<= 1)
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (!(e & st)) {
        const float lo = v[e], hi = v[e + st];
        v[e] = lo + hi;
        v[e + st] = lo - hi;
      }
  auto stage = [&](auto mc) __attribute__((always_inline)) {
    constexpr int M = decltype(mc)::value;
    const bool hi = l16 & M;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float y = xor16<M>(v[e]);
      v[e] = hi ? y - v[e] : v[e] + y;
    }
  };
  stage(std::integral_constant<int, 1>{});
  stage(std::integral_constant<int, 2>{});
  stage(std::integral_constant<int, 4>{});
  stage(std::integral_constant<int, 8>{});
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = v[e] * 0.08838834764831845f;
}

// absmax of the 16-lane row (lanes of one row group)
__device__ __forceinline__ float row_amax16(const float* v) {
  float amax = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[e]));
  amax = fmaxf(amax, xor16<8>(amax));
  amax = fmaxf(amax, xor16<4>(amax));
  amax = fmaxf(amax, xor16<2>(amax));
  amax = fmaxf(amax, xor16<1>(amax));
  return amax;
}

// per-token INT8 of the 16-lane row (attn_int8.cu:157-163): sc = max(amax, 1e-8) / 127, q = rint(x * (1 / sc));
// returns sc, writes the lane's 8 codes
__device__ __forceinline__ float token_quant_row(const float* v, uint2& codes) {
  const float sc = fmaxf(row_amax16(v), 1e-8f) / 127.0f;
  const float inv = 1.0f / sc;
  uint32_t b[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) b[e] = static_cast<uint32_t>(static_cast<int32_t>(rintf(v[e] * inv))) & 0xffu;
  codes.x = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
  codes.y = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
  return sc;
}

}  // namespace attn
}  // namespace rh3
