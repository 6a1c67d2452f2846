// Per-token activation quantizers (HBM-bound, one read of the input, one write of the codes).
//
// One 64-lane wavefront owns one row: lane l loads the 16-byte chunks at columns 512*j + 8*l
// (j = 0..NCH-1), so each load instruction of a wave covers 1 KiB of contiguous row. The row stays
// in VGPRs between the absmax and the quantize step (the reference's Triton kernels read it twice,
// triton_fp8.py:37-54). Row absmax by a wavefront butterfly; s = max(amax / QMAX, 1e-12);
// q = round_half_even(v / s) with IEEE quotient semantics (kernels.py:75-82).
//
// Prologues (triton_fp8.py:128-148):
//   KIND_PLAIN   v = x
//   KIND_SWIGLU  v = (g * sigmoid(g)) * u, x = [g | u]
//   KIND_NORMMOD v = ((x * rstd) * w) * (1 + scale[idx]) + shift[idx], rstd = 1/sqrt(sum x^2 / K + eps)
//   KIND_HEADS   v = o[k / 128][m][k % 128] (head-major attention output gathered per token)
// The RMSNorm sum of squares is accumulated per lane over (j, e) in order, then added across lanes by
// a butterfly over distances 32..1; the CPU oracle (oracle/quant.py sumsq_rows) uses the same order.
#include "rh3_common.hpp"

namespace rh3 {
namespace {

enum Kind { KIND_PLAIN = 0, KIND_SWIGLU = 1, KIND_NORMMOD = 2, KIND_HEADS = 3 };

struct QuantArgs {
  const uint16_t* x;
  int64_t ldx;       // row stride (PLAIN, SWIGLU, NORMMOD) or token stride (HEADS)
  int64_t ld_head;   // HEADS: head stride
  int64_t M, K;      // K = quantized width (SWIGLU: F; HEADS: H * 128)
  const uint16_t* w; // NORMMOD weight or nullptr
  float eps;
  const int32_t* idx;
  const void* shift;
  const void* scale;
  int64_t ld_tab;
  void* q;
  int64_t ldq;
  float* s;
};

template <typename T> __device__ __forceinline__ float tab_load(const void* p, int64_t i);
template <> __device__ __forceinline__ float tab_load<float>(const void* p, int64_t i) {
  return static_cast<const float*>(p)[i];
}
template <> __device__ __forceinline__ float tab_load<uint16_t>(const void* p, int64_t i) {
  return bf2f(static_cast<const uint16_t*>(p)[i]);
}

// 8 consecutive table values at element i (VEC: 16-byte loads; the launcher checked the alignment)
template <typename TabT, bool VEC>
__device__ __forceinline__ void tab_load8(const void* p, int64_t i, float* t) {
  if (VEC && sizeof(TabT) == 4) {
    const float4* q = reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
    const float4 u0 = q[0], u1 = q[1];
    t[0] = u0.x; t[1] = u0.y; t[2] = u0.z; t[3] = u0.w; t[4] = u1.x; t[5] = u1.y; t[6] = u1.z; t[7] = u1.w;
  } else if (VEC) {
    unpack8(*reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + i), t);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) t[e] = tab_load<TabT>(p, i + e);
  }
}

__device__ __forceinline__ float silu_mul(float g, float u) {
  const float sig = 1.0f / (1.0f + __expf(-g));
  return (g * sig) * u;
}

// OCP e4m3fn encode, round to nearest even, |t| <= 448 (the caller clamps)
__device__ __forceinline__ uint32_t fp8_e4m3(float t) {
  const uint32_t u = __float_as_uint(t);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7fffffffu;
  uint32_t code;
  if (a < 0x3c800000u) {  // |t| < 2^-6: subnormal grid step 2^-9, exact scaling then rint
    code = static_cast<uint32_t>(rintf(__uint_as_float(a) * 512.0f));
  } else {
    const uint32_t r = a + 0x7ffffu + ((a >> 20) & 1u);
    code = (r >> 20) - 960u;  // (biased exponent - 120) << 3 | top 3 mantissa bits
  }
  return code | sign;
}

// 16-byte row loads; STREAM: the row is read once (streaming hint), else it may be read again from L2
template <bool STREAM>
__device__ __forceinline__ uint4 ld_row16(const uint16_t* p) {
  if constexpr (STREAM) return ld_stream16(p);
  else return *reinterpret_cast<const uint4*>(p);
}

template <int KIND, bool STREAM = false>
__device__ __forceinline__ void load_chunk(const QuantArgs& a, int64_t m, int64_t c, float* v) {
  if (KIND == KIND_HEADS) {
    const uint16_t* p = a.x + (c >> 7) * a.ld_head + m * a.ldx + (c & 127);
    unpack8(ld_row16<STREAM>(p), v);
  } else if (KIND == KIND_SWIGLU) {
    const uint16_t* p = a.x + m * a.ldx + c;
    float g[8], u[8];
    unpack8(ld_row16<STREAM>(p), g);
    unpack8(ld_row16<STREAM>(p + a.K), u);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = silu_mul(g[e], u[e]);
  } else {
    unpack8(ld_row16<STREAM>(a.x + m * a.ldx + c), v);
  }
}

// NCH = 512-column chunks held in registers per lane (row width <= 512 * NCH). PLAIN and HEADS keep the
// raw bf16 words (4 VGPRs per 8 columns) and unpack them again for the quantization; the prologue kinds
// keep fp32 values.
template <int NCH, int KIND, bool FP8, typename TabT, bool VEC>
__global__ void __launch_bounds__(256) quant_rows_kernel(const QuantArgs a) {
  constexpr bool RAW = KIND == KIND_PLAIN || KIND == KIND_HEADS;
  const int lane = threadIdx.x & 63;
  const int64_t m = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (m >= a.M) return;
  uint4 raw[RAW ? NCH : 1];
  float v[RAW ? 1 : NCH][8];
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int64_t c = 512 * j + 8 * lane;
    if (RAW) {
      if (c < a.K) {
        const uint16_t* p = KIND == KIND_HEADS ? a.x + (c >> 7) * a.ld_head + m * a.ldx + (c & 127) : a.x + m * a.ldx + c;
        raw[j] = ld_stream16(p);
      } else {
        raw[j] = make_uint4(0, 0, 0, 0);
      }
    } else if (c < a.K) {
      load_chunk<KIND, true>(a, m, c, v[j]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[j][e] = 0.0f;
    }
  }
  auto vals = [&](int j, float* out) __attribute__((always_inline)) {
    if (RAW) unpack8(raw[j], out);
    else {
#pragma unroll
      for (int e = 0; e < 8; ++e) out[e] = v[j][e];
    }
  };
  if (KIND == KIND_NORMMOD) {
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NCH; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(v[j][e], v[j][e], ss);  // x*x exact (bf16 x): same as ss + x*x
    ss = wave_sum_tree(ss);
    const float rstd = 1.0f / sqrtf(ss / static_cast<float>(a.K) + a.eps);
    const int64_t t = static_cast<int64_t>(a.idx[m]) * a.ld_tab;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int64_t c = 512 * j + 8 * lane;
      if (c < a.K) {
        float wv[8], sc[8], sh[8];
        if (a.w) unpack8(*reinterpret_cast<const uint4*>(a.w + c), wv);
        tab_load8<TabT, VEC>(a.scale, t + c, sc);
        tab_load8<TabT, VEC>(a.shift, t + c, sh);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float y = v[j][e] * rstd;
          if (a.w) y = y * wv[e];
          v[j][e] = y * (1.0f + sc[e]) + sh[e];
        }
      }
    }
  }
  float amax = 0.0f;
  if constexpr (RAW) {  // on the raw bf16 words: magnitude bits, two per 32-bit lane
    uint32_t m2 = 0;
#pragma unroll
    for (int j = 0; j < NCH; ++j) m2 = absmax8_bf16(m2, raw[j]);
    amax = amax_of_pair(m2);
  } else {
#pragma unroll
    for (int j = 0; j < NCH; ++j)
#pragma unroll
      for (int e = 0; e < 8; e += 2) amax = max3_abs(amax, v[j][e], v[j][e + 1]);
  }
  amax = wave_max(amax);
  if (RAW) {
    // the raw words are unpacked again below rather than kept as floats (the empty asm hides the first
    // unpack from common-subexpression elimination, which would hold 8 floats per chunk live)
#pragma unroll
    for (int j = 0; j < (RAW ? NCH : 0); ++j) asm volatile("" : "+v"(raw[j].x), "+v"(raw[j].y), "+v"(raw[j].z), "+v"(raw[j].w));
  }
  const float qmax = FP8 ? 448.0f : 127.0f;
  const float s = fmaxf(amax / qmax, 1e-12f);
  const float inv = 1.0f / s;
  if (lane == 0) a.s[m] = s;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int64_t c = 512 * j + 8 * lane;
    if (c >= a.K) continue;
    float x[8];
    vals(j, x);
    uint2 out;
    if (FP8) {
      uint32_t b[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) b[e] = fp8_e4m3(fminf(fmaxf(x[e] / s, -448.0f), 448.0f));
      out.x = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
      out.y = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
    } else {
      out = quant8_i8(x, s, inv);
    }
    st_stream8(static_cast<int8_t*>(a.q) + m * a.ldq + c, out);
  }
}

// KIND_NORMMOD with the modulation rows and the norm weight staged in LDS: every token of a segment reads
// the same table row, so a workgroup copies the row of its first token once (as fp32, plus the weight) and
// each wavefront then quantizes NM_RPW rows from LDS; a row with another table index reads its values from
// global memory. Same arithmetic and order as quant_rows_kernel<NCH, KIND_NORMMOD>.
constexpr int NM_RPW = 4, NM_WAVES = 4;
static_assert(NM_RPW * NM_WAVES <= 64, "one lane per row of a workgroup holds the row's table index");
template <int NCH, typename TabT>
__global__ void __launch_bounds__(64 * NM_WAVES) quant_normmod_lds_kernel(const QuantArgs a) {
  extern __shared__ float4 nm_lds[];   // [K] 1 + scale, [K] shift, [K] weight (fp32)
  float* sc_s = reinterpret_cast<float*>(nm_lds);
  float* sh_s = sc_s + a.K;
  float* w_s = sh_s + a.K;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * NM_WAVES * NM_RPW;
  // the table indices of the workgroup's rows, one per lane (read once, so no row waits on a load of its own)
  const int32_t idx_rows = lane < NM_WAVES * NM_RPW && r0 + lane < a.M ? a.idx[r0 + lane] : 0;
  const int32_t staged = __builtin_amdgcn_readfirstlane(idx_rows);
  const int64_t t0 = static_cast<int64_t>(staged) * a.ld_tab;
  for (int64_t c = threadIdx.x * 4; c < a.K; c += 64 * NM_WAVES * 4) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      sc_s[c + e] = 1.0f + tab_load<TabT>(a.scale, t0 + c + e);  // the (1 + scale) of every token of the row
      sh_s[c + e] = tab_load<TabT>(a.shift, t0 + c + e);
    }
  }
  // without a weight the staged row is 1.0 (x * 1 is x exactly), so the row loop multiplies unconditionally
  for (int64_t c = threadIdx.x * 8; c < a.K; c += 64 * NM_WAVES * 8) {
    float wv[8] = {1, 1, 1, 1, 1, 1, 1, 1};
    if (a.w) unpack8(*reinterpret_cast<const uint4*>(a.w + c), wv);
    float4* d = reinterpret_cast<float4*>(w_s + c);
    d[0] = make_float4(wv[0], wv[1], wv[2], wv[3]);
    d[1] = make_float4(wv[4], wv[5], wv[6], wv[7]);
  }
  // Row loads and code stores go through a buffer resource per row (base = the row, size = its K elements, 0 for a
  // row past M or a load not wanted): lanes past the row end read zeros and their stores are dropped by the
  // hardware's range check, so neither needs a branch, and the lane offsets stay fixed (no per-row vector address
  // arithmetic). Every row issues its successor's load, so the loop carries the row registers without copies.
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  auto load_raw = [&](int64_t m, uint4* raw, bool want) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(a.x + m * a.ldx), 0, want && m < a.M ? static_cast<int>(a.K * 2) : 0, BUF_RSRC_WORD3);
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const u32x4_t t = __builtin_amdgcn_raw_buffer_load_b128(r, lane * 16 + j * 1024, 0, BUF_NT);
      raw[j] = make_uint4(t[0], t[1], t[2], t[3]);
    }
  };
  uint4 raw[NCH];
  load_raw(r0 + wv, raw, true);
  __syncthreads();
  for (int i = 0; i < NM_RPW; ++i) {
    const int64_t m = r0 + static_cast<int64_t>(i) * NM_WAVES + wv;
    if (m >= a.M) break;
    float v[NCH][8];
#pragma unroll
    for (int j = 0; j < NCH; ++j) unpack8(raw[j], v[j]);
    // the next row is in flight while this one is reduced and written (the last row's load reads nothing)
    load_raw(m + NM_WAVES, raw, i + 1 < NM_RPW);
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NCH; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(v[j][e], v[j][e], ss);  // x*x exact (bf16 x): same as ss + x*x
    ss = wave_sum_tree(ss);
    const float rstd = 1.0f / sqrtf(ss / static_cast<float>(a.K) + a.eps);
    const int32_t im = __builtin_amdgcn_readlane(idx_rows, i * NM_WAVES + wv);
    const int64_t t = static_cast<int64_t>(im) * a.ld_tab;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int64_t c = 512 * j + 8 * lane;
      if (c < a.K) {
        float wv[8], sc[8], sh[8];
        {
          const float4* pw = reinterpret_cast<const float4*>(w_s + c);
          const float4 w0 = pw[0], w1 = pw[1];
          wv[0] = w0.x; wv[1] = w0.y; wv[2] = w0.z; wv[3] = w0.w; wv[4] = w1.x; wv[5] = w1.y; wv[6] = w1.z; wv[7] = w1.w;
        }
        if (im == staged) {
          const float4* ps = reinterpret_cast<const float4*>(sc_s + c);
          const float4* ph = reinterpret_cast<const float4*>(sh_s + c);
          const float4 s0 = ps[0], s1 = ps[1], h0 = ph[0], h1 = ph[1];
          sc[0] = s0.x; sc[1] = s0.y; sc[2] = s0.z; sc[3] = s0.w; sc[4] = s1.x; sc[5] = s1.y; sc[6] = s1.z; sc[7] = s1.w;
          sh[0] = h0.x; sh[1] = h0.y; sh[2] = h0.z; sh[3] = h0.w; sh[4] = h1.x; sh[5] = h1.y; sh[6] = h1.z; sh[7] = h1.w;
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            sc[e] = 1.0f + tab_load<TabT>(a.scale, t + c + e);
            sh[e] = tab_load<TabT>(a.shift, t + c + e);
          }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float y = v[j][e] * rstd;
          y = y * wv[e];
          v[j][e] = y * sc[e] + sh[e];
        }
      }
    }
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < NCH; ++j)
#pragma unroll
      for (int e = 0; e < 8; e += 2) amax = max3_abs(amax, v[j][e], v[j][e + 1]);
    amax = wave_max(amax);
    const float s = fmaxf(amax / 127.0f, 1e-12f);
    const float inv = 1.0f / s;
    if (lane == 0) a.s[m] = s;
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(static_cast<int8_t*>(a.q) + m * a.ldq, 0,
                                                                       static_cast<int>(a.K), BUF_RSRC_WORD3);
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const uint2 c8 = quant8_i8(v[j], s, inv);
      const u32x2_t t = {c8.x, c8.y};
      __builtin_amdgcn_raw_buffer_store_b64(t, rq, lane * 8 + j * 512, 0, BUF_NT);
    }
  }
}

// Rows wider than 8192: same arithmetic, re-reading the row (from L2) instead of holding it.
template <int KIND, bool FP8, typename TabT, bool VEC>
__global__ void __launch_bounds__(256) quant_rows_wide_kernel(const QuantArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t m = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (m >= a.M) return;
  const int64_t nch = (a.K + 511) / 512;
  float rstd = 0.0f;
  int64_t t = 0;
  if (KIND == KIND_NORMMOD) {
    float ss = 0.0f;
    for (int64_t j = 0; j < nch; ++j) {
      const int64_t c = 512 * j + 8 * lane;
      float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      if (c < a.K) load_chunk<KIND>(a, m, c, v);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = ss + v[e] * v[e];
    }
    ss = wave_sum_tree(ss);
    rstd = 1.0f / sqrtf(ss / static_cast<float>(a.K) + a.eps);
    t = static_cast<int64_t>(a.idx[m]) * a.ld_tab;
  }
  auto value = [&](int64_t c, float* v) {
    load_chunk<KIND>(a, m, c, v);
    if (KIND == KIND_NORMMOD) {
      float wv[8], sc[8], sh[8];
      if (a.w) unpack8(*reinterpret_cast<const uint4*>(a.w + c), wv);
      tab_load8<TabT, VEC>(a.scale, t + c, sc);
      tab_load8<TabT, VEC>(a.shift, t + c, sh);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float y = v[e] * rstd;
        if (a.w) y = y * wv[e];
        v[e] = y * (1.0f + sc[e]) + sh[e];
      }
    }
  };
  float amax = 0.0f;
  for (int64_t j = 0; j < nch; ++j) {
    const int64_t c = 512 * j + 8 * lane;
    if (c >= a.K) continue;
    float v[8];
    value(c, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[e]));
  }
  amax = wave_max(amax);
  const float qmax = FP8 ? 448.0f : 127.0f;
  const float s = fmaxf(amax / qmax, 1e-12f);
  const float inv = 1.0f / s;
  if (lane == 0) a.s[m] = s;
  for (int64_t j = 0; j < nch; ++j) {
    const int64_t c = 512 * j + 8 * lane;
    if (c >= a.K) continue;
    float v[8];
    value(c, v);
    uint32_t b[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (FP8) {
        b[e] = fp8_e4m3(fminf(fmaxf(v[e] / s, -448.0f), 448.0f));
      } else {
        const float r = fminf(fmaxf(rint_div(v[e], s, inv), -127.0f), 127.0f);
        b[e] = static_cast<uint32_t>(static_cast<int32_t>(r)) & 0xffu;
      }
    }
    uint2 out;
    out.x = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
    out.y = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
    *reinterpret_cast<uint2*>(static_cast<int8_t*>(a.q) + m * a.ldq + c) = out;
  }
}

template <int KIND, bool FP8, typename TabT, bool VEC>
void launch_vec(const QuantArgs& a, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>((a.M + 3) / 4)), block(256);
  const int64_t nch = (a.K + 511) / 512;
  if (nch <= 1) hipLaunchKernelGGL((quant_rows_kernel<1, KIND, FP8, TabT, VEC>), grid, block, 0, st, a);
  else if (nch <= 2) hipLaunchKernelGGL((quant_rows_kernel<2, KIND, FP8, TabT, VEC>), grid, block, 0, st, a);
  else if (nch <= 4) hipLaunchKernelGGL((quant_rows_kernel<4, KIND, FP8, TabT, VEC>), grid, block, 0, st, a);
  else if (nch <= 6) hipLaunchKernelGGL((quant_rows_kernel<6, KIND, FP8, TabT, VEC>), grid, block, 0, st, a);
  else if (nch <= 8) hipLaunchKernelGGL((quant_rows_kernel<8, KIND, FP8, TabT, VEC>), grid, block, 0, st, a);
  else if (nch <= 12) hipLaunchKernelGGL((quant_rows_kernel<12, KIND, FP8, TabT, VEC>), grid, block, 0, st, a);
  else if (nch <= 16) hipLaunchKernelGGL((quant_rows_kernel<16, KIND, FP8, TabT, VEC>), grid, block, 0, st, a);
  else hipLaunchKernelGGL((quant_rows_wide_kernel<KIND, FP8, TabT, VEC>), grid, block, 0, st, a);
}

// Plain rows wider than 4096 columns: one workgroup per row, its 4 wavefronts taking every 4th 512-column
// chunk (at most 8 each, so the row stays in 32 VGPRs per lane and occupancy stays high); the row absmax
// goes through LDS. Same arithmetic as quant_rows_kernel<NCH, KIND_PLAIN, FP8> (max is order-free).
template <int NCHW, bool FP8>
__global__ void __launch_bounds__(256) quant_rows_split_kernel(const QuantArgs a) {
  __shared__ float wmax[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t m = blockIdx.x;
  uint4 raw[NCHW];
#pragma unroll
  for (int i = 0; i < NCHW; ++i) {
    const int64_t c = 512 * (4 * i + wave) + 8 * lane;
    raw[i] = c < a.K ? ld_stream16(a.x + m * a.ldx + c) : make_uint4(0, 0, 0, 0);
  }
  uint32_t m2 = 0;  // on the raw bf16 words: magnitude bits, two per 32-bit lane
#pragma unroll
  for (int i = 0; i < NCHW; ++i) m2 = absmax8_bf16(m2, raw[i]);
  float amax = wave_max(amax_of_pair(m2));
  if (lane == 0) wmax[wave] = amax;
  // the raw words are unpacked again below rather than kept as floats
#pragma unroll
  for (int i = 0; i < NCHW; ++i) asm volatile("" : "+v"(raw[i].x), "+v"(raw[i].y), "+v"(raw[i].z), "+v"(raw[i].w));
  __syncthreads();
  amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  const float qmax = FP8 ? 448.0f : 127.0f;
  const float s = fmaxf(amax / qmax, 1e-12f);
  const float inv = 1.0f / s;
  if (threadIdx.x == 0) a.s[m] = s;
#pragma unroll
  for (int i = 0; i < NCHW; ++i) {
    const int64_t c = 512 * (4 * i + wave) + 8 * lane;
    if (c >= a.K) continue;
    float x[8];
    unpack8(raw[i], x);
    uint2 out;
    if (FP8) {
      uint32_t b[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) b[e] = fp8_e4m3(fminf(fmaxf(x[e] / s, -448.0f), 448.0f));
      out.x = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
      out.y = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
    } else {
      out = quant8_i8(x, s, inv);
    }
    st_stream8(static_cast<int8_t*>(a.q) + m * a.ldq + c, out);
  }
}

template <int KIND, bool FP8, typename TabT>
int launch(const QuantArgs& a, hipStream_t st, const char* name) {
  if (a.M == 0) return RH3_OK;
  if (KIND == KIND_PLAIN && a.K > 4096 && a.K <= 16384 && a.M < (1ll << 31)) {
    const dim3 grid(static_cast<unsigned>(a.M)), block(256);
    if (a.K <= 8192) hipLaunchKernelGGL((quant_rows_split_kernel<4, FP8>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((quant_rows_split_kernel<8, FP8>), grid, block, 0, st, a);
    return launch_status(name);
  }
  // up to 6144 columns the staged table and weight rows fit in 72 KB of LDS
  if (KIND == KIND_NORMMOD && !FP8 && a.K <= 6144 && a.K % 8 == 0) {
    const dim3 grid(static_cast<unsigned>((a.M + NM_WAVES * NM_RPW - 1) / (NM_WAVES * NM_RPW))), block(64 * NM_WAVES);
    const size_t lds = static_cast<size_t>(a.K) * (4 + 4 + 4);
    const int64_t nch = (a.K + 511) / 512;
    if (nch <= 2) hipLaunchKernelGGL((quant_normmod_lds_kernel<2, TabT>), grid, block, lds, st, a);
    else if (nch <= 4) hipLaunchKernelGGL((quant_normmod_lds_kernel<4, TabT>), grid, block, lds, st, a);
    else if (nch <= 6) hipLaunchKernelGGL((quant_normmod_lds_kernel<6, TabT>), grid, block, lds, st, a);
    else if (nch <= 8) hipLaunchKernelGGL((quant_normmod_lds_kernel<8, TabT>), grid, block, lds, st, a);
    else hipLaunchKernelGGL((quant_normmod_lds_kernel<12, TabT>), grid, block, lds, st, a);
    return launch_status(name);
  }
  // 16-byte modulation-table loads when every table row start is 16-byte aligned
  const bool vec = KIND != KIND_NORMMOD || (aligned16(a.shift) && aligned16(a.scale) &&
                                            (a.ld_tab * static_cast<int64_t>(sizeof(TabT))) % 16 == 0);
  if (vec) launch_vec<KIND, FP8, TabT, true>(a, st);
  else launch_vec<KIND, FP8, TabT, false>(a, st);
  return launch_status(name);
}

int check_common(const void* x, int64_t M, int64_t K, const void* q, int64_t ldq, const float* s) {
  RH3_REQUIRE(M >= 0 && K >= 0, "quant: negative size (M=%lld, K=%lld)", (long long)M, (long long)K);
  RH3_REQUIRE(K % 8 == 0, "quant: K=%lld must be a multiple of 8", (long long)K);
  if (M == 0) return RH3_OK;
  RH3_REQUIRE(K > 0, "quant: K must be positive");
  RH3_REQUIRE(x && q && s, "quant: null pointer");
  RH3_REQUIRE(ldq >= K && ldq % 8 == 0, "quant: output row stride %lld (K=%lld) must be >= K and a multiple of 8",
              (long long)ldq, (long long)K);
  RH3_REQUIRE(aligned16(x) && (reinterpret_cast<uintptr_t>(q) & 7) == 0, "quant: x must be 16-byte and q 8-byte aligned");
  return RH3_OK;
}

}  // namespace
}  // namespace rh3

using namespace rh3;

extern "C" int rh3_quant_rows_i8(const uint16_t* x, int64_t ldx, int64_t M, int64_t K, int8_t* q, int64_t ldq,
                                 float* s, hipStream_t stream) {
  clear_error();
  if (int e = check_common(x, M, K, q, ldq, s)) return e;
  RH3_REQUIRE(M == 0 || (ldx >= K && ldx % 8 == 0), "quant_rows_i8: row stride %lld invalid for K=%lld",
              (long long)ldx, (long long)K);
  QuantArgs a{x, ldx, 0, M, K, nullptr, 0.f, nullptr, nullptr, nullptr, 0, q, ldq, s};
  return launch<KIND_PLAIN, false, float>(a, stream, "quant_rows_i8");
}

extern "C" int rh3_quant_rows_fp8(const uint16_t* x, int64_t ldx, int64_t M, int64_t K, uint8_t* q, int64_t ldq,
                                  float* s, hipStream_t stream) {
  clear_error();
  if (int e = check_common(x, M, K, q, ldq, s)) return e;
  RH3_REQUIRE(M == 0 || (ldx >= K && ldx % 8 == 0), "quant_rows_fp8: row stride %lld invalid for K=%lld",
              (long long)ldx, (long long)K);
  QuantArgs a{x, ldx, 0, M, K, nullptr, 0.f, nullptr, nullptr, nullptr, 0, q, ldq, s};
  return launch<KIND_PLAIN, true, float>(a, stream, "quant_rows_fp8");
}

extern "C" int rh3_quant_norm_mod_i8(const uint16_t* x, int64_t ldx, int64_t M, int64_t K, const uint16_t* weight,
                                     float eps, const int32_t* idx, const void* shift, const void* scale,
                                     int tab_dtype, int64_t ld_tab, int8_t* q, int64_t ldq, float* s,
                                     hipStream_t stream) {
  clear_error();
  if (int e = check_common(x, M, K, q, ldq, s)) return e;
  if (M == 0) return RH3_OK;
  RH3_REQUIRE(ldx >= K && ldx % 8 == 0, "quant_norm_mod_i8: row stride %lld invalid for K=%lld", (long long)ldx,
              (long long)K);
  RH3_REQUIRE(idx && shift && scale, "quant_norm_mod_i8: idx, shift and scale are required");
  RH3_REQUIRE(ld_tab >= K, "quant_norm_mod_i8: table row stride %lld < K=%lld", (long long)ld_tab, (long long)K);
  RH3_REQUIRE(!weight || aligned16(weight), "quant_norm_mod_i8: weight must be 16-byte aligned");
  RH3_REQUIRE(tab_dtype == RH3_DTYPE_F32 || tab_dtype == RH3_DTYPE_BF16, "quant_norm_mod_i8: tab_dtype %d",
              tab_dtype);
  QuantArgs a{x, ldx, 0, M, K, weight, eps, idx, shift, scale, ld_tab, q, ldq, s};
  if (tab_dtype == RH3_DTYPE_F32) return launch<KIND_NORMMOD, false, float>(a, stream, "quant_norm_mod_i8");
  return launch<KIND_NORMMOD, false, uint16_t>(a, stream, "quant_norm_mod_i8");
}

extern "C" int rh3_quant_heads_i8(const uint16_t* o, int64_t H, int64_t M, int64_t ld_head, int64_t ld_row,
                                  int8_t* q, int64_t ldq, float* s, hipStream_t stream) {
  clear_error();
  RH3_REQUIRE(H > 0, "quant_heads_i8: H=%lld", (long long)H);
  if (int e = check_common(o, M, H * 128, q, ldq, s)) return e;
  if (M == 0) return RH3_OK;
  RH3_REQUIRE(ld_head % 8 == 0 && ld_row % 8 == 0 && ld_row >= 0 && ld_head >= 0,
              "quant_heads_i8: strides must be multiples of 8 elements");
  QuantArgs a{o, ld_row, ld_head, M, H * 128, nullptr, 0.f, nullptr, nullptr, nullptr, 0, q, ldq, s};
  return launch<KIND_HEADS, false, float>(a, stream, "quant_heads_i8");
}

extern "C" int rh3_quant_swiglu_i8(const uint16_t* x, int64_t ldx, int64_t M, int64_t F, int8_t* q, int64_t ldq,
                                   float* s, hipStream_t stream) {
  clear_error();
  if (int e = check_common(x, M, F, q, ldq, s)) return e;
  if (M == 0) return RH3_OK;
  RH3_REQUIRE(ldx >= 2 * F && ldx % 8 == 0, "quant_swiglu_i8: row stride %lld invalid for 2F=%lld", (long long)ldx,
              (long long)(2 * F));
  QuantArgs a{x, ldx, 0, M, F, nullptr, 0.f, nullptr, nullptr, nullptr, 0, q, ldq, s};
  return launch<KIND_SWIGLU, false, float>(a, stream, "quant_swiglu_i8");
}

// ---------------------------------------------------------------- NVFP4 round trip (verification modes)
namespace rh3 {
namespace {

// |x| max of the whole [M, K] tensor into *amax (non-negative floats order like their bit patterns, so an
// unsigned atomic max is exact and order-free); *amax is zeroed by fill_zero_kernel first
template <typename T>
__global__ void __launch_bounds__(256) absmax_kernel(const T* __restrict__ x, int64_t ldx, int64_t M, int64_t K,
                                                     unsigned int* __restrict__ amax) {
  __shared__ float red[4];
  float m = 0.0f;
  const int64_t n = M * K;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t r = i / K, c = i % K;
    float v;
    if constexpr (sizeof(T) == 2) v = bf2f(x[r * ldx + c]);
    else v = x[r * ldx + c];
    m = fmaxf(m, fabsf(v));
  }
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) atomicMax(amax, __float_as_uint(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]))));
}

__global__ void fill_zero_kernel(unsigned int* p) { *p = 0u; }

// one thread per 16-element block along the rows (K % 16 == 0): kernels.fake_nvfp4 (kernels.py:38-49) then the
// bf16 cast of its callers (:56, :122)
template <typename T>
__global__ void __launch_bounds__(256) fake_nvfp4_kernel(const T* __restrict__ x, int64_t ldx, int64_t M, int64_t K,
                                                         uint16_t* __restrict__ out, int64_t ldo,
                                                         const unsigned int* __restrict__ amax) {
  const int64_t b = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x, nb = K / 16;
  if (b >= M * nb) return;
  const int64_t r = b / nb, c0 = (b % nb) * 16;
  float v[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    if constexpr (sizeof(T) == 2) v[e] = bf2f(x[r * ldx + c0 + e]);
    else v[e] = x[r * ldx + c0 + e];
  }
  const float gs = fmaxf(__uint_as_float(*amax) / 2688.0f, 1e-12f);
  float bm = 0.0f;
#pragma unroll
  for (int e = 0; e < 16; ++e) bm = fmaxf(bm, fabsf(v[e]));
  const float sb = fminf((bm / 6.0f) / gs, 448.0f);
  // e4m3fn round to nearest even (0 <= sb <= 448), decoded back to fp32
  const uint32_t code = __builtin_amdgcn_cvt_pk_fp8_f32(sb, 0.0f, 0, false) & 0xffu;
  const uint32_t ex = (code >> 3) & 0xfu, mt = code & 7u;
  const float dec = ex ? __uint_as_float(((ex + 120u) << 23) | (mt << 20)) : static_cast<float>(mt) * 0x1p-9f;
  float s = dec * gs;
  if (s == 0.0f) s = 1.0f;
  uint32_t w[8];
#pragma unroll
  for (int e = 0; e < 16; e += 2) {
    float y[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const float q = v[e + u] / s;
      const float a = fminf(fabsf(q), 6.0f);
      // the e2m1 grid point of torch.bucketize over the midpoints (a tie goes to the lower point)
      const float g = a <= 0.25f ? 0.0f : a <= 0.75f ? 0.5f : a <= 1.25f ? 1.0f : a <= 1.75f ? 1.5f
                    : a <= 2.5f ? 2.0f : a <= 3.5f ? 3.0f : a <= 5.0f ? 4.0f : 6.0f;
      const float sg = q > 0.0f ? 1.0f : (q < 0.0f ? -1.0f : 0.0f);
      y[u] = (g * sg) * s;
    }
    w[e >> 1] = pack_bf2(y[0], y[1]);
  }
  uint4* o = reinterpret_cast<uint4*>(out + r * ldo + c0);
  o[0] = make_uint4(w[0], w[1], w[2], w[3]);
  o[1] = make_uint4(w[4], w[5], w[6], w[7]);
}

}  // namespace
}  // namespace rh3

extern "C" int rh3_fake_nvfp4(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, uint16_t* out,
                              int64_t ldo, float* amax_ws, hipStream_t stream) {
  using namespace rh3;
  clear_error();
  RH3_REQUIRE(M >= 0 && K >= 0 && K % 16 == 0, "fake_nvfp4: K=%lld must be a multiple of 16", (long long)K);
  if (M == 0 || K == 0) return RH3_OK;
  RH3_REQUIRE(x && out && amax_ws, "fake_nvfp4: null pointer");
  RH3_REQUIRE(x_dtype == RH3_DTYPE_BF16 || x_dtype == RH3_DTYPE_F32, "fake_nvfp4: x_dtype %d", x_dtype);
  RH3_REQUIRE(ldx >= K && ldo >= K && ldo % 8 == 0 && aligned16(out), "fake_nvfp4: strides / alignment");
  RH3_REQUIRE(M * (K / 16) < (1ll << 31) * 256ll, "fake_nvfp4: tensor too large");
  unsigned int* am = reinterpret_cast<unsigned int*>(amax_ws);
  hipLaunchKernelGGL(fill_zero_kernel, dim3(1), dim3(1), 0, stream, am);
  const int64_t n = M * K;
  const unsigned grid = static_cast<unsigned>(std::min<int64_t>((n + 255) / 256, 4096));
  const unsigned gq = static_cast<unsigned>((M * (K / 16) + 255) / 256);
  if (x_dtype == RH3_DTYPE_BF16) {
    hipLaunchKernelGGL(absmax_kernel<uint16_t>, dim3(grid), dim3(256), 0, stream, static_cast<const uint16_t*>(x), ldx, M, K, am);
    hipLaunchKernelGGL(fake_nvfp4_kernel<uint16_t>, dim3(gq), dim3(256), 0, stream, static_cast<const uint16_t*>(x), ldx, M, K,
                       out, ldo, am);
  } else {
    hipLaunchKernelGGL(absmax_kernel<float>, dim3(grid), dim3(256), 0, stream, static_cast<const float*>(x), ldx, M, K, am);
    hipLaunchKernelGGL(fake_nvfp4_kernel<float>, dim3(gq), dim3(256), 0, stream, static_cast<const float*>(x), ldx, M, K,
                       out, ldo, am);
  }
  return launch_status("fake_nvfp4");
}

// ---------------------------------------------------------------- quantizer of any float input
// Inputs the fused quantizers do not take: fp16 / fp32 rows and FP8 with one scale per tensor. The reference's
// torch path (kernels.py:57-82, :125-128) casts with .float(), takes the absmax, s = max(amax / QMAX, 1e-12) and
// q = round(x / s) clamped (int8) or e4m3(clamp(x / s)) (FP8), with the IEEE quotient. One workgroup per row;
// per-element code (these are load-time or verification paths, not the per-step quantizers).
namespace rh3 {
namespace {

template <int DT>
__device__ __forceinline__ float ld_any(const void* p, int64_t i) {
  if constexpr (DT == RH3_DTYPE_F32) return static_cast<const float*>(p)[i];
  else if constexpr (DT == RH3_DTYPE_F16) return static_cast<float>(static_cast<const _Float16*>(p)[i]);
  else return bf2f(static_cast<const uint16_t*>(p)[i]);
}

template <int DT>
__global__ void __launch_bounds__(256) absmax_any_kernel(const void* __restrict__ x, int64_t ldx, int64_t M, int64_t K,
                                                         unsigned int* __restrict__ amax) {
  __shared__ float red[4];
  float m = 0.0f;
  const int64_t n = M * K;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256)
    m = fmaxf(m, fabsf(ld_any<DT>(x, (i / K) * ldx + i % K)));
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) atomicMax(amax, __float_as_uint(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]))));
}

// MODE 0: int8 per row; 1: FP8 per row; 2: FP8 per tensor (amax from absmax_any_kernel)
template <int DT, int MODE>
__global__ void __launch_bounds__(256) quant_any_kernel(const void* __restrict__ x, int64_t ldx, int64_t K,
                                                        uint8_t* __restrict__ q, int64_t ldq, float* __restrict__ s,
                                                        const unsigned int* __restrict__ amax_t) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x;
  float amax;
  if constexpr (MODE == 2) {
    amax = __uint_as_float(*amax_t);
  } else {
    float m = 0.0f;
    for (int64_t k = tid; k < K; k += 256) m = fmaxf(m, fabsf(ld_any<DT>(x, r * ldx + k)));
    m = wave_max(m);
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  }
  const float sc = fmaxf(amax / (MODE == 0 ? 127.0f : 448.0f), 1e-12f);
  if (tid == 0 && (MODE != 2 || r == 0)) s[MODE == 2 ? 0 : r] = sc;
  for (int64_t k = tid; k < K; k += 256) {
    const float t = ld_any<DT>(x, r * ldx + k) / sc;
    q[r * ldq + k] = MODE == 0 ? static_cast<uint8_t>(static_cast<int8_t>(fminf(fmaxf(rintf(t), -127.0f), 127.0f)))
                               : static_cast<uint8_t>(fp8_e4m3(fminf(fmaxf(t, -448.0f), 448.0f)));
  }
}

template <int DT>
int launch_any(const void* x, int64_t ldx, int64_t M, int64_t K, int mode, void* q, int64_t ldq, float* s,
               float* amax_ws, hipStream_t st) {
  uint8_t* qb = static_cast<uint8_t*>(q);
  if (mode == 0) {
    hipLaunchKernelGGL((quant_any_kernel<DT, 0>), dim3(static_cast<unsigned>(M)), dim3(256), 0, st, x, ldx, K, qb, ldq, s,
                       nullptr);
  } else if (mode == 1) {
    hipLaunchKernelGGL((quant_any_kernel<DT, 1>), dim3(static_cast<unsigned>(M)), dim3(256), 0, st, x, ldx, K, qb, ldq, s,
                       nullptr);
  } else {
    unsigned int* am = reinterpret_cast<unsigned int*>(amax_ws);
    hipLaunchKernelGGL(fill_zero_kernel, dim3(1), dim3(1), 0, st, am);
    const unsigned grid = static_cast<unsigned>(std::min<int64_t>((M * K + 255) / 256, 4096));
    hipLaunchKernelGGL(absmax_any_kernel<DT>, dim3(grid), dim3(256), 0, st, x, ldx, M, K, am);
    hipLaunchKernelGGL((quant_any_kernel<DT, 2>), dim3(static_cast<unsigned>(M)), dim3(256), 0, st, x, ldx, K, qb, ldq, s,
                       am);
  }
  return launch_status("quant_any");
}

}  // namespace
}  // namespace rh3

extern "C" int rh3_quant_any(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, int mode, void* q,
                             int64_t ldq, float* s, float* amax_ws, hipStream_t stream) {
  using namespace rh3;
  clear_error();
  RH3_REQUIRE(M >= 0 && K >= 0 && M < (1ll << 31), "quant_any: bad sizes M=%lld K=%lld", (long long)M, (long long)K);
  RH3_REQUIRE(mode >= 0 && mode <= 2, "quant_any: mode %d (0 int8 rows, 1 fp8 rows, 2 fp8 tensor)", mode);
  if (M == 0 || K == 0) return RH3_OK;
  RH3_REQUIRE(x && q && s && (mode != 2 || amax_ws), "quant_any: null pointer");
  RH3_REQUIRE(ldx >= K && ldq >= K, "quant_any: row strides (%lld, %lld) must be >= K=%lld", (long long)ldx,
              (long long)ldq, (long long)K);
  switch (x_dtype) {
    case RH3_DTYPE_BF16: return launch_any<RH3_DTYPE_BF16>(x, ldx, M, K, mode, q, ldq, s, amax_ws, stream);
    case RH3_DTYPE_F32: return launch_any<RH3_DTYPE_F32>(x, ldx, M, K, mode, q, ldq, s, amax_ws, stream);
    case RH3_DTYPE_F16: return launch_any<RH3_DTYPE_F16>(x, ldx, M, K, mode, q, ldq, s, amax_ws, stream);
    default: RH3_REQUIRE(false, "quant_any: x_dtype %d (1 bf16, 2 fp32, 3 fp16)", x_dtype);
  }
}
