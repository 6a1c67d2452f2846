// ConvRot (int8_rot) quantizers: the activation or weight row is rotated by blockdiag(H256) before the
// per-row INT8 quantization, H256 = the 4x4 regular Hadamard [[1,1,1,-1],[1,1,-1,1],[1,-1,1,1],[-1,1,1,1]]
// to the 4th Kronecker power, normalized (triton_fp8.py:70-90).
//
// Activations (triton_fp8.py:102-116, :218-233, :277-351): per 256-column group the prologue values v
// (fp32, same arithmetic as quant.hip) are rounded to bf16 and split into four 64-column chunks X_k;
// Z_k = X_k H64^T (H64 normalized, entries +-1/8) is the fp32 rounding of the exact dot products (the
// reference takes it from a bf16 tensor-core dot with fp32 accumulation, whose summation order is not
// specified; here every product is exact and the 64-term sums are formed exactly in float64, then rounded
// once); the four chunks are combined in fp32 in the reference's order
//   y0 = ((z0 + z1) + z2 - z3) * 0.5,  y1 = ((z0 + z1) - z2 + z3) * 0.5,
//   y2 = ((z0 - z1) + z2 + z3) * 0.5,  y3 = ((z1 + z2) + z3 - z0) * 0.5;
// then s = max(amax / 127, 1e-12), q = rint(clamp(y * (1 / s), -127, 127)).
//
// Weights (kernels.py:52-72, quantize_weight mode int8_rot): w @ blockdiag(H256)^T as the fp32 rounding of
// the exact product (float64 butterflies), then the int8_rowwise quantizer q = rint(w_rot / s).
//
// Layout: one wavefront per row; lane l owns the 64-column chunk 64*p + l of pass p, so the H64 part of the
// transform runs in the lane's registers (three radix-4 stages, H4 x = sum(x) - 2 reverse(x), in float64)
// and the four chunks of a 256-group sit in one lane quad, combined through quad DPP broadcasts.
#include "rh3_common.hpp"

namespace rh3 {
namespace {

enum RotKind { ROT_PLAIN = 0, ROT_SWIGLU = 1, ROT_NORMMOD = 2, ROT_HEADS = 3 };

struct RotArgs {
  const uint16_t* x;
  int64_t ldx;       // row stride (PLAIN, SWIGLU, NORMMOD) or token stride (HEADS)
  int64_t ld_head;   // HEADS: head stride
  int64_t M, K;      // K = rotated / quantized width (SWIGLU: F; HEADS: H * 128), K % 256 == 0
  const uint16_t* w; // NORMMOD weight or nullptr
  float eps;
  const int32_t* idx;
  const void* shift;
  const void* scale;
  int64_t ld_tab;
  int8_t* q;
  int64_t ldq;
  float* s;
};

template <typename T> __device__ __forceinline__ float tab_at(const void* p, int64_t i);
template <> __device__ __forceinline__ float tab_at<float>(const void* p, int64_t i) {
  return static_cast<const float*>(p)[i];
}
template <> __device__ __forceinline__ float tab_at<uint16_t>(const void* p, int64_t i) {
  return bf2f(static_cast<const uint16_t*>(p)[i]);
}

typedef __bf16 v2bf_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pk_bf16_hw(float a, float b) {
  const v2bf_t v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float silu_mul_f(float g, float u) {
  const float sig = 1.0f / (1.0f + __expf(-g));
  return (g * sig) * u;
}

// one radix-4 stage of H64 on the elements i, i+S, i+2S, i+3S of every group (exact in float64 for
// values within 2^38 of each other)
template <int S>
__device__ __forceinline__ void h4_stage(double (&d)[64]) {
#pragma unroll
  for (int g = 0; g < 16; ++g) {
    const int i = (g / S) * 4 * S + (g % S);
    const double x0 = d[i], x1 = d[i + S], x2 = d[i + 2 * S], x3 = d[i + 3 * S];
    const double t = ((x0 + x1) + x2) + x3;
    // fma(-2, x, t) rounds t - 2x once, like the subtraction (2x is exact)
    d[i] = fma(-2.0, x3, t);
    d[i + S] = fma(-2.0, x2, t);
    d[i + 2 * S] = fma(-2.0, x1, t);
    d[i + 3 * S] = fma(-2.0, x0, t);
  }
}

__device__ __forceinline__ void h64(double (&d)[64]) {
  h4_stage<1>(d);
  h4_stage<4>(d);
  h4_stage<16>(d);
}

// lane q of every quad receives lane CTRL[2q+1:2q] of the quad (DPP quad_perm; every source lane is inside
// the quad, so bound_ctrl never applies)
template <int CTRL>
__device__ __forceinline__ float quad_f(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, true));
}
template <int CTRL>
__device__ __forceinline__ double quad_d(double v) {
  const uint64_t u = __double_as_longlong(v);
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(u & 0xffffffffu), CTRL, 0xf, 0xf, true));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(u >> 32), CTRL, 0xf, 0xf, true));
  return __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hi) << 32) | lo));
}

// 8 consecutive modulation-table values at element i (VEC: 16-byte loads, the caller checked alignment)
template <typename TabT, bool VEC>
__device__ __forceinline__ void tab8(const void* p, int64_t i, float* t) {
  if (VEC && sizeof(TabT) == 4) {
    const float4* q = reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
    const float4 u0 = q[0], u1 = q[1];
    t[0] = u0.x; t[1] = u0.y; t[2] = u0.z; t[3] = u0.w; t[4] = u1.x; t[5] = u1.y; t[6] = u1.z; t[7] = u1.w;
  } else if (VEC) {
    unpack8(*reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + i), t);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) t[e] = tab_at<TabT>(p, i + e);
  }
}

// prologue values of the 8 columns c..c+7 of row m (the plain row, silu(g) * u, or the head-major gather)
template <int KIND>
__device__ __forceinline__ void prologue8(const RotArgs& a, int64_t m, int64_t c, float* v) {
  if (KIND == ROT_HEADS) {
    unpack8(*reinterpret_cast<const uint4*>(a.x + (c >> 7) * a.ld_head + m * a.ldx + (c & 127)), v);
  } else if (KIND == ROT_SWIGLU) {
    const uint16_t* p = a.x + m * a.ldx + c;
    float g[8], u[8];
    unpack8(*reinterpret_cast<const uint4*>(p), g);
    unpack8(*reinterpret_cast<const uint4*>(p + a.K), u);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = silu_mul_f(g[e], u[e]);
  } else {
    unpack8(*reinterpret_cast<const uint4*>(a.x + m * a.ldx + c), v);
  }
}

// The fp32 H4 combine of four chunk values z of a lane quad, before the halving: lane q computes
// t_q = ((sA A + sB B) + sC C) + sD D with (A, B, C, D) its quad's z in the order of the reference's formula for y_q
// (lanes 0-2: z0, z1, z2, z3; lane 3: z1, z2, z3, z0) and the lane's signs times a power of two (the H64
// normalization 1/8, applied here instead of to each z). The first term is one v_mul_f32 and each further term one
// v_fmac_f32 whose first operand arrives through a DPP quad permutation; the products with +-2^-k are exact, so each
// step is the reference's add or subtract of the scaled z rounded once, and scaling by a power of two commutes with
// the rounding. Four elements per block; s_nop 1 gives the DPP reads of z the two wait states a VALU write needs
// before them.
__device__ __forceinline__ void quad_combine4(const float* z, float sa, float sb, float sc, float sd, float* t) {
  asm volatile(
      "s_nop 1\n\t"
      "v_mul_f32_dpp %0, %4, %11 quad_perm:[0,0,0,1] row_mask:0xf bank_mask:0xf\n\t"
      "v_mul_f32_dpp %1, %5, %11 quad_perm:[0,0,0,1] row_mask:0xf bank_mask:0xf\n\t"
      "v_mul_f32_dpp %2, %6, %11 quad_perm:[0,0,0,1] row_mask:0xf bank_mask:0xf\n\t"
      "v_mul_f32_dpp %3, %7, %11 quad_perm:[0,0,0,1] row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %0, %4, %8 quad_perm:[1,1,1,2] row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %1, %5, %8 quad_perm:[1,1,1,2] row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %2, %6, %8 quad_perm:[1,1,1,2] row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %3, %7, %8 quad_perm:[1,1,1,2] row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %0, %4, %9 quad_perm:[2,2,2,3] row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %1, %5, %9 quad_perm:[2,2,2,3] row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %2, %6, %9 quad_perm:[2,2,2,3] row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %3, %7, %9 quad_perm:[2,2,2,3] row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %0, %4, %10 quad_perm:[3,3,3,0] row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %1, %5, %10 quad_perm:[3,3,3,0] row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %2, %6, %10 quad_perm:[3,3,3,0] row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %3, %7, %10 quad_perm:[3,3,3,0] row_mask:0xf bank_mask:0xf"
      : "=&v"(t[0]), "=&v"(t[1]), "=&v"(t[2]), "=&v"(t[3])
      : "v"(z[0]), "v"(z[1]), "v"(z[2]), "v"(z[3]), "v"(sb), "v"(sc), "v"(sd), "v"(sa));
}

// H64 of the lane's chunk d (bf16 values, exact in float64), rounded once to fp32, then the fp32 H4 combine of
// the quad's four chunks in the reference's order. The H64 normalization 1/8 rides on the combine's signs: fp32(d)/8
// is fp32(d/8) (a power-of-two scaling commutes with the rounding; below 2^-126, where the two could differ, every
// code is 0 and the scale sits at its 1e-12 floor either way; |d| stays below 2^128 for inputs below 2^122, the
// range in which t = 2 y below is finite too). t = 2 y: the reference's final halving is folded
// into the quantization scale (rot_scale), which gives the same scale and codes (see there).
__device__ __forceinline__ void rot_combine(double (&d)[64], float sb, float sc, float sd, float (&t)[64]) {
  h64(d);
  float z[64];
#pragma unroll
  for (int i = 0; i < 64; ++i) z[i] = static_cast<float>(d[i]);
  const float qb = sb * 0.125f, qc = sc * 0.125f, qd = sd * 0.125f;
#pragma unroll
  for (int i = 0; i < 64; i += 4) quad_combine4(z + i, 0.125f, qb, qc, qd, t + i);
}

// Row scale and quantization multiplier from the largest |t| (t = 2 y). With y = t / 2 the reference computes
// s = max(max|y| / 127, 1e-12) and q = rint(clamp(y * (1 / s), +-127)). Halving is exact for every normal t, so
// max|y| = max|t| / 2 and y * inv = t * (inv / 2); where t / 2 would be subnormal (|t| < 2^-125) both products lie
// below 2^-125 * 1e12 and round to the code 0, and a subnormal max|t| / 2 leaves s at its 1e-12 floor either way.
// The clamp never binds: |y * inv| <= 127 (1 + 2^-22) < 127.5.
__device__ __forceinline__ float rot_scale(float amax_t, float* inv_half) {
  const float s = fmaxf((amax_t * 0.5f) / 127.0f, 1e-12f);
  *inv_half = (1.0f / s) * 0.5f;
  return s;
}

// y = the rotated values (times 2) of chunk ch. A lane past the row (valid false; its whole quad is past it) works on
// chunk 0 of its row instead, an in-bounds read whose results the caller discards.
template <int KIND>
__device__ __forceinline__ void rot_act_chunk(const RotArgs& a, int64_t m, int64_t ch, bool valid, float sb, float sc,
                                              float sd, float (&y)[64]) {
  double d[64];
  const int64_t c0 = valid ? ch * 64 : 0;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    float v[8];
    prologue8<KIND>(a, m, c0 + 8 * t, v);
    if constexpr (KIND == ROT_SWIGLU) {
#pragma unroll
      for (int e = 0; e < 8; e += 2) {  // bf16 round to nearest even (v_cvt_pk_bf16_f32), back to fp32 exactly
        const uint32_t pk = pk_bf16_hw(v[e], v[e + 1]);
        d[8 * t + e] = static_cast<double>(__uint_as_float(pk << 16));
        d[8 * t + e + 1] = static_cast<double>(__uint_as_float(pk & 0xffff0000u));
      }
    } else {  // the plain and head-major values are bf16 already: the rounding would give them back unchanged
#pragma unroll
      for (int e = 0; e < 8; ++e) d[8 * t + e] = static_cast<double>(v[e]);
    }
  }
  rot_combine(d, sb, sc, sd, y);
}

// codes rint(t * inv_half) of the 64 values of a chunk: pack4_codes rounds to nearest even by its magic-number add
// (|t * inv_half| < 127.5 < 2^22) and packs the low bytes
__device__ __forceinline__ void store64(int8_t* q, const float (&t)[64], float inv_half) {
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    float n[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) n[e] = t[8 * k + e] * inv_half;
    *reinterpret_cast<uint2*>(q + 8 * k) = make_uint2(pack4_codes(n), pack4_codes(n + 4));
  }
}

// NP = passes of 64 chunks (K <= 4096 * NP). With one pass the rotated values stay in registers between
// the absmax and the quantization; with more, the values of passes 0..NP-2 wait in LDS (64 floats per
// lane, lane-interleaved float4s, a private region per wave) until the row scale is known.
template <int NP> constexpr int rot_waves() { return NP <= 2 ? 4 : 2; }

template <int KIND, int NP>
__global__ void __launch_bounds__(64 * rot_waves<NP>()) rot_quant_kernel(const RotArgs a) {
  constexpr int W = rot_waves<NP>();
  __shared__ float4 stash[NP > 1 ? W * (NP - 1) * 16 * 64 : 1];  // [wave][pass][i / 4][lane]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t m = static_cast<int64_t>(blockIdx.x) * W + wave;
  if (m >= a.M) return;  // whole wavefront: DPP partners never leave; no workgroup barrier below
  const int q4 = lane & 3;
  const float sb = q4 == 2 ? -1.0f : 1.0f, sc = q4 == 1 ? -1.0f : 1.0f, sd = (q4 == 0 || q4 == 3) ? -1.0f : 1.0f;
  static_assert(KIND != ROT_NORMMOD, "RMSNorm + modulation runs in rot_normmod_kernel");
  const int64_t nchunks = a.K / 64;
  float4* my = stash + wave * (NP - 1) * 16 * 64 + lane;
  float y[64];
  float amax = 0.0f;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int64_t ch = 64 * p + lane;
    rot_act_chunk<KIND>(a, m, ch, ch < nchunks, sb, sc, sd, y);
    float am = 0.0f;
#pragma unroll
    for (int i = 0; i < 64; i += 2) am = max3_abs(am, y[i], y[i + 1]);
    if (ch < nchunks) amax = fmaxf(amax, am);
    if (p < NP - 1) {
#pragma unroll
      for (int t = 0; t < 16; ++t) my[(p * 16 + t) * 64] = make_float4(y[4 * t], y[4 * t + 1], y[4 * t + 2], y[4 * t + 3]);
    }
  }
  amax = wave_max(amax);
  float inv;
  const float s = rot_scale(amax, &inv);
  if (lane == 0) a.s[m] = s;
  const int64_t last = 64 * (NP - 1) + lane;
  if (last < nchunks) store64(a.q + m * a.ldq + 64 * last, y, inv);
#pragma unroll
  for (int p = 0; p < NP - 1; ++p) {
    const int64_t ch = 64 * p + lane;
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      const float4 u = my[(p * 16 + t) * 64];
      y[4 * t] = u.x; y[4 * t + 1] = u.y; y[4 * t + 2] = u.z; y[4 * t + 3] = u.w;
    }
    if (ch < nchunks) store64(a.q + m * a.ldq + 64 * ch, y, inv);
  }
}

// RMSNorm + modulation, rotation and INT8 with the prologue staged through LDS. Phase 1 works in the coalesced
// layout of the sum of squares (lane l holds columns 512 j + 8 l .. +7): the row, the norm weight and both
// modulation rows are read with whole-wave 16-byte accesses, the prologue values are computed there (the same
// operations in the same order as the unrotated quantizer's prologue) and written to the wave's LDS region as bf16,
// chunk-major with a 144-byte chunk pitch (lanes reading their own chunk then hit 16 distinct bank quads). Phase 2 is
// the rotation of rot_quant_kernel with each lane's chunk read from LDS instead of gathered from global memory. A wave
// can walk RPW consecutive rows, issuing the next row's loads before the current row's rotation; that holds the loaded
// row through the rotation (222 registers, 2 waves per SIMD) and measured slower than one row per wave at 3 waves per
// SIMD (0.71 vs 0.64 ms at 145,152 x 3072), so RPW is 1. A wave uses only its own LDS region (in order: a row's
// phase-1 writes follow the previous row's phase-2 reads), so no workgroup barrier is needed.
constexpr int STAGE_PITCH = 144;
template <int NP> constexpr int nm_waves() { return NP == 1 ? 4 : (NP == 2 ? 2 : 1); }
template <int NP> constexpr int nm_rows() { return 1; }

template <typename TabT, int NP, bool VEC>
__global__ void __launch_bounds__(64 * nm_waves<NP>()) rot_normmod_kernel(const RotArgs a) {
  constexpr int W = nm_waves<NP>(), RPW = nm_rows<NP>();
  __shared__ __attribute__((aligned(16))) uint8_t stage[W * 64 * NP * STAGE_PITCH];
  __shared__ float4 stash[NP > 1 ? W * (NP - 1) * 16 * 64 : 1];  // [wave][pass][i / 4][lane]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t m0 = (static_cast<int64_t>(blockIdx.x) * W + wave) * RPW;
  if (m0 >= a.M) return;  // whole wavefront: DPP partners never leave; no workgroup barrier below
  const int nrows = static_cast<int>(min(static_cast<int64_t>(RPW), a.M - m0));
  uint8_t* st = stage + wave * 64 * NP * STAGE_PITCH;
  const int q4 = lane & 3;
  const float sb = q4 == 2 ? -1.0f : 1.0f, sc = q4 == 1 ? -1.0f : 1.0f, sd = (q4 == 0 || q4 == 3) ? -1.0f : 1.0f;
  const int64_t nchunks = a.K / 64;
  float4* my = stash + wave * (NP - 1) * 16 * 64 + lane;
  // the row's loads, all issued before the first product (K <= 4096 * NP, so j < 8 * NP)
  uint4 r[8 * NP];
  auto load_row = [&](int64_t m) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 8 * NP; ++j) {
      const int64_t c = 512 * j + 8 * lane;
      r[j] = c < a.K ? *reinterpret_cast<const uint4*>(a.x + m * a.ldx + c) : make_uint4(0, 0, 0, 0);
    }
  };
  load_row(m0);
  for (int ri = 0; ri < nrows; ++ri) {
    const int64_t m = m0 + ri;
    const int64_t trow = static_cast<int64_t>(a.idx[m]) * a.ld_tab;
    // phase 1. Sum of squares in the order of quant.hip (lane chunks 512 j + 8 l, (j, e) sequential, butterfly)
    float xv[8 * NP][8];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < 8 * NP; ++j) {
      unpack8(r[j], xv[j]);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(xv[j][e], xv[j][e], ss);  // x * x is exact (bf16 x): = ss + x * x
    }
    if (ri + 1 < nrows) load_row(m + 1);
    ss = wave_sum_tree(ss);
    const float rstd = 1.0f / sqrtf(ss / static_cast<float>(a.K) + a.eps);
#pragma unroll
    for (int j = 0; j < 8 * NP; ++j) {
      const int64_t c = 512 * j + 8 * lane;
      if (c < a.K) {
        float* v = xv[j];
        float wv[8], scl[8], shf[8];
        if (a.w) unpack8(*reinterpret_cast<const uint4*>(a.w + c), wv);
        tab8<TabT, VEC>(a.scale, trow + c, scl);
        tab8<TabT, VEC>(a.shift, trow + c, shf);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float y = v[e] * rstd;
          if (a.w) y = y * wv[e];
          v[e] = y * (1.0f + scl[e]) + shf[e];
        }
        uint4 o;
        o.x = pk_bf16_hw(v[0], v[1]);
        o.y = pk_bf16_hw(v[2], v[3]);
        o.z = pk_bf16_hw(v[4], v[5]);
        o.w = pk_bf16_hw(v[6], v[7]);
        *reinterpret_cast<uint4*>(st + (c >> 6) * STAGE_PITCH + (c & 63) * 2) = o;
      }
    }
    // the wave's own LDS writes are complete before its lanes read each other's columns
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
    // phase 2: lane l rotates chunk 64 p + l
    float y[64];
    float amax = 0.0f;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int64_t ch = 64 * p + lane;
      // a lane past the row (its whole quad is) reads its slot of the wave's region all the same (ch < 64 NP) and
      // its results are discarded
      double d[64];
      const uint8_t* src = st + ch * STAGE_PITCH;
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const uint4 u = *reinterpret_cast<const uint4*>(src + 16 * t);
        const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          d[8 * t + 2 * e] = static_cast<double>(__uint_as_float(w4[e] << 16));
          d[8 * t + 2 * e + 1] = static_cast<double>(__uint_as_float(w4[e] & 0xffff0000u));
        }
      }
      rot_combine(d, sb, sc, sd, y);
      float am = 0.0f;
#pragma unroll
      for (int i = 0; i < 64; i += 2) am = max3_abs(am, y[i], y[i + 1]);
      if (ch < nchunks) amax = fmaxf(amax, am);
      if (p < NP - 1) {
#pragma unroll
        for (int t = 0; t < 16; ++t) my[(p * 16 + t) * 64] = make_float4(y[4 * t], y[4 * t + 1], y[4 * t + 2], y[4 * t + 3]);
      }
    }
    amax = wave_max(amax);
    float inv;
    const float s = rot_scale(amax, &inv);
    if (lane == 0) a.s[m] = s;
    const int64_t last = 64 * (NP - 1) + lane;
    if (last < nchunks) store64(a.q + m * a.ldq + 64 * last, y, inv);
#pragma unroll
    for (int p = 0; p < NP - 1; ++p) {
      const int64_t ch = 64 * p + lane;
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        const float4 u = my[(p * 16 + t) * 64];
        y[4 * t] = u.x; y[4 * t + 1] = u.y; y[4 * t + 2] = u.z; y[4 * t + 3] = u.w;
      }
      if (ch < nchunks) store64(a.q + m * a.ldq + 64 * ch, y, inv);
    }
  }
}

// ---------------------------------------------------------------- exact H256 rotation of weights
struct ExactArgs {
  const void* x;     // bf16 or fp32 rows
  int64_t ldx;
  int64_t M, K;
  float* y;          // OUT_F32: rotated rows
  int64_t ldy;
  int8_t* q;         // otherwise: int8 codes + per-row scale
  int64_t ldq;
  float* s;
};

// the exactly rotated chunk ch, rounded once to fp32
template <bool IN_F32>
__device__ __forceinline__ void rot_exact_chunk(const ExactArgs& a, int64_t m, int64_t ch, bool valid,
                                                float (&y)[64]) {
  double d[64];
  if (valid) {
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int64_t c = ch * 64 + 8 * t;
      float v[8];
      if (IN_F32) {
        const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(a.x) + m * a.ldx + c);
        const float4 u0 = p[0], u1 = p[1];
        v[0] = u0.x; v[1] = u0.y; v[2] = u0.z; v[3] = u0.w; v[4] = u1.x; v[5] = u1.y; v[6] = u1.z; v[7] = u1.w;
      } else {
        unpack8(*reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.x) + m * a.ldx + c), v);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) d[8 * t + e] = static_cast<double>(v[e]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 64; ++i) d[i] = 0.0;
  }
  h64(d);
  // the fourth radix-4 stage runs across the lane quad: y_q = sum_k d_k - 2 d_(3-q)
#pragma unroll
  for (int i = 0; i < 64; ++i) {
    const double b0 = quad_d<0x00>(d[i]), b1 = quad_d<0x55>(d[i]), b2 = quad_d<0xAA>(d[i]), b3 = quad_d<0xFF>(d[i]);
    const double mir = quad_d<0x1B>(d[i]);
    const double t = ((b0 + b1) + b2) + b3;
    y[i] = static_cast<float>((t - 2.0 * mir) * 0.0625);
  }
}

template <bool IN_F32, bool OUT_F32, int NP>
__global__ void __launch_bounds__(256) rot_exact_kernel(const ExactArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t m = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (m >= a.M) return;
  const int64_t nchunks = a.K / 64;
  float y[64];
  if (OUT_F32) {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int64_t ch = 64 * p + lane;
      rot_exact_chunk<IN_F32>(a, m, ch, ch < nchunks, y);
      if (ch < nchunks) {
        float4* o = reinterpret_cast<float4*>(a.y + m * a.ldy + 64 * ch);
#pragma unroll
        for (int t = 0; t < 16; ++t) o[t] = make_float4(y[4 * t], y[4 * t + 1], y[4 * t + 2], y[4 * t + 3]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    return;
  }
  float amax = 0.0f;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int64_t ch = 64 * p + lane;
    rot_exact_chunk<IN_F32>(a, m, ch, ch < nchunks, y);
#pragma unroll
    for (int i = 0; i < 64; ++i) amax = fmaxf(amax, fabsf(y[i]));
    __builtin_amdgcn_sched_barrier(0);
  }
  amax = wave_max(amax);
  const float s = fmaxf(amax / 127.0f, 1e-12f);
  const float inv = 1.0f / s;
  if (lane == 0) a.s[m] = s;
  // int8_rowwise weight codes: round(w / s) with IEEE quotient semantics (kernels.py:69-71)
  auto emit = [&](int64_t ch) {
    int8_t* q = a.q + m * a.ldq + 64 * ch;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      uint32_t b[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float r = fminf(fmaxf(rint_div(y[8 * t + e], s, inv), -127.0f), 127.0f);
        b[e] = static_cast<uint32_t>(static_cast<int32_t>(r)) & 0xffu;
      }
      uint2 o;
      o.x = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
      o.y = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
      *reinterpret_cast<uint2*>(q + 8 * t) = o;
    }
  };
  if (NP == 1) {
    if (lane < nchunks) emit(lane);
  } else {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int64_t ch = 64 * p + lane;
      rot_exact_chunk<IN_F32>(a, m, ch, ch < nchunks, y);
      if (ch < nchunks) emit(ch);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

template <typename TabT, bool VEC>
void launch_normmod(const RotArgs& a, hipStream_t st) {
  if (a.K <= 4096)
    hipLaunchKernelGGL((rot_normmod_kernel<TabT, 1, VEC>), dim3(static_cast<unsigned>((a.M + 3) / 4)), dim3(256), 0, st,
                       a);
  else if (a.K <= 8192)
    hipLaunchKernelGGL((rot_normmod_kernel<TabT, 2, VEC>), dim3(static_cast<unsigned>((a.M + 1) / 2)), dim3(128), 0, st,
                       a);
  else
    hipLaunchKernelGGL((rot_normmod_kernel<TabT, 4, VEC>), dim3(static_cast<unsigned>(a.M)), dim3(64), 0, st, a);
}

template <int KIND>
void launch_rot(const RotArgs& a, hipStream_t st) {
  if (a.K <= 4096)
    hipLaunchKernelGGL((rot_quant_kernel<KIND, 1>), dim3(static_cast<unsigned>((a.M + 3) / 4)), dim3(256), 0, st, a);
  else if (a.K <= 8192)
    hipLaunchKernelGGL((rot_quant_kernel<KIND, 2>), dim3(static_cast<unsigned>((a.M + 3) / 4)), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((rot_quant_kernel<KIND, 4>), dim3(static_cast<unsigned>((a.M + 1) / 2)), dim3(128), 0, st, a);
}

template <int KIND, typename TabT>
int launch_act(const RotArgs& a, hipStream_t st, const char* name) {
  if (a.M == 0) return RH3_OK;
  if constexpr (KIND == ROT_NORMMOD) {
    // 16-byte modulation-table loads when every row start is 16-byte aligned
    if (aligned16(a.shift) && aligned16(a.scale) && (a.ld_tab * static_cast<int64_t>(sizeof(TabT))) % 16 == 0)
      launch_normmod<TabT, true>(a, st);
    else
      launch_normmod<TabT, false>(a, st);
  } else {
    launch_rot<KIND>(a, st);
  }
  return launch_status(name);
}

template <bool IN_F32, bool OUT_F32>
void launch_exact(const ExactArgs& a, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>((a.M + 3) / 4)), block(256);
  if (a.K <= 4096) hipLaunchKernelGGL((rot_exact_kernel<IN_F32, OUT_F32, 1>), grid, block, 0, st, a);
  else if (a.K <= 8192) hipLaunchKernelGGL((rot_exact_kernel<IN_F32, OUT_F32, 2>), grid, block, 0, st, a);
  else hipLaunchKernelGGL((rot_exact_kernel<IN_F32, OUT_F32, 4>), grid, block, 0, st, a);
}

int check_rot(const char* name, const void* x, int64_t M, int64_t K, const void* q, int64_t ldq, const void* s) {
  RH3_REQUIRE(M >= 0 && K >= 0, "%s: negative size (M=%lld, K=%lld)", name, (long long)M, (long long)K);
  RH3_REQUIRE(K % 256 == 0, "%s: K=%lld must be a multiple of the rotation group 256", name, (long long)K);
  RH3_REQUIRE(K <= 16384, "%s: K=%lld exceeds the 16384-column limit of the rotation kernels", name, (long long)K);
  if (M == 0) return RH3_OK;
  RH3_REQUIRE(K > 0, "%s: K must be positive", name);
  RH3_REQUIRE(M < (int64_t{1} << 31) * 4, "%s: M=%lld too large", name, (long long)M);
  RH3_REQUIRE(x && q && s, "%s: null pointer", name);
  RH3_REQUIRE(ldq >= K && ldq % 8 == 0, "%s: output row stride %lld (K=%lld) must be >= K and a multiple of 8", name,
              (long long)ldq, (long long)K);
  RH3_REQUIRE(aligned16(x) && (reinterpret_cast<uintptr_t>(q) & 7) == 0, "%s: x must be 16-byte and q 8-byte aligned",
              name);
  return RH3_OK;
}

}  // namespace
}  // namespace rh3

using namespace rh3;

extern "C" int rh3_rot_quant_rows_i8(const uint16_t* x, int64_t ldx, int64_t M, int64_t K, int8_t* q, int64_t ldq,
                                     float* s, hipStream_t stream) {
  clear_error();
  if (int e = check_rot("rot_quant_rows_i8", x, M, K, q, ldq, s)) return e;
  RH3_REQUIRE(M == 0 || (ldx >= K && ldx % 8 == 0), "rot_quant_rows_i8: row stride %lld invalid for K=%lld",
              (long long)ldx, (long long)K);
  RotArgs a{x, ldx, 0, M, K, nullptr, 0.f, nullptr, nullptr, nullptr, 0, q, ldq, s};
  return launch_act<ROT_PLAIN, float>(a, stream, "rot_quant_rows_i8");
}

extern "C" int rh3_swiglu_rot_quant_rows_i8(const uint16_t* x, int64_t ldx, int64_t M, int64_t F, int8_t* q,
                                            int64_t ldq, float* s, hipStream_t stream) {
  clear_error();
  if (int e = check_rot("swiglu_rot_quant_rows_i8", x, M, F, q, ldq, s)) return e;
  RH3_REQUIRE(M == 0 || (ldx >= 2 * F && ldx % 8 == 0), "swiglu_rot_quant_rows_i8: row stride %lld invalid for 2F=%lld",
              (long long)ldx, (long long)(2 * F));
  RotArgs a{x, ldx, 0, M, F, nullptr, 0.f, nullptr, nullptr, nullptr, 0, q, ldq, s};
  return launch_act<ROT_SWIGLU, float>(a, stream, "swiglu_rot_quant_rows_i8");
}

extern "C" int rh3_norm_mod_rot_quant_i8(const uint16_t* x, int64_t ldx, int64_t M, int64_t K, const uint16_t* weight,
                                         float eps, const int32_t* idx, const void* shift, const void* scale,
                                         int tab_dtype, int64_t ld_tab, int8_t* q, int64_t ldq, float* s,
                                         hipStream_t stream) {
  clear_error();
  if (int e = check_rot("norm_mod_rot_quant_i8", x, M, K, q, ldq, s)) return e;
  if (M == 0) return RH3_OK;
  RH3_REQUIRE(ldx >= K && ldx % 8 == 0, "norm_mod_rot_quant_i8: row stride %lld invalid for K=%lld", (long long)ldx,
              (long long)K);
  RH3_REQUIRE(idx && shift && scale, "norm_mod_rot_quant_i8: idx, shift and scale are required");
  RH3_REQUIRE(ld_tab >= K, "norm_mod_rot_quant_i8: table row stride %lld < K=%lld", (long long)ld_tab, (long long)K);
  RH3_REQUIRE(!weight || aligned16(weight), "norm_mod_rot_quant_i8: weight must be 16-byte aligned");
  RH3_REQUIRE(tab_dtype == RH3_DTYPE_F32 || tab_dtype == RH3_DTYPE_BF16, "norm_mod_rot_quant_i8: tab_dtype %d",
              tab_dtype);
  RotArgs a{x, ldx, 0, M, K, weight, eps, idx, shift, scale, ld_tab, q, ldq, s};
  if (tab_dtype == RH3_DTYPE_F32) return launch_act<ROT_NORMMOD, float>(a, stream, "norm_mod_rot_quant_i8");
  return launch_act<ROT_NORMMOD, uint16_t>(a, stream, "norm_mod_rot_quant_i8");
}

extern "C" int rh3_rot_quant_heads_i8(const uint16_t* o, int64_t H, int64_t M, int64_t ld_head, int64_t ld_row,
                                      int8_t* q, int64_t ldq, float* s, hipStream_t stream) {
  clear_error();
  RH3_REQUIRE(H > 0 && H < (int64_t{1} << 24), "rot_quant_heads_i8: H=%lld", (long long)H);
  if (int e = check_rot("rot_quant_heads_i8", o, M, H * 128, q, ldq, s)) return e;
  if (M == 0) return RH3_OK;
  RH3_REQUIRE(ld_head % 8 == 0 && ld_row % 8 == 0 && ld_row >= 0 && ld_head >= 0,
              "rot_quant_heads_i8: strides must be non-negative multiples of 8 elements");
  RotArgs a{o, ld_row, ld_head, M, H * 128, nullptr, 0.f, nullptr, nullptr, nullptr, 0, q, ldq, s};
  return launch_act<ROT_HEADS, float>(a, stream, "rot_quant_heads_i8");
}

extern "C" int rh3_convrot_f32(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, float* y, int64_t ldy,
                               hipStream_t stream) {
  clear_error();
  RH3_REQUIRE(M >= 0 && K >= 0 && K % 256 == 0, "convrot_f32: K=%lld must be a non-negative multiple of 256",
              (long long)K);
  if (M == 0 || K == 0) return RH3_OK;
  RH3_REQUIRE(x && y, "convrot_f32: null pointer");
  RH3_REQUIRE(x_dtype == RH3_DTYPE_BF16 || x_dtype == RH3_DTYPE_F32, "convrot_f32: x_dtype %d", x_dtype);
  RH3_REQUIRE(ldx >= K && ldx % 8 == 0 && ldy >= K && ldy % 4 == 0, "convrot_f32: invalid row strides");
  RH3_REQUIRE(aligned16(x) && aligned16(y), "convrot_f32: x and y must be 16-byte aligned");
  RH3_REQUIRE(K <= 16384, "convrot_f32: K=%lld exceeds the 16384-column limit", (long long)K);
  RH3_REQUIRE(M < (int64_t{1} << 31) * 4, "convrot_f32: M=%lld too large", (long long)M);
  ExactArgs a{x, ldx, M, K, y, ldy, nullptr, 0, nullptr};
  if (x_dtype == RH3_DTYPE_F32) launch_exact<true, true>(a, stream);
  else launch_exact<false, true>(a, stream);
  return launch_status("convrot_f32");
}

extern "C" int rh3_quant_weight_rot_i8(const void* w, int w_dtype, int64_t ldw, int64_t N, int64_t K, int8_t* q,
                                       int64_t ldq, float* s, hipStream_t stream) {
  clear_error();
  if (int e = check_rot("quant_weight_rot_i8", w, N, K, q, ldq, s)) return e;
  if (N == 0) return RH3_OK;
  RH3_REQUIRE(w_dtype == RH3_DTYPE_BF16 || w_dtype == RH3_DTYPE_F32, "quant_weight_rot_i8: w_dtype %d", w_dtype);
  RH3_REQUIRE(ldw >= K && ldw % 8 == 0, "quant_weight_rot_i8: row stride %lld invalid for K=%lld", (long long)ldw,
              (long long)K);
  ExactArgs a{w, ldw, N, K, nullptr, 0, q, ldq, s};
  if (w_dtype == RH3_DTYPE_F32) launch_exact<true, false>(a, stream);
  else launch_exact<false, false>(a, stream);
  return launch_status("quant_weight_rot_i8");
}
