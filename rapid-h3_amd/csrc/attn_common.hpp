// Device helpers shared by the attention kernels of librh3 (attn.hip: the per-128-block recipe with bf16
// P.V; attn_u8.hip: the reference's production numerics): head_dim 128, the per-head RMSNorm + RoPE
// prologue of a 16-lane row, K statistics, and the asynchronous global -> LDS copy.
#pragma once

#include "rh3_common.hpp"

namespace rh3 {
namespace attn {
namespace {  // each translation unit keeps its own copy of the kernels below

constexpr int D = 128;
constexpr int CHUNK = 256;   // statistics chunk (tokens)

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

struct RR {
  const uint16_t* tab;  // [S][rot/2][2][2] bf16, nullptr = no RMSNorm/RoPE
  const uint16_t* w;    // [128] bf16
  float eps;
  int rot;
};

__device__ __forceinline__ void load8(const uint16_t* p, float* v) {
  unpack8(*reinterpret_cast<const uint4*>(p), v);
}

// Per-head RMSNorm + split-half RoPE of one 128-channel row held by 16 lanes (8 channels each,
// lane l16 owns channels 8*l16..8*l16+7). Fixed order: per-lane x*x sum over e, then xor 8,4,2,1.
__device__ __forceinline__ void rms_rope8(float* x, int lane, const RR& rr, int64_t s) {
  const int l16 = lane & 15;
  float ss = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss = ss + x[e] * x[e];
  ss = ss + __shfl_xor(ss, 8, 64);
  ss = ss + __shfl_xor(ss, 4, 64);
  ss = ss + __shfl_xor(ss, 2, 64);
  ss = ss + __shfl_xor(ss, 1, 64);
  const float r = 1.0f / sqrtf(ss / 128.0f + rr.eps);
  float w[8];
  load8(rr.w + 8 * l16, w);
  float y[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = round_bf((r * x[e]) * w[e]);
  const int hr = rr.rot >> 1, step = hr >> 3;  // partner lane distance in 8-channel units
  const int c0 = 8 * l16;
  int src = l16;
  if (c0 < hr) src = l16 + step;
  else if (c0 < rr.rot) src = l16 - step;
  float py[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) py[e] = __shfl(y[e], (lane & ~15) + src, 64);
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
      x[e] = first ? round_bf((a * tv[4 * e + 0]) + (b * tv[4 * e + 1]))
                   : round_bf((a * tv[4 * e + 2]) + (b * tv[4 * e + 3]));
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = y[e];
  }
}

// ------------------------------------------------------------------ statistics
// grid (nchunk, H), 256 threads = 16 token slots x 16 lanes
__global__ void __launch_bounds__(256) stats_kernel(const uint16_t* __restrict__ k, int64_t k_ss, int64_t k_sh,
                                                    int64_t S, RR rr, double* __restrict__ part) {
  __shared__ double red[16][D];
  const int h = blockIdx.y, c = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
  const int slot = tid >> 4, l16 = tid & 15;
  double acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int it = 0; it < CHUNK / 16; ++it) {
    const int64_t s = static_cast<int64_t>(c) * CHUNK + it * 16 + slot;
    const bool ok = s < S;  // uniform per 16-lane group
    float x[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (ok) load8(k + s * k_ss + h * k_sh + 8 * l16, x);
    if (rr.tab) {
      // the shuffles inside rms_rope8 need every lane of the wave; out-of-range rows use token 0's table
      rms_rope8(x, lane, rr, ok ? s : 0);
    }
    if (ok) {
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += static_cast<double>(x[e]);
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) red[slot][8 * l16 + e] = acc[e];
  __syncthreads();
  if (tid < D) {
    double t = 0.0;
    for (int i = 0; i < 16; ++i) t += red[i][tid];
    part[(static_cast<int64_t>(h) * gridDim.x + c) * D + tid] = t;
  }
}

__global__ void zero_kernel(float* __restrict__ p, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.0f;
}

__global__ void kmean_kernel(const double* __restrict__ part, int nchunk, int64_t S, float* __restrict__ kmean) {
  const int h = blockIdx.x, d = threadIdx.x;
  double t = 0.0;
  for (int c = 0; c < nchunk; ++c) t += part[(static_cast<int64_t>(h) * nchunk + c) * D + d];
  kmean[h * D + d] = static_cast<float>(t / static_cast<double>(S));
}

typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) const v4i lds_v4i;

__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  const v2bf v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};  // v_cvt_pk_bf16_f32, RNE
  return __builtin_bit_cast(uint32_t, v);
}

// 16-byte LDS read at a byte address (the immediate offset folds into ds_read_b128)
__device__ __forceinline__ v4i lds_read16(uint32_t addr) {
  return *reinterpret_cast<lds_v4i*>(static_cast<uintptr_t>(addr));
}

// max of lane l and lane l ^ 32 (v_permlane32_swap exchanges the wave's halves)
__device__ __forceinline__ int max_halves(int v) {
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return max(static_cast<int>(r[0]), static_cast<int>(r[1]));
}

// Global -> LDS copy of 16 bytes per lane: lane l of the wave writes LDS byte offset lds_base + 16*l
// (M0 holds the wave-uniform base). Issued from inline assembly so that the compiler adds no wait of
// its own for it: the calling kernel accounts for these loads itself (s_waitcnt vmcnt) and issues no
// other vector-memory loads while they are in flight. M0 is a reserved register, so the statement
// restores the value it found; gfx9 requires one wait state between writing M0 and an LDS DMA that
// reads it.
__device__ __forceinline__ void lds_dma16(const void* gptr, uint32_t lds_base) {
  uint32_t saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off\n\t"
               "s_nop 0\n\ts_mov_b32 m0, %0"
               : "=&s"(saved)
               : "v"(gptr), "s"(lds_base)
               : "memory");
}

}  // namespace
}  // namespace attn
}  // namespace rh3
