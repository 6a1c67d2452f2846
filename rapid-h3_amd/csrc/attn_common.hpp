// Device helpers shared by the attention kernels of librh3 (attn.hip: the per-128-block recipe with bf16
// P.V; attn_u8.hip: the reference's production numerics): head_dim 128, the per-head RMSNorm + RoPE
// prologue of a 16-lane row, K statistics, and the asynchronous global -> LDS copy.
#pragma once

#include "attn_prologue.hpp"

namespace rh3 {
namespace attn {
namespace {  // each translation unit keeps its own copy of the kernels below

constexpr int D = 128;
constexpr int CHUNK = 256;   // statistics chunk (tokens)

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

// ------------------------------------------------------------------ statistics
// Sums of bf16 values in float64 are exact here (a few hundred thousand values of 8 significant bits within a
// few dozen binades), so every summation order below gives the same bits.
//
// grid (H, nchunk) (heads fastest: the workgroups of one chunk run together and share its rope-table rows in
// L2), STATS_NT threads = 16 token slots x 16 lanes. A row and its rope-table row are loaded together; rows past
// S read row S - 1 and are not added, so no lane-divergent branch stands between the loads.
constexpr int STATS_NT = 256;
template <bool RRON>
__global__ void __launch_bounds__(STATS_NT) stats_kernel(const uint16_t* __restrict__ k, int64_t k_ss, int64_t k_sh,
                                                    int64_t S, RR rr, double* __restrict__ part,
                                                    uint16_t* __restrict__ kn, int64_t kn_sh) {
  __shared__ double red[16][D];
  const int h = blockIdx.x, c = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
  const int slot = tid >> 4, l16 = tid & 15;
  double acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  float w[8];
  if constexpr (RRON) load8(rr.w + 8 * l16, w);
  for (int it = 0; it < CHUNK / 16; ++it) {
    const int64_t s = static_cast<int64_t>(c) * CHUNK + it * 16 + slot;
    const int64_t sl = s < S ? s : S - 1;
    const uint4 rx = *reinterpret_cast<const uint4*>(k + sl * k_ss + h * k_sh + 8 * l16);
    uint4 rt[4];
    if constexpr (RRON) rope_tab8_raw(rr, l16, sl, rt);
    float x[8];
    unpack8(rx, x);
    if constexpr (RRON) rms_rope8_raw(x, lane, rr, w, rt);
    if (s < S) {
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += static_cast<double>(x[e]);
      if (RRON && kn) {  // the RMSNorm + RoPE'd row (bf16 values: the packing is exact) for the K quantizer
        uint4 o;
        o.x = pack_bf2(x[0], x[1]);
        o.y = pack_bf2(x[2], x[3]);
        o.z = pack_bf2(x[4], x[5]);
        o.w = pack_bf2(x[6], x[7]);
        *reinterpret_cast<uint4*>(kn + h * kn_sh + s * D + 8 * l16) = o;
      }
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) red[slot][8 * l16 + e] = acc[e];
  __syncthreads();
  if (tid < D) {
    double t = 0.0;
    for (int i = 0; i < 16; ++i) t += red[i][tid];
    part[(static_cast<int64_t>(h) * gridDim.y + c) * D + tid] = t;
  }
}

// the K statistics of one launch: stats_kernel with or without the RMSNorm + RoPE prologue; with the prologue and
// kn, also the prologue's rows as bf16 into kn [H][..][128] (head stride kn_sh elements)
inline void launch_stats(dim3 grid, hipStream_t st, const uint16_t* k, int64_t k_ss, int64_t k_sh, int64_t S,
                         const RR& rr, double* part, uint16_t* kn = nullptr, int64_t kn_sh = 0) {
  if (rr.tab)
    hipLaunchKernelGGL(stats_kernel<true>, grid, dim3(STATS_NT), 0, st, k, k_ss, k_sh, S, rr, part, kn, kn_sh);
  else
    hipLaunchKernelGGL(stats_kernel<false>, grid, dim3(STATS_NT), 0, st, k, k_ss, k_sh, S, rr, part, nullptr,
                       int64_t{0});
}

__global__ void zero_kernel(float* __restrict__ p, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.0f;
}

// The main kernels' work items, claimed per XCD. The dispatcher deals workgroups to the 8 XCDs round-robin (linear
// workgroup id bid on XCD bid % 8); XCD x owns the contiguous share [x nmain / 8, (x + 1) nmain / 8) of the main items,
// whose order (query blocks fastest) makes a share a few whole heads, so the K / V tiles its workgroups stream stay
// in that XCD's L2. A workgroup takes the next item of its own XCD's share, then of the other XCDs' shares in turn
// (so a fast XCD finishes a slow one's share), then of the tail items [nmain, nmain + ntail); -1 when every item is
// taken. ctr[0 .. 8] are zero at launch. The grid holds more workgroups than items, so every item is taken: a
// workgroup that gets -1 saw every counter past its end.
__device__ __forceinline__ int claim_item(int* ctr, int nmain, int ntail, int bid) {
  const int x = bid & 7;
#pragma unroll 1
  for (int k = 0; k < 8; ++k) {
    const int y = (x + k) & 7;
    const int lo = static_cast<int>((static_cast<int64_t>(y) * nmain) >> 3);
    const int n = static_cast<int>((static_cast<int64_t>(y + 1) * nmain) >> 3) - lo;
    if (__hip_atomic_load(ctr + y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= n) continue;
    const int c = atomicAdd(ctr + y, 1);
    if (c < n) return lo + c;
  }
  const int c = atomicAdd(ctr + 8, 1);
  return c < ntail ? nmain + c : -1;
}
constexpr int64_t CLAIM_COUNTERS = 9;

// grid (H), KMEAN_NT threads: group j of 128 channels sums chunks j, j + 8, ..., then the 8 groups
constexpr int KMEAN_NT = 1024;
__global__ void __launch_bounds__(KMEAN_NT) kmean_kernel(const double* __restrict__ part, int nchunk, int64_t S,
                                                         float* __restrict__ kmean) {
  constexpr int G = KMEAN_NT / D;
  __shared__ double red[G][D];
  const int h = blockIdx.x, d = threadIdx.x % D, j = threadIdx.x / D;
  const double* p = part + static_cast<int64_t>(h) * nchunk * D + d;
  double t0 = 0.0, t1 = 0.0;
  int c = j;
  for (; c + G < nchunk; c += 2 * G) {
    t0 += p[static_cast<int64_t>(c) * D];
    t1 += p[static_cast<int64_t>(c + G) * D];
  }
  if (c < nchunk) t0 += p[static_cast<int64_t>(c) * D];
  red[j][d] = t0 + t1;
  __syncthreads();
  if (j == 0) {
    double t = 0.0;
#pragma unroll
    for (int i = 0; i < G; ++i) t += red[i][d];
    kmean[h * D + d] = static_cast<float>(t / static_cast<double>(S));
  }
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

// Issue order of a run of N (LDS read, MFMA) pairs: the first A reads, then each MFMA followed by the next read,
// then the last A MFMAs, so that every operand is read A MFMAs (>= 32 A pipe cycles) before its use. Left alone,
// the scheduler places each read right before its MFMA and waits for it there.
template <int N, int A>
__device__ __forceinline__ void read_ahead() {
  __builtin_amdgcn_sched_group_barrier(0x100, A, 0);  // 0x100: LDS reads
#pragma unroll
  for (int i = 0; i < N - A; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 0x008: MFMA
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
  }
  __builtin_amdgcn_sched_group_barrier(0x008, A, 0);
}

}  // namespace
}  // namespace attn
}  // namespace rh3
