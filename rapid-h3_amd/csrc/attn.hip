// INT8 flash attention for gfx950, head_dim 128, non-causal.
//
// Pre-pass (HBM-bound):
//   stats_kernel   per (256-token chunk, head): float64 channel sums of K (after the optional per-head
//                  RMSNorm + RoPE) -> part [H][nchunk][128]           (attn_int8.cu:80-109 semantics)
//   kmean_kernel   kmean[h][d] = fp32(sum_chunks part / Sk)            (attn_int8.cu:95-109)
//   quant_kernel   per (128-token block, head): [RMSNorm + RoPE] -> [- kmean] -> one scale per block
//                  sc = max(amax, 1e-8) / 127, q = rint(x / sc)        (attn_int8.cu:402-443,
//                  bench/attn_emulate.py:10-18) -> codes [H][Spad][128] int8, scales [H][Spad/128]
//   vt_kernel      V [S][H][128] bf16 -> Vt [H][128][Skpad] bf16, keys permuted inside 32-key groups
//                  so that the P.V operand of each lane is one 16-byte LDS read
// Main kernel: per (384-query block, head) workgroup of 12 waves, 32 queries per wave, 64-key steps.
//   S^T = K8 . Q8^T on v_mfma_i32_32x32x32_i8 (keys on rows, queries on lanes), one fp32 dequant
//   multiply per score c = qs[qblock] * ks[kblock] * scale * log2(e) (the 128x128 tile shares both
//   block scales), online softmax in the exp2 domain, P rounded to bf16, and O^T += Vt . P^T on
//   v_mfma_f32_32x32x16_bf16 (D on rows, queries on lanes, so the per-query rescale is per lane).
//   The row sum l adds the same bf16-rounded P the MFMA consumes (attn_int8.cu:8-10, :652-656).
//   K and Vt tiles (8 + 16 KiB per step) go through a 4-slot LDS ring with XOR-swizzled 16-byte chunks.
//   With one workgroup per CU the grid runs in rounds; a last round at most half full runs as two key
//   halves per workgroup (fp32 partials), merged by attn_combine_kernel.
#include <cstdlib>
#include <mutex>
#include <type_traits>

#include "attn_common.hpp"
#include "attn_layout.hpp"

namespace rh3 {
namespace {

using namespace attn;

constexpr int BLK = 128;     // quantization block and attention tile (tokens)

// ------------------------------------------------------------------ per-block quantizer
// grid (H, Spad/128) (heads fastest, so the workgroups of one token block run together and share its rope-table
// rows in L2), 256 threads: wave w handles tokens w*32 .. w*32+31 of the block, 4 per pass
// knorm (K only, may be null): per block, an upper bound of the largest L2 norm of a token's 128 int8 codes,
// which lets the main kernel bound every logit of the block without scanning its scores
__global__ void __launch_bounds__(256) quant_kernel(const uint16_t* __restrict__ x, int64_t x_ss, int64_t x_sh,
                                                    int64_t S, int64_t Spad, RR rr, const float* __restrict__ mean,
                                                    int8_t* __restrict__ codes, float* __restrict__ scales,
                                                    float* __restrict__ knorm) {
  __shared__ float wmax[4];
  __shared__ int wnorm[4];
  const int h = blockIdx.x, blk = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, sub = lane >> 4;
  float mv[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (mean) {
    const float4 a = *reinterpret_cast<const float4*>(mean + h * D + 8 * l16);
    const float4 b = *reinterpret_cast<const float4*>(mean + h * D + 8 * l16 + 4);
    mv[0] = a.x; mv[1] = a.y; mv[2] = a.z; mv[3] = a.w; mv[4] = b.x; mv[5] = b.y; mv[6] = b.z; mv[7] = b.w;
  }
  float w[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (rr.tab) load8(rr.w + 8 * l16, w);
  float v[8][8];
  float amax = 0.0f;
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const int64_t s = static_cast<int64_t>(blk) * BLK + wave * 32 + p * 4 + sub;
    const bool ok = s < S;
    // the row and its rope-table row are loaded together (rows past S read row S - 1 and are zeroed below)
    const int64_t sl = ok ? s : S - 1;
    const uint4 rx = *reinterpret_cast<const uint4*>(x + sl * x_ss + h * x_sh + 8 * l16);
    uint4 rt[4];
    if (rr.tab) rope_tab8_raw(rr, l16, sl, rt);
    unpack8(rx, v[p]);
    if (rr.tab) rms_rope8_raw(v[p], lane, rr, w, rt);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v[p][e] = ok ? v[p][e] - mv[e] : 0.0f;
      amax = fmaxf(amax, fabsf(v[p][e]));
    }
  }
  amax = wave_max(amax);
  if (lane == 0) wmax[wave] = amax;
  __syncthreads();
  const float bm = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  const float sc = fmaxf(bm, 1e-8f) / 127.0f;
  const float inv = 1.0f / sc;
  if (tid == 0) scales[static_cast<int64_t>(h) * (Spad / BLK) + blk] = sc;
  int n2 = 0;  // largest sum of squared codes over this lane's rows (each row's sum spans its 16 lanes)
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const int64_t s = static_cast<int64_t>(blk) * BLK + wave * 32 + p * 4 + sub;
    // rint(x / sc) clamped to +-127: the multiply by 1/sc decides all lanes but those within 2^-12 of a
    // half-integer, and one wave vote per 8 values sends only those through the IEEE division
    const uint2 c8 = quant8_i8(v[p], sc, inv);
    *reinterpret_cast<uint2*>(codes + (static_cast<int64_t>(h) * Spad + s) * D + 8 * l16) = c8;
    if (knorm) {
      int r = __builtin_amdgcn_sdot4(static_cast<int>(c8.x), static_cast<int>(c8.x), 0, false);
      r = __builtin_amdgcn_sdot4(static_cast<int>(c8.y), static_cast<int>(c8.y), r, false);
      r = row_sum16_i(r);
      n2 = max(n2, r);
    }
  }
  if (knorm) {
#pragma unroll
    for (int o = 16; o < 64; o <<= 1) n2 = max(n2, __shfl_xor(n2, o, 64));
    if (lane == 0) wnorm[wave] = n2;
    __syncthreads();
    if (tid == 0) {
      // the integer is exact in fp32 (<= 128 * 127^2); sqrt rounded, then pushed up past any rounding
      const int m = max(max(wnorm[0], wnorm[1]), max(wnorm[2], wnorm[3]));
      knorm[static_cast<int64_t>(h) * (Spad / BLK) + blk] = sqrtf(static_cast<float>(m)) * 1.0001f;
    }
  }
}

void launch_quant(dim3 grid, hipStream_t st, const uint16_t* x, int64_t x_ss, int64_t x_sh, int64_t S, int64_t Spad,
                  const RR& rr, const float* mean, int8_t* codes, float* scales, float* knorm) {
  hipLaunchKernelGGL(quant_kernel, grid, dim3(256), 0, st, x, x_ss, x_sh, S, Spad, rr, mean, codes, scales, knorm);
}

// ------------------------------------------------------------------ V transpose
// Position p of a 32-key group holds key perm32(p): p = 16*m + 8*g + e  <->  key = 16*m + 8*(e/4) + 4*g + e%4,
// the key order of lane group g's B fragment (registers 8m..8m+7 of the S^T accumulator).
__device__ __forceinline__ int perm32(int p) {
  const int m = p >> 4, g = (p >> 3) & 1, e = p & 7;
  return 16 * m + 8 * (e >> 2) + 4 * g + (e & 3);
}

// grid (H, Skpad/64) (heads fastest, so a block's token rows are read together), 256 threads
__global__ void __launch_bounds__(256) vt_kernel(const uint16_t* __restrict__ v, int64_t v_ss, int64_t v_sh,
                                                 int64_t S, int64_t Spad, uint16_t* __restrict__ vt) {
  constexpr int T = 64, P = D + 8;
  __shared__ uint16_t tile[T * P];
  const int h = blockIdx.x, tid = threadIdx.x;
  const int64_t s0 = static_cast<int64_t>(blockIdx.y) * T;
  for (int i = tid; i < T * D / 8; i += 256) {
    const int r = i / (D / 8), c8 = (i % (D / 8)) * 8;
    uint4 val = make_uint4(0, 0, 0, 0);
    if (s0 + r < S) val = *reinterpret_cast<const uint4*>(v + (s0 + r) * v_ss + h * v_sh + c8);
    *reinterpret_cast<uint4*>(&tile[r * P + c8]) = val;
  }
  __syncthreads();
  for (int i = tid; i < D * (T / 8); i += 256) {
    const int d = i / (T / 8), pc = (i % (T / 8)) * 8;  // positions pc..pc+7 of this 64-key slab
    uint16_t o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int p = pc + e;
      const int key = (p & ~31) + perm32(p & 31);
      o[e] = tile[key * P + d];
    }
    uint4 pk;
    pk.x = o[0] | (static_cast<uint32_t>(o[1]) << 16);
    pk.y = o[2] | (static_cast<uint32_t>(o[3]) << 16);
    pk.z = o[4] | (static_cast<uint32_t>(o[5]) << 16);
    pk.w = o[6] | (static_cast<uint32_t>(o[7]) << 16);
    *reinterpret_cast<uint4*>(vt + (static_cast<int64_t>(h) * D + d) * Spad + s0 + pc) = pk;
  }
}

// ------------------------------------------------------------------ main kernel
struct FwdArgs {
  const int8_t* q8;  // [H][Sqpad][128]
  const float* qs;   // [H][Sqpad/128]
  const int8_t* k8;  // [H][Skpad][128]
  const float* ks;   // [H][Skpad/128]
  const float* kn;   // [H][Skpad/128] bound of the largest L2 norm of a key's codes per block
  const uint16_t* vt;  // [H][128][Skpad]
  uint16_t* out;
  int64_t o_ss, o_sh;
  int64_t Sq, Sk, Sqpad, Skpad;
  float scale_log2;
  int nqb;      // query blocks per head; (head, query block) id = h * nqb + qb (query blocks fastest)
  int nmain;    // workgroups 0 .. nmain-1 run ids 0 .. nmain-1 whole
  int npair;    // items nmain + i and nmain + npair + i run the two key halves of id nmain + i
  float* tail;  // [2][npair][FWD_BQ][TAIL_ROW] fp32 partials of the split ids
  int* ctr;     // CLAIM_COUNTERS work counters, zero at launch (claim_item)
};

// a wave-uniform float (lane 0's value), held in an SGPR
__device__ __forceinline__ float uniform(float x) {
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x)));
}

// XOR swizzle of the 16-byte chunks of a V^T slot row d (128 B rows): chunk c at c ^ vsw(d). gfx950 serves a
// 16-byte LDS read 16 lanes at a time over 64 banks; the 16 lanes of a P.V fragment read rows d .. d+15 at one
// chunk, and rows d and d+8 share a bank group under c ^ (d & 7) (a 2-way conflict on every V read, 40 % of the
// kernel's LDS cycles). Folding in d >> 3 spreads the 16 rows over 16 groups.
__device__ __forceinline__ int vsw(int d) { return ((d & 31) ^ ((d & 31) >> 3)) & 7; }

// 12 waves (3 per SIMD), 32 queries each = 384 queries per workgroup (three 128-query scale blocks);
// at most 168 registers per wave, so a step covers 64 keys. Per wave and step: 8 i8 MFMAs (S^T = K Q^T), 16 bf16
// MFMAs (O^T += V^T P^T) and ~105 VALU instructions (the softmax of 32 scores per lane). Each 32x32 MFMA also
// holds the SIMD's VALU issue for a few cycles, so the kernel is bound by VALU issue as much as by the MFMA pipe:
// every vector instruction the step does not need is taken out (no vector address arithmetic for the copies, and
// no score scan while a bound proves the running max is still good).
constexpr int FWD_WAVES = 12, FWD_NT = FWD_WAVES * 64, FWD_BQ = FWD_WAVES * 32;
static_assert(FWD_BQ == attn_ws::FWD_BQ, "workspace layout constants");
constexpr int TAIL_ROW = attn_ws::TAIL_ROW;
constexpr int MAGIC_I = 0x4B400000;  // bits of 1.5 * 2^23
constexpr float MAGIC_F = 12582912.0f;
constexpr int STEP = 64;  // keys per step
// lazy rescale: after a scan, the reference max moves only when the step max exceeds it by more than 2^8
constexpr float RESCALE_LOG2 = 8.0f;
// no scan while every logit of the step is provably below mref + 2^6 (then P < 2^64: O and l stay far from the
// fp32 range for |v| < 2^40, and bf16 P keeps its relative precision at any magnitude)
constexpr float BOUND_LOG2 = 64.0f;
constexpr int KSLOT = STEP * D;      // K tile: 64 keys x 128 B, chunk c of row r at c ^ ((r ^ (r >> 3)) & 7)
constexpr int VSLOT = D * STEP * 2;  // V^T tile: 128 d x 64 keys x 2 B, chunk c of row d at c ^ vsw(d)
constexpr int NRING = 4;             // slots of the K ring and of the V^T ring

// Step j reads K(j) and V^T(j) from ring slot u = (j - j0) % 4 and first copies K(j+2), V^T(j+2) into slot
// (u + 2) % 4, last read in step j-2 (every wave has passed the end-of-step barrier of step j-1). Steps past Sk
// are not run; the ragged last step is a separate instantiation, so the full steps carry no key mask.
// SPLIT: bid < npair runs the first half of the steps of id nmain + bid, bid >= npair the second half of id
// nmain + bid - npair, and each writes its unnormalised O, running max and row sum to the tail partials.
template <bool SPLIT>
__device__ __forceinline__ void fwd_body(const FwdArgs& a, const int bid, int8_t* kring, int8_t* vring,
                                         float2* kscale) {
  const int half = SPLIT ? bid / a.npair : 0;
  const int id = SPLIT ? a.nmain + bid - half * a.npair : bid;
  const int h = id / a.nqb, qb = id - h * a.nqb;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, g = lane >> 5;
  const int64_t q = static_cast<int64_t>(qb) * FWD_BQ + wave * 32 + l32;

  // the Q operands are padded to 128 queries; a workgroup's last blocks may lie past them (then they are
  // computed on zero codes and never stored)
  const bool qin = q < a.Sqpad;
  v4i qf[4];
  {
    const int8_t* qp = a.q8 + (static_cast<int64_t>(h) * a.Sqpad + q) * D + g * 16;
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) qf[ds] = qin ? *reinterpret_cast<const v4i*>(qp + ds * 32) : v4i{0, 0, 0, 0};
  }
  // a wave's 32 queries lie in one 128-query scale block, all below Sqpad or all past it: the scale is uniform
  const float qscale = uniform((qin ? a.qs[static_cast<int64_t>(h) * (a.Sqpad / BLK) + (q >> 7)] : 0.0f) * a.scale_log2);
  // |q8 . k8| <= |q8| |k8|: the wave's largest query norm (each lane's 64 codes plus the partner lane's 64),
  // pushed up past the roundings of the bound below, times the query scale
  float qbound;
  {
    int n2 = 0;
#pragma unroll
    for (int ds = 0; ds < 4; ++ds)
#pragma unroll
      for (int e = 0; e < 4; ++e) n2 = __builtin_amdgcn_sdot4(qf[ds][e], qf[ds][e], n2, false);
    n2 += __shfl_xor(n2, 32, 64);
#pragma unroll
    for (int o = 1; o < 32; o <<= 1) n2 = max(n2, __shfl_xor(n2, o, 64));
    qbound = uniform(qscale * (sqrtf(static_cast<float>(n2)) * 1.0001f));
  }
  const int nkb = static_cast<int>(a.Skpad / BLK);
  for (int i = tid; i < nkb; i += FWD_NT) {
    const float ksc = a.ks[static_cast<int64_t>(h) * nkb + i];
    kscale[i] = make_float2(ksc, ksc * a.kn[static_cast<int64_t>(h) * nkb + i]);
  }

  // Copies go global -> LDS directly (lane l of a wave writes LDS base + 16*l), so the XOR swizzles are applied on
  // the global side. K slot: 512 chunk positions (64 rows x 8), one copy each for waves 0-7; V^T slot: 1024
  // positions (128 rows x 8), waves 0-7 one copy each (positions 64w + lane), waves 8-11 two each (positions
  // 512 + 64(2(w-8) + i) + lane). Position p of a slot is its byte 16p. Each copy is a per-step scalar base plus a
  // fixed lane offset.
  const int8_t* kbase = a.k8 + static_cast<int64_t>(h) * a.Skpad * D;
  const int8_t* vbase = reinterpret_cast<const int8_t*>(a.vt + static_cast<int64_t>(h) * D * a.Skpad);
  auto kpos = [&](int p) { const int row = p >> 3, pc = p & 7; return row * 128 + ((pc ^ ((row ^ (row >> 3)) & 7)) << 4); };
  auto vpos = [&](int p) {
    const int d = p >> 3, pc = p & 7;
    return static_cast<int>(d * a.Skpad * 2 + ((pc ^ vsw(d)) << 4));
  };
  const bool kwave = wave < 8;
  const uint32_t go0 = static_cast<uint32_t>(kwave ? kpos(wave * 64 + lane) : vpos(512 + 2 * (wave - 8) * 64 + lane));
  const uint32_t go1 = static_cast<uint32_t>(kwave ? vpos(wave * 64 + lane) : vpos(512 + (2 * (wave - 8) + 1) * 64 + lane));
  const uint32_t ds0 = static_cast<uint32_t>(kwave ? wave * 1024 : 8192 + 2 * (wave - 8) * 1024);
  const uint32_t ds1 = static_cast<uint32_t>(kwave ? wave * 1024 : 8192 + (2 * (wave - 8) + 1) * 1024);
  const uint32_t kring_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(kring));
  const uint32_t vring_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(vring));
  const int nfull = static_cast<int>(a.Sk / STEP), rem = static_cast<int>(a.Sk % STEP);
  const int nsteps = nfull + (rem > 0);
  // steps [j0, j1) of this workgroup; a split's first half holds only full steps (nsteps / 2 <= nfull)
  const int j0 = half ? nsteps / 2 : 0, j1 = SPLIT && !half ? nsteps / 2 : nsteps;
  auto load_step = [&](int j) __attribute__((always_inline)) {
    const uint32_t u = static_cast<uint32_t>(j - j0) & (NRING - 1);
    const int jj = min(j, nsteps - 1);  // clamped: every step issues the same copies; the copy lands unread
    const int8_t* vb = vbase + static_cast<int64_t>(jj) * (STEP * 2);
    if (kwave) {
      lds_dma16_s(kbase + static_cast<int64_t>(jj) * KSLOT, go0, kring_lds + u * KSLOT + ds0);
      lds_dma16_s(vb, go1, vring_lds + u * VSLOT + ds1);
    } else {
      lds_dma16_s(vb, go0, vring_lds + u * VSLOT + ds0);
      lds_dma16_s(vb, go1, vring_lds + u * VSLOT + ds1);
    }
  };

  // Lane parts of the LDS read addresses inside slot 0. K fragment (kb, ds): row kb*32 + l32, chunk
  // 2ds + g, stored at chunk ^ ((row ^ (row >> 3)) & 7) = (2ds ^ 4kb) ^ y with y = (g ^ l32 ^ (l32 >> 3)) & 7,
  // so the 8 reads use 4 lane offsets koff[(2ds ^ 4kb) / 2] plus the slot's u*KSLOT and the immediate kb*4096. V^T
  // fragment (kb, m, db): row db*32 + l32, chunk 4kb + 2m + g at chunk ^ vsw(l32): 4 lane offsets voff[2kb + m]
  // plus u*VSLOT and the immediate db*4096.
  uint32_t koff[4], voff[4];
  {
    const int y = (g ^ l32 ^ (l32 >> 3)) & 7;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      koff[i] = kring_lds + l32 * 128 + (((2 * i) ^ y) << 4);
      voff[i] = vring_lds + l32 * 128 + (((2 * i + g) ^ vsw(l32)) << 4);
    }
  }

  v16f o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[i][r] = 0.0f;
  float mref = -INFINITY, lrow = 0.0f;
  const v2bf ones = {static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)};
  // S^T accumulators start at the bits of 1.5*2^23: the integer register then reads as the float
  // 1.5*2^23 + acc (|acc| <= 128 * 127^2 < 2^22), so the exponent needs no int -> float conversion
  v16i magic;
#pragma unroll
  for (int r = 0; r < 16; ++r) magic[r] = MAGIC_I;

  // S^T[key][query] = K8 . Q8^T of the step in slot U: lane (l32, g) of s[kb] holds query l32 and step keys
  // kb*32 + 8*(r/4) + 4*g + r%4
  v16i s[2];
  auto qk = [&](const uint32_t u) __attribute__((always_inline)) {
    uint32_t ka[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ka[i] = koff[i] + u * KSLOT;
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const v4i kf = lds_read16(ka[ds ^ (2 * kb)] + kb * 4096);
        s[kb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(kf, qf[ds], ds == 0 ? magic : s[kb], 0, 0, 0);
      }
    }
    read_ahead<8, 3>();
  };
  // online softmax of step j's scores and O^T += V^T(j) . P^T; TAIL steps hold 1..63 keys below Sk
  uint32_t pk[2][8];  // P of the current step, bf16 pairs, the B operand of the P.V MFMAs
  // kk: the step's key-block (scale, scale x code-norm bound), read from LDS before the step's Q.K^T so that the
  // read's latency runs under the MFMAs (read after them, the wave waited for it: 0.7 % of the kernel)
  auto softmax = [&](const int j, auto tail, const float2 kk) __attribute__((always_inline)) {
    constexpr bool TAIL = decltype(tail)::value;
    const int nvalid = TAIL ? static_cast<int>(a.Sk - static_cast<int64_t>(j) * STEP) : STEP;
    const float c = qscale * kk.x;
    // Every logit of the step is at most qbound * kk.y (Cauchy-Schwarz on the codes, in the exp2 domain). While
    // that is below mref + 64 for all the wave's queries the step needs no max; otherwise scan the step's
    // scores (c > 0, so the max score is c * the max int32 accumulator over the valid keys; a tail step holds key
    // j*64, so every query's max covers at least one key) and move mref if the max passed it by 2^8.
    float mt = -INFINITY;
    if (__builtin_amdgcn_ballot_w64(qbound * kk.y > mref + BOUND_LOG2) != 0) {
      int mi = INT_MIN;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (!TAIL || kb * 32 + 8 * (r >> 2) + 4 * g + (r & 3) < nvalid) mi = max(mi, s[kb][r]);
      mi = max_halves(mi);
      mt = static_cast<float>(mi - MAGIC_I) * c;
    }
    if (__builtin_amdgcn_ballot_w64(mt > mref + RESCALE_LOG2) != 0) {
      const float mnew = fmaxf(mref, mt);
      const float alpha = __builtin_amdgcn_exp2f(mref - mnew);
      mref = mnew;
      lrow = lrow * alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] = o[db][r] * alpha;
    }
    // the accumulator holds the bits of 1.5*2^23 + acc, so fma(bits, c, nb) = acc c - mref with the constant
    // nb = -1.5*2^23 c - mref rounded once: the same rounding error for every score of this query and step
    const float nb = fmaf(-MAGIC_F, c, -mref);
    // P = 2^(t - mref) in bf16 (P < 2^64); keys past Sk get P = 0 (lane mask on the packed words)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const float p0 = __builtin_amdgcn_exp2f(fmaf(__int_as_float(s[kb][r]), c, nb));
        const float p1 = __builtin_amdgcn_exp2f(fmaf(__int_as_float(s[kb][r + 1]), c, nb));
        pk[kb][r >> 1] = pk_bf16(p0, p1);
      }
    if constexpr (TAIL) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int w = 0; w < 8; ++w) {
          const int key = kb * 32 + 8 * (w >> 1) + 4 * g + 2 * (w & 1);  // keys of bf16 halves lo / hi
          const uint32_t lo = key < nvalid ? 0x0000ffffu : 0u, hi = key + 1 < nvalid ? 0xffff0000u : 0u;
          pk[kb][w] &= lo | hi;
        }
    }
    // the row sum adds exactly the bf16 values the P.V MFMA consumes
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int w = 0; w < 8; ++w)
        lrow = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2bf, pk[kb][w]), ones, lrow, false);
  };
  // O^T[d][query] += V^T . P^T of the step in slot u
  auto pv = [&](const uint32_t u) __attribute__((always_inline)) {
    uint32_t va[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) va[i] = voff[i] + u * VSLOT;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        v4i pw;
        pw[0] = pk[kb][4 * m + 0]; pw[1] = pk[kb][4 * m + 1]; pw[2] = pk[kb][4 * m + 2]; pw[3] = pk[kb][4 * m + 3];
        const v8bf pf = __builtin_bit_cast(v8bf, pw);
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          const v4i vw = lds_read16(va[2 * kb + m] + db * 4096);
          o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, vw), pf, o[db], 0, 0, 0);
        }
      }
    }
    read_ahead<16, 3>();
  };

  // Barrier B_j ends the use of ring slot j: every wave meets it after pv(j). Each wave issues the copies of step
  // j+2 right after B_(j-1), into the slot last read in step j-2; before B_j it waits for its copies of step j+1
  // (vmcnt(2) leaves the two issued in step j in flight), so slot j+1 is complete past B_j.
  auto barrier = [&]() __attribute__((always_inline)) {
    asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  auto step = [&](const int j, auto tail) __attribute__((always_inline)) {
    const uint32_t slot = static_cast<uint32_t>(j - j0) & (NRING - 1);
    const float2 kk = kscale[j >> 1];
    load_step(j + 2);
    qk(slot);
    softmax(j, tail, kk);
    pv(slot);
    barrier();
  };

  load_step(j0);
  load_step(j0 + 1);
  // vmcnt(0) through the builtin, so the compiler also sees the Q loads above as complete and adds no
  // wait of its own inside the loop (gfx9 s_waitcnt: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8])
  __builtin_amdgcn_s_waitcnt(0x0f70);
  __syncthreads();
  const int jf = min(j1, nfull);
  for (int j = j0; j < jf; ++j) step(j, std::false_type{});
  if (rem > 0 && j1 == nsteps) step(nfull, std::true_type{});
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no global->LDS copy outlives the workgroup

  const float lt = lrow + __shfl_xor(lrow, 32, 64);
  if constexpr (SPLIT) {
    if (q < a.Sq) {
      float* tp = a.tail + ((static_cast<int64_t>(half) * a.npair + (id - a.nmain)) * FWD_BQ + wave * 32 + l32) * TAIL_ROW;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq)
          *reinterpret_cast<float4*>(tp + db * 32 + 8 * rq + 4 * g) =
              make_float4(o[db][4 * rq], o[db][4 * rq + 1], o[db][4 * rq + 2], o[db][4 * rq + 3]);
      if (g == 0) *reinterpret_cast<float2*>(tp + D) = make_float2(mref, lt);
    }
    return;
  }
  const float il = 1.0f / lt;
  if (q < a.Sq) {
    uint16_t* op = a.out + q * a.o_ss + static_cast<int64_t>(h) * a.o_sh;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int d = db * 32 + 8 * rq + 4 * g;
        uint2 w;
        w.x = pk_bf16(o[db][4 * rq + 0] * il, o[db][4 * rq + 1] * il);
        w.y = pk_bf16(o[db][4 * rq + 2] * il, o[db][4 * rq + 3] * il);
        *reinterpret_cast<uint2*>(op + d) = w;
      }
  }
}

// One launch over nmain + 2 npair items, the unsplit ids first, then the split halves (which take CUs as the last
// unsplit items finish). A workgroup runs the item it claims when it starts (claim_item: its XCD's share of the
// unsplit ids first), not the one its position names: the grid is dealt to the XCDs in fixed shares, and the XCDs
// run at different clocks (workgroup times differ by up to 7 % between them), so fixed items would leave the fast
// XCDs idle while the slowest finishes. The grid holds more workgroups than items; a fast XCD starts its queued
// workgroups sooner and takes more items, and the workgroups that find the items gone return at once. The LDS rings and scale table are
// declared once, shared by both bodies.
__global__ void __launch_bounds__(FWD_NT, 1) attn_fwd_kernel(const FwdArgs a) {
  __shared__ __attribute__((aligned(16))) int8_t ring[NRING * (KSLOT + VSLOT)];
  __shared__ float2 kscale[4096];  // per-128-key-block (K scale, K scale x key-norm bound) of this head
  __shared__ int item_s;
  if (threadIdx.x == 0) item_s = claim_item(a.ctr, a.nmain, 2 * a.npair, blockIdx.x);
  __syncthreads();
  const int item = __builtin_amdgcn_readfirstlane(item_s);
  if (item < 0) return;
  if (item < a.nmain)
    fwd_body<false>(a, item, ring, ring + NRING * KSLOT, kscale);
  else
    fwd_body<true>(a, item - a.nmain, ring, ring + NRING * KSLOT, kscale);
}

// Merge of the two key halves of a split workgroup: m = max(m0, m1), O = (O0 2^(m0-m) + O1 2^(m1-m)) / l with
// l = l0 2^(m0-m) + l1 2^(m1-m). grid (npair, FWD_BQ / 16), 256 threads: 16 queries x 16 lanes of 8 dims.
__global__ void __launch_bounds__(256) attn_combine_kernel(const float* __restrict__ tail, int npair, int nmain,
                                                           int nqb, int64_t Sq, uint16_t* __restrict__ out,
                                                           int64_t o_ss, int64_t o_sh) {
  const int pair = blockIdx.x, ql = blockIdx.y * 16 + (threadIdx.x >> 4), c = threadIdx.x & 15;
  const int id = nmain + pair, h = id / nqb, qb = id - h * nqb;
  const int64_t q = static_cast<int64_t>(qb) * FWD_BQ + ql;
  if (q >= Sq) return;
  const float* t0 = tail + (static_cast<int64_t>(pair) * FWD_BQ + ql) * TAIL_ROW;
  const float* t1 = t0 + static_cast<int64_t>(npair) * FWD_BQ * TAIL_ROW;
  const float2 ml0 = *reinterpret_cast<const float2*>(t0 + D), ml1 = *reinterpret_cast<const float2*>(t1 + D);
  const float m = fmaxf(ml0.x, ml1.x);
  const float a0 = __builtin_amdgcn_exp2f(ml0.x - m), a1 = __builtin_amdgcn_exp2f(ml1.x - m);
  const float il = 1.0f / (ml0.y * a0 + ml1.y * a1);
  float r[8];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float4 x = *reinterpret_cast<const float4*>(t0 + 8 * c + 4 * i);
    const float4 y = *reinterpret_cast<const float4*>(t1 + 8 * c + 4 * i);
    r[4 * i + 0] = (x.x * a0 + y.x * a1) * il;
    r[4 * i + 1] = (x.y * a0 + y.y * a1) * il;
    r[4 * i + 2] = (x.z * a0 + y.z * a1) * il;
    r[4 * i + 3] = (x.w * a0 + y.w * a1) * il;
  }
  // two 8-byte stores, the alignment the entry points require of out (its strides are multiples of 4 elements)
  uint16_t* op = out + q * o_ss + static_cast<int64_t>(h) * o_sh + 8 * c;
  *reinterpret_cast<uint2*>(op) = make_uint2(pk_bf16(r[0], r[1]), pk_bf16(r[2], r[3]));
  *reinterpret_cast<uint2*>(op + 4) = make_uint2(pk_bf16(r[4], r[5]), pk_bf16(r[6], r[7]));
}

// ------------------------------------------------------------------ host
using attn_ws::pad;
using attn_ws::Work;
using attn_ws::layout;

int check_qkv(const char* name, const uint16_t* q, int64_t q_ss, int64_t q_sh, const uint16_t* k, int64_t k_ss,
              int64_t k_sh, const uint16_t* v, int64_t v_ss, int64_t v_sh, int64_t Sq, int64_t Sk, int64_t H) {
  RH3_REQUIRE(Sq > 0 && Sk > 0 && H > 0, "%s: sizes must be positive (Sq=%lld Sk=%lld H=%lld)", name, (long long)Sq,
              (long long)Sk, (long long)H);
  // the pre-pass grids are (H, token blocks): at most 65,535 blocks of 128 tokens on either side
  RH3_REQUIRE(pad(Sq) / BLK < 65536 && H < 65536, "%s: Sq=%lld exceeds the 8,388,480-token grid limit", name,
              (long long)Sq);
  RH3_REQUIRE(pad(Sk) / BLK <= 4096, "%s: Sk=%lld exceeds the 524288-key limit of the attention kernel", name,
              (long long)Sk);
  RH3_REQUIRE(q && k && v, "%s: null q/k/v", name);
  RH3_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v), "%s: q/k/v must be 16-byte aligned", name);
  RH3_REQUIRE(q_ss % 8 == 0 && q_sh % 8 == 0 && k_ss % 8 == 0 && k_sh % 8 == 0 && v_ss % 8 == 0 && v_sh % 8 == 0,
              "%s: token/head strides must be multiples of 8 elements", name);
  return RH3_OK;
}

int prepass(const uint16_t* q, int64_t q_ss, int64_t q_sh, const uint16_t* k, int64_t k_ss, int64_t k_sh,
            const uint16_t* v, int64_t v_ss, int64_t v_sh, int64_t Sq, int64_t Sk, int64_t H, const RR& rq,
            const RR& rk, int smooth_k, const Work& w, hipStream_t st) {
  const int64_t sqp = pad(Sq), skp = pad(Sk);
  const int nchunk = static_cast<int>((Sk + CHUNK - 1) / CHUNK);
  const float* mean = nullptr;
  // With smoothing and the RMSNorm + RoPE prologue, the statistics pass already computes every K row's prologue:
  // it stores those rows (bf16, [H][Skpad][128]) in the V^T region, which vt_kernel fills only afterwards, and the K
  // quantizer reads them back without running the prologue a second time (the same values, so the same codes).
  const bool staged = smooth_k && rk.tab;
  if (smooth_k) {
    launch_stats(dim3(H, nchunk), st, k, k_ss, k_sh, Sk, rk, w.part, staged ? w.vt : nullptr, skp * D);
    hipLaunchKernelGGL(kmean_kernel, dim3(H), dim3(KMEAN_NT), 0, st, w.part, nchunk, Sk, w.kmean);
    mean = w.kmean;
  } else {
    // a fill kernel, not hipMemsetAsync, so the call stays safe inside a captured HIP graph
    hipLaunchKernelGGL(zero_kernel, dim3((H * D + 255) / 256), dim3(256), 0, st, w.kmean, H * D);
  }
  launch_quant(dim3(H, sqp / BLK), st, q, q_ss, q_sh, Sq, sqp, rq, static_cast<const float*>(nullptr), w.q8, w.qs,
               nullptr);
  if (staged)
    launch_quant(dim3(H, skp / BLK), st, w.vt, D, skp * D, Sk, skp, RR{nullptr, nullptr, 0.f, 0}, mean, w.k8, w.ks,
                 w.kn);
  else
    launch_quant(dim3(H, skp / BLK), st, k, k_ss, k_sh, Sk, skp, rk, mean, w.k8, w.ks, w.kn);
  hipLaunchKernelGGL(vt_kernel, dim3(H, skp / 64), dim3(256), 0, st, v, v_ss, v_sh, Sk, skp, w.vt);
  return launch_status("attention prepass");
}

int forward(const Work& w, int64_t Sq, int64_t Sk, int64_t H, float scale, uint16_t* out, int64_t o_ss,
            int64_t o_sh, hipStream_t st) {
  const int64_t nwg = attn_ws::fwd_blocks(Sq, H);
  RH3_REQUIRE(nwg < (int64_t{1} << 30) / FWD_NT, "attention forward: %lld workgroups exceed the grid limit",
              (long long)nwg);
  const int nqb = static_cast<int>((Sq + FWD_BQ - 1) / FWD_BQ);
  // One workgroup per CU: the grid runs in rounds of `cus` workgroups. When the last round is at most half
  // full, its workgroups run as two key halves each (a round half as long) and a merge kernel combines them.
  const int cus = device_cus();
  const int64_t last = cus > 0 ? nwg % cus : 0;
  const int64_t nsteps = (Sk + STEP - 1) / STEP;
  // The split changes how a split workgroup's keys are summed (two fp32 halves merged), so a head's output can
  // differ in the last bits with the grid (H, Sq, the CU count). RH3_ATTN_SPLIT=0 turns it off for callers that
  // need the same bits on every grid.
  const char* env = getenv("RH3_ATTN_SPLIT");
  const bool split_ok = !(env && env[0] == '0');
  const int npair = split_ok && w.tail && nwg > cus && last > 0 && 2 * last <= cus && last <= attn_ws::TAIL_MAX &&
                            nsteps >= 8
                        ? static_cast<int>(last) : 0;
  const int nmain = static_cast<int>(nwg - npair);
  const FwdArgs f{w.q8, w.qs, w.k8, w.ks, w.kn, w.vt, out, o_ss, o_sh, Sq, Sk, pad(Sq), pad(Sk),
                  scale * 1.4426950408889634f, nqb, nmain, npair, w.tail, w.ctr};
  // a quarter more workgroups than items: room for the fastest XCD to take a quarter more than its share
  const int64_t items = nmain + 2 * static_cast<int64_t>(npair);
  const int64_t grid = items + (items + 3) / 4;
  // the counter is cleared by a fill kernel, not hipMemsetAsync, so the call stays safe inside a captured HIP graph
  hipLaunchKernelGGL(zero_kernel, dim3(1), dim3(64), 0, st, reinterpret_cast<float*>(w.ctr), CLAIM_COUNTERS);
  hipLaunchKernelGGL(attn_fwd_kernel, dim3(static_cast<uint32_t>(grid)), dim3(FWD_NT), 0, st, f);
  if (npair > 0)
    hipLaunchKernelGGL(attn_combine_kernel, dim3(npair, FWD_BQ / 16), dim3(256), 0, st, w.tail, npair, nmain, nqb, Sq,
                       out, o_ss, o_sh);
  return launch_status("attention forward");
}

// ------------------------------------------------------------------ standalone RMSNorm + RoPE (in place)
// The per-head prologue of the pre-pass on its own, for callers that hand the roped q / k to another attention:
// 16 lanes per (token, head) row, heads fastest (rows of one token are contiguous in the qkv output), grid.y 0 = q,
// 1 = k. rms_rope8 is the function the pre-pass applies, so the results are the pre-pass's own operands bit for bit.
// Lanes past the last row compute on a clamped row (the RoPE partner exchange needs every lane) and store nothing.
__global__ void __launch_bounds__(256) rms_rope_kernel(uint16_t* q, int64_t q_ss, int64_t q_sh, uint16_t* k,
                                                       int64_t k_ss, int64_t k_sh, int64_t S, int64_t H, RR rq,
                                                       RR rk) {
  const int lane = threadIdx.x & 63;
  const bool isk = blockIdx.y != 0;
  const int64_t rows = S * H;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 16 + (threadIdx.x >> 4);
  const int64_t rc = r < rows ? r : rows - 1;
  const int64_t s = rc / H, h = rc - s * H;
  uint16_t* p = (isk ? k + s * k_ss + h * k_sh : q + s * q_ss + h * q_sh) + 8 * (lane & 15);
  float x[8];
  load8(p, x);
  rms_rope8(x, lane, isk ? rk : rq, s);
  if (r < rows) {
    uint4 o;
    o.x = pack_bf2(x[0], x[1]);
    o.y = pack_bf2(x[2], x[3]);
    o.z = pack_bf2(x[4], x[5]);
    o.w = pack_bf2(x[6], x[7]);
    *reinterpret_cast<uint4*>(p) = o;
  }
}

int check_rr(const char* name, const uint16_t* tab, int rot, const uint16_t* qw, const uint16_t* kw) {
  RH3_REQUIRE(tab && qw && kw, "%s: tab, qw and kw are required", name);
  RH3_REQUIRE(rot == 96 || rot == 128, "%s: rot_dim %d (96 or 128 supported)", name, rot);
  RH3_REQUIRE(aligned16(tab) && aligned16(qw) && aligned16(kw), "%s: tab/qw/kw must be 16-byte aligned", name);
  return RH3_OK;
}

}  // namespace
}  // namespace rh3

// ------------------------------------------------------------------ allocation-free variant
// The workspace of rh3_int8_attention_noalloc: a file-scope device array, one copy per GPU for the life of the
// process. It is part of the code object, so every process that loads the library holds these 16 MiB on each GPU
// where the module is loaded, whether or not it calls this entry point. Host code never passes `scratch` itself (in host code the name is only a stand-in): each device's
// address comes from hipGetSymbolAddress once, with that device current, and is kept in g_scratch.
constexpr int64_t NOALLOC_SCRATCH_BYTES = int64_t{16} << 20;
static __device__ __align__(256) char scratch[NOALLOC_SCRATCH_BYTES];

namespace rh3 {
namespace {
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch[MAX_DEVICES] = {};

// this GPU's scratch address: the device of the stream (the current device for the null stream)
int scratch_of(hipStream_t stream, void** out) {
  int cur = 0;
  RH3_REQUIRE(hipGetDevice(&cur) == hipSuccess, "int8_attention_noalloc: no current HIP device");
  int dev = cur;
  if (stream) RH3_REQUIRE(hipStreamGetDevice(stream, &dev) == hipSuccess, "int8_attention_noalloc: bad stream");
  RH3_REQUIRE(dev >= 0 && dev < MAX_DEVICES, "int8_attention_noalloc: device %d beyond %d", dev, MAX_DEVICES);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    if (dev != cur) RH3_REQUIRE(hipSetDevice(dev) == hipSuccess, "int8_attention_noalloc: hipSetDevice(%d)", dev);
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) (void)hipSetDevice(cur);
    RH3_REQUIRE(e == hipSuccess && p, "int8_attention_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                hipGetErrorString(e));
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return RH3_OK;
}
}  // namespace
}  // namespace rh3

using namespace rh3;

// rh3_int8_attention without a workspace argument: the pre-pass operands live in this GPU's 16 MiB scratch array,
// and the main kernel runs every workgroup whole (no split last round, whose partials would need more room). The
// pre-pass writes every element the main kernel reads, so nothing is cleared first. Calls that overlap on one GPU
// (two streams, or two host threads) share the array and race.
extern "C" int rh3_int8_attention_noalloc(const uint16_t* q, int64_t q_ss, int64_t q_sh, const uint16_t* k,
                                          int64_t k_ss, int64_t k_sh, const uint16_t* v, int64_t v_ss, int64_t v_sh,
                                          int64_t Sq, int64_t Sk, int64_t H, float scale, int smooth_k, uint16_t* out,
                                          int64_t o_ss, int64_t o_sh, hipStream_t stream) {
  clear_error();
  if (int e = check_qkv("int8_attention_noalloc", q, q_ss, q_sh, k, k_ss, k_sh, v, v_ss, v_sh, Sq, Sk, H)) return e;
  RH3_REQUIRE(out && (reinterpret_cast<uintptr_t>(out) & 7) == 0 && o_ss % 4 == 0 && o_sh % 4 == 0,
              "int8_attention_noalloc: out must be 8-byte aligned with strides multiple of 4");
  const int64_t need = layout(nullptr, Sq, Sk, H, false).bytes;
  RH3_REQUIRE(need <= NOALLOC_SCRATCH_BYTES,
              "int8_attention_noalloc: Sq=%lld Sk=%lld H=%lld needs %lld bytes of scratch, beyond its %lld-byte maximum "
              "(rh3_int8_attention takes a workspace of any size)", (long long)Sq, (long long)Sk, (long long)H,
              (long long)need, (long long)NOALLOC_SCRATCH_BYTES);
  void* base = nullptr;
  if (int e = scratch_of(stream, &base)) return e;
  const Work w = layout(base, Sq, Sk, H, false);
  const RR none{nullptr, nullptr, 0.f, 0};
  if (int e = prepass(q, q_ss, q_sh, k, k_ss, k_sh, v, v_ss, v_sh, Sq, Sk, H, none, none, smooth_k, w, stream))
    return e;
  return forward(w, Sq, Sk, H, scale, out, o_ss, o_sh, stream);
}

extern "C" int64_t rh3_attention_workspace_bytes(int64_t Sq, int64_t Sk, int64_t H) {
  if (Sq <= 0 || Sk <= 0 || H <= 0) return 0;
  return layout(nullptr, Sq, Sk, H).bytes;
}

extern "C" int rh3_attention_prepass(const uint16_t* q, int64_t q_ss, int64_t q_sh, const uint16_t* k, int64_t k_ss,
                                     int64_t k_sh, const uint16_t* v, int64_t v_ss, int64_t v_sh, int64_t Sq,
                                     int64_t Sk, int64_t H, const uint16_t* tab, int rot, const uint16_t* qw,
                                     const uint16_t* kw, float eps, int smooth_k, void* workspace,
                                     int64_t workspace_bytes, void** ptrs, hipStream_t stream) {
  clear_error();
  if (int e = check_qkv("attention_prepass", q, q_ss, q_sh, k, k_ss, k_sh, v, v_ss, v_sh, Sq, Sk, H)) return e;
  RH3_REQUIRE(ptrs, "attention_prepass: ptrs required");
  const Work w = layout(workspace, Sq, Sk, H);
  RH3_REQUIRE(workspace && aligned16(workspace) && workspace_bytes >= w.bytes,
              "attention_prepass: workspace %lld bytes < required %lld", (long long)workspace_bytes,
              (long long)w.bytes);
  RR rq{nullptr, nullptr, 0.f, 0}, rk{nullptr, nullptr, 0.f, 0};
  if (tab) {
    if (int e = check_rr("attention_prepass", tab, rot, qw, kw)) return e;
    RH3_REQUIRE(Sq == Sk, "attention_prepass: RMSNorm+RoPE needs self-attention (Sq == Sk)");
    rq = RR{tab, qw, eps, rot};
    rk = RR{tab, kw, eps, rot};
  }
  if (int e = prepass(q, q_ss, q_sh, k, k_ss, k_sh, v, v_ss, v_sh, Sq, Sk, H, rq, rk, smooth_k, w, stream)) return e;
  ptrs[0] = w.q8; ptrs[1] = w.qs; ptrs[2] = w.k8; ptrs[3] = w.ks; ptrs[4] = w.kmean; ptrs[5] = w.vt;
  return RH3_OK;
}

extern "C" int rh3_attention_prepass_qkv(const uint16_t* k, int64_t k_ss, int64_t k_sh, const uint16_t* v,
                                         int64_t v_ss, int64_t v_sh, int64_t S, int64_t H, const uint16_t* tab,
                                         int rot, const uint16_t* kw, float eps, int smooth_k, void* workspace,
                                         int64_t workspace_bytes, void** ptrs, hipStream_t stream) {
  clear_error();
  if (int e = check_qkv("attention_prepass_qkv", k, k_ss, k_sh, k, k_ss, k_sh, v, v_ss, v_sh, S, S, H)) return e;
  RH3_REQUIRE(ptrs, "attention_prepass_qkv: ptrs required");
  const Work w = layout(workspace, S, S, H);
  RH3_REQUIRE(workspace && aligned16(workspace) && workspace_bytes >= w.bytes,
              "attention_prepass_qkv: workspace %lld bytes < required %lld", (long long)workspace_bytes,
              (long long)w.bytes);
  RR rk{nullptr, nullptr, 0.f, 0};
  if (tab) {
    RH3_REQUIRE(kw && (rot == 96 || rot == 128) && aligned16(tab) && aligned16(kw),
                "attention_prepass_qkv: kw (16-byte aligned) and rot_dim 96 or 128 required with tab");
    rk = RR{tab, kw, eps, rot};
  }
  // q8, qs and the K channel sums come from rh3_gemm_i8_qkv (numerics 0) on this workspace
  const int64_t skp = pad(S);
  const int nchunk = static_cast<int>((S + CHUNK - 1) / CHUNK);
  const float* mean = nullptr;
  if (smooth_k) {
    hipLaunchKernelGGL(kmean_kernel, dim3(H), dim3(KMEAN_NT), 0, stream, w.part, nchunk, S, w.kmean);
    mean = w.kmean;
  } else {
    hipLaunchKernelGGL(zero_kernel, dim3((H * D + 255) / 256), dim3(256), 0, stream, w.kmean, H * D);
  }
  launch_quant(dim3(H, skp / BLK), stream, k, k_ss, k_sh, S, skp, rk, mean, w.k8, w.ks, w.kn);
  hipLaunchKernelGGL(vt_kernel, dim3(H, skp / 64), dim3(256), 0, stream, v, v_ss, v_sh, S, skp, w.vt);
  if (int e = launch_status("attention prepass_qkv")) return e;
  ptrs[0] = w.q8; ptrs[1] = w.qs; ptrs[2] = w.k8; ptrs[3] = w.ks; ptrs[4] = w.kmean; ptrs[5] = w.vt;
  return RH3_OK;
}

extern "C" int rh3_attention_forward(int64_t Sq, int64_t Sk, int64_t H, float scale, uint16_t* out, int64_t o_ss,
                                     int64_t o_sh, void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  clear_error();
  RH3_REQUIRE(Sq > 0 && Sk > 0 && H > 0, "attention_forward: sizes must be positive");
  // the limits check_qkv applies to the pre-pass that filled the workspace (the main kernel's K-scale table
  // holds pad(Sk)/128 <= 4096 entries)
  RH3_REQUIRE(pad(Sq) / BLK < 65536 && H < 65536, "attention_forward: Sq=%lld exceeds the 8,388,480-token grid limit",
              (long long)Sq);
  RH3_REQUIRE(pad(Sk) / BLK <= 4096, "attention_forward: Sk=%lld exceeds the 524288-key limit of the attention kernel",
              (long long)Sk);
  RH3_REQUIRE(out && (reinterpret_cast<uintptr_t>(out) & 7) == 0 && o_ss % 4 == 0 && o_sh % 4 == 0,
              "attention_forward: out must be 8-byte aligned with strides multiple of 4");
  const Work w = layout(workspace, Sq, Sk, H);
  RH3_REQUIRE(workspace && aligned16(workspace) && workspace_bytes >= w.bytes,
              "attention_forward: workspace %lld bytes < required %lld", (long long)workspace_bytes,
              (long long)w.bytes);
  return forward(w, Sq, Sk, H, scale, out, o_ss, o_sh, stream);
}

extern "C" int rh3_int8_attention(const uint16_t* q, int64_t q_ss, int64_t q_sh, const uint16_t* k, int64_t k_ss,
                                  int64_t k_sh, const uint16_t* v, int64_t v_ss, int64_t v_sh, int64_t Sq, int64_t Sk,
                                  int64_t H, float scale, int smooth_k, uint16_t* out, int64_t o_ss, int64_t o_sh,
                                  void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  clear_error();
  if (int e = check_qkv("int8_attention", q, q_ss, q_sh, k, k_ss, k_sh, v, v_ss, v_sh, Sq, Sk, H)) return e;
  RH3_REQUIRE(out && (reinterpret_cast<uintptr_t>(out) & 7) == 0 && o_ss % 4 == 0 && o_sh % 4 == 0,
              "int8_attention: out must be 8-byte aligned with strides multiple of 4");
  const Work w = layout(workspace, Sq, Sk, H);
  RH3_REQUIRE(workspace && aligned16(workspace) && workspace_bytes >= w.bytes,
              "int8_attention: workspace %lld bytes < required %lld", (long long)workspace_bytes, (long long)w.bytes);
  const RR none{nullptr, nullptr, 0.f, 0};
  if (int e = prepass(q, q_ss, q_sh, k, k_ss, k_sh, v, v_ss, v_sh, Sq, Sk, H, none, none, smooth_k, w, stream))
    return e;
  return forward(w, Sq, Sk, H, scale, out, o_ss, o_sh, stream);
}

extern "C" int rh3_int8_attention_rr(const uint16_t* q, int64_t q_ss, int64_t q_sh, const uint16_t* k, int64_t k_ss,
                                     int64_t k_sh, const uint16_t* v, int64_t v_ss, int64_t v_sh, int64_t S,
                                     int64_t H, const uint16_t* tab, int rot, const uint16_t* qw, const uint16_t* kw,
                                     float eps, float scale, int smooth_k, uint16_t* out, int64_t o_ss, int64_t o_sh,
                                     void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  clear_error();
  if (int e = check_qkv("int8_attention_rr", q, q_ss, q_sh, k, k_ss, k_sh, v, v_ss, v_sh, S, S, H)) return e;
  if (int e = check_rr("int8_attention_rr", tab, rot, qw, kw)) return e;
  RH3_REQUIRE(out && (reinterpret_cast<uintptr_t>(out) & 7) == 0 && o_ss % 4 == 0 && o_sh % 4 == 0,
              "int8_attention_rr: out must be 8-byte aligned with strides multiple of 4");
  const Work w = layout(workspace, S, S, H);
  RH3_REQUIRE(workspace && aligned16(workspace) && workspace_bytes >= w.bytes,
              "int8_attention_rr: workspace %lld bytes < required %lld", (long long)workspace_bytes,
              (long long)w.bytes);
  const RR rq{tab, qw, eps, rot}, rk{tab, kw, eps, rot};
  if (int e = prepass(q, q_ss, q_sh, k, k_ss, k_sh, v, v_ss, v_sh, S, S, H, rq, rk, smooth_k, w, stream)) return e;
  return forward(w, S, S, H, scale, out, o_ss, o_sh, stream);
}

// RMSNorm + RoPE of q and k in place ([S, H, 128] bf16, any token / head strides in elements, multiples of 8),
// the prologue every rh3_*_rr / prepass entry point applies before quantizing.
extern "C" int rh3_rms_rope_qk(uint16_t* q, int64_t q_ss, int64_t q_sh, uint16_t* k, int64_t k_ss, int64_t k_sh,
                               int64_t S, int64_t H, const uint16_t* tab, int rot, const uint16_t* qw,
                               const uint16_t* kw, float eps, hipStream_t stream) {
  clear_error();
  RH3_REQUIRE(S >= 0 && H > 0, "rms_rope_qk: bad sizes S=%lld H=%lld", (long long)S, (long long)H);
  if (S == 0) return RH3_OK;
  if (int e = check_rr("rms_rope_qk", tab, rot, qw, kw)) return e;
  RH3_REQUIRE(q && k && aligned16(q) && aligned16(k), "rms_rope_qk: q and k must be 16-byte aligned");
  RH3_REQUIRE(q_ss % 8 == 0 && q_sh % 8 == 0 && k_ss % 8 == 0 && k_sh % 8 == 0,
              "rms_rope_qk: strides must be multiples of 8 elements");
  const int64_t blocks = (S * H + 15) / 16;
  RH3_REQUIRE(blocks < (int64_t{1} << 31), "rms_rope_qk: S*H=%lld rows exceed the grid", (long long)(S * H));
  hipLaunchKernelGGL(rms_rope_kernel, dim3(static_cast<unsigned>(blocks), 2), dim3(256), 0, stream, q, q_ss, q_sh,
                     k, k_ss, k_sh, S, H, RR{tab, qw, eps, rot}, RR{tab, kw, eps, rot});
  return launch_status("rms_rope_qk");
}
