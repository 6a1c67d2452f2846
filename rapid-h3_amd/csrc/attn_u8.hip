// INT8 flash attention with the reference's production numerics (attn_int8.cu config 80 = attn_fwd8
// :2250-2511; configs 90/94 run the same math on a persistent schedule, and 1xx add the q/k RMSNorm + RoPE
// pre-pass), gfx950, head_dim 128, non-causal.
//
// Pre-pass (HBM-bound; attn_int8.cu:2568-2644):
//   stats_kernel   float64 channel sums of K (after the optional RMSNorm + RoPE), per 256-token chunk
//   vstats_kernel  float64 channel sums, max and min of V, per 256-token chunk
//   kmean_kernel   kmean = fp32(sum / Sk)                                      (attn_int8.cu:97-109)
//   vfinal_kernel  vmean = fp32(sum / Sk) (0 without smooth_v),
//                  vscale = max(max(vmax - vmean, vmean - vmin), 1e-6) / 127  (attn_int8.cu:97-109)
//   tokq_kernel    per (token, head) row: [RMSNorm + RoPE] -> [- kmean] -> [normalized H128] -> one scale
//                  sc = max(amax, 1e-8) / 127, q = rint(x * (1 / sc))         (attn_int8.cu:113-170, :298-340);
//                  for K also the per-key pair (sc, -1.5*2^23 * sc); padded keys get (0, -inf)
//   vq_kernel      per (128-key tile, head): int8 V codes rint((v - vmean) / vscale) (attn_int8.cu:452-475),
//                  transposed to [H][128][Skpad] in the key order of the P.V operand, and the tile's P.V
//                  accumulator start 1.5*2^23 bits + 128 * (sum of its codes) per channel
// Main kernel: per (256-query block, head) workgroup of 8 waves, 32 queries per wave, 128-key tiles.
//   S^T = K8 . Q8^T on v_mfma_i32_32x32x32_i8 (keys on rows, queries on lanes), the accumulator starting at
//   the bits of 1.5*2^23 so that t = fma(float bits, s_j, b_j) is the dequantized score in one instruction;
//   tile max tm, n = max(m, tm), a = 2^((m - n) c), ts = 2^((tm - n) c); P = rint(2^(fma(t, c, log2 255 - tm c)))
//   in [0, 255]; row sums of the integer P; O^T += V8^T . P^T on v_mfma_i32_32x32x32_i8 with P - 128 as the
//   signed operand (the tile's 128 * sum(V codes) is the accumulator start, so the integer result is the
//   reference's u8 x s8 product exactly); O = fma(ts, acc bits, fma(O, a, -ts * 1.5*2^23)); out =
//   bf16(fma(O (1 / l), vscale, vmean)). Text bias (attn_cake.cuh:97-99, :210-240): t += bias*log2(e) / c on
//   keys [0, nbias).
// Configs 60-61 (attn_fwd6 :1786-1962): the same kernel with BK = true and blockk_kernel (quant_k_block :404-443)
//   in place of the per-token K quantizer: one K scale per 128-key tile, integer tile max, no per-key dequant.
#include "attn_common.hpp"
#include "attn_layout.hpp"

namespace rh3 {
namespace {

using namespace attn;

constexpr int TILE = 128;                 // keys per tile (the tile max of the u8 P)
constexpr int SIDE = 2048;                // bytes per (head, tile): 128 (s, b) pairs, 128 int32 starts, pad
constexpr int SIDE_VINIT = 1024;          // byte offset of the accumulator starts inside a side record
constexpr int MAGIC_I = 0x4B400000;       // bits of 1.5 * 2^23
constexpr float MAGIC_F = 12582912.0f;
constexpr float LOG2_255 = 7.99435343685886f;       // attn_int8.cu:24
constexpr float LOG2_448 = 8.807354922057604f;      // attn_int8.cu:1557
constexpr float V_STRETCH = 448.0f / 127.0f;        // attn_int8.cu:468
constexpr float V_UNSTRETCH = 127.0f / 448.0f;      // attn_int8.cu:2642
constexpr float INV_SQRT128 = 0.08838834764831845f;  // attn_int8.cu:127

// ------------------------------------------------------------------ V statistics
// grid (H, nchunk) (heads fastest, so a chunk's token rows are read together), 256 threads = 16 token slots x 16
// lanes (8 channels each)
__global__ void __launch_bounds__(256) vstats_kernel(const uint16_t* __restrict__ v, int64_t v_ss, int64_t v_sh,
                                                     int64_t S, double* __restrict__ vsum,
                                                     float* __restrict__ vmax, float* __restrict__ vmin) {
  __shared__ double red[16][D];
  __shared__ float rmx[16][D], rmn[16][D];
  const int h = blockIdx.x, c = blockIdx.y, tid = threadIdx.x;
  const int slot = tid >> 4, l16 = tid & 15;
  double acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  float mx[8], mn[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) { mx[e] = -INFINITY; mn[e] = INFINITY; }
  // the rows of four iterations are loaded before any is used (rows past S read row S - 1 and are skipped)
  for (int it0 = 0; it0 < CHUNK / 16; it0 += 4) {
    uint4 rx[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t s = static_cast<int64_t>(c) * CHUNK + (it0 + i) * 16 + slot;
      rx[i] = *reinterpret_cast<const uint4*>(v + (s < S ? s : S - 1) * v_ss + h * v_sh + 8 * l16);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (static_cast<int64_t>(c) * CHUNK + (it0 + i) * 16 + slot < S) {
        float x[8];
        unpack8(rx[i], x);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          acc[e] += static_cast<double>(x[e]);
          mx[e] = fmaxf(mx[e], x[e]);
          mn[e] = fminf(mn[e], x[e]);
        }
      }
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    red[slot][8 * l16 + e] = acc[e];
    rmx[slot][8 * l16 + e] = mx[e];
    rmn[slot][8 * l16 + e] = mn[e];
  }
  __syncthreads();
  if (tid < D) {
    double t = 0.0;
    float a = -INFINITY, b = INFINITY;
    for (int i = 0; i < 16; ++i) {
      t += red[i][tid];
      a = fmaxf(a, rmx[i][tid]);
      b = fminf(b, rmn[i][tid]);
    }
    const int64_t o = (static_cast<int64_t>(h) * gridDim.y + c) * D + tid;
    vsum[o] = t;
    vmax[o] = a;
    vmin[o] = b;
  }
}

// grid H, VFINAL_NT threads: group j of 128 channels folds chunks j, j + 8, ..., then the 8 groups (the float64
// sums of bf16 values are exact and max / min are order-free, so the grouping does not change the result)
constexpr int VFINAL_NT = 1024;
__global__ void __launch_bounds__(VFINAL_NT) vfinal_kernel(const double* __restrict__ vsum,
                                                           const float* __restrict__ vmax,
                                                           const float* __restrict__ vmin, int nchunk, int64_t S,
                                                           int smooth_v, float* __restrict__ vmean,
                                                           float* __restrict__ vscale) {
  constexpr int G = VFINAL_NT / D;
  __shared__ double rs[G][D];
  __shared__ float rmx[G][D], rmn[G][D];
  const int h = blockIdx.x, d = threadIdx.x % D, j = threadIdx.x / D;
  double t = 0.0;
  float a = -INFINITY, b = INFINITY;
  for (int c = j; c < nchunk; c += G) {
    const int64_t o = (static_cast<int64_t>(h) * nchunk + c) * D + d;
    t += vsum[o];
    a = fmaxf(a, vmax[o]);
    b = fminf(b, vmin[o]);
  }
  rs[j][d] = t;
  rmx[j][d] = a;
  rmn[j][d] = b;
  __syncthreads();
  if (j != 0) return;
#pragma unroll
  for (int i = 1; i < G; ++i) {
    t += rs[i][d];
    a = fmaxf(a, rmx[i][d]);
    b = fminf(b, rmn[i][d]);
  }
  const float vm = smooth_v ? static_cast<float>(t / static_cast<double>(S)) : 0.0f;
  vmean[h * D + d] = vm;
  vscale[h * D + d] = fmaxf(fmaxf(a - vm, vm - b), 1e-6f) / 127.0f;
}

// ------------------------------------------------------------------ per-token Q / K quantizer
// 256 threads = 16 rows of 16 lanes; row g = blockIdx.x * 16 + tid / 16 is (token g / H, head g % H), heads
// fastest. grid = Spad * H / 16 (Spad is a multiple of 128).
__global__ void __launch_bounds__(256) tokq_kernel(const uint16_t* __restrict__ x, int64_t x_ss, int64_t x_sh,
                                                   int64_t S, int64_t Spad, int64_t H, RR rr,
                                                   const float* __restrict__ mean, int rotate,
                                                   int8_t* __restrict__ codes, float* __restrict__ scales,
                                                   float* __restrict__ side) {
  const int tid = threadIdx.x, lane = tid & 63, l16 = tid & 15;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 16 + (tid >> 4);
  const int64_t s = row / H, h = row % H;
  const int64_t co = (h * Spad + s) * D + 8 * l16;
  if (s >= S) {  // uniform per 16-lane row: padded rows and keys
    *reinterpret_cast<uint2*>(codes + co) = make_uint2(0, 0);
    if (l16 == 0) {
      scales[h * Spad + s] = 0.0f;
      if (side) {
        float* p = side + ((h * (Spad / TILE) + s / TILE) * SIDE) / 4 + 2 * (s % TILE);
        *reinterpret_cast<float2*>(p) = make_float2(0.0f, -INFINITY);
      }
    }
    return;
  }
  // the row, the rope-table row and the norm weights are loaded together, before any arithmetic
  const uint4 rx = *reinterpret_cast<const uint4*>(x + s * x_ss + h * x_sh + 8 * l16);
  uint4 rt[4];
  uint4 rw = make_uint4(0, 0, 0, 0);
  if (rr.tab) {
    rope_tab8_raw(rr, l16, s, rt);
    rw = *reinterpret_cast<const uint4*>(rr.w + 8 * l16);
  }
  float v[8];
  unpack8(rx, v);
  if (rr.tab) {
    float w[8];
    unpack8(rw, w);
    rms_rope8_raw(v, lane, rr, w, rt);
  }
  if (mean) {
    float m[8];
    const float4 a = *reinterpret_cast<const float4*>(mean + h * D + 8 * l16);
    const float4 b = *reinterpret_cast<const float4*>(mean + h * D + 8 * l16 + 4);
    m[0] = a.x; m[1] = a.y; m[2] = a.z; m[3] = a.w; m[4] = b.x; m[5] = b.y; m[6] = b.z; m[7] = b.w;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = v[e] - m[e];
  }
  if (rotate) wht128_row(v, l16);
  uint2 o;
  const float sc = token_quant_row(v, o);
  *reinterpret_cast<uint2*>(codes + co) = o;
  if (l16 == 0) {
    scales[h * Spad + s] = sc;
    if (side) {
      float* p = side + ((h * (Spad / TILE) + s / TILE) * SIDE) / 4 + 2 * (s % TILE);
      *reinterpret_cast<float2*>(p) = make_float2(sc, -MAGIC_F * sc);
    }
  }
}

// ------------------------------------------------------------------ per-block K (configs 60-61)
// grid (H, Skpad / 128) (heads fastest), 256 threads: wave w quantizes tokens 32 w .. 32 w + 31 of the block, four 16-lane rows
// per pass. K - kmean -> [normalized H128] -> one scale per (head, 128-key block) sc = max(amax, 1e-8) / 127,
// codes rint(x * (1 / sc)) (quant_k_block, attn_int8.cu:404-443); sc goes to kbs [H][Skpad/128] and to the first
// float of the block's side record, where the main kernel reads it. Padded tokens are zero rows.
__global__ void __launch_bounds__(256) blockk_kernel(const uint16_t* __restrict__ k, int64_t k_ss, int64_t k_sh,
                                                     int64_t S, int64_t Spad, const float* __restrict__ mean,
                                                     int rotate, int8_t* __restrict__ codes,
                                                     float* __restrict__ kbs, float* __restrict__ side) {
  __shared__ float wmax[4];
  const int h = blockIdx.x, blk = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, sub = lane >> 4;
  float m[8];
  {
    const float4 a = *reinterpret_cast<const float4*>(mean + h * D + 8 * l16);
    const float4 b = *reinterpret_cast<const float4*>(mean + h * D + 8 * l16 + 4);
    m[0] = a.x; m[1] = a.y; m[2] = a.z; m[3] = a.w; m[4] = b.x; m[5] = b.y; m[6] = b.z; m[7] = b.w;
  }
  float v[8][8];
  float amax = 0.0f;
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const int64_t s = static_cast<int64_t>(blk) * TILE + wave * 32 + p * 4 + sub;
    const bool ok = s < S;  // uniform per 16-lane row
#pragma unroll
    for (int e = 0; e < 8; ++e) v[p][e] = 0.0f;
    if (ok) {
      load8(k + s * k_ss + h * k_sh + 8 * l16, v[p]);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[p][e] = v[p][e] - m[e];
    }
    if (rotate) wht128_row(v[p], l16);  // every lane joins the row shuffles; zero rows stay zero
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[p][e]));
  }
  amax = wave_max(amax);
  if (lane == 0) wmax[wave] = amax;
  __syncthreads();
  const float bm = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  const float sc = fmaxf(bm, 1e-8f) / 127.0f;
  const float inv = 1.0f / sc;
  if (tid == 0) {
    kbs[static_cast<int64_t>(h) * (Spad / TILE) + blk] = sc;
    side[((static_cast<int64_t>(h) * (Spad / TILE) + blk) * SIDE) / 4] = sc;
  }
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const int64_t s = static_cast<int64_t>(blk) * TILE + wave * 32 + p * 4 + sub;
    uint32_t b[8];
    // |x * inv| <= 127 (1 + 2^-23): rint stays within the int8 range without a clamp
#pragma unroll
    for (int e = 0; e < 8; ++e) b[e] = static_cast<uint32_t>(static_cast<int32_t>(rintf(v[p][e] * inv))) & 0xffu;
    uint2 o;
    o.x = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
    o.y = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
    *reinterpret_cast<uint2*>(codes + (static_cast<int64_t>(h) * Spad + s) * D + 8 * l16) = o;
  }
}

// ------------------------------------------------------------------ V codes, transposed
// Position p of a 32-key block holds key perm_u8(p): p = 16 g + r <-> key 8 (r / 4) + 4 g + r % 4, the key of
// register r of lane group g in the S^T accumulator, so that a lane's 16 P bytes are its P.V B operand.
__device__ __forceinline__ int perm_u8(int p) {
  const int g = p >> 4, r = p & 15;
  return 8 * (r >> 2) + 4 * g + (r & 3);
}

// Position p of a 64-key chunk of the e4m3 layout holds key perm_f8(p): p = 32 g + 16 h + r <-> key 32 h + 8 (r / 4)
// + 4 g + r % 4, the key of register r of 32-key block h in lane group g's S^T accumulator, so that a lane's 32 P
// bytes of the chunk are its B operand of the 64-deep FP8 MFMA.
__device__ __forceinline__ int perm_f8(int p) {
  const int g = p >> 5, hh = (p >> 4) & 1, r = p & 15;
  return 32 * hh + 8 * (r >> 2) + 4 * g + (r & 3);
}

// grid (H, Skpad / 128) (heads fastest), 256 threads. F8 (configs 50-56): e4m3 codes of ((v - vmean) / vscale) *
// fp32(448 / 127) (attn_int8.cu:467-473) in the perm_f8 order, and no accumulator starts.
template <bool F8>
__global__ void __launch_bounds__(256) vq_kernel(const uint16_t* __restrict__ v, int64_t v_ss, int64_t v_sh,
                                                 int64_t S, int64_t Spad, const float* __restrict__ vmean,
                                                 const float* __restrict__ vscale, int8_t* __restrict__ vt,
                                                 int32_t* __restrict__ side) {
  constexpr int P = D + 16;  // row pitch of the key-major code tile
  __shared__ int8_t tile[TILE * P];
  const int h = blockIdx.x, tid = threadIdx.x, l16 = tid & 15;
  const int64_t s0 = static_cast<int64_t>(blockIdx.y) * TILE;
  float vm[8], vs[8], iv[8];
  {
    const float4 a = *reinterpret_cast<const float4*>(vmean + h * D + 8 * l16);
    const float4 b = *reinterpret_cast<const float4*>(vmean + h * D + 8 * l16 + 4);
    const float4 c = *reinterpret_cast<const float4*>(vscale + h * D + 8 * l16);
    const float4 d = *reinterpret_cast<const float4*>(vscale + h * D + 8 * l16 + 4);
    vm[0] = a.x; vm[1] = a.y; vm[2] = a.z; vm[3] = a.w; vm[4] = b.x; vm[5] = b.y; vm[6] = b.z; vm[7] = b.w;
    vs[0] = c.x; vs[1] = c.y; vs[2] = c.z; vs[3] = c.w; vs[4] = d.x; vs[5] = d.y; vs[6] = d.z; vs[7] = d.w;
#pragma unroll
    for (int e = 0; e < 8; ++e) iv[e] = 1.0f / vs[e];
  }
  // 128 keys x 16 lanes: 8 passes of 16 keys
  for (int r = tid >> 4; r < TILE; r += 16) {
    uint2 o = make_uint2(0, 0);
    if (s0 + r < S) {
      float x[8];
      load8(v + (s0 + r) * v_ss + h * v_sh + 8 * l16, x);
      if constexpr (F8) {
        float y[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = fminf(fmaxf(((x[e] - vm[e]) / vs[e]) * V_STRETCH, -448.0f), 448.0f);
        o.x = __builtin_amdgcn_cvt_pk_fp8_f32(y[2], y[3], __builtin_amdgcn_cvt_pk_fp8_f32(y[0], y[1], 0, false), true);
        o.y = __builtin_amdgcn_cvt_pk_fp8_f32(y[6], y[7], __builtin_amdgcn_cvt_pk_fp8_f32(y[4], y[5], 0, false), true);
      } else {
        uint32_t b[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          b[e] = static_cast<uint32_t>(static_cast<int32_t>(rint_div(x[e] - vm[e], vs[e], iv[e]))) & 0xffu;
        o.x = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
        o.y = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
      }
    }
    *reinterpret_cast<uint2*>(&tile[r * P + 8 * l16]) = o;
  }
  __syncthreads();
  // V^T rows: channel d, 16 positions per store (8 stores of 16 B per row)
  for (int i = tid; i < D * (TILE / 16); i += 256) {
    const int d = i >> 3, pc = (i & 7) * 16;  // positions pc..pc+15 of this tile
    uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int p = pc + e;
      const int key = F8 ? (p & ~63) + perm_f8(p & 63) : (p & ~31) + perm_u8(p & 31);
      w[e >> 2] |= (static_cast<uint32_t>(static_cast<uint8_t>(tile[key * P + d]))) << (8 * (e & 3));
    }
    *reinterpret_cast<uint4*>(vt + (static_cast<int64_t>(h) * D + d) * Spad + s0 + pc) =
        make_uint4(w[0], w[1], w[2], w[3]);
  }
  // accumulator starts: 1.5*2^23 bits + 128 * (sum of the tile's codes of channel d); the pad is zeroed
  if constexpr (F8) return;
  int32_t* rec = side + (static_cast<int64_t>(h) * (Spad / TILE) + blockIdx.y) * (SIDE / 4);
  if (tid < D) {
    int sum = 0;
    for (int k = 0; k < TILE; ++k) sum += static_cast<int8_t>(tile[k * P + tid]);
    rec[SIDE_VINIT / 4 + tid] = MAGIC_I + 128 * sum;
  } else {
    rec[SIDE_VINIT / 4 + tid] = 0;
  }
}

// ------------------------------------------------------------------ main kernel
struct U8Args {
  const int8_t* q8;    // [H][Sqpad][128]
  const float* qs;     // [H][Sqpad]
  const int8_t* k8;    // [H][Skpad][128]
  const int8_t* side;  // [H][Skpad/128][2048 B]: (s, b) pairs, accumulator starts
  const int8_t* vt;    // [H][128][Skpad]
  const float* vscale;  // [H][128]
  const float* vmean;   // [H][128]
  uint16_t* out;
  int64_t o_ss, o_sh;
  int64_t Sq, Sk, Sqpad, Skpad;
  float scale_log2;
  int nbias;
  float bias_log2;
  int nqb;   // query blocks per head; item = h * nqb + qb (query blocks fastest)
  int* ctr;  // work counter, zero at launch: a starting workgroup takes item ctr++
};

constexpr int U8_WAVES = 8, U8_NT = U8_WAVES * 64, U8_BQ = U8_WAVES * 32;

typedef __attribute__((address_space(3))) const v4i lds_v4i_u8;
typedef __attribute__((address_space(3))) const float lds_f32_u8;

// max of three floats in one instruction (fmaxf chains get a NaN-quieting max inserted per operand)
__device__ __forceinline__ float max3f(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// Tile j reads K(j), V^T(j) and its side record from ring slot j % 4 and first loads tile j + 2 into slot
// (j + 2) % 4, whose last reader ran before the barrier that ended tile j - 1 (see the barrier comment).
// A slot holds K: 128 keys x 128 B (chunk c of row r at c ^ ((r ^ (r >> 3)) & 7)), V^T: 128 channels x 128
// keys (the same swizzle), then the 2 KiB side record. Padded keys carry b = -inf, so every tile runs unmasked.
// BK (configs 60-61, attn_fwd6 :1786-1962): one K scale kb per 128-key tile (the first float of the side record)
// instead of the per-key pairs: the tile max is the integer max ti of the raw accumulators (keys past Sk forced to
// 1.5*2^23 - 2^22 first), cc = c kb, tv = (ti - 1.5*2^23) cc, n = max(m, tv), a = 2^(m - n), ts = 2^(tv - n),
// P = rint(2^(fma(acc bits, cc, fma(-ti bits, cc, log2 255)))); the P.V, row sums and fold are the same.
// MODE 2 (FP8 P.V, configs 50-56, attn_fwd5 :1563-1785): the per-key dequant of MODE 0, then per group of MAXG keys
// (64 or 128, the reference's tile) the group max updates the running max m exactly (O and l scaled by
// 2^((m_old - m) c) when it grows), P = 2^(fma(t, c, fma(-m, c, log2 448))) in e4m3 (v_cvt_pk_fp8_f32: OCP e4m3fn,
// round to nearest even), l += P unquantized, and O^T += V^T . P^T on v_mfma_scale_f32_32x32x64_f8f6f4 (e4m3 V
// from vq_kernel<true>) straight into the fp32 accumulators: no per-tile fold.
template <int MODE, int MAXG = 128>
__global__ void __launch_bounds__(U8_NT, 1) attn_u8_kernel(const U8Args a) {
  constexpr bool BK = MODE == 1;
  constexpr int KB = TILE * D, VB = D * TILE, SLOT = KB + VB + SIDE;
  __shared__ __attribute__((aligned(16))) int8_t ring[4 * SLOT];
  // the workgroup runs the item it takes from one work counter when it starts (a fast XCD takes more; see the
  // launch), the (head, query block) pair h * nqb + qb. Per-XCD shares (claim_item) measured 1.6 % slower here
  // (180.3 vs 177.4 ms at C4), so this kernel keeps the single counter.
  __shared__ int item_s;
  if (threadIdx.x == 0) item_s = atomicAdd(a.ctr, 1);
  __syncthreads();
  const int item = __builtin_amdgcn_readfirstlane(item_s);
  if (item >= static_cast<int>(gridDim.y) * a.nqb) return;
  const int h = item / a.nqb, qb = item - h * a.nqb;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, g = lane >> 5;
  const int64_t q = static_cast<int64_t>(qb) * U8_BQ + wave * 32 + l32;
  const int ntiles = static_cast<int>(a.Skpad / TILE);

  // Q operands are padded to 128 queries; a workgroup's last rows may lie past them (computed on zero codes
  // with c = 0 and never stored)
  const bool qin = q < a.Sqpad;
  v4i qf[4];
  {
    const int8_t* qp = a.q8 + (static_cast<int64_t>(h) * a.Sqpad + q) * D + g * 16;
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) qf[ds] = qin ? *reinterpret_cast<const v4i*>(qp + ds * 32) : v4i{0, 0, 0, 0};
  }
  const float c = (qin ? a.qs[static_cast<int64_t>(h) * a.Sqpad + q] : 0.0f) * a.scale_log2;
  const float ib = (a.nbias > 0 && c > 0.0f) ? a.bias_log2 / c : 0.0f;

  // global -> LDS copies (lane l of a wave writes LDS base + 16 l; the swizzle is applied on the global side):
  // K and V^T positions p = 64 w + lane and 512 + 64 w + lane (rows p / 8 and p / 8 + 64, same swizzle) for
  // every wave, the 128 side chunks by waves 0 and 1. Waves 0-1 issue 5 copies per tile, waves 2-7 issue 4.
  const int8_t* kbase = a.k8 + static_cast<int64_t>(h) * a.Skpad * D;
  const int8_t* vbase = a.vt + static_cast<int64_t>(h) * D * a.Skpad;
  const int8_t* sbase = a.side + static_cast<int64_t>(h) * ntiles * SIDE;
  const int p0 = wave * 64 + lane, row0 = p0 >> 3, pc0 = p0 & 7, sw0 = (pc0 ^ ((row0 ^ (row0 >> 3)) & 7)) << 4;
  const int8_t* ksrc = kbase + row0 * D + sw0;
  const int8_t* vsrc = vbase + static_cast<int64_t>(row0) * a.Skpad + sw0;
  const int8_t* ssrc = sbase + p0 * 16;  // waves 0, 1 only
  const int64_t vhalf = 64 * a.Skpad;
  const uint32_t ring_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(ring));
  const uint32_t kdst = ring_lds + wave * 1024, vdst = kdst + KB, sdst = ring_lds + KB + VB + wave * 1024;
  const bool side_wave = wave < 2;
  auto load_tile = [&](int j) __attribute__((always_inline)) {
    const uint32_t so = static_cast<uint32_t>(j & 3) * SLOT;
    j = min(j, ntiles - 1);  // clamped: every tile issues the same copies; a copy past the end lands unread
    const int8_t* kp = ksrc + static_cast<int64_t>(j) * KB;
    const int8_t* vp = vsrc + static_cast<int64_t>(j) * TILE;
    lds_dma16(kp, kdst + so);
    lds_dma16(kp + 64 * D, kdst + so + 8192);
    lds_dma16(vp, vdst + so);
    lds_dma16(vp + vhalf, vdst + so + 8192);
    if (side_wave) lds_dma16(ssrc + static_cast<int64_t>(j) * SIDE, sdst + so);
  };

  // lane parts of the LDS reads inside a slot. K fragment (kb, ds): row 32 kb + l32, chunk 2 ds + g, stored at
  // chunk ^ ((row ^ (row >> 3)) & 7) = (2 ds ^ 4 (kb & 1)) ^ y, y = (g ^ l32 ^ (l32 >> 3)) & 7: lane offsets
  // koff[ds ^ 2 (kb & 1)] plus the immediate 4096 kb. V^T fragment (db, kc) likewise, plus KB.
  uint32_t koff[4];
  {
    const int y = (g ^ l32 ^ (l32 >> 3)) & 7;
#pragma unroll
    for (int i = 0; i < 4; ++i) koff[i] = ring_lds + l32 * 128 + (((2 * i) ^ y) << 4);
  }
  // side record: pairs of keys 32 kb + 8 i + 4 g .. +3 at byte 8 key, accumulator starts of channels
  // 32 db + 8 i + 4 g .. +3 at SIDE_VINIT + 4 d
  const uint32_t soff = ring_lds + KB + VB + 32 * g;
  const uint32_t ioff = ring_lds + KB + VB + SIDE_VINIT + 16 * g;
  // MODE 2: the e4m3 V^T fragment (db, 64-key chunk cc) of lane (l32, g) is logical chunks 4 cc + 2 g + h (h = 0, 1)
  // of row 32 db + l32, stored at chunk ^ ((row ^ (row >> 3)) & 7) = (4 (cc ^ (db & 1)) + 2 g + h) ^ y2
  uint32_t voff8[2][2];
  {
    const int y2 = (l32 ^ (l32 >> 3)) & 7;
#pragma unroll
    for (int c2 = 0; c2 < 2; ++c2)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) voff8[c2][hh] = ring_lds + KB + l32 * 128 + (((4 * c2 + 2 * g + hh) ^ y2) << 4);
  }

  v16f o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[i][r] = 0.0f;
  float mx = -INFINITY, lrow = 0.0f;
  v16i magic;
#pragma unroll
  for (int r = 0; r < 16; ++r) magic[r] = MAGIC_I;

  // S^T of tile j: lane (l32, g) of s[kb] holds query l32 and keys 32 kb + 8 (r / 4) + 4 g + r % 4
  v16i s[4];
  auto qk = [&](const int j) __attribute__((always_inline)) {
    const uint32_t so = static_cast<uint32_t>(j & 3) * SLOT;
    uint32_t ka[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ka[i] = koff[i] + so;
    // key-block outer, so that block kb is complete while the MFMAs of block kb + 1 still run
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int ds = 0; ds < 4; ++ds) {
        const v4i kf = *reinterpret_cast<lds_v4i_u8*>(static_cast<uintptr_t>(ka[ds ^ (2 * (kb & 1))] + kb * 4096));
        s[kb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(kf, qf[ds], ds == 0 ? magic : s[kb], 0, 0, 0);
      }
    read_ahead<16, 3>();
  };

  auto softmax_pv = [&](const int j) __attribute__((always_inline)) {
    const uint32_t so = static_cast<uint32_t>(j & 3) * SLOT;
    // exponent of P: 2^(fma(t, cx, bb)); u8: t the dequantized score, cx = c; BK: t the accumulator bits, cx = c kb
    float t[4][16];
    float cx, bb, al, ts;
    if constexpr (BK) {
      if ((j + 1) * TILE > a.Sk) {  // the ragged last tile (uniform branch): padded keys far below every score
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (j * TILE + 32 * kb + 8 * (r >> 2) + 4 * g + (r & 3) >= a.Sk) s[kb][r] = MAGIC_I - (1 << 22);
      }
      int ti = s[0][0];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int r = 0; r < 16; r += 2) ti = max(ti, max(s[kb][r], s[kb][r + 1]));
      {
        const auto sw = __builtin_amdgcn_permlane32_swap(ti, ti, false, false);
        ti = max(static_cast<int>(sw[0]), static_cast<int>(sw[1]));
      }
      const float kbv = *reinterpret_cast<lds_f32_u8*>(static_cast<uintptr_t>(ring_lds + KB + VB + so));
      cx = c * kbv;
      const float tif = __int_as_float(ti);
      const float tv = (tif - MAGIC_F) * cx;
      const float n = fmaxf(mx, tv);
      al = __builtin_amdgcn_exp2f(mx - n);
      ts = __builtin_amdgcn_exp2f(tv - n);
      mx = n;
      bb = fmaf(-tif, cx, LOG2_255);
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) t[kb][r] = __int_as_float(s[kb][r]);
    } else {
    // t = fma(1.5*2^23 + acc, s_key, b_key), in place over the accumulator registers
    float tm = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const v4i p01 = *reinterpret_cast<lds_v4i_u8*>(static_cast<uintptr_t>(soff + so + kb * 256 + i * 64));
        const v4i p23 = *reinterpret_cast<lds_v4i_u8*>(static_cast<uintptr_t>(soff + so + kb * 256 + i * 64 + 16));
        const float ps[4] = {__int_as_float(p01[0]), __int_as_float(p01[2]), __int_as_float(p23[0]),
                             __int_as_float(p23[2])};
        const float pb[4] = {__int_as_float(p01[1]), __int_as_float(p01[3]), __int_as_float(p23[1]),
                             __int_as_float(p23[3])};
#pragma unroll
        for (int e = 0; e < 4; ++e) t[kb][4 * i + e] = fmaf(__int_as_float(s[kb][4 * i + e]), ps[e], pb[e]);
      }
    if (a.nbias > j * TILE) {  // text bias on keys [0, nbias) (uniform branch)
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = j * TILE + 32 * kb + 8 * (r >> 2) + 4 * g + (r & 3);
          if (key < a.nbias) t[kb][r] = t[kb][r] + ib;
        }
    }
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int r = 0; r < 16; r += 2) tm = max3f(tm, t[kb][r], t[kb][r + 1]);
    {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_int(tm), __float_as_int(tm), false, false);
      tm = fmaxf(__int_as_float(sw[0]), __int_as_float(sw[1]));
    }
    const float n = fmaxf(mx, tm);
    al = __builtin_amdgcn_exp2f((mx - n) * c);
    ts = __builtin_amdgcn_exp2f((tm - n) * c);
    mx = n;
    bb = fmaf(-tm, c, LOG2_255);
    cx = c;
    }
    // P = sat_u8(rint(2^x)) with v_cvt_pk_u8_f32 (round to nearest even, saturating at 0 and 255: the
    // reference's cvt.pack.sat.u8 of __float2int_rn), four per word; the signed operand of the MFMA is P - 128
    uint32_t pw[4][4];
    uint32_t rs = 0;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        uint32_t x = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          x = __builtin_amdgcn_cvt_pk_u8_f32(__builtin_amdgcn_exp2f(fmaf(t[kb][4 * w + e], cx, bb)), e, x);
        rs = __builtin_amdgcn_udot4(x, 0x01010101u, rs, false);
        pw[kb][w] = x ^ 0x80808080u;
      }
    // l adds the integer row sum of P (the lane's 64 keys)
    lrow = fmaf(ts, static_cast<float>(rs), lrow * al);
    const float nm = -ts * MAGIC_F;
    uint32_t va[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) va[i] = koff[i] + so + KB;
    // O^T[d][query] += V^T . P^T per 32-channel block db, then the fold into fp32
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      v16i acc;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const v4i st = *reinterpret_cast<lds_v4i_u8*>(static_cast<uintptr_t>(ioff + so + db * 128 + i * 32));
        acc[4 * i + 0] = st[0]; acc[4 * i + 1] = st[1]; acc[4 * i + 2] = st[2]; acc[4 * i + 3] = st[3];
      }
#pragma unroll
      for (int kc = 0; kc < 4; ++kc) {
        const v4i vf = *reinterpret_cast<lds_v4i_u8*>(static_cast<uintptr_t>(va[kc ^ (2 * (db & 1))] + db * 4096));
        v4i pf;
        pf[0] = pw[kc][0]; pf[1] = pw[kc][1]; pf[2] = pw[kc][2]; pf[3] = pw[kc][3];
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(vf, pf, acc, 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) o[db][r] = fmaf(ts, __int_as_float(acc[r]), fmaf(o[db][r], al, nm));
    }
    // issue order: 8 of the 32 LDS reads (per block: 4 accumulator starts, 4 V^T fragments) first, then each
    // P.V MFMA followed by two more reads, so the reads run ahead of the MFMAs that consume them
    __builtin_amdgcn_sched_group_barrier(0x100, 8, 1);  // 0x100: LDS reads
#pragma unroll
    for (int i = 0; i < 12; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);  // 0x008: MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4, 1);
  };

  auto softmax_pv_f8 = [&](const int j) __attribute__((always_inline)) {
    const uint32_t so = static_cast<uint32_t>(j & 3) * SLOT;
    float t[4][16];
    // t of blocks kb0 .. kb1 - 1 (MAXG 64: per 64-key chunk, so that only one chunk's scores are live at a time)
    auto dequant = [&](const int kb0, const int kb1) __attribute__((always_inline)) {
#pragma unroll
    for (int kb = kb0; kb < kb1; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const v4i p01 = *reinterpret_cast<lds_v4i_u8*>(static_cast<uintptr_t>(soff + so + kb * 256 + i * 64));
        const v4i p23 = *reinterpret_cast<lds_v4i_u8*>(static_cast<uintptr_t>(soff + so + kb * 256 + i * 64 + 16));
        const float ps[4] = {__int_as_float(p01[0]), __int_as_float(p01[2]), __int_as_float(p23[0]),
                             __int_as_float(p23[2])};
        const float pb[4] = {__int_as_float(p01[1]), __int_as_float(p01[3]), __int_as_float(p23[1]),
                             __int_as_float(p23[3])};
#pragma unroll
        for (int e = 0; e < 4; ++e) t[kb][4 * i + e] = fmaf(__int_as_float(s[kb][4 * i + e]), ps[e], pb[e]);
      }
    };
    if constexpr (MAXG == 128) dequant(0, 4);
    float bb = 0.0f;
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
      if constexpr (MAXG == 64) dequant(2 * cc, 2 * cc + 2);
      if (MAXG == 64 || cc == 0) {
        float tm = -INFINITY;
#pragma unroll
        for (int kb = 2 * cc; kb < 2 * cc + MAXG / 32; ++kb)
#pragma unroll
          for (int r = 0; r < 16; r += 2) tm = max3f(tm, t[kb][r], t[kb][r + 1]);
        {
          const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_int(tm), __float_as_int(tm), false, false);
          tm = fmaxf(__int_as_float(sw[0]), __int_as_float(sw[1]));
        }
        if (__builtin_amdgcn_ballot_w64(tm > mx) != 0) {  // a = 1 exactly on the rows whose max stays
          const float n = fmaxf(mx, tm);
          const float al = __builtin_amdgcn_exp2f((mx - n) * c);
          lrow = lrow * al;
#pragma unroll
          for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[db][r] = o[db][r] * al;
          mx = n;
        }
        bb = fmaf(-mx, c, LOG2_448);
      }
      // P of the chunk's two 32-key blocks in e4m3, four per word: the B operand of the 64-deep MFMA
      v8i pf;
#pragma unroll
      for (int hb = 0; hb < 2; ++hb)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int kb = 2 * cc + hb;
          const float p0 = __builtin_amdgcn_exp2f(fmaf(t[kb][4 * w + 0], c, bb));
          const float p1 = __builtin_amdgcn_exp2f(fmaf(t[kb][4 * w + 1], c, bb));
          const float p2 = __builtin_amdgcn_exp2f(fmaf(t[kb][4 * w + 2], c, bb));
          const float p3 = __builtin_amdgcn_exp2f(fmaf(t[kb][4 * w + 3], c, bb));
          lrow = lrow + (p0 + p1);
          lrow = lrow + (p2 + p3);
          uint32_t x = __builtin_amdgcn_cvt_pk_fp8_f32(p0, p1, 0, false);
          x = __builtin_amdgcn_cvt_pk_fp8_f32(p2, p3, x, true);
          pf[4 * hb + w] = static_cast<int>(x);
        }
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const uint32_t base = so + db * 4096;
        const v4i lo = *reinterpret_cast<lds_v4i_u8*>(static_cast<uintptr_t>(voff8[cc ^ (db & 1)][0] + base));
        const v4i hi = *reinterpret_cast<lds_v4i_u8*>(static_cast<uintptr_t>(voff8[cc ^ (db & 1)][1] + base));
        v8i vf;
        vf[0] = lo[0]; vf[1] = lo[1]; vf[2] = lo[2]; vf[3] = lo[3];
        vf[4] = hi[0]; vf[5] = hi[1]; vf[6] = hi[2]; vf[7] = hi[3];
        // cbsz / blgp type 0 = FP8 E4M3 for both operands; zero scale operands select the unscaled form
        o[db] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(vf, pf, o[db], 0, 0, 0, 0, 0, 0);
      }
    }
  };

  // Barrier B_j ends the use of ring slot j. Leading waves reach B_j after softmax_pv(j), lagging waves after
  // qk(j), so between B_(j-1) and B_j a lagging wave runs softmax_pv(j-1) while a leading wave runs qk(j). Each
  // wave issues its copies of tile j+2 right after B_(j-1), into slot (j+2) % 4, whose last reader
  // (softmax_pv(j-2) of a lagging wave) ran before B_(j-1); before B_j it waits for its copies of tile j+1
  // (vmcnt(n) leaves the n issued after B_(j-1) in flight), so slot j+1 is complete past B_j.
  const bool lag = (wave >> 2) == 1;  // waves 4-7 (one per SIMD) run half a tile behind
  auto barrier = [&]() __attribute__((always_inline)) {
    if (side_wave) asm volatile("s_waitcnt vmcnt(5)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  load_tile(0);
  load_tile(1);
  // vmcnt(0) through the builtin, so the compiler also sees the Q loads above as complete and adds no wait of
  // its own inside the loop (gfx9 s_waitcnt: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8])
  __builtin_amdgcn_s_waitcnt(0x0f70);
  __syncthreads();
  if (lag) load_tile(2);
  for (int j = 0; j < ntiles; ++j) {
    if (!lag) load_tile(j + 2);
    qk(j);
    if (lag) {
      barrier();
      load_tile(j + 3);
    }
    if constexpr (MODE == 2) softmax_pv_f8(j);
    else softmax_pv(j);
    if (!lag) barrier();
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no global->LDS copy outlives the workgroup

  const float lt = lrow + __shfl_xor(lrow, 32, 64);
  const float il = 1.0f / lt;
  if (q < a.Sq) {
    uint16_t* op = a.out + q * a.o_ss + static_cast<int64_t>(h) * a.o_sh;
    const float* vs = a.vscale + h * D;
    const float* vm = a.vmean + h * D;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = db * 32 + 8 * i + 4 * g;
        float4 s4 = *reinterpret_cast<const float4*>(vs + d);
        if constexpr (MODE == 2) {  // the e4m3 V codes were stretched by 448 / 127 (attn_int8.cu:2642)
          s4.x = s4.x * V_UNSTRETCH; s4.y = s4.y * V_UNSTRETCH; s4.z = s4.z * V_UNSTRETCH; s4.w = s4.w * V_UNSTRETCH;
        }
        const float4 m4 = *reinterpret_cast<const float4*>(vm + d);
        uint2 w;
        w.x = pack_bf2(fmaf(o[db][4 * i + 0] * il, s4.x, m4.x), fmaf(o[db][4 * i + 1] * il, s4.y, m4.y));
        w.y = pack_bf2(fmaf(o[db][4 * i + 2] * il, s4.z, m4.z), fmaf(o[db][4 * i + 3] * il, s4.w, m4.w));
        *reinterpret_cast<uint2*>(op + d) = w;
      }
  }
}

// ------------------------------------------------------------------ host
static_assert(TILE == attn_ws::BLK && SIDE == attn_ws::SIDE, "workspace layout constants");
using attn_ws::WorkU8;
using attn_ws::layout_u8;
inline int64_t padk(int64_t s) { return attn_ws::pad(s); }

int check_qkv_u8(const char* name, const uint16_t* q, int64_t q_ss, int64_t q_sh, const uint16_t* k, int64_t k_ss,
                 int64_t k_sh, const uint16_t* v, int64_t v_ss, int64_t v_sh, int64_t Sq, int64_t Sk, int64_t H) {
  RH3_REQUIRE(Sq > 0 && Sk > 0 && H > 0, "%s: sizes must be positive (Sq=%lld Sk=%lld H=%lld)", name, (long long)Sq,
              (long long)Sk, (long long)H);
  RH3_REQUIRE(H < 65536 && (Sq + U8_BQ - 1) / U8_BQ < (1ll << 31), "%s: grid too large", name);
  RH3_REQUIRE(padk(Sq) * H < (1ll << 31) && padk(Sk) * H < (1ll << 31), "%s: Spad * H must stay below 2^31", name);
  // the key-side pre-pass grids are (H, key blocks): at most 65,535 blocks of 128 keys
  RH3_REQUIRE(padk(Sk) / TILE < 65536, "%s: Sk=%lld exceeds the 8,388,480-key grid limit", name, (long long)Sk);
  RH3_REQUIRE(q && k && v, "%s: null q/k/v", name);
  RH3_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v), "%s: q/k/v must be 16-byte aligned", name);
  RH3_REQUIRE(q_ss % 8 == 0 && q_sh % 8 == 0 && k_ss % 8 == 0 && k_sh % 8 == 0 && v_ss % 8 == 0 && v_sh % 8 == 0,
              "%s: token/head strides must be multiples of 8 elements", name);
  return RH3_OK;
}

int check_rr_u8(const char* name, const uint16_t* tab, int rot, const uint16_t* qw, const uint16_t* kw) {
  RH3_REQUIRE(tab && qw && kw, "%s: tab, qw and kw are required", name);
  RH3_REQUIRE(rot == 96 || rot == 128, "%s: rot_dim %d (96 or 128 supported)", name, rot);
  RH3_REQUIRE(aligned16(tab) && aligned16(qw) && aligned16(kw), "%s: tab/qw/kw must be 16-byte aligned", name);
  return RH3_OK;
}

int prepass_u8(const uint16_t* q, int64_t q_ss, int64_t q_sh, const uint16_t* k, int64_t k_ss, int64_t k_sh,
               const uint16_t* v, int64_t v_ss, int64_t v_sh, int64_t Sq, int64_t Sk, int64_t H, const RR& rq,
               const RR& rk, int smooth_k, int smooth_v, int rotate, const WorkU8& w, hipStream_t st,
               bool f8 = false) {
  const int64_t sqp = padk(Sq), skp = padk(Sk);
  const int nchunk = static_cast<int>((Sk + CHUNK - 1) / CHUNK);
  const float* mean = nullptr;
  if (smooth_k) {
    launch_stats(dim3(H, nchunk), st, k, k_ss, k_sh, Sk, rk, w.kpart);
    hipLaunchKernelGGL(kmean_kernel, dim3(H), dim3(KMEAN_NT), 0, st, w.kpart, nchunk, Sk, w.kmean);
    mean = w.kmean;
  } else {
    // a fill kernel, not hipMemsetAsync, so the call stays safe inside a captured HIP graph
    hipLaunchKernelGGL(zero_kernel, dim3((H * D + 255) / 256), dim3(256), 0, st, w.kmean, H * D);
  }
  hipLaunchKernelGGL(vstats_kernel, dim3(H, nchunk), dim3(256), 0, st, v, v_ss, v_sh, Sk, w.vsum, w.vmax, w.vmin);
  hipLaunchKernelGGL(vfinal_kernel, dim3(H), dim3(VFINAL_NT), 0, st, w.vsum, w.vmax, w.vmin, nchunk, Sk, smooth_v, w.vmean,
                     w.vscale);
  hipLaunchKernelGGL(tokq_kernel, dim3(sqp * H / 16), dim3(256), 0, st, q, q_ss, q_sh, Sq, sqp, H, rq,
                     static_cast<const float*>(nullptr), rotate, w.q8, w.qs, static_cast<float*>(nullptr));
  hipLaunchKernelGGL(tokq_kernel, dim3(skp * H / 16), dim3(256), 0, st, k, k_ss, k_sh, Sk, skp, H, rk, mean, rotate,
                     w.k8, w.ks, reinterpret_cast<float*>(w.side));
  if (f8)  // configs 50-56: e4m3 V codes (attn_int8.cu:2639-2642)
    hipLaunchKernelGGL(vq_kernel<true>, dim3(H, skp / TILE), dim3(256), 0, st, v, v_ss, v_sh, Sk, skp, w.vmean,
                       w.vscale, w.vt, reinterpret_cast<int32_t*>(w.side));
  else
    hipLaunchKernelGGL(vq_kernel<false>, dim3(H, skp / TILE), dim3(256), 0, st, v, v_ss, v_sh, Sk, skp, w.vmean,
                       w.vscale, w.vt, reinterpret_cast<int32_t*>(w.side));
  return launch_status("attention_u8 prepass");
}

// Grid of the main kernel, whose workgroups take their (head, query block) items from a work counter: the grid is
// dealt to the XCDs in fixed shares and the XCDs run at different clocks, so the grid holds a quarter more
// workgroups than items (room for the fastest XCD to take a quarter more than its share); the extra ones return
// at once. gridDim.y carries H. The counter is cleared first by a fill kernel (no hipMemsetAsync: graph-safe).
dim3 claim_grid(U8Args& f, const WorkU8& w, int64_t Sq, int64_t H, hipStream_t st) {
  f.nqb = static_cast<int>((Sq + U8_BQ - 1) / U8_BQ);
  f.ctr = w.ctr;
  const int64_t per_head = f.nqb + (f.nqb + 3) / 4;
  hipLaunchKernelGGL(zero_kernel, dim3(1), dim3(64), 0, st, reinterpret_cast<float*>(w.ctr), int64_t{1});
  return dim3(static_cast<uint32_t>(per_head), static_cast<uint32_t>(H));
}

// configs 50-56: the FP8 P.V main kernel; tile = the reference's BN (64 or 128 keys per running-max update)
int forward_f8(const WorkU8& w, int64_t Sq, int64_t Sk, int64_t H, float scale, int tile, uint16_t* out, int64_t o_ss,
               int64_t o_sh, hipStream_t st) {
  U8Args f{w.q8, w.qs, w.k8, w.side, w.vt, w.vscale, w.vmean, out, o_ss, o_sh, Sq, Sk, padk(Sq), padk(Sk),
           scale * 1.4426950408889634f, 0, 0.0f};
  const dim3 grid = claim_grid(f, w, Sq, H, st);  // sets f.nqb and f.ctr: before f is passed
  if (tile == 64) hipLaunchKernelGGL((attn_u8_kernel<2, 64>), grid, dim3(U8_NT), 0, st, f);
  else hipLaunchKernelGGL((attn_u8_kernel<2, 128>), grid, dim3(U8_NT), 0, st, f);
  return launch_status("attention_f8 forward");
}

int forward_u8(const WorkU8& w, int64_t Sq, int64_t Sk, int64_t H, float scale, int nbias, double bias, uint16_t* out,
               int64_t o_ss, int64_t o_sh, hipStream_t st) {
  U8Args f{w.q8, w.qs, w.k8, w.side, w.vt, w.vscale, w.vmean, out, o_ss, o_sh, Sq, Sk, padk(Sq), padk(Sk),
           scale * 1.4426950408889634f, nbias, static_cast<float>(bias * 1.4426950408889634)};
  const dim3 grid = claim_grid(f, w, Sq, H, st);  // sets f.nqb and f.ctr: before f is passed
  hipLaunchKernelGGL(attn_u8_kernel<0>, grid, dim3(U8_NT), 0, st, f);
  return launch_status("attention_u8 forward");
}

// configs 60-61: Q per token as prepass_u8 (no RMSNorm + RoPE: the reference has none for these configs), K one
// scale per 128-key block after the smoothing and the optional H128 (into ks [H][Skpad/128] and the side records),
// V as prepass_u8 (attn_int8.cu:2618-2641)
int prepass_bk(const uint16_t* q, int64_t q_ss, int64_t q_sh, const uint16_t* k, int64_t k_ss, int64_t k_sh,
               const uint16_t* v, int64_t v_ss, int64_t v_sh, int64_t Sq, int64_t Sk, int64_t H, int smooth_k,
               int smooth_v, int rotate, const WorkU8& w, hipStream_t st) {
  const int64_t sqp = padk(Sq), skp = padk(Sk);
  const int nchunk = static_cast<int>((Sk + CHUNK - 1) / CHUNK);
  const RR none{nullptr, nullptr, 0.f, 0};
  if (smooth_k) {
    launch_stats(dim3(H, nchunk), st, k, k_ss, k_sh, Sk, none, w.kpart);
    hipLaunchKernelGGL(kmean_kernel, dim3(H), dim3(KMEAN_NT), 0, st, w.kpart, nchunk, Sk, w.kmean);
  } else {
    hipLaunchKernelGGL(zero_kernel, dim3((H * D + 255) / 256), dim3(256), 0, st, w.kmean, H * D);
  }
  hipLaunchKernelGGL(vstats_kernel, dim3(H, nchunk), dim3(256), 0, st, v, v_ss, v_sh, Sk, w.vsum, w.vmax, w.vmin);
  hipLaunchKernelGGL(vfinal_kernel, dim3(H), dim3(VFINAL_NT), 0, st, w.vsum, w.vmax, w.vmin, nchunk, Sk, smooth_v,
                     w.vmean, w.vscale);
  hipLaunchKernelGGL(tokq_kernel, dim3(sqp * H / 16), dim3(256), 0, st, q, q_ss, q_sh, Sq, sqp, H, none,
                     static_cast<const float*>(nullptr), rotate, w.q8, w.qs, static_cast<float*>(nullptr));
  hipLaunchKernelGGL(blockk_kernel, dim3(H, skp / TILE), dim3(256), 0, st, k, k_ss, k_sh, Sk, skp,
                     static_cast<const float*>(w.kmean), rotate, w.k8, w.ks, reinterpret_cast<float*>(w.side));
  hipLaunchKernelGGL(vq_kernel<false>, dim3(H, skp / TILE), dim3(256), 0, st, v, v_ss, v_sh, Sk, skp, w.vmean, w.vscale,
                     w.vt, reinterpret_cast<int32_t*>(w.side));
  return launch_status("attention_bk prepass");
}

int forward_bk(const WorkU8& w, int64_t Sq, int64_t Sk, int64_t H, float scale, uint16_t* out, int64_t o_ss,
               int64_t o_sh, hipStream_t st) {
  U8Args f{w.q8, w.qs, w.k8, w.side, w.vt, w.vscale, w.vmean, out, o_ss, o_sh, Sq, Sk, padk(Sq), padk(Sk),
           scale * 1.4426950408889634f, 0, 0.0f};
  const dim3 grid = claim_grid(f, w, Sq, H, st);  // sets f.nqb and f.ctr: before f is passed
  hipLaunchKernelGGL(attn_u8_kernel<1>, grid, dim3(U8_NT), 0, st, f);
  return launch_status("attention_bk forward");
}

int check_out_u8(const char* name, const uint16_t* out, int64_t o_ss, int64_t o_sh) {
  RH3_REQUIRE(out && (reinterpret_cast<uintptr_t>(out) & 7) == 0 && o_ss % 4 == 0 && o_sh % 4 == 0,
              "%s: out must be 8-byte aligned with strides multiple of 4", name);
  return RH3_OK;
}

int check_bias_u8(const char* name, int nbias, int64_t Sk) {
  RH3_REQUIRE(nbias >= 0 && nbias <= Sk, "%s: nbias %d outside [0, Sk=%lld]", name, nbias, (long long)Sk);
  return RH3_OK;
}

}  // namespace
}  // namespace rh3

using namespace rh3;

extern "C" int rh3_attention_workspace_layout(int numerics, int64_t Sq, int64_t Sk, int64_t H, int64_t* offsets) {
  clear_error();
  RH3_REQUIRE(Sq > 0 && Sk > 0 && H > 0 && offsets, "attention_workspace_layout: sizes must be positive, offsets set");
  char* const b = reinterpret_cast<char*>(static_cast<uintptr_t>(256));  // any aligned base; offsets relative
  auto off = [&](const void* p) { return static_cast<int64_t>(static_cast<const char*>(p) - b); };
  if (numerics == 0) {
    const attn_ws::Work w = attn_ws::layout(b, Sq, Sk, H);
    const void* ps[8] = {w.q8, w.qs, w.k8, w.ks, w.kmean, w.part, w.vt, w.kn};
    for (int i = 0; i < 8; ++i) offsets[i] = off(ps[i]);
    offsets[8] = w.bytes;
    return RH3_OK;
  }
  RH3_REQUIRE(numerics == 1, "attention_workspace_layout: numerics %d (0 per-block, 1 production)", numerics);
  const WorkU8 w = layout_u8(b, Sq, Sk, H);
  const void* ps[13] = {w.q8, w.qs, w.k8, w.ks, w.side, w.vt, w.kmean, w.vmean, w.vscale,
                        w.kpart, w.vsum, w.vmax, w.vmin};
  for (int i = 0; i < 13; ++i) offsets[i] = off(ps[i]);
  offsets[13] = w.bytes;
  return RH3_OK;
}

extern "C" int64_t rh3_attention_u8_workspace_bytes(int64_t Sq, int64_t Sk, int64_t H) {
  if (Sq <= 0 || Sk <= 0 || H <= 0) return 0;
  return layout_u8(nullptr, Sq, Sk, H).bytes;
}

extern "C" int rh3_attention_u8_prepass(const uint16_t* q, int64_t q_ss, int64_t q_sh, const uint16_t* k,
                                        int64_t k_ss, int64_t k_sh, const uint16_t* v, int64_t v_ss, int64_t v_sh,
                                        int64_t Sq, int64_t Sk, int64_t H, const uint16_t* tab, int rot,
                                        const uint16_t* qw, const uint16_t* kw, float eps, int smooth_k, int smooth_v,
                                        int rotate, void* workspace, int64_t workspace_bytes, void** ptrs,
                                        hipStream_t stream) {
  clear_error();
  if (int e = check_qkv_u8("attention_u8_prepass", q, q_ss, q_sh, k, k_ss, k_sh, v, v_ss, v_sh, Sq, Sk, H)) return e;
  RH3_REQUIRE(ptrs, "attention_u8_prepass: ptrs required");
  const WorkU8 w = layout_u8(workspace, Sq, Sk, H);
  RH3_REQUIRE(workspace && aligned16(workspace) && workspace_bytes >= w.bytes,
              "attention_u8_prepass: workspace %lld bytes < required %lld", (long long)workspace_bytes,
              (long long)w.bytes);
  RR rq{nullptr, nullptr, 0.f, 0}, rk{nullptr, nullptr, 0.f, 0};
  if (tab) {
    if (int e = check_rr_u8("attention_u8_prepass", tab, rot, qw, kw)) return e;
    RH3_REQUIRE(Sq == Sk, "attention_u8_prepass: RMSNorm+RoPE needs self-attention (Sq == Sk)");
    rq = RR{tab, qw, eps, rot};
    rk = RR{tab, kw, eps, rot};
  }
  if (int e = prepass_u8(q, q_ss, q_sh, k, k_ss, k_sh, v, v_ss, v_sh, Sq, Sk, H, rq, rk, smooth_k, smooth_v, rotate,
                         w, stream))
    return e;
  ptrs[0] = w.q8; ptrs[1] = w.qs; ptrs[2] = w.k8; ptrs[3] = w.ks; ptrs[4] = w.side; ptrs[5] = w.vt;
  ptrs[6] = w.kmean; ptrs[7] = w.vscale; ptrs[8] = w.vmean;
  return RH3_OK;
}

extern "C" int rh3_attention_u8_prepass_qkv(const uint16_t* k, int64_t k_ss, int64_t k_sh, const uint16_t* v,
                                            int64_t v_ss, int64_t v_sh, int64_t S, int64_t H, const uint16_t* tab,
                                            int rot, const uint16_t* kw, float eps, int smooth_k, int smooth_v,
                                            int rotate, void* workspace, int64_t workspace_bytes, void** ptrs,
                                            hipStream_t stream) {
  clear_error();
  if (int e = check_qkv_u8("attention_u8_prepass_qkv", k, k_ss, k_sh, k, k_ss, k_sh, v, v_ss, v_sh, S, S, H)) return e;
  RH3_REQUIRE(ptrs, "attention_u8_prepass_qkv: ptrs required");
  const WorkU8 w = layout_u8(workspace, S, S, H);
  RH3_REQUIRE(workspace && aligned16(workspace) && workspace_bytes >= w.bytes,
              "attention_u8_prepass_qkv: workspace %lld bytes < required %lld", (long long)workspace_bytes,
              (long long)w.bytes);
  RR rk{nullptr, nullptr, 0.f, 0};
  if (tab) {
    RH3_REQUIRE(kw && (rot == 96 || rot == 128) && aligned16(tab) && aligned16(kw),
                "attention_u8_prepass_qkv: kw (16-byte aligned) and rot_dim 96 or 128 required with tab");
    rk = RR{tab, kw, eps, rot};
  }
  // q8, qs and the K / V channel statistics come from rh3_gemm_i8_qkv (numerics 1) on this workspace
  const int64_t skp = padk(S);
  const int nchunk = static_cast<int>((S + CHUNK - 1) / CHUNK);
  const float* mean = nullptr;
  if (smooth_k) {
    hipLaunchKernelGGL(kmean_kernel, dim3(H), dim3(KMEAN_NT), 0, stream, w.kpart, nchunk, S, w.kmean);
    mean = w.kmean;
  } else {
    hipLaunchKernelGGL(zero_kernel, dim3((H * D + 255) / 256), dim3(256), 0, stream, w.kmean, H * D);
  }
  hipLaunchKernelGGL(vfinal_kernel, dim3(H), dim3(VFINAL_NT), 0, stream, w.vsum, w.vmax, w.vmin, nchunk, S, smooth_v, w.vmean,
                     w.vscale);
  hipLaunchKernelGGL(tokq_kernel, dim3(skp * H / 16), dim3(256), 0, stream, k, k_ss, k_sh, S, skp, H, rk, mean, rotate,
                     w.k8, w.ks, reinterpret_cast<float*>(w.side));
  hipLaunchKernelGGL(vq_kernel<false>, dim3(H, skp / TILE), dim3(256), 0, stream, v, v_ss, v_sh, S, skp, w.vmean, w.vscale,
                     w.vt, reinterpret_cast<int32_t*>(w.side));
  if (int e = launch_status("attention_u8 prepass_qkv")) return e;
  ptrs[0] = w.q8; ptrs[1] = w.qs; ptrs[2] = w.k8; ptrs[3] = w.ks; ptrs[4] = w.side; ptrs[5] = w.vt;
  ptrs[6] = w.kmean; ptrs[7] = w.vscale; ptrs[8] = w.vmean;
  return RH3_OK;
}

extern "C" int rh3_attention_u8_forward(int64_t Sq, int64_t Sk, int64_t H, float scale, int nbias, double bias,
                                        uint16_t* out, int64_t o_ss, int64_t o_sh, void* workspace,
                                        int64_t workspace_bytes, hipStream_t stream) {
  clear_error();
  RH3_REQUIRE(Sq > 0 && Sk > 0 && H > 0, "attention_u8_forward: sizes must be positive");
  if (int e = check_out_u8("attention_u8_forward", out, o_ss, o_sh)) return e;
  if (int e = check_bias_u8("attention_u8_forward", nbias, Sk)) return e;
  const WorkU8 w = layout_u8(workspace, Sq, Sk, H);
  RH3_REQUIRE(workspace && aligned16(workspace) && workspace_bytes >= w.bytes,
              "attention_u8_forward: workspace %lld bytes < required %lld", (long long)workspace_bytes,
              (long long)w.bytes);
  return forward_u8(w, Sq, Sk, H, scale, nbias, bias, out, o_ss, o_sh, stream);
}

extern "C" int rh3_int8_attention_u8(const uint16_t* q, int64_t q_ss, int64_t q_sh, const uint16_t* k, int64_t k_ss,
                                     int64_t k_sh, const uint16_t* v, int64_t v_ss, int64_t v_sh, int64_t Sq,
                                     int64_t Sk, int64_t H, const uint16_t* tab, int rot, const uint16_t* qw,
                                     const uint16_t* kw, float eps, float scale, int nbias, double bias, int smooth_k,
                                     int smooth_v, int rotate, uint16_t* out, int64_t o_ss, int64_t o_sh,
                                     void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  clear_error();
  if (int e = check_qkv_u8("int8_attention_u8", q, q_ss, q_sh, k, k_ss, k_sh, v, v_ss, v_sh, Sq, Sk, H)) return e;
  if (int e = check_out_u8("int8_attention_u8", out, o_ss, o_sh)) return e;
  if (int e = check_bias_u8("int8_attention_u8", nbias, Sk)) return e;
  const WorkU8 w = layout_u8(workspace, Sq, Sk, H);
  RH3_REQUIRE(workspace && aligned16(workspace) && workspace_bytes >= w.bytes,
              "int8_attention_u8: workspace %lld bytes < required %lld", (long long)workspace_bytes,
              (long long)w.bytes);
  RR rq{nullptr, nullptr, 0.f, 0}, rk{nullptr, nullptr, 0.f, 0};
  if (tab) {
    if (int e = check_rr_u8("int8_attention_u8", tab, rot, qw, kw)) return e;
    RH3_REQUIRE(Sq == Sk, "int8_attention_u8: RMSNorm+RoPE needs self-attention (Sq == Sk)");
    rq = RR{tab, qw, eps, rot};
    rk = RR{tab, kw, eps, rot};
  }
  if (int e = prepass_u8(q, q_ss, q_sh, k, k_ss, k_sh, v, v_ss, v_sh, Sq, Sk, H, rq, rk, smooth_k, smooth_v, rotate,
                         w, stream))
    return e;
  return forward_u8(w, Sq, Sk, H, scale, nbias, bias, out, o_ss, o_sh, stream);
}

extern "C" int rh3_attention_bk_prepass(const uint16_t* q, int64_t q_ss, int64_t q_sh, const uint16_t* k,
                                        int64_t k_ss, int64_t k_sh, const uint16_t* v, int64_t v_ss, int64_t v_sh,
                                        int64_t Sq, int64_t Sk, int64_t H, int smooth_k, int smooth_v, int rotate,
                                        void* workspace, int64_t workspace_bytes, void** ptrs, hipStream_t stream) {
  clear_error();
  if (int e = check_qkv_u8("attention_bk_prepass", q, q_ss, q_sh, k, k_ss, k_sh, v, v_ss, v_sh, Sq, Sk, H)) return e;
  RH3_REQUIRE(ptrs, "attention_bk_prepass: ptrs required");
  const WorkU8 w = layout_u8(workspace, Sq, Sk, H);
  RH3_REQUIRE(workspace && aligned16(workspace) && workspace_bytes >= w.bytes,
              "attention_bk_prepass: workspace %lld bytes < required %lld", (long long)workspace_bytes,
              (long long)w.bytes);
  if (int e = prepass_bk(q, q_ss, q_sh, k, k_ss, k_sh, v, v_ss, v_sh, Sq, Sk, H, smooth_k, smooth_v, rotate, w, stream))
    return e;
  ptrs[0] = w.q8; ptrs[1] = w.qs; ptrs[2] = w.k8; ptrs[3] = w.ks; ptrs[4] = w.side; ptrs[5] = w.vt;
  ptrs[6] = w.kmean; ptrs[7] = w.vscale; ptrs[8] = w.vmean;
  return RH3_OK;
}

extern "C" int rh3_attention_bk_forward(int64_t Sq, int64_t Sk, int64_t H, float scale, uint16_t* out, int64_t o_ss,
                                        int64_t o_sh, void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  clear_error();
  RH3_REQUIRE(Sq > 0 && Sk > 0 && H > 0, "attention_bk_forward: sizes must be positive");
  if (int e = check_out_u8("attention_bk_forward", out, o_ss, o_sh)) return e;
  const WorkU8 w = layout_u8(workspace, Sq, Sk, H);
  RH3_REQUIRE(workspace && aligned16(workspace) && workspace_bytes >= w.bytes,
              "attention_bk_forward: workspace %lld bytes < required %lld", (long long)workspace_bytes,
              (long long)w.bytes);
  return forward_bk(w, Sq, Sk, H, scale, out, o_ss, o_sh, stream);
}

extern "C" int rh3_int8_attention_bk(const uint16_t* q, int64_t q_ss, int64_t q_sh, const uint16_t* k, int64_t k_ss,
                                     int64_t k_sh, const uint16_t* v, int64_t v_ss, int64_t v_sh, int64_t Sq,
                                     int64_t Sk, int64_t H, float scale, int smooth_k, int smooth_v, int rotate,
                                     uint16_t* out, int64_t o_ss, int64_t o_sh, void* workspace,
                                     int64_t workspace_bytes, hipStream_t stream) {
  clear_error();
  if (int e = check_qkv_u8("int8_attention_bk", q, q_ss, q_sh, k, k_ss, k_sh, v, v_ss, v_sh, Sq, Sk, H)) return e;
  if (int e = check_out_u8("int8_attention_bk", out, o_ss, o_sh)) return e;
  const WorkU8 w = layout_u8(workspace, Sq, Sk, H);
  RH3_REQUIRE(workspace && aligned16(workspace) && workspace_bytes >= w.bytes,
              "int8_attention_bk: workspace %lld bytes < required %lld", (long long)workspace_bytes,
              (long long)w.bytes);
  if (int e = prepass_bk(q, q_ss, q_sh, k, k_ss, k_sh, v, v_ss, v_sh, Sq, Sk, H, smooth_k, smooth_v, rotate, w, stream))
    return e;
  return forward_bk(w, Sq, Sk, H, scale, out, o_ss, o_sh, stream);
}

extern "C" int rh3_attention_f8_prepass(const uint16_t* q, int64_t q_ss, int64_t q_sh, const uint16_t* k,
                                        int64_t k_ss, int64_t k_sh, const uint16_t* v, int64_t v_ss, int64_t v_sh,
                                        int64_t Sq, int64_t Sk, int64_t H, const uint16_t* tab, int rot,
                                        const uint16_t* qw, const uint16_t* kw, float eps, int smooth_k, int smooth_v,
                                        int rotate, void* workspace, int64_t workspace_bytes, void** ptrs,
                                        hipStream_t stream) {
  clear_error();
  if (int e = check_qkv_u8("attention_f8_prepass", q, q_ss, q_sh, k, k_ss, k_sh, v, v_ss, v_sh, Sq, Sk, H)) return e;
  RH3_REQUIRE(ptrs, "attention_f8_prepass: ptrs required");
  const WorkU8 w = layout_u8(workspace, Sq, Sk, H);
  RH3_REQUIRE(workspace && aligned16(workspace) && workspace_bytes >= w.bytes,
              "attention_f8_prepass: workspace %lld bytes < required %lld", (long long)workspace_bytes,
              (long long)w.bytes);
  RR rq{nullptr, nullptr, 0.f, 0}, rk{nullptr, nullptr, 0.f, 0};
  if (tab) {
    if (int e = check_rr_u8("attention_f8_prepass", tab, rot, qw, kw)) return e;
    RH3_REQUIRE(Sq == Sk, "attention_f8_prepass: RMSNorm+RoPE needs self-attention (Sq == Sk)");
    rq = RR{tab, qw, eps, rot};
    rk = RR{tab, kw, eps, rot};
  }
  if (int e = prepass_u8(q, q_ss, q_sh, k, k_ss, k_sh, v, v_ss, v_sh, Sq, Sk, H, rq, rk, smooth_k, smooth_v, rotate,
                         w, stream, true))
    return e;
  ptrs[0] = w.q8; ptrs[1] = w.qs; ptrs[2] = w.k8; ptrs[3] = w.ks; ptrs[4] = w.side; ptrs[5] = w.vt;
  ptrs[6] = w.kmean; ptrs[7] = w.vscale; ptrs[8] = w.vmean;
  return RH3_OK;
}

extern "C" int rh3_attention_f8_forward(int64_t Sq, int64_t Sk, int64_t H, float scale, int tile, uint16_t* out,
                                        int64_t o_ss, int64_t o_sh, void* workspace, int64_t workspace_bytes,
                                        hipStream_t stream) {
  clear_error();
  RH3_REQUIRE(Sq > 0 && Sk > 0 && H > 0, "attention_f8_forward: sizes must be positive");
  RH3_REQUIRE(tile == 64 || tile == 128, "attention_f8_forward: tile %d (64 or 128 keys)", tile);
  if (int e = check_out_u8("attention_f8_forward", out, o_ss, o_sh)) return e;
  const WorkU8 w = layout_u8(workspace, Sq, Sk, H);
  RH3_REQUIRE(workspace && aligned16(workspace) && workspace_bytes >= w.bytes,
              "attention_f8_forward: workspace %lld bytes < required %lld", (long long)workspace_bytes,
              (long long)w.bytes);
  return forward_f8(w, Sq, Sk, H, scale, tile, out, o_ss, o_sh, stream);
}

extern "C" int rh3_int8_attention_f8(const uint16_t* q, int64_t q_ss, int64_t q_sh, const uint16_t* k, int64_t k_ss,
                                     int64_t k_sh, const uint16_t* v, int64_t v_ss, int64_t v_sh, int64_t Sq,
                                     int64_t Sk, int64_t H, const uint16_t* tab, int rot, const uint16_t* qw,
                                     const uint16_t* kw, float eps, float scale, int tile, int smooth_k, int smooth_v,
                                     int rotate, uint16_t* out, int64_t o_ss, int64_t o_sh, void* workspace,
                                     int64_t workspace_bytes, hipStream_t stream) {
  void* ptrs[9];
  if (int e = rh3_attention_f8_prepass(q, q_ss, q_sh, k, k_ss, k_sh, v, v_ss, v_sh, Sq, Sk, H, tab, rot, qw, kw, eps,
                                       smooth_k, smooth_v, rotate, workspace, workspace_bytes, ptrs, stream))
    return e;
  return rh3_attention_f8_forward(Sq, Sk, H, scale, tile, out, o_ss, o_sh, workspace, workspace_bytes, stream);
}
