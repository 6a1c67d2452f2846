// Row-wise W8A8 (int8) and FP8 (OCP e4m3fn) GEMMs on CDNA4 MFMA with fused epilogues.
//
//   acc[m, n] = sum_k xq[m, k] * wq[n, k]        (both operands K-contiguous: the "TN" GEMM)
//   y = (fp32(acc) * xs[m]) * ws[n]               fp8_rowwise.cu:294-304 (EVT order)
//   EPI_PLAIN   out = bf16(y [+ bias[n]])
//   EPI_SWIGLU  g, u = bf16(y) over the swiglu_perm interleave; h = bf16((g * sigmoid(g)) * u) at n / 2
//   EPI_GATED   resid = bf16(fma(bf16(y), gate[n], resid))     (in place)
//   EPI_ACC     raw int32 accumulators (verification)
//
// Schedule: 256x256 output tile per workgroup, 8 waves (2 per SIMD, so each hides the other's LDS and
// barrier latency) in a 2x4 grid, 128x64 per wave held in registers (int8: 2x4 v_mfma_i32_32x32x32_i8
// tiles; fp8: v_mfma_f32_32x32x64_f8f6f4). K advances 64 bytes per step through a 4-stage LDS ring
// (4 x 32 KiB) filled by asynchronous global->LDS loads three steps ahead; each step waits only for the
// loads of the next step, then one barrier. LDS rows are 64 B; 16-byte chunks are XOR-swizzled by row so
// the ds_read_b128 fragment loads of 16 consecutive rows hit distinct banks.
//
// MFMA roles: the weight tile is the A operand (rows = n) and the activation tile the B operand
// (columns = m), so each lane's accumulator holds one token m and runs of 4 consecutive n — the
// epilogue writes 8-byte bf16 vectors along n. Workgroups are mapped XCD-aware: consecutive
// workgroup ids land on different XCDs, so the tile order is remapped to give every XCD a
// contiguous run of tiles that walk N fastest (one activation panel stays in that XCD's L2).
#include "rh3_common.hpp"

namespace rh3 {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

enum Epi { EPI_PLAIN = 0, EPI_SWIGLU = 1, EPI_GATED = 2, EPI_ACC = 3 };

constexpr int BM = 256, BN = 256, BK = 64, NT = 512;
// 8 waves in a 2 (m) x 4 (n) grid, 128 x 64 outputs per wave: 2 waves per SIMD hide each other's LDS and
// barrier latency
constexpr int WAVES = NT / 64, WM = 128, WN = 64, TI = WN / 32, TJ = WM / 32;
constexpr int TILE_BYTES = BM * BK;  // per operand per stage (BM == BN)

struct GemmArgs {
  const int8_t* x;  // [M, K] int8 or e4m3 codes
  int64_t ldx;
  const int8_t* w;  // [N, K]
  int64_t ldw;
  const float* xs;
  const float* ws;
  const uint16_t* bias;
  const uint16_t* gate;
  void* out;  // bf16 out / resid / int32 acc
  int64_t ldo;
  int64_t M, N, K;
  int tiles_m, tiles_n;
};

// 16-byte chunk c (0..3) of LDS row r: rows r, r+1 share a 128-byte line; the XOR keeps 16
// consecutive rows of one chunk column on 16 distinct 16-byte bank groups.
__device__ __forceinline__ int swz(int r, int c) {
  return r * BK + ((c ^ (((r >> 1) & 3) ^ ((r >> 3) & 1))) << 4);
}

__device__ __forceinline__ float silu_mul(float g, float u) {
  const float sig = 1.0f / (1.0f + __expf(-g));
  return (g * sig) * u;
}

template <bool FP8>
struct Mma;

template <>
struct Mma<false> {  // int8: 2 MFMAs of k = 32 per 64-byte step, 16-byte fragments
  typedef v16i acc_t;
  static constexpr int KSUB = 2;
  typedef v4i frag_t;
  __device__ static frag_t load(const int8_t* lds, int row, int ks, int g) {
    return *reinterpret_cast<const v4i*>(lds + swz(row, ks * 2 + g));
  }
  __device__ static acc_t mma(frag_t a, frag_t b, acc_t c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
  }
  __device__ static float val(const acc_t& c, int r) { return static_cast<float>(c[r]); }
};

template <>
struct Mma<true> {  // e4m3: 1 MFMA of k = 64 per step, 32-byte fragments (two 16-byte chunks)
  typedef v16f acc_t;
  static constexpr int KSUB = 1;
  typedef v8i frag_t;
  __device__ static frag_t load(const int8_t* lds, int row, int, int g) {
    const v4i lo = *reinterpret_cast<const v4i*>(lds + swz(row, 2 * g));
    const v4i hi = *reinterpret_cast<const v4i*>(lds + swz(row, 2 * g + 1));
    frag_t f;
    f[0] = lo[0]; f[1] = lo[1]; f[2] = lo[2]; f[3] = lo[3];
    f[4] = hi[0]; f[5] = hi[1]; f[6] = hi[2]; f[7] = hi[3];
    return f;
  }
  __device__ static acc_t mma(frag_t a, frag_t b, acc_t c) {
    // cbsz / blgp type 0 = FP8 E4M3 for both operands; zero scale operands select the unscaled form
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
  }
  __device__ static float val(const acc_t& c, int r) { return c[r]; }
};

template <bool FP8, int EPI>
__global__ void __launch_bounds__(NT, 2) gemm_kernel(const GemmArgs a) {
  using MM = Mma<FP8>;
  using acc_t = typename MM::acc_t;
  // 4-stage ring, each stage its own LDS object {x tile, w tile} (2 x 16 KiB) named statically: the
  // asynchronous global->LDS loads into one stage then provably do not alias the reads of another
  __shared__ __attribute__((aligned(16))) int8_t st0[2 * TILE_BYTES], st1[2 * TILE_BYTES], st2[2 * TILE_BYTES],
      st3[2 * TILE_BYTES];

  // XCD-aware tile order: workgroup id b runs on XCD b % 8; give XCD x the contiguous logical range
  const int nb = a.tiles_m * a.tiles_n;
  const int b = blockIdx.x;
  const int xcd = b % 8, slot = b / 8;
  const int lt = xcd * (nb / 8) + min(xcd, nb % 8) + slot;  // XCD x owns logical tiles [prefix(x), prefix(x+1))
  const int tm = lt / a.tiles_n, tn = lt % a.tiles_n;
  const int64_t m0 = static_cast<int64_t>(tm) * BM, n0 = static_cast<int64_t>(tn) * BN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3;
  const int l32 = lane & 31, g = lane >> 5;

  // Global -> LDS loads bypass VGPRs (global_load_lds_dwordx4: lane l of a wave writes LDS base + 16*l),
  // so the XOR swizzle is applied on the global side: stage position p (16-byte units, 1024 per operand)
  // holds row p / 4, logical chunk (p % 4) ^ f(row) (swz is an involution on the chunk index). Wave w
  // fills positions (2w + i)*64 + lane, i = 0, 1, of each operand.
  const int8_t* xp[2];
  const int8_t* wp[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int p = (2 * wave + i) * 64 + lane, r = p >> 2;
    const int c = (p & 3) ^ (((r >> 1) & 3) ^ ((r >> 3) & 1));
    int64_t mr = m0 + r, nr = n0 + r;
    mr = mr < a.M ? mr : a.M - 1;
    nr = nr < a.N ? nr : a.N - 1;
    xp[i] = a.x + mr * a.ldx + c * 16;
    wp[i] = a.w + nr * a.ldw + c * 16;
  }
  const int nk = static_cast<int>(a.K / BK);
  // loads of k-step kt into a stage (clamped to the last step so every step issues the same four
  // loads and the vmcnt bookkeeping stays exact; a clamped load lands in a stage nobody reads again)
  auto gload = [&](int kt, int8_t* stg) __attribute__((always_inline)) {
    const int64_t k0 = static_cast<int64_t>(min(kt, nk - 1)) * BK;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      __builtin_amdgcn_global_load_lds(xp[i] + k0, stg + (2 * wave + i) * 1024, 16, 0, 0);
      __builtin_amdgcn_global_load_lds(wp[i] + k0, stg + TILE_BYTES + (2 * wave + i) * 1024, 16, 0, 0);
    }
  };

  acc_t acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  // k-step kt: load step kt+3 into the stage step kt-1 used, compute from this stage, then wait for
  // step kt+1's loads (the 8 most recent loads, steps kt+2 and kt+3, stay in flight) and barrier
  auto step = [&](const int kt, const int8_t* cur, int8_t* nxt3) __attribute__((always_inline)) {
    gload(kt + 3, nxt3);
    const int8_t* ldx = cur;
    const int8_t* ldw = cur + TILE_BYTES;
#pragma unroll
    for (int ks = 0; ks < MM::KSUB; ++ks) {
      typename MM::frag_t fa[TI], fb[TJ];
#pragma unroll
      for (int i = 0; i < TI; ++i) fa[i] = MM::load(ldw, wn * WN + i * 32 + l32, ks, g);
#pragma unroll
      for (int j = 0; j < TJ; ++j) fb[j] = MM::load(ldx, wm * WM + j * 32 + l32, ks, g);
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = MM::mma(fa[i], fb[j], acc[i][j]);
    }
    // s_waitcnt on gfx9: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14];
    // vmcnt(8) expcnt(7) lgkmcnt(0) = 8 | 0x70
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0x0078);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  gload(0, st0);
  gload(1, st1);
  gload(2, st2);
  asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  __syncthreads();
  int kt = 0;
  for (; kt + 4 <= nk; kt += 4) {
    step(kt + 0, st0, st3);
    step(kt + 1, st1, st0);
    step(kt + 2, st2, st1);
    step(kt + 3, st3, st2);
  }
  const int rem = nk - kt;  // steps left: they read stages 0, 1, 2 in order
  if (rem >= 1) step(kt + 0, st0, st3);
  if (rem >= 2) step(kt + 1, st1, st0);
  if (rem >= 3) step(kt + 2, st2, st1);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no global->LDS load outlives the workgroup

  // epilogue: acc[i][j] register r holds m = m0 + wm*128 + j*32 + l32,
  //           n = n0 + wn*64 + i*32 + 8*(r/4) + 4*g + (r%4)
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const int64_t m = m0 + wm * WM + j * 32 + l32;
    const bool mok = m < a.M;
    const float xsm = (EPI != EPI_ACC && mok) ? a.xs[m] : 0.0f;
#pragma unroll
    for (int i = 0; i < TI; ++i) {
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int64_t n = n0 + wn * WN + i * 32 + 8 * rq + 4 * g;
        const bool ok = mok && n < a.N;
        if constexpr (EPI == EPI_ACC) {
          static_assert(!FP8, "raw accumulators are an int8 feature");
          if (ok) {
            int4 v;
            v.x = acc[i][j][4 * rq + 0];
            v.y = acc[i][j][4 * rq + 1];
            v.z = acc[i][j][4 * rq + 2];
            v.w = acc[i][j][4 * rq + 3];
            *reinterpret_cast<int4*>(static_cast<int32_t*>(a.out) + m * a.ldo + n) = v;
          }
          continue;
        }
        float y[4];
        float4 wsn = make_float4(0.f, 0.f, 0.f, 0.f);
        if (n < a.N) wsn = *reinterpret_cast<const float4*>(a.ws + n);
        const float wsv[4] = {wsn.x, wsn.y, wsn.z, wsn.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = (MM::val(acc[i][j], 4 * rq + e) * xsm) * wsv[e];
        if constexpr (EPI == EPI_PLAIN) {
          if (ok) {
            if (a.bias) {
              const uint2 bb = *reinterpret_cast<const uint2*>(a.bias + n);
              y[0] = y[0] + __uint_as_float(bb.x << 16);
              y[1] = y[1] + __uint_as_float(bb.x & 0xffff0000u);
              y[2] = y[2] + __uint_as_float(bb.y << 16);
              y[3] = y[3] + __uint_as_float(bb.y & 0xffff0000u);
            }
            uint2 o;
            o.x = pack_bf2(y[0], y[1]);
            o.y = pack_bf2(y[2], y[3]);
            *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.out) + m * a.ldo + n) = o;
          }
        } else if constexpr (EPI == EPI_GATED) {
          if (ok) {
            uint16_t* rp = static_cast<uint16_t*>(a.out) + m * a.ldo + n;
            const uint2 rr = *reinterpret_cast<const uint2*>(rp);
            const uint2 gg = *reinterpret_cast<const uint2*>(a.gate + n);
            const float rv[4] = {__uint_as_float(rr.x << 16), __uint_as_float(rr.x & 0xffff0000u),
                                 __uint_as_float(rr.y << 16), __uint_as_float(rr.y & 0xffff0000u)};
            const float gv[4] = {__uint_as_float(gg.x << 16), __uint_as_float(gg.x & 0xffff0000u),
                                 __uint_as_float(gg.y << 16), __uint_as_float(gg.y & 0xffff0000u)};
            float o4[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) o4[e] = fmaf(round_bf(y[e]), gv[e], rv[e]);
            uint2 o;
            o.x = pack_bf2(o4[0], o4[1]);
            o.y = pack_bf2(o4[2], o4[3]);
            *reinterpret_cast<uint2*>(rp) = o;
          }
        } else {  // EPI_SWIGLU: lanes g = 0 hold gate columns 4j..4j+3, lanes g = 1 the matching up columns
          float other[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) other[e] = __shfl_xor(y[e], 32, 64);
          if (g == 0 && ok) {
            float h[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) h[e] = silu_mul(round_bf(y[e]), round_bf(other[e]));
            uint2 o;
            o.x = pack_bf2(h[0], h[1]);
            o.y = pack_bf2(h[2], h[3]);
            *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.out) + m * a.ldo + n / 2) = o;
          }
        }
      }
    }
  }
}

template <bool FP8, int EPI>
int run(GemmArgs a, hipStream_t st, const char* name) {
  if (a.M == 0 || a.N == 0) return RH3_OK;
  a.tiles_m = static_cast<int>((a.M + BM - 1) / BM);
  a.tiles_n = static_cast<int>((a.N + BN - 1) / BN);
  const int64_t nb = static_cast<int64_t>(a.tiles_m) * a.tiles_n;
  RH3_REQUIRE(nb < (1ll << 31), "%s: too many tiles", name);
  hipLaunchKernelGGL((gemm_kernel<FP8, EPI>), dim3(static_cast<unsigned>(nb)), dim3(NT), 0, st, a);
  return launch_status(name);
}

int check(const char* name, const void* xq, int64_t ldx, const void* wq, int64_t ldw, const void* out, int64_t ldo,
          int64_t M, int64_t N, int64_t K, int64_t out_cols) {
  RH3_REQUIRE(M >= 0 && N >= 0 && K > 0, "%s: bad sizes M=%lld N=%lld K=%lld", name, (long long)M, (long long)N,
              (long long)K);
  RH3_REQUIRE(K % BK == 0, "%s: K=%lld must be a multiple of %d", name, (long long)K, BK);
  RH3_REQUIRE(N % 8 == 0, "%s: N=%lld must be a multiple of 8", name, (long long)N);
  if (M == 0 || N == 0) return RH3_OK;
  RH3_REQUIRE(xq && wq && out, "%s: null pointer", name);
  RH3_REQUIRE(ldx >= K && ldw >= K && ldx % 16 == 0 && ldw % 16 == 0,
              "%s: operand row strides (%lld, %lld) must be >= K and multiples of 16", name, (long long)ldx,
              (long long)ldw);
  RH3_REQUIRE(ldo >= out_cols && ldo % 4 == 0, "%s: output row stride %lld invalid (need >= %lld, multiple of 4)",
              name, (long long)ldo, (long long)out_cols);
  RH3_REQUIRE(aligned16(xq) && aligned16(wq) && aligned16(out), "%s: operands must be 16-byte aligned", name);
  return RH3_OK;
}

}  // namespace
}  // namespace rh3

using namespace rh3;

extern "C" int rh3_gemm_i8(const int8_t* xq, int64_t ldx, const float* xs, const int8_t* wq, int64_t ldw,
                           const float* ws, const uint16_t* bias, uint16_t* out, int64_t ldo, int64_t M, int64_t N,
                           int64_t K, hipStream_t stream) {
  clear_error();
  if (int e = check("gemm_i8", xq, ldx, wq, ldw, out, ldo, M, N, K, N)) return e;
  RH3_REQUIRE(M == 0 || N == 0 || (xs && ws && aligned16(ws)), "gemm_i8: scales required (ws 16-byte aligned)");
  GemmArgs a{xq, ldx, wq, ldw, xs, ws, bias, nullptr, out, ldo, M, N, K, 0, 0};
  return run<false, EPI_PLAIN>(a, stream, "gemm_i8");
}

extern "C" int rh3_gemm_i8_swiglu(const int8_t* xq, int64_t ldx, const float* xs, const int8_t* wq_perm, int64_t ldw,
                                  const float* ws_perm, uint16_t* out, int64_t ldo, int64_t M, int64_t N, int64_t K,
                                  hipStream_t stream) {
  clear_error();
  if (int e = check("gemm_i8_swiglu", xq, ldx, wq_perm, ldw, out, ldo, M, N, K, N / 2)) return e;
  RH3_REQUIRE(M == 0 || N == 0 || (xs && ws_perm && aligned16(ws_perm)), "gemm_i8_swiglu: scales required");
  GemmArgs a{xq, ldx, wq_perm, ldw, xs, ws_perm, nullptr, nullptr, out, ldo, M, N, K, 0, 0};
  return run<false, EPI_SWIGLU>(a, stream, "gemm_i8_swiglu");
}

extern "C" int rh3_gemm_i8_gated(const int8_t* xq, int64_t ldx, const float* xs, const int8_t* wq, int64_t ldw,
                                 const float* ws, const uint16_t* gate, uint16_t* resid, int64_t ldr, int64_t M,
                                 int64_t N, int64_t K, hipStream_t stream) {
  clear_error();
  if (int e = check("gemm_i8_gated", xq, ldx, wq, ldw, resid, ldr, M, N, K, N)) return e;
  RH3_REQUIRE(M == 0 || N == 0 || (xs && ws && gate && aligned16(ws)), "gemm_i8_gated: scales and gate required");
  GemmArgs a{xq, ldx, wq, ldw, xs, ws, nullptr, gate, resid, ldr, M, N, K, 0, 0};
  return run<false, EPI_GATED>(a, stream, "gemm_i8_gated");
}

extern "C" int rh3_gemm_i8_acc(const int8_t* xq, int64_t ldx, const int8_t* wq, int64_t ldw, int32_t* acc,
                               int64_t ldc, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  clear_error();
  if (int e = check("gemm_i8_acc", xq, ldx, wq, ldw, acc, ldc, M, N, K, N)) return e;
  GemmArgs a{xq, ldx, wq, ldw, nullptr, nullptr, nullptr, nullptr, acc, ldc, M, N, K, 0, 0};
  return run<false, EPI_ACC>(a, stream, "gemm_i8_acc");
}

extern "C" int rh3_gemm_fp8(const uint8_t* xq, int64_t ldx, const float* xs, const uint8_t* wq, int64_t ldw,
                            const float* ws, const uint16_t* bias, uint16_t* out, int64_t ldo, int64_t M, int64_t N,
                            int64_t K, hipStream_t stream) {
  clear_error();
  if (int e = check("gemm_fp8", xq, ldx, wq, ldw, out, ldo, M, N, K, N)) return e;
  RH3_REQUIRE(M == 0 || N == 0 || (xs && ws && aligned16(ws)), "gemm_fp8: scales required (ws 16-byte aligned)");
  GemmArgs a{reinterpret_cast<const int8_t*>(xq), ldx, reinterpret_cast<const int8_t*>(wq), ldw, xs, ws, bias,
             nullptr, out, ldo, M, N, K, 0, 0};
  return run<true, EPI_PLAIN>(a, stream, "gemm_fp8");
}
