// Row-wise W8A8 (int8) and FP8 (OCP e4m3fn) GEMMs on CDNA4 MFMA with fused epilogues.
//
//   acc[m, n] = sum_k xq[m, k] * wq[n, k]        (both operands K-contiguous: the "TN" GEMM)
//   y = (fp32(acc) * xs[m]) * ws[n]               fp8_rowwise.cu:294-304 (EVT order)
//   EPI_PLAIN   out = bf16(y [+ bias[n]])
//   EPI_SWIGLU  g, u = bf16(y) over the swiglu_perm interleave; h = bf16((g * sigmoid(g)) * u) at n / 2
//   EPI_GATED   resid = bf16(fma(bf16(y), gate[n], resid))     (in place)
//   EPI_GATED_ROWS  the same with gate[gidx[m]][n], a gate table row per output row (per-token modulation)
//   EPI_ACC     raw accumulators: int32 (int8 operands) or fp32 (e4m3 operands)
//   EPI_QKV     the qkv projection with the attention pre-pass partly fused (the reference's config 3xx,
//               fp8_rowwise.cu:108-272): the 256x256 tile (two heads of q, k or v, 256 tokens = one statistics
//               chunk) is staged whole in LDS; q: per-head RMSNorm + RoPE and the Q quantization of the
//               attention numerics (per 128-token block, or per token after the H128 rotation), the bf16 q is
//               not written; k: written, plus the float64 channel sums of RMSNorm + RoPE(k); v: written, plus
//               (production numerics) float64 channel sums, max and min
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
#include "attn_layout.hpp"
#include "attn_prologue.hpp"

namespace rh3 {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

enum Epi { EPI_PLAIN = 0, EPI_SWIGLU = 1, EPI_GATED = 2, EPI_ACC = 3, EPI_QKV = 4, EPI_GATED_ROWS = 5 };

constexpr int BM = 256, BN = 256, BK = 64;
// NW waves in a 2 (m) x NW/2 (n) grid, 128 x (512 / NW) outputs per wave. The library builds NW = 8 (GEMM_NW):
// 2 waves per SIMD hide each other's LDS and barrier latency. (One wave per SIMD with 128 x 128 outputs, NW = 4,
// reads a third less LDS per MFMA but measured slower; its branches below are not instantiated.)
constexpr int GEMM_NW = 8;
template <int NW>
struct Cfg {
  static constexpr int NT = NW * 64, WM = 128, WN = BN / (NW / 2), TI = WN / 32, TJ = WM / 32;
  static constexpr int LOADS = 2 * (BM * BK / 16) / NT;  // global->LDS loads per wave per k-step (both operands)
};
constexpr int GROUP_M = 4;
constexpr int TILE_BYTES = BM * BK;  // per operand per stage (BM == BN)

// EPI_QKV operands (pointers into the attention workspace of the chosen numerics)
struct QkvPrep {
  int64_t H, Spad;           // heads, tokens padded to 128
  int mode;                  // 0: one Q scale per (head, 128-token block); 1: per token after the H128 rotation
  int rotate;
  attn::RR rq, rk;           // q / k RMSNorm + RoPE (tab null: none)
  int8_t* q8;                // [H][Spad][128]
  float* qs;                 // mode 0: [H][Spad/128]; mode 1: [H][Spad]
  double* kpart;             // [H][nchunk][128] channel sums of the (RMSNorm + RoPE'd) k
  double* vsum;              // mode 1: [H][nchunk][128]
  float* vmax;
  float* vmin;
};

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
  QkvPrep qp;
  const int32_t* gidx;  // EPI_GATED_ROWS: gate table row of each output row (the gate is [R, ldg] bf16)
  int64_t ldg;
  int* ctr;  // persistent kernel: per-XCD tile counters (8 ints, zero at launch) or null (fixed tile shares)
};

// 16-byte chunk c (0..3) of LDS row r: rows r, r+1 share a 128-byte line; the XOR keeps 16
// consecutive rows of one chunk column on 16 distinct 16-byte bank groups.
__device__ __forceinline__ int swz(int r, int c) {
  return r * BK + ((c ^ (((r >> 1) & 3) ^ ((r >> 3) & 1))) << 4);
}

// g * sigmoid(g) * u with the sigmoid's reciprocal on v_rcp_f32 (1 ulp) instead of the IEEE division
// sequence (~10 instructions): the exp is approximate on both sides already, so the bf16 result moves by at
// most one ulp on a small fraction of elements, the tolerance the SwiGLU epilogue is held to
__device__ __forceinline__ float silu_mul(float g, float u) {
  const float sig = __builtin_amdgcn_rcpf(1.0f + __expf(-g));
  return (g * sig) * u;
}

// EPI_ACC stores the accumulator registers as they are: int32 values (int8) or fp32 bit patterns (e4m3)
__device__ __forceinline__ int acc_bits(int v) { return v; }
__device__ __forceinline__ int acc_bits(float v) { return __builtin_bit_cast(int, v); }

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


template <bool FP8, int EPI, int NW>
__global__ void __launch_bounds__(GEMM_NW * 64, GEMM_NW / 4) gemm_kernel(const GemmArgs a) {
  static_assert(NW == GEMM_NW, "the launch bounds are those of the built wave count");
  using MM = Mma<FP8>;
  using acc_t = typename MM::acc_t;
  constexpr int NT = Cfg<NW>::NT, WM = Cfg<NW>::WM, WN = Cfg<NW>::WN, TI = Cfg<NW>::TI, TJ = Cfg<NW>::TJ;
  // loads per operand per wave per k-step (from GEMM_NW, not NW: an array sized by a template-dependent
  // constant makes clang's host pass drop the kernel's launch stub)
  constexpr int NL = (BM * BK / 16) / (GEMM_NW * 64);
  static_assert(NL == Cfg<NW>::LOADS / 2, "load count");
  // 4-stage ring, each stage its own LDS object {x tile, w tile} (2 x 16 KiB) named statically: the
  // asynchronous global->LDS loads into one stage then provably do not alias the reads of another
  __shared__ __attribute__((aligned(16))) int8_t st0[2 * TILE_BYTES], st1[2 * TILE_BYTES], st2[2 * TILE_BYTES],
      st3[2 * TILE_BYTES];

  // XCD-aware tile order: workgroup id b runs on XCD b % 8; give XCD x the contiguous logical range
  const int nb = a.tiles_m * a.tiles_n;
  const int b = blockIdx.x;
  const int xcd = b % 8, slot = b / 8;
  const int lt = xcd * (nb / 8) + min(xcd, nb % 8) + slot;  // XCD x owns logical tiles [prefix(x), prefix(x+1))
  // grouped order: GROUP_M consecutive M tiles per N column, so the ~32 tiles an XCD runs at once form a
  // GROUP_M x (32 / GROUP_M) block that shares activation and weight panels in that XCD's L2
  const int group = lt / (GROUP_M * a.tiles_n), first_m = group * GROUP_M;
  const int gsz = min(a.tiles_m - first_m, GROUP_M);
  const int tm = first_m + (lt % (GROUP_M * a.tiles_n)) % gsz;
  const int tn = (lt % (GROUP_M * a.tiles_n)) / gsz;
  const int64_t m0 = static_cast<int64_t>(tm) * BM, n0 = static_cast<int64_t>(tn) * BN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / (NW / 2), wn = wave % (NW / 2);
  const int l32 = lane & 31, g = lane >> 5;

  // Global -> LDS loads bypass VGPRs (global_load_lds_dwordx4: lane l of a wave writes LDS base + 16*l),
  // so the XOR swizzle is applied on the global side: stage position p (16-byte units, 1024 per operand)
  // holds row p / 4, logical chunk (p % 4) ^ f(row) (swz is an involution on the chunk index). Wave w
  // fills positions (NL*w + i)*64 + lane, i = 0 .. NL-1, of each operand.
  const int8_t* xp[NL];
  const int8_t* wp[NL];
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const int p = (NL * wave + i) * 64 + lane, r = p >> 2;
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
    for (int i = 0; i < NL; ++i) {
      __builtin_amdgcn_global_load_lds(xp[i] + k0, stg + (NL * wave + i) * 1024, 16, 0, 0);
      __builtin_amdgcn_global_load_lds(wp[i] + k0, stg + TILE_BYTES + (NL * wave + i) * 1024, 16, 0, 0);
    }
  };

  acc_t acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  // s_waitcnt on gfx9: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]; wait_next is vmcnt(2 x
  // the loads of one k-step) expcnt(7) lgkmcnt(0): the loads of the next k-step have landed, the two after
  // it stay in flight. The empty asm statements keep the compiler from moving memory accesses across.
  static_assert(2 * Cfg<NW>::LOADS == (NW == 8 ? 8 : 16), "vmcnt immediates below");
  auto wait_next = [&]() __attribute__((always_inline)) {
    if constexpr (NW == 8) __builtin_amdgcn_s_waitcnt(0x0078);   // vmcnt(8)
    else __builtin_amdgcn_s_waitcnt(0x4070);                     // vmcnt(16)
  };
  auto sync_next = [&]() __attribute__((always_inline)) {
    asm volatile("" ::: "memory");
    wait_next();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  typename MM::frag_t fa0[TI], fb0[TJ], fa1[TI], fb1[TJ];
  auto load_frags = [&](const int8_t* stg, const int ks, typename MM::frag_t* fa, typename MM::frag_t* fb)
      __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < TI; ++i) fa[i] = MM::load(stg + TILE_BYTES, wn * WN + i * 32 + l32, ks, g);
#pragma unroll
    for (int j = 0; j < TJ; ++j) fb[j] = MM::load(stg, wm * WM + j * 32 + l32, ks, g);
  };
  auto mma_all = [&](const typename MM::frag_t* fa, const typename MM::frag_t* fb) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int j = 0; j < TJ; ++j) acc[i][j] = MM::mma(fa[i], fb[j], acc[i][j]);
  };
  // k-step kt, reading stage cur; loads step kt+3 into nxt3 (the stage of step kt-1, whose readers all
  // passed the previous step's barrier). int8 (two k = 32 halves): the fragments of half 0 were read at
  // the end of the previous step; read half 1, run half 0's MFMAs, wait for step kt+1's loads (the 8 most
  // recent loads, steps kt+2 and kt+3, stay in flight) and barrier, then read half 0 of step kt+1 while
  // half 1's MFMAs run, so the LDS latency after the barrier hides behind the MFMA tail.
  auto step = [&](const int kt, const int8_t* cur, const int8_t* nxt1, int8_t* nxt3) __attribute__((always_inline)) {
    gload(kt + 3, nxt3);
    if constexpr (MM::KSUB == 2) {
      load_frags(cur, 1, fa1, fb1);
      mma_all(fa0, fb0);
      sync_next();
      load_frags(nxt1, 0, fa0, fb0);
      mma_all(fa1, fb1);
    } else {
      load_frags(cur, 0, fa1, fb1);
      mma_all(fa1, fb1);
      sync_next();
    }
  };

  gload(0, st0);
  gload(1, st1);
  gload(2, st2);
  wait_next();  // step 0 has landed
  __syncthreads();
  if constexpr (MM::KSUB == 2) load_frags(st0, 0, fa0, fb0);
  int kt = 0;
  for (; kt + 4 <= nk; kt += 4) {
    step(kt + 0, st0, st1, st3);
    step(kt + 1, st1, st2, st0);
    step(kt + 2, st2, st3, st1);
    step(kt + 3, st3, st0, st2);
  }
  const int rem = nk - kt;  // steps left: they read stages 0, 1, 2 in order
  if (rem >= 1) step(kt + 0, st0, st1, st3);
  if (rem >= 2) step(kt + 1, st1, st2, st0);
  if (rem >= 3) step(kt + 2, st2, st3, st1);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no global->LDS load outlives the workgroup

  // epilogue: acc[i][j] register r holds m = m0 + wm*128 + j*32 + l32,
  //           n = n0 + wn*64 + i*32 + 8*(r/4) + 4*g + (r%4)
  if constexpr (EPI == EPI_ACC) {
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      const int64_t m = m0 + wm * WM + j * 32 + l32;
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const int64_t n = n0 + wn * WN + i * 32 + 8 * rq + 4 * g;
          if (m < a.M && n < a.N) {
            int4 v;
            v.x = acc_bits(acc[i][j][4 * rq + 0]);
            v.y = acc_bits(acc[i][j][4 * rq + 1]);
            v.z = acc_bits(acc[i][j][4 * rq + 2]);
            v.w = acc_bits(acc[i][j][4 * rq + 3]);
            *reinterpret_cast<int4*>(static_cast<int32_t*>(a.out) + m * a.ldo + n) = v;
          }
        }
    }
  } else if constexpr (EPI == EPI_QKV) {
    static_assert(NT == 512 && BM == 256 && BN == 256 && 2 * TILE_BYTES == 64 * 512, "tile staging layout");
    // the whole 256 x 256 bf16 tile in the idle ring: row r in stage r / 64 at (r % 64) * 512, 16-byte chunk c
    // (columns 8c..8c+7) at c ^ (r % 32), so 32 rows of one chunk and one row's 32 chunks are both spread
    // over the banks
    __shared__ float qred[64];  // per-group block absmax (mode 0), then the block scales
    auto tp = [&](int r, int c) __attribute__((always_inline)) -> int8_t* {
      const int sidx = r >> 6;
      int8_t* const stg = sidx == 0 ? st0 : sidx == 1 ? st1 : sidx == 2 ? st2 : st3;
      return stg + (r & 63) * 512 + ((c ^ (r & 31)) << 4);
    };
    __syncthreads();  // every wave is done reading the ring
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      const int row = wm * WM + j * 32 + l32;
      const int64_t m = m0 + row;
      const float xsm = m < a.M ? a.xs[m] : 0.0f;
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const int col = wn * WN + i * 32 + 8 * rq + 4 * g;
          const int64_t n = n0 + col;
          const float4 wsn = *reinterpret_cast<const float4*>(a.ws + n);
          float y[4] = {(MM::val(acc[i][j], 4 * rq + 0) * xsm) * wsn.x, (MM::val(acc[i][j], 4 * rq + 1) * xsm) * wsn.y,
                        (MM::val(acc[i][j], 4 * rq + 2) * xsm) * wsn.z, (MM::val(acc[i][j], 4 * rq + 3) * xsm) * wsn.w};
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
          *reinterpret_cast<uint2*>(tp(row, col >> 3) + 8 * g) = o;
        }
    }
    __syncthreads();
    const QkvPrep& qp = a.qp;
    const int64_t hd = qp.H * 128;
    const int role = static_cast<int>(n0 / hd);    // 0 q, 1 k, 2 v (a 256-column tile never straddles two)
    const int64_t hb = (n0 % hd) / 128;            // first of the tile's two heads
    const int grp = tid >> 4, l16 = tid & 15, hh = grp & 1;
    const int64_t nrows = a.M - m0 < 256 ? a.M - m0 : 256;
    const int64_t nchunk = attn_ws::nchunks(a.M);
    // 16-lane row groups: group grp handles head hb + (grp & 1) and rows 16 it + grp / 2, it = 0..15
    auto load_row = [&](int row, float* v) __attribute__((always_inline)) {
      unpack8(*reinterpret_cast<const uint4*>(tp(row, hh * 16 + l16)), v);
    };
    // rows are taken 4 at a time per group, all their loads (tile values, rope-table values) issued before any
    // arithmetic, so the table latency is paid once per 4 rows; the norm weights are loaded once
    constexpr int R = 4;
    const attn::RR& rr = role == 0 ? qp.rq : qp.rk;
    float wn8[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (rr.tab) attn::load8(rr.w + 8 * l16, wn8);
    auto load_batch = [&](int it0, float (*v)[8], float (*tv)[32]) __attribute__((always_inline)) {
#pragma unroll
      for (int u = 0; u < R; ++u) {
        const int row = (it0 + u) * 16 + (grp >> 1);
        const int64_t s = m0 + row;
        load_row(row, v[u]);
        if (rr.tab) attn::rope_tab8(rr, l16, s < a.M ? s : a.M - 1, tv[u]);
      }
    };
    if (role == 0 && qp.mode == 1) {
      for (int it0 = 0; it0 < 16; it0 += R) {
        float v[R][8], tv[R][32];
        load_batch(it0, v, tv);
#pragma unroll
        for (int u = 0; u < R; ++u) {
          const int row = (it0 + u) * 16 + (grp >> 1);
          const int64_t s = m0 + row, h = hb + hh;
          if (s >= qp.Spad) continue;  // uniform per row group
          int8_t* co = qp.q8 + (h * qp.Spad + s) * 128 + 8 * l16;
          if (s >= a.M) {
            *reinterpret_cast<uint2*>(co) = make_uint2(0, 0);
            if (l16 == 0) qp.qs[h * qp.Spad + s] = 0.0f;
            continue;
          }
          if (rr.tab) attn::rms_rope8_pre(v[u], lane, rr, wn8, tv[u]);
          if (qp.rotate) attn::wht128_row(v[u], l16);
          uint2 codes;
          const float sc = attn::token_quant_row(v[u], codes);
          *reinterpret_cast<uint2*>(co) = codes;
          if (l16 == 0) qp.qs[h * qp.Spad + s] = sc;
        }
      }
    } else if (role == 0) {
      // one scale per (head, 128-token block): the RMSNorm + RoPE'd rows (bf16 values) go back into the tile
      // while the block absmax accumulates, then the codes are made from them (rows past M count as 0, as in
      // the pre-pass quantizer)
      float bmax[2] = {0.0f, 0.0f};
      for (int it0 = 0; it0 < 16; it0 += R) {
        float v[R][8], tv[R][32];
        load_batch(it0, v, tv);
#pragma unroll
        for (int u = 0; u < R; ++u) {
          const int row = (it0 + u) * 16 + (grp >> 1);
          if (m0 + row >= a.M) continue;
          if (rr.tab) {
            attn::rms_rope8_pre(v[u], lane, rr, wn8, tv[u]);
            uint4 o;
            o.x = pack_bf2(v[u][0], v[u][1]);
            o.y = pack_bf2(v[u][2], v[u][3]);
            o.z = pack_bf2(v[u][4], v[u][5]);
            o.w = pack_bf2(v[u][6], v[u][7]);
            *reinterpret_cast<uint4*>(tp(row, hh * 16 + l16)) = o;
          }
          float am = 0.0f;
#pragma unroll
          for (int e = 0; e < 8; ++e) am = fmaxf(am, fabsf(v[u][e]));
          bmax[(it0 + u) >> 3] = fmaxf(bmax[(it0 + u) >> 3], am);
        }
      }
#pragma unroll
      for (int b = 0; b < 2; ++b) {
#pragma unroll
        for (int m = 8; m > 0; m >>= 1) bmax[b] = fmaxf(bmax[b], __shfl_xor(bmax[b], m, 64));
      }
      if (l16 == 0) {
        qred[2 * grp] = bmax[0];
        qred[2 * grp + 1] = bmax[1];
      }
      __syncthreads();
      float sc[2], inv[2];
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        float am = 0.0f;
        for (int gg = hh; gg < 32; gg += 2) am = fmaxf(am, qred[2 * gg + b]);
        sc[b] = fmaxf(am, 1e-8f) / 127.0f;
        inv[b] = 1.0f / sc[b];
      }
      if (tid < 4) {  // scale of (head hb + th, block b), reduced over that head's row groups
        const int th = tid & 1, b = tid >> 1;
        float am = 0.0f;
        for (int gg = th; gg < 32; gg += 2) am = fmaxf(am, qred[2 * gg + b]);
        const int64_t blk = m0 / 128 + b;
        if (blk * 128 < qp.Spad) qp.qs[(hb + th) * (qp.Spad / 128) + blk] = fmaxf(am, 1e-8f) / 127.0f;
      }
      for (int it = 0; it < 16; ++it) {
        const int row = it * 16 + (grp >> 1), b = it >> 3;
        const int64_t s = m0 + row, h = hb + hh;
        if (s >= qp.Spad) continue;
        float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if (s < a.M) load_row(row, v);
        uint32_t cb[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float r = fminf(fmaxf(rint_div(v[e], sc[b], inv[b]), -127.0f), 127.0f);
          cb[e] = static_cast<uint32_t>(static_cast<int32_t>(r)) & 0xffu;
        }
        uint2 o;
        o.x = cb[0] | (cb[1] << 8) | (cb[2] << 16) | (cb[3] << 24);
        o.y = cb[4] | (cb[5] << 8) | (cb[6] << 16) | (cb[7] << 24);
        *reinterpret_cast<uint2*>(qp.q8 + (h * qp.Spad + s) * 128 + 8 * l16) = o;
      }
    } else {
      // k / v: the bf16 columns go out as whole 512-byte row segments
      for (int it = 0; it < 16; ++it) {
        const int qi = it * 512 + tid, row = qi >> 5, ch = qi & 31;
        if (row < nrows)
          *reinterpret_cast<uint4*>(static_cast<uint16_t*>(a.out) + (m0 + row) * a.ldo + n0 + ch * 8) =
              *reinterpret_cast<const uint4*>(tp(row, ch));
      }
      const bool vstats = role == 2 && qp.mode == 1;
      if (role == 1 || vstats) {
        // channel statistics of this 256-token chunk: float64 sums of bf16 values are exact, so the partial
        // equals the pre-pass statistics kernel's bit for bit whatever the summation order
        double acc8[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        float mx[8], mn[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) { mx[e] = -INFINITY; mn[e] = INFINITY; }
        const bool rope = role == 1 && rr.tab;
        for (int it0 = 0; it0 < 16; it0 += R) {
          float v[R][8], tv[R][32];
          if (rope) {
            load_batch(it0, v, tv);
          } else {
#pragma unroll
            for (int u = 0; u < R; ++u) load_row((it0 + u) * 16 + (grp >> 1), v[u]);
          }
#pragma unroll
          for (int u = 0; u < R; ++u) {
            const int row = (it0 + u) * 16 + (grp >> 1);
            if (row >= nrows) continue;
            if (rope) attn::rms_rope8_pre(v[u], lane, rr, wn8, tv[u]);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              acc8[e] += static_cast<double>(v[u][e]);
              mx[e] = fmaxf(mx[e], v[u][e]);
              mn[e] = fminf(mn[e], v[u][e]);
            }
          }
        }
        __syncthreads();  // the tile is no longer read: stage 0 / 1 take the per-group partials
        double* red = reinterpret_cast<double*>(st0);     // [32 groups][128 channels]
        float* rmx = reinterpret_cast<float*>(st1);       // [32][128]
        float* rmn = rmx + 32 * 128;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          red[grp * 128 + 8 * l16 + e] = acc8[e];
          rmx[grp * 128 + 8 * l16 + e] = mx[e];
          rmn[grp * 128 + 8 * l16 + e] = mn[e];
        }
        __syncthreads();
        if (tid < 256) {
          const int th = tid >> 7, d = tid & 127;
          double t = 0.0;
          float x = -INFINITY, y = INFINITY;
          for (int gg = th; gg < 32; gg += 2) {
            t += red[gg * 128 + d];
            x = fmaxf(x, rmx[gg * 128 + d]);
            y = fminf(y, rmn[gg * 128 + d]);
          }
          const int64_t o = ((hb + th) * nchunk + m0 / 256) * 128 + d;
          if (role == 1) {
            qp.kpart[o] = t;
          } else {
            qp.vsum[o] = t;
            qp.vmax[o] = x;
            qp.vmin[o] = y;
          }
        }
      }
    }
  } else {
    // bf16(y) (plain: bf16(y + bias)) goes through LDS so that the global side reads and writes whole
    // row segments of WN columns: each wave stages its 128 x WN block (row r at r * PITCH, 16-byte chunk c
    // at c ^ (r % CPR)) in the now idle ring, then lane l handles row RPI*it + l/CPR, columns
    // 8*(l%CPR)..+7.
    constexpr int PITCH = WN * 2, CPR = PITCH / 16, RPI = 64 / CPR;
    __syncthreads();  // every wave is done reading the ring
    constexpr int PER_STAGE = 2 * TILE_BYTES / (WM * PITCH);  // staged wave blocks per ring stage
    const int sidx = wave / PER_STAGE;
    int8_t* const stage = sidx == 0 ? st0 : sidx == 1 ? st1 : sidx == 2 ? st2 : st3;
    int8_t* const ep = stage + (wave % PER_STAGE) * (WM * PITCH);
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      const int row = j * 32 + l32;
      const int64_t m = m0 + wm * WM + row;
      const float xsm = m < a.M ? a.xs[m] : 0.0f;
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const int col = i * 32 + 8 * rq + 4 * g;
          const int64_t n = n0 + wn * WN + col;
          float4 wsn = make_float4(0.f, 0.f, 0.f, 0.f);
          if (n < a.N) wsn = *reinterpret_cast<const float4*>(a.ws + n);
          float y[4] = {(MM::val(acc[i][j], 4 * rq + 0) * xsm) * wsn.x, (MM::val(acc[i][j], 4 * rq + 1) * xsm) * wsn.y,
                        (MM::val(acc[i][j], 4 * rq + 2) * xsm) * wsn.z, (MM::val(acc[i][j], 4 * rq + 3) * xsm) * wsn.w};
          if constexpr (EPI == EPI_PLAIN) {
            if (a.bias && n < a.N) {
              const uint2 bb = *reinterpret_cast<const uint2*>(a.bias + n);
              y[0] = y[0] + __uint_as_float(bb.x << 16);
              y[1] = y[1] + __uint_as_float(bb.x & 0xffff0000u);
              y[2] = y[2] + __uint_as_float(bb.y << 16);
              y[3] = y[3] + __uint_as_float(bb.y & 0xffff0000u);
            }
          }
          uint2 o;
          o.x = pack_bf2(y[0], y[1]);
          o.y = pack_bf2(y[2], y[3]);
          const int ch = col >> 3;  // 16-byte chunk; this lane's 8 bytes are its half g
          *reinterpret_cast<uint2*>(ep + row * PITCH + ((ch ^ (row % CPR)) << 4) + 8 * g) = o;
        }
    }
    // each lane reads back what other lanes of its own wave wrote: LDS executes a wave's accesses in
    // order, and the compiler keeps the reads after the writes (same array)
    const int ch = lane % CPR;
    const int64_t n = n0 + wn * WN + ch * 8;
    const bool nok = n < a.N;
    float gv[8];
    if constexpr (EPI == EPI_GATED) {
      if (nok) unpack8(*reinterpret_cast<const uint4*>(a.gate + n), gv);
    }
    (void)gv;
#pragma unroll 4
    for (int it = 0; it < WM / RPI; ++it) {
      const int row = it * RPI + lane / CPR;
      const int64_t m = m0 + wm * WM + row;
      const uint4 v = *reinterpret_cast<const uint4*>(ep + row * PITCH + ((ch ^ (row % CPR)) << 4));
      if (m >= a.M || !nok) continue;
      if constexpr (EPI == EPI_PLAIN) {
        *reinterpret_cast<uint4*>(static_cast<uint16_t*>(a.out) + m * a.ldo + n) = v;
      } else if constexpr (EPI == EPI_GATED || EPI == EPI_GATED_ROWS) {
        uint16_t* rp = static_cast<uint16_t*>(a.out) + m * a.ldo + n;
        float yv[8], rv[8];
        if constexpr (EPI == EPI_GATED_ROWS)
          unpack8(*reinterpret_cast<const uint4*>(a.gate + static_cast<int64_t>(a.gidx[m]) * a.ldg + n), gv);
        unpack8(v, yv);
        unpack8(*reinterpret_cast<const uint4*>(rp), rv);
        uint4 o;
        o.x = pack_bf2(fmaf(yv[0], gv[0], rv[0]), fmaf(yv[1], gv[1], rv[1]));
        o.y = pack_bf2(fmaf(yv[2], gv[2], rv[2]), fmaf(yv[3], gv[3], rv[3]));
        o.z = pack_bf2(fmaf(yv[4], gv[4], rv[4]), fmaf(yv[5], gv[5], rv[5]));
        o.w = pack_bf2(fmaf(yv[6], gv[6], rv[6]), fmaf(yv[7], gv[7], rv[7]));
        *reinterpret_cast<uint4*>(rp) = o;
      } else {  // EPI_SWIGLU: the 8 columns are one [gate 4j..4j+3 | up 4j..4j+3] group of swiglu_perm
        float yv[8];
        unpack8(v, yv);
        uint2 o;
        o.x = pack_bf2(silu_mul(yv[0], yv[4]), silu_mul(yv[1], yv[5]));
        o.y = pack_bf2(silu_mul(yv[2], yv[6]), silu_mul(yv[3], yv[7]));
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.out) + m * a.ldo + n / 2) = o;
      }
    }
  }
}

// The next tile of a persistent workgroup on XCD xcd, taken from the per-XCD counters: its own XCD's range first,
// then the other XCDs' (so an XCD that runs faster takes over the tiles of a slower one at the end). Range x holds
// tiles [lo_x, hi_x); its first (grid - x + 7) / 8 tiles went out as the workgroups' first tiles, the rest are
// handed out in order by counter x. -1: no tile left.
__device__ __forceinline__ int claim_tile(int* ctr, int xcd, int nb, int grid) {
  // opaque to the compiler, so the range bounds below are computed here, at the claim, and not hoisted out of the
  // caller's tile loop into registers held for the whole kernel
  asm volatile("" : "+s"(nb), "+s"(grid));
#pragma unroll 1
  for (int d = 0; d < 8; ++d) {
    const int x = (xcd + d) & 7;
    const int lo = x * (nb / 8) + min(x, nb % 8);
    const int hi = lo + nb / 8 + (x < nb % 8 ? 1 : 0);
    const int first = lo + (grid - x + 7) / 8;
    if (first >= hi) continue;
    const int c = atomicAdd(ctr + x, 1);
    if (first + c < hi) return first + c;
  }
  return -1;
}

__global__ void zero_ctr_kernel(int* p) {
  if (threadIdx.x < 8) p[threadIdx.x] = 0;
}

// Persistent form of gemm_kernel (every epilogue but EPI_QKV; K a multiple of 4 k-steps, at least 8): one workgroup
// per CU walks a strided share of its XCD's tile range, in the same grouped order. The k-loop runs on
// across tile boundaries: the loads of the next tile's first three k-steps are issued by the current
// tile's last three steps into the ring stages those steps free, so a new tile starts with its operands
// already in LDS. The epilogue no longer owns the ring: it stages one 32 x 32 bf16 block at a time through
// a 2 KiB per-wave LDS area and its global stores drain while the next tile's MFMAs run. The row scales,
// column scales and bias / gate of a tile are loaded into registers at the tile start and parked in LDS
// after its first four k-steps. Same arithmetic as gemm_kernel, element for element.
template <bool FP8, int EPI, bool CLAIM>
__global__ void __launch_bounds__(512, 2) gemm_persistent_kernel(const GemmArgs a) {
  static_assert(EPI != EPI_QKV, "the qkv epilogue stages the whole tile in the ring");
  constexpr int NW = 8;
  using MM = Mma<FP8>;
  using acc_t = typename MM::acc_t;
  constexpr int WM = Cfg<NW>::WM, WN = Cfg<NW>::WN, TI = Cfg<NW>::TI, TJ = Cfg<NW>::TJ;
  constexpr int NL = (BM * BK / 16) / (NW * 64);
  static_assert(NL == 2 && WM == 128 && WN == 64 && TI == 2 && TJ == 4, "layout below");
  __shared__ __attribute__((aligned(16))) int8_t st0[2 * TILE_BYTES], st1[2 * TILE_BYTES], st2[2 * TILE_BYTES],
      st3[2 * TILE_BYTES];
  __shared__ __attribute__((aligned(16))) int8_t ep_lds[NW * 2048];  // per-wave 32 x 32 bf16 staging block
  __shared__ __attribute__((aligned(16))) float rec[3 * BM];         // xs[256], ws[256], bias / gate[256]
  __shared__ int next_tile;

  // XCD-aware share: workgroup b runs on XCD b % 8; XCD x owns the logical tiles [lo, hi) and its nslot
  // workgroups take them round robin, so the ~32 tiles in flight on an XCD are consecutive in the grouped
  // order (shared activation and weight panels in that XCD's L2). With counters (a.ctr), a workgroup's first tile
  // is the same, and each later one is taken from the counters one tile ahead (claim_tile): the XCDs run at
  // different clocks, and fixed shares leave the fast ones idle while the slowest finishes (3-5 % of a launch)
  const int nb = a.tiles_m * a.tiles_n;
  const int b = blockIdx.x, xcd = b % 8, slot = b / 8;
  const int nslot = (static_cast<int>(gridDim.x) - xcd + 7) / 8;
  const int lo = xcd * (nb / 8) + min(xcd, nb % 8);
  const int hi = lo + nb / 8 + (xcd < nb % 8 ? 1 : 0);
  int lt = lo + slot;
  if (lt >= hi) return;  // whole workgroup: no tile here
  auto tile_origin = [&](int t, int64_t& m0, int64_t& n0) __attribute__((always_inline)) {
    const int group = t / (GROUP_M * a.tiles_n), first_m = group * GROUP_M;
    const int gsz = min(a.tiles_m - first_m, GROUP_M);
    const int r = t % (GROUP_M * a.tiles_n);
    m0 = static_cast<int64_t>(first_m + r % gsz) * BM;
    n0 = static_cast<int64_t>(r / gsz) * BN;
  };

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / (NW / 2), wn = wave % (NW / 2);
  const int l32 = lane & 31, g = lane >> 5;

  // global -> LDS copy geometry as in gemm_kernel (swizzle applied on the global side), held as a tile base
  // (uniform, so in scalar registers) plus a 32-bit byte offset per lane (row r clamped to the last valid row,
  // 16-byte chunk c): half the vector registers of 64-bit lane pointers, which the epilogues need (the host
  // keeps 255 * ld + 64 below 2^32)
  const int8_t* xb = a.x;
  const int8_t* wb = a.w;
  uint32_t xo[NL], wo[NL];
  auto tile_ptrs = [&](int64_t m0, int64_t n0) __attribute__((always_inline)) {
    xb = a.x + m0 * a.ldx;
    wb = a.w + n0 * a.ldw;
    const int rmx = static_cast<int>(min<int64_t>(BM - 1, a.M - 1 - m0));
    const int rmw = static_cast<int>(min<int64_t>(BN - 1, a.N - 1 - n0));
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int p = (NL * wave + i) * 64 + lane, r = p >> 2;
      const int c = (p & 3) ^ (((r >> 1) & 3) ^ ((r >> 3) & 1));
      xo[i] = static_cast<uint32_t>(min(r, rmx)) * static_cast<uint32_t>(a.ldx) + c * 16;
      wo[i] = static_cast<uint32_t>(min(r, rmw)) * static_cast<uint32_t>(a.ldw) + c * 16;
    }
  };
  const int nk = static_cast<int>(a.K / BK);
  // the saddr form: the tile base + k0 in scalar registers, the lane offsets fixed (no vector address arithmetic)
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  auto gload = [&](int kt, int8_t* stg) __attribute__((always_inline)) {
    const int64_t k0 = static_cast<int64_t>(kt) * BK;
    const uint32_t dst = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(stg)) + NL * wv * 1024;
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      lds_dma16_s(xb + k0, xo[i], dst + i * 1024);
      lds_dma16_s(wb + k0, wo[i], dst + TILE_BYTES + i * 1024);
    }
  };

  acc_t acc[TI][TJ];
  auto zero_acc = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int j = 0; j < TJ; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
  };
  // vmcnt(8): the loads of the next k-step have landed, the two k-steps after it stay in flight (loads
  // or stores issued in between only make the wait stronger)
  auto sync_next = [&]() __attribute__((always_inline)) {
    // int8: every MFMA of the half step is issued before the barrier (left alone, the scheduler moved the last
    // ones past it, so a wave waiting there had no MFMA queued; about 0.5-1 % on the C2 shapes); fp8 is faster
    // with the scheduler's order
    if constexpr (MM::KSUB == 2) __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0x0078);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  typename MM::frag_t fa0[TI], fb0[TJ], fa1[TI], fb1[TJ];
  auto load_frags = [&](const int8_t* stg, const int ks, typename MM::frag_t* fa, typename MM::frag_t* fb)
      __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < TI; ++i) fa[i] = MM::load(stg + TILE_BYTES, wn * WN + i * 32 + l32, ks, g);
#pragma unroll
    for (int j = 0; j < TJ; ++j) fb[j] = MM::load(stg, wm * WM + j * 32 + l32, ks, g);
  };
  auto mma_all = [&](const typename MM::frag_t* fa, const typename MM::frag_t* fb) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int j = 0; j < TJ; ++j) acc[i][j] = MM::mma(fa[i], fb[j], acc[i][j]);
  };
  // one k-step reading stage cur, after first loading k-step kload of the current pointers into nxt3 (the
  // stage of the previous k-step, whose readers all passed the previous barrier); as in gemm_kernel
  // issue order of a half step (int8): one MFMA, then each of the 6 fragment reads of the other half followed
  // by an MFMA, then the last one, so that the reads go out under the MFMAs instead of after them
  auto interleave = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);    // 0x008: MFMA
#pragma unroll
    for (int i = 0; i < TI + TJ; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 0x100: LDS read
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, TI * TJ - TI - TJ - 1, 0);
  };
  auto step = [&](const int kload, const int8_t* cur, const int8_t* nxt1, int8_t* nxt3) __attribute__((always_inline)) {
    gload(kload, nxt3);
    if constexpr (MM::KSUB == 2) {
      load_frags(cur, 1, fa1, fb1);
      mma_all(fa0, fb0);
      interleave();
      sync_next();
      load_frags(nxt1, 0, fa0, fb0);
      mma_all(fa1, fb1);
      interleave();
    } else {
      load_frags(cur, 0, fa1, fb1);
      mma_all(fa1, fb1);
      sync_next();
    }
  };

  int64_t m0, n0;
  tile_origin(lt, m0, n0);
  tile_ptrs(m0, n0);
  zero_acc();
  gload(0, st0);
  gload(1, st1);
  gload(2, st2);
  __builtin_amdgcn_s_waitcnt(0x0078);  // k-step 0 has landed
  __syncthreads();
  if constexpr (MM::KSUB == 2) load_frags(st0, 0, fa0, fb0);

  constexpr bool HAS_BG = EPI == EPI_PLAIN || EPI == EPI_GATED;
  const uint16_t* bg = EPI == EPI_GATED ? a.gate : a.bias;
  while (true) {
    // this tile's scales (and bias / gate) into registers now, into LDS before the last k-step
    float rv0 = 0.0f, rv1 = 0.0f;
    if constexpr (EPI != EPI_ACC) {
      if (tid < BM) {
        const int64_t m = m0 + tid;
        if (m < a.M) rv0 = a.xs[m];
      } else {
        const int64_t n = n0 + (tid - BM);
        if (n < a.N) {
          rv0 = a.ws[n];
          if (HAS_BG && bg) rv1 = bf2f(bg[n]);
        }
      }
    }
    // the next tile: claimed by thread 0 now, read by every thread past the barrier of the first k-step
    if (CLAIM && tid == 0) next_tile = claim_tile(a.ctr, xcd, nb, static_cast<int>(gridDim.x));

    // k-steps 0..3, then the record goes to LDS: every wave has finished the previous tile's epilogue (it
    // passed this tile's barriers since), and the barriers of the k-steps left publish it to this tile's
    step(3, st0, st1, st3);
    const int ltn = CLAIM ? __builtin_amdgcn_readfirstlane(next_tile) : lt + nslot;
    const bool more = CLAIM ? ltn >= 0 : ltn < hi;
    int64_t m0n = m0, n0n = n0;
    if (more) tile_origin(ltn, m0n, n0n);
    step(4, st1, st2, st0);
    step(5, st2, st3, st1);
    step(6, st3, st0, st2);
    if constexpr (EPI != EPI_ACC) {
      rec[tid] = rv0;
      if (tid >= BM) rec[BM + tid] = rv1;
    }
    for (int kt = 4; kt + 4 < nk; kt += 4) {
      step(kt + 3, st0, st1, st3);
      step(kt + 4, st1, st2, st0);
      step(kt + 5, st2, st3, st1);
      step(kt + 6, st3, st0, st2);
    }
    // the last four k-steps; the three after them are the next tile's k-steps 0..2 (with no next tile:
    // the current tile's last k-step again, into stages nobody reads)
    step(nk - 1, st0, st1, st3);
    if (more) tile_ptrs(m0n, n0n);
    const int k0n = more ? 0 : nk - 1, k1n = more ? 1 : nk - 1, k2n = more ? 2 : nk - 1;
    step(k0n, st1, st2, st0);
    step(k1n, st2, st3, st1);
    step(k2n, st3, st0, st2);

    // epilogue: acc[i][j] register r holds m = m0 + wm*128 + j*32 + l32,
    //           n = n0 + wn*64 + i*32 + 8*(r/4) + 4*g + (r%4)
    if constexpr (EPI == EPI_ACC) {
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        const int64_t m = m0 + wm * WM + j * 32 + l32;
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
          for (int rq = 0; rq < 4; ++rq) {
            const int64_t n = n0 + wn * WN + i * 32 + 8 * rq + 4 * g;
            if (m < a.M && n < a.N) {
              int4 v;
              v.x = acc_bits(acc[i][j][4 * rq + 0]);
              v.y = acc_bits(acc[i][j][4 * rq + 1]);
              v.z = acc_bits(acc[i][j][4 * rq + 2]);
              v.w = acc_bits(acc[i][j][4 * rq + 3]);
              *reinterpret_cast<int4*>(static_cast<int32_t*>(a.out) + m * a.ldo + n) = v;
            }
          }
      }
    } else {
      // block (j, i) = rows j*32.., columns i*32.. of the wave's 128 x 64: bf16(y) (plain: bf16(y + bias))
      // staged with row r at r * 64 B, 16-byte chunk c at c ^ ((r >> 2) & 3), then lane l handles row
      // 16*it + l/4, columns 8*(l%4)..+7, so global accesses are 64-byte row segments
      int8_t* const ep = ep_lds + wave * 2048;
      const float* xs_s = rec;
      const float* ws_s = rec + BM;
      const float* bg_s = rec + 2 * BM;
      const int chr = lane & 3;
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        const int row = j * 32 + l32;
        const float xsm = xs_s[wm * WM + row];
        // the residual segments of this row block (gated): issued before the staging so their latency
        // runs under it
        uint4 rres[TI][2];
        if constexpr (EPI == EPI_GATED || EPI == EPI_GATED_ROWS) {
#pragma unroll
          for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int it = 0; it < 2; ++it) {
              const int64_t m = m0 + wm * WM + j * 32 + it * 16 + (lane >> 2);
              const int64_t n = n0 + wn * WN + i * 32 + chr * 8;
              rres[i][it] = (m < a.M && n < a.N)
                                ? *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.out) + m * a.ldo + n)
                                : make_uint4(0, 0, 0, 0);
            }
        }
#pragma unroll
        for (int i = 0; i < TI; ++i) {
#pragma unroll
          for (int rq = 0; rq < 4; ++rq) {
            const int col = wn * WN + i * 32 + 8 * rq + 4 * g;  // tile column of acc register 4*rq
            const float4 wsn = *reinterpret_cast<const float4*>(ws_s + col);
            float y[4] = {(MM::val(acc[i][j], 4 * rq + 0) * xsm) * wsn.x, (MM::val(acc[i][j], 4 * rq + 1) * xsm) * wsn.y,
                          (MM::val(acc[i][j], 4 * rq + 2) * xsm) * wsn.z, (MM::val(acc[i][j], 4 * rq + 3) * xsm) * wsn.w};
            if constexpr (EPI == EPI_PLAIN) {
              if (a.bias) {
                const float4 bb = *reinterpret_cast<const float4*>(bg_s + col);
                y[0] = y[0] + bb.x;
                y[1] = y[1] + bb.y;
                y[2] = y[2] + bb.z;
                y[3] = y[3] + bb.w;
              }
            }
            uint2 o;
            o.x = pack_bf2(y[0], y[1]);
            o.y = pack_bf2(y[2], y[3]);
            *reinterpret_cast<uint2*>(ep + l32 * 64 + ((rq ^ ((l32 >> 2) & 3)) << 4) + 8 * g) = o;
          }
          // each lane reads back what other lanes of its own wave wrote: LDS executes a wave's accesses
          // in order, and the compiler keeps the reads after the writes (same array)
#pragma unroll
          for (int it = 0; it < 2; ++it) {
            const int r = it * 16 + (lane >> 2);
            const uint4 v = *reinterpret_cast<const uint4*>(ep + r * 64 + ((chr ^ ((r >> 2) & 3)) << 4));
            const int64_t m = m0 + wm * WM + j * 32 + r;
            const int64_t n = n0 + wn * WN + i * 32 + chr * 8;
            if (m < a.M && n < a.N) {
              if constexpr (EPI == EPI_PLAIN) {
                *reinterpret_cast<uint4*>(static_cast<uint16_t*>(a.out) + m * a.ldo + n) = v;
              } else if constexpr (EPI == EPI_GATED || EPI == EPI_GATED_ROWS) {
                float4 g0, g1;
                if constexpr (EPI == EPI_GATED) {
                  g0 = *reinterpret_cast<const float4*>(bg_s + (n - n0));
                  g1 = *reinterpret_cast<const float4*>(bg_s + (n - n0) + 4);
                } else {  // this row's gate row, from global memory (per-token modulation)
                  float gv[8];
                  unpack8(*reinterpret_cast<const uint4*>(a.gate + static_cast<int64_t>(a.gidx[m]) * a.ldg + n), gv);
                  g0 = make_float4(gv[0], gv[1], gv[2], gv[3]);
                  g1 = make_float4(gv[4], gv[5], gv[6], gv[7]);
                }
                float yv[8], rv[8];
                unpack8(v, yv);
                unpack8(rres[i][it], rv);
                uint4 o;
                o.x = pack_bf2(fmaf(yv[0], g0.x, rv[0]), fmaf(yv[1], g0.y, rv[1]));
                o.y = pack_bf2(fmaf(yv[2], g0.z, rv[2]), fmaf(yv[3], g0.w, rv[3]));
                o.z = pack_bf2(fmaf(yv[4], g1.x, rv[4]), fmaf(yv[5], g1.y, rv[5]));
                o.w = pack_bf2(fmaf(yv[6], g1.z, rv[6]), fmaf(yv[7], g1.w, rv[7]));
                *reinterpret_cast<uint4*>(static_cast<uint16_t*>(a.out) + m * a.ldo + n) = o;
              } else {  // EPI_SWIGLU: the 8 columns are one [gate 4j..4j+3 | up 4j..4j+3] group of swiglu_perm
                float yv[8];
                unpack8(v, yv);
                uint2 o;
                o.x = pack_bf2(silu_mul(yv[0], yv[4]), silu_mul(yv[1], yv[5]));
                o.y = pack_bf2(silu_mul(yv[2], yv[6]), silu_mul(yv[3], yv[7]));
                *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.out) + m * a.ldo + n / 2) = o;
              }
            }
          }
        }
      }
    }
    if (!more) break;
    lt = ltn;
    m0 = m0n;
    n0 = n0n;
    zero_acc();
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no global->LDS load outlives the workgroup
}

template <bool FP8, int EPI>
int run(GemmArgs a, hipStream_t st, const char* name) {
  if (a.M == 0 || a.N == 0) return RH3_OK;
  a.tiles_m = static_cast<int>((a.M + BM - 1) / BM);
  a.tiles_n = static_cast<int>((a.N + BN - 1) / BN);
  const int64_t nb = static_cast<int64_t>(a.tiles_m) * a.tiles_n;
  RH3_REQUIRE(nb < (1ll << 31), "%s: too many tiles", name);
  if constexpr (EPI != EPI_QKV) {
    const int64_t nk = a.K / BK;
    const int cus = device_cus();
    // the persistent kernel's 32-bit lane offsets reach 255 rows of either operand
    const bool off32 = 255 * a.ldx + 64 < (1ll << 32) && 255 * a.ldw + 64 < (1ll << 32);
    if (nk % 4 == 0 && nk >= 8 && cus > 0 && off32) {
      const int64_t grid = nb < cus ? nb : cus;  // one workgroup per CU (the LDS use admits no second)
      // the counters are cleared by a fill kernel (no hipMemsetAsync: the call stays graph-safe)
      const dim3 g(static_cast<unsigned>(grid));
      if (a.ctr != nullptr) {
        hipLaunchKernelGGL(zero_ctr_kernel, dim3(1), dim3(64), 0, st, a.ctr);
        hipLaunchKernelGGL((gemm_persistent_kernel<FP8, EPI, true>), g, dim3(512), 0, st, a);
      } else {
        hipLaunchKernelGGL((gemm_persistent_kernel<FP8, EPI, false>), g, dim3(512), 0, st, a);
      }
      return launch_status(name);
    }
  }
  hipLaunchKernelGGL((gemm_kernel<FP8, EPI, GEMM_NW>), dim3(static_cast<unsigned>(nb)), dim3(GEMM_NW * 64), 0,
                     st, a);
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
  RH3_REQUIRE(ldo >= out_cols && ldo % 8 == 0, "%s: output row stride %lld invalid (need >= %lld, multiple of 8)",
              name, (long long)ldo, (long long)out_cols);
  RH3_REQUIRE(aligned16(xq) && aligned16(wq) && aligned16(out), "%s: operands must be 16-byte aligned", name);
  return RH3_OK;
}

}  // namespace
}  // namespace rh3

using namespace rh3;

extern "C" int rh3_gemm_i8(const int8_t* xq, int64_t ldx, const float* xs, const int8_t* wq, int64_t ldw,
                           const float* ws, const uint16_t* bias, uint16_t* out, int64_t ldo, int64_t M, int64_t N,
                           int64_t K, int32_t* ctr, hipStream_t stream) {
  clear_error();
  if (int e = check("gemm_i8", xq, ldx, wq, ldw, out, ldo, M, N, K, N)) return e;
  RH3_REQUIRE(M == 0 || N == 0 || (xs && ws && aligned16(ws)), "gemm_i8: scales required (ws 16-byte aligned)");
  GemmArgs a{xq, ldx, wq, ldw, xs, ws, bias, nullptr, out, ldo, M, N, K, 0, 0};
  RH3_REQUIRE((reinterpret_cast<uintptr_t>(ctr) & 3) == 0, "%s: ctr must be 4-byte aligned", "gemm_i8");
  a.ctr = reinterpret_cast<int*>(ctr);
  return run<false, EPI_PLAIN>(a, stream, "gemm_i8");
}

extern "C" int rh3_gemm_i8_swiglu(const int8_t* xq, int64_t ldx, const float* xs, const int8_t* wq_perm, int64_t ldw,
                                  const float* ws_perm, uint16_t* out, int64_t ldo, int64_t M, int64_t N, int64_t K,
                                  int32_t* ctr, hipStream_t stream) {
  clear_error();
  if (int e = check("gemm_i8_swiglu", xq, ldx, wq_perm, ldw, out, ldo, M, N, K, N / 2)) return e;
  RH3_REQUIRE(M == 0 || N == 0 || (xs && ws_perm && aligned16(ws_perm)), "gemm_i8_swiglu: scales required");
  GemmArgs a{xq, ldx, wq_perm, ldw, xs, ws_perm, nullptr, nullptr, out, ldo, M, N, K, 0, 0};
  RH3_REQUIRE((reinterpret_cast<uintptr_t>(ctr) & 3) == 0, "%s: ctr must be 4-byte aligned", "gemm_i8_swiglu");
  a.ctr = reinterpret_cast<int*>(ctr);
  return run<false, EPI_SWIGLU>(a, stream, "gemm_i8_swiglu");
}

extern "C" int rh3_gemm_i8_gated_rows(const int8_t* xq, int64_t ldx, const float* xs, const int8_t* wq, int64_t ldw,
                                      const float* ws, const uint16_t* gate, int64_t ldg, const int32_t* gidx,
                                      uint16_t* resid, int64_t ldr, int64_t M, int64_t N, int64_t K,
                                      int32_t* ctr, hipStream_t stream) {
  clear_error();
  if (int e = check("gemm_i8_gated_rows", xq, ldx, wq, ldw, resid, ldr, M, N, K, N)) return e;
  RH3_REQUIRE(M == 0 || N == 0 || (xs && ws && gate && gidx && aligned16(ws) && aligned16(gate)),
              "gemm_i8_gated_rows: scales, gate table and row indices required (ws, gate 16-byte aligned)");
  RH3_REQUIRE(ldg >= N && ldg % 8 == 0, "gemm_i8_gated_rows: gate row stride %lld invalid (need >= N, multiple of 8)",
              (long long)ldg);
  GemmArgs a{xq, ldx, wq, ldw, xs, ws, nullptr, gate, resid, ldr, M, N, K, 0, 0};
  a.gidx = gidx;
  a.ldg = ldg;
  RH3_REQUIRE((reinterpret_cast<uintptr_t>(ctr) & 3) == 0, "%s: ctr must be 4-byte aligned", "gemm_i8_gated_rows");
  a.ctr = reinterpret_cast<int*>(ctr);
  return run<false, EPI_GATED_ROWS>(a, stream, "gemm_i8_gated_rows");
}

extern "C" int rh3_gemm_i8_gated(const int8_t* xq, int64_t ldx, const float* xs, const int8_t* wq, int64_t ldw,
                                 const float* ws, const uint16_t* gate, uint16_t* resid, int64_t ldr, int64_t M,
                                 int64_t N, int64_t K, int32_t* ctr, hipStream_t stream) {
  clear_error();
  if (int e = check("gemm_i8_gated", xq, ldx, wq, ldw, resid, ldr, M, N, K, N)) return e;
  RH3_REQUIRE(M == 0 || N == 0 || (xs && ws && gate && aligned16(ws)), "gemm_i8_gated: scales and gate required");
  GemmArgs a{xq, ldx, wq, ldw, xs, ws, nullptr, gate, resid, ldr, M, N, K, 0, 0};
  RH3_REQUIRE((reinterpret_cast<uintptr_t>(ctr) & 3) == 0, "%s: ctr must be 4-byte aligned", "gemm_i8_gated");
  a.ctr = reinterpret_cast<int*>(ctr);
  return run<false, EPI_GATED>(a, stream, "gemm_i8_gated");
}

extern "C" int rh3_gemm_i8_acc(const int8_t* xq, int64_t ldx, const int8_t* wq, int64_t ldw, int32_t* acc,
                               int64_t ldc, int64_t M, int64_t N, int64_t K, int32_t* ctr, hipStream_t stream) {
  clear_error();
  if (int e = check("gemm_i8_acc", xq, ldx, wq, ldw, acc, ldc, M, N, K, N)) return e;
  GemmArgs a{xq, ldx, wq, ldw, nullptr, nullptr, nullptr, nullptr, acc, ldc, M, N, K, 0, 0};
  RH3_REQUIRE((reinterpret_cast<uintptr_t>(ctr) & 3) == 0, "%s: ctr must be 4-byte aligned", "gemm_i8_acc");
  a.ctr = reinterpret_cast<int*>(ctr);
  return run<false, EPI_ACC>(a, stream, "gemm_i8_acc");
}

extern "C" int rh3_gemm_i8_qkv(const int8_t* xq, int64_t ldx, const float* xs, const int8_t* wq, int64_t ldw,
                               const float* ws, const uint16_t* bias, uint16_t* out, int64_t ldo, int64_t M, int64_t H,
                               int64_t K, const uint16_t* tab, int rot, const uint16_t* qw, const uint16_t* kw,
                               float eps, int numerics, int rotate, void* workspace, int64_t workspace_bytes,
                               hipStream_t stream) {
  clear_error();
  RH3_REQUIRE(H > 0 && H % 2 == 0 && H < 65536, "gemm_i8_qkv: H=%lld must be even (two heads per 256-column tile)",
              (long long)H);
  RH3_REQUIRE(numerics == 0 || numerics == 1, "gemm_i8_qkv: numerics %d (0 per-block, 1 production)", numerics);
  RH3_REQUIRE(M > 0, "gemm_i8_qkv: M must be positive");
  const int64_t N = 3 * H * 128;
  if (int e = check("gemm_i8_qkv", xq, ldx, wq, ldw, out, ldo, M, N, K, N)) return e;
  RH3_REQUIRE(xs && ws && aligned16(ws), "gemm_i8_qkv: scales required (ws 16-byte aligned)");
  RH3_REQUIRE(!bias || aligned16(bias), "gemm_i8_qkv: bias must be 16-byte aligned");
  QkvPrep qp{};
  qp.H = H;
  qp.Spad = attn_ws::pad(M);
  qp.mode = numerics;
  qp.rotate = rotate;
  if (tab) {
    RH3_REQUIRE(qw && kw && (rot == 96 || rot == 128) && aligned16(tab) && aligned16(qw) && aligned16(kw),
                "gemm_i8_qkv: tab, qw, kw (16-byte aligned) and rot_dim 96 or 128 required");
    qp.rq = attn::RR{tab, qw, eps, rot};
    qp.rk = attn::RR{tab, kw, eps, rot};
  } else {
    qp.rq = attn::RR{nullptr, nullptr, 0.f, 0};
    qp.rk = qp.rq;
  }
  int64_t need = 0;
  if (numerics == 0) {
    const attn_ws::Work w = attn_ws::layout(workspace, M, M, H);
    need = w.bytes;
    qp.q8 = w.q8; qp.qs = w.qs; qp.kpart = w.part;
  } else {
    const attn_ws::WorkU8 w = attn_ws::layout_u8(workspace, M, M, H);
    need = w.bytes;
    qp.q8 = w.q8; qp.qs = w.qs; qp.kpart = w.kpart; qp.vsum = w.vsum; qp.vmax = w.vmax; qp.vmin = w.vmin;
  }
  RH3_REQUIRE(workspace && aligned16(workspace) && workspace_bytes >= need,
              "gemm_i8_qkv: workspace %lld bytes < required %lld", (long long)workspace_bytes, (long long)need);
  GemmArgs a{xq, ldx, wq, ldw, xs, ws, bias, nullptr, out, ldo, M, N, K, 0, 0, qp};
  return run<false, EPI_QKV>(a, stream, "gemm_i8_qkv");
}

extern "C" int rh3_gemm_fp8(const uint8_t* xq, int64_t ldx, const float* xs, const uint8_t* wq, int64_t ldw,
                            const float* ws, const uint16_t* bias, uint16_t* out, int64_t ldo, int64_t M, int64_t N,
                            int64_t K, int32_t* ctr, hipStream_t stream) {
  clear_error();
  if (int e = check("gemm_fp8", xq, ldx, wq, ldw, out, ldo, M, N, K, N)) return e;
  RH3_REQUIRE(M == 0 || N == 0 || (xs && ws && aligned16(ws)), "gemm_fp8: scales required (ws 16-byte aligned)");
  GemmArgs a{reinterpret_cast<const int8_t*>(xq), ldx, reinterpret_cast<const int8_t*>(wq), ldw, xs, ws, bias,
             nullptr, out, ldo, M, N, K, 0, 0};
  RH3_REQUIRE((reinterpret_cast<uintptr_t>(ctr) & 3) == 0, "%s: ctr must be 4-byte aligned", "gemm_fp8");
  a.ctr = reinterpret_cast<int*>(ctr);
  return run<true, EPI_PLAIN>(a, stream, "gemm_fp8");
}

extern "C" int rh3_gemm_fp8_acc(const uint8_t* xq, int64_t ldx, const uint8_t* wq, int64_t ldw, float* acc,
                                int64_t ldc, int64_t M, int64_t N, int64_t K, int32_t* ctr, hipStream_t stream) {
  clear_error();
  if (int e = check("gemm_fp8_acc", xq, ldx, wq, ldw, acc, ldc, M, N, K, N)) return e;
  GemmArgs a{reinterpret_cast<const int8_t*>(xq), ldx, reinterpret_cast<const int8_t*>(wq), ldw, nullptr, nullptr,
             nullptr, nullptr, acc, ldc, M, N, K, 0, 0};
  RH3_REQUIRE((reinterpret_cast<uintptr_t>(ctr) & 3) == 0, "%s: ctr must be 4-byte aligned", "gemm_fp8_acc");
  a.ctr = reinterpret_cast<int*>(ctr);
  return run<true, EPI_ACC>(a, stream, "gemm_fp8_acc");
}
