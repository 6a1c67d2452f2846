// Workspace layouts of the two attention numerics, shared by the attention pre-pass / main kernels and by the
// qkv GEMM whose epilogue writes the Q operands and the K / V statistics straight into the workspace.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace rh3 {
namespace attn_ws {

constexpr int D = 128;
constexpr int BLK = 128;    // token padding, quantization block, production key tile
constexpr int CHUNK = 256;  // statistics chunk (tokens)
constexpr int SIDE = 2048;  // production side record bytes per (head, 128-key tile)

__host__ __device__ inline int64_t pad(int64_t s) { return (s + BLK - 1) / BLK * BLK; }
__host__ __device__ inline int64_t up256(int64_t b) { return (b + 255) / 256 * 256; }
__host__ __device__ inline int64_t nchunks(int64_t s) { return (s + CHUNK - 1) / CHUNK; }

// per-128-block recipe (bf16 P.V)
constexpr int FWD_BQ = 384;     // queries per main-kernel workgroup
constexpr int TAIL_MAX = 128;   // most (head, query block) workgroups whose keys the main kernel splits in two
constexpr int TAIL_ROW = D + 4; // floats per query of a split partial: O[128], running max, row sum, 2 unused

// (head, query block) workgroups of the main kernel
__host__ __device__ inline int64_t fwd_blocks(int64_t Sq, int64_t H) { return (Sq + FWD_BQ - 1) / FWD_BQ * H; }

struct Work {
  int8_t* q8; float* qs; int8_t* k8; float* ks; float* kmean; double* part; uint16_t* vt;
  float* kn;    // [H][Skpad/128]: per 128-key block, an upper bound of the largest L2 norm of a key's int8 codes
  float* tail;  // [2][npair][FWD_BQ][TAIL_ROW] partials of the split last round; null when not reserved
  int* ctr;     // the main kernel's work counter (cleared before each launch)
  int64_t bytes;
};

// split false: no room for the split-last-round partials (the main kernel then runs every workgroup whole)
inline Work layout(void* base, int64_t Sq, int64_t Sk, int64_t H, bool split = true) {
  const int64_t sqp = pad(Sq), skp = pad(Sk), nchunk = nchunks(Sk);
  char* p = static_cast<char*>(base);
  int64_t off = 0;
  Work w{};
  auto take = [&](int64_t n) { char* r = p ? p + off : nullptr; off += up256(n); return r; };
  w.q8 = reinterpret_cast<int8_t*>(take(H * sqp * D));
  w.qs = reinterpret_cast<float*>(take(H * (sqp / BLK) * 4));
  w.k8 = reinterpret_cast<int8_t*>(take(H * skp * D));
  w.ks = reinterpret_cast<float*>(take(H * (skp / BLK) * 4));
  w.kmean = reinterpret_cast<float*>(take(H * D * 4));
  w.part = reinterpret_cast<double*>(take(H * nchunk * D * 8));
  w.vt = reinterpret_cast<uint16_t*>(take(H * D * skp * 2));
  w.kn = reinterpret_cast<float*>(take(H * (skp / BLK) * 4));
  // only a grid larger than TAIL_MAX workgroups can leave a last round worth splitting
  const int64_t nwg = fwd_blocks(Sq, H);
  w.tail = split && nwg > TAIL_MAX ? reinterpret_cast<float*>(take(int64_t{2} * TAIL_MAX * FWD_BQ * TAIL_ROW * 4))
                                   : nullptr;
  w.ctr = reinterpret_cast<int*>(take(256));
  w.bytes = off;
  return w;
}

// production numerics (u8 P, int8 V)
struct WorkU8 {
  int8_t* q8; float* qs; int8_t* k8; float* ks; int8_t* side; int8_t* vt;
  float* kmean; float* vmean; float* vscale;
  double* kpart; double* vsum; float* vmax; float* vmin;
  int* ctr;  // the main kernel's work counter (cleared before each launch)
  int64_t bytes;
};

inline WorkU8 layout_u8(void* base, int64_t Sq, int64_t Sk, int64_t H) {
  const int64_t sqp = pad(Sq), skp = pad(Sk), nchunk = nchunks(Sk);
  char* p = static_cast<char*>(base);
  int64_t off = 0;
  WorkU8 w{};
  auto take = [&](int64_t n) { char* r = p ? p + off : nullptr; off += up256(n); return r; };
  w.q8 = reinterpret_cast<int8_t*>(take(H * sqp * D));
  w.qs = reinterpret_cast<float*>(take(H * sqp * 4));
  w.k8 = reinterpret_cast<int8_t*>(take(H * skp * D));
  w.ks = reinterpret_cast<float*>(take(H * skp * 4));
  w.side = reinterpret_cast<int8_t*>(take(H * (skp / BLK) * SIDE));
  w.vt = reinterpret_cast<int8_t*>(take(H * D * skp));
  w.kmean = reinterpret_cast<float*>(take(H * D * 4));
  w.vmean = reinterpret_cast<float*>(take(H * D * 4));
  w.vscale = reinterpret_cast<float*>(take(H * D * 4));
  w.kpart = reinterpret_cast<double*>(take(H * nchunk * D * 8));
  w.vsum = reinterpret_cast<double*>(take(H * nchunk * D * 8));
  w.vmax = reinterpret_cast<float*>(take(H * nchunk * D * 4));
  w.vmin = reinterpret_cast<float*>(take(H * nchunk * D * 4));
  w.ctr = reinterpret_cast<int*>(take(256));
  w.bytes = off;
  return w;
}

}  // namespace attn_ws
}  // namespace rh3
