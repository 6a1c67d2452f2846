/* rh3.h — C ABI of the MI355X (gfx950) DiT hot-path library librh3.so.
 *
 * Plain pointers, int64 sizes and strides (in elements), a hipStream_t, and an int status
 * (0 = success; on failure rh3_last_error() returns the message for the calling thread). Every
 * pointer is device memory unless stated. Nothing here allocates device memory: callers own the
 * outputs and, for attention, a workspace sized by rh3_attention_workspace_bytes().
 *
 * Element types travel as their bit patterns: bf16 as uint16_t, OCP e4m3fn as uint8_t.
 *
 * Each entry point names the reference interface it replaces (paths under
 * /root/reference/custom_nodes/rapid_h3/). The reference reaches those through pybind11 modules
 * built by torch.utils.cpp_extension; this library is loaded with ctypes instead.
 */
#ifndef RH3_H
#define RH3_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RH3_OK 0
#define RH3_EINVAL 1   /* bad argument: shape, stride, alignment, null pointer */
#define RH3_ELAUNCH 2  /* HIP reported an error for a launch */

#define RH3_DTYPE_BF16 1
#define RH3_DTYPE_F32 2
#define RH3_DTYPE_F16 3

/* Message of the last failed call on this thread ("" if none). */
const char* rh3_last_error(void);
/* Library ABI version (increments when a signature changes). */
int rh3_abi_version(void);

/* ---------------------------------------------------------------------------------------------
 * Per-token activation quantizers: one HBM pass, s[m] = max(amax_m / QMAX, 1e-12),
 * q = round_half_even(x / s) clamped (int8: +-127; fp8: +-448 then e4m3fn RNE).
 * x [M, K] bf16 row stride ldx; q [M, K] row stride ldq; s [M] fp32. K % 8 == 0, ldx % 8 == 0,
 * ldq % 8 == 0, 16-byte aligned rows.
 * ------------------------------------------------------------------------------------------- */

/* replaces triton_fp8.quant_rows_i8 (triton_fp8.py:57-64) and the int8_rowwise
 * kernels.quantize_rows (kernels.py:75-80) */
int rh3_quant_rows_i8(const uint16_t* x, int64_t ldx, int64_t M, int64_t K,
                      int8_t* q, int64_t ldq, float* s, hipStream_t stream);

/* replaces triton_fp8.quant_rows (triton_fp8.py:449-455) and the fp8 kernels.quantize_rows (kernels.py:81-82) */
int rh3_quant_rows_fp8(const uint16_t* x, int64_t ldx, int64_t M, int64_t K,
                       uint8_t* q, int64_t ldq, float* s, hipStream_t stream);

/* RMSNorm + modulation prologue, then per-token int8:
 *   v = ((x * rstd) * w) * (1 + scale[idx[m]]) + shift[idx[m]],  rstd = 1 / sqrt(sum(x^2) / K + eps)
 * weight [K] bf16 or NULL; idx [M] int32; shift/scale [R, K] of tab_dtype (RH3_DTYPE_BF16 or
 * RH3_DTYPE_F32) sharing row stride ld_tab, unit column stride.
 * replaces triton_fp8.norm_mod_rot_quant_rows_i8 (triton_fp8.py:442-446), KIND 2 prologue
 * (triton_fp8.py:141-147), for the int8_rowwise recipe (no ConvRot) */
int rh3_quant_norm_mod_i8(const uint16_t* x, int64_t ldx, int64_t M, int64_t K,
                          const uint16_t* weight, float eps, const int32_t* idx,
                          const void* shift, const void* scale, int tab_dtype, int64_t ld_tab,
                          int8_t* q, int64_t ldq, float* s, hipStream_t stream);

/* Head-major attention output o [H, M, 128] bf16 (head stride ld_head, token stride ld_row) ->
 * per-token int8 of the row [M, H*128] (column k = head k/128, dim k%128), without the transpose.
 * replaces triton_fp8.rot_quant_heads_i8 (triton_fp8.py:429-434), KIND 3 gather (:133-135) */
int rh3_quant_heads_i8(const uint16_t* o, int64_t H, int64_t M, int64_t ld_head, int64_t ld_row,
                       int8_t* q, int64_t ldq, float* s, hipStream_t stream);

/* x [M, 2F] = [gate | up] bf16 -> per-token int8 of (g * sigmoid(g)) * u, [M, F].
 * replaces triton_fp8.swiglu_rot_quant_rows_i8 (triton_fp8.py:437-439), KIND 1 prologue (:137-139) */
int rh3_quant_swiglu_i8(const uint16_t* x, int64_t ldx, int64_t M, int64_t F,
                        int8_t* q, int64_t ldq, float* s, hipStream_t stream);

/* ---------------------------------------------------------------------------------------------
 * ConvRot (int8_rot) quantizers: the prologue row is rotated by blockdiag(H256) (H256 = normalized 4th
 * Kronecker power of the 4x4 regular Hadamard) before the per-token int8 quantization. Per 256-group:
 * bf16(v) in four 64-chunks, z_k = fp32(exact X_k H64^T), the fixed-order fp32 H4/2 combine of the
 * chunks, s = max(amax/127, 1e-12), q = rint(clamp(y * (1/s))). K % 256 == 0, K <= 16384.
 * ------------------------------------------------------------------------------------------- */

/* replaces triton_fp8.rot_quant_rows_i8 (triton_fp8.py:424-427), KIND 0 of _rot_quant_wide_kernel */
int rh3_rot_quant_rows_i8(const uint16_t* x, int64_t ldx, int64_t M, int64_t K,
                          int8_t* q, int64_t ldq, float* s, hipStream_t stream);

/* replaces triton_fp8.swiglu_rot_quant_rows_i8 (triton_fp8.py:437-439): x [M, 2F] = [gate | up] */
int rh3_swiglu_rot_quant_rows_i8(const uint16_t* x, int64_t ldx, int64_t M, int64_t F,
                                 int8_t* q, int64_t ldq, float* s, hipStream_t stream);

/* replaces triton_fp8.norm_mod_rot_quant_rows_i8 (triton_fp8.py:442-446): RMSNorm + modulation
 * prologue as rh3_quant_norm_mod_i8, then the rotation */
int rh3_norm_mod_rot_quant_i8(const uint16_t* x, int64_t ldx, int64_t M, int64_t K,
                              const uint16_t* weight, float eps, const int32_t* idx,
                              const void* shift, const void* scale, int tab_dtype, int64_t ld_tab,
                              int8_t* q, int64_t ldq, float* s, hipStream_t stream);

/* replaces triton_fp8.rot_quant_heads_i8 (triton_fp8.py:429-434): head-major o [H, M, 128] gathered
 * per token as in rh3_quant_heads_i8, then rotated */
int rh3_rot_quant_heads_i8(const uint16_t* o, int64_t H, int64_t M, int64_t ld_head, int64_t ld_row,
                           int8_t* q, int64_t ldq, float* s, hipStream_t stream);

/* replaces triton_fp8.convrot (triton_fp8.py:86-90): y = x @ blockdiag(H256)^T as the fp32 rounding of
 * the exact product; x bf16 (RH3_DTYPE_BF16) or fp32 (RH3_DTYPE_F32) rows, y fp32 */
int rh3_convrot_f32(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K,
                    float* y, int64_t ldy, hipStream_t stream);

/* NVFP4 round trip of the verification modes nvfp4_fake / nvfp4_rot_fake: replaces kernels.fake_nvfp4
 * (kernels.py:38-49) followed by the callers' bf16 cast (kernels.py:56, :122). x [M, K] bf16 (RH3_DTYPE_BF16)
 * or fp32 (RH3_DTYPE_F32), K % 16 == 0; out [M, K] bf16 (row stride ldo % 8 == 0, 16-byte aligned);
 * amax_ws: one device float of caller scratch (the tensor absmax, written before it is read). One fp32 scale
 * per tensor gs = max(amax / 2688, 1e-12); per 16-element block s = e4m3(min(amax_b / 6 / gs, 448)) * gs (1 where
 * 0); values rounded to the e2m1 grid of x / s with ties to the lower point, times s. */
int rh3_fake_nvfp4(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, uint16_t* out, int64_t ldo,
                   float* amax_ws, hipStream_t stream);

/* Quantizer of any float input (bf16, fp16 or fp32 rows; x_dtype RH3_DTYPE_*), for what the fused quantizers
 * above do not take: the reference's torch path casts any float with .float() (kernels.py:57-82). mode 0: per-row
 * int8, s[m] = max(amax_m / 127, 1e-12), q = clamp(rint(x / s), +-127); mode 1: per-row FP8, s[m] = max(amax_m /
 * 448, 1e-12), q = e4m3(clamp(x / s, +-448)); mode 2: FP8 with one scale per tensor (the fp8_tensor mode,
 * kernels.py:64-66, :125-128), s[0] = max(amax / 448, 1e-12), amax_ws one float of caller scratch. IEEE quotient.
 * q [M, K] int8 / e4m3 bytes (row stride ldq).
 * replaces kernels.quantize_weight / quantize_rows and the fp8_tensor quantization of kernels.linear for
 * non-bf16 inputs */
int rh3_quant_any(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, int mode,
                  void* q, int64_t ldq, float* s, float* amax_ws, hipStream_t stream);

/* replaces kernels.quantize_weight(w, "int8_rot") (kernels.py:62-72): convrot(w) (exact, rounded to
 * fp32), then per-row s = max(amax/127, 1e-12), q = round(w_rot / s); w [N, K] bf16 or fp32 */
int rh3_quant_weight_rot_i8(const void* w, int w_dtype, int64_t ldw, int64_t N, int64_t K,
                            int8_t* q, int64_t ldq, float* s, hipStream_t stream);

/* ---------------------------------------------------------------------------------------------
 * Row-wise W8A8 GEMMs on int8 MFMA: acc[m,n] = sum_k xq[m,k] * wq[n,k] (int32, exact),
 * y = (fp32(acc) * xs[m]) * ws[n]. xq [M, K] int8 (row stride ldx), wq [N, K] int8 (row stride ldw),
 * xs [M], ws [N] fp32. K % 64 == 0, N % 8 == 0, strides % 16 == 0, 16-byte aligned rows.
 * ctr: NULL, or 8 int32 of device memory (4-byte aligned) that the call owns while it runs on `stream`: the
 * large shapes run one workgroup per CU over a tile sequence, and with ctr the workgroups of a faster XCD take
 * over tiles of a slower one (per-XCD tile counters, cleared by a fill kernel on `stream` at each call, so the
 * call stays capturable). Calls that may run concurrently (different streams) need different ctr. Same
 * results with and without it; NULL keeps fixed per-XCD tile shares.
 * ------------------------------------------------------------------------------------------- */

/* out = bf16_RNE(y [+ bias[n]]); bias [N] bf16 or NULL; out [M, N] row stride ldo.
 * replaces cutlass_fp8.int8_gemm -> int8_rowwise_gemm (cutlass_fp8.py:37-39, fp8_rowwise.cu:546-584) */
int rh3_gemm_i8(const int8_t* xq, int64_t ldx, const float* xs, const int8_t* wq, int64_t ldw,
                const float* ws, const uint16_t* bias, uint16_t* out, int64_t ldo,
                int64_t M, int64_t N, int64_t K, int32_t* ctr, hipStream_t stream);

/* SwiGLU epilogue for fc1 rows in swiglu_perm order ([g 4j..4j+3 | u 4j..4j+3] per 8 columns):
 * g, u = bf16(y); h[m, n/2..] = bf16((g * sigmoid(g)) * u); out [M, N/2] row stride ldo.
 * replaces cutlass_fp8.int8_gemm_swiglu (cutlass_fp8.py:65-67, fp8_rowwise.cu:611-629) */
int rh3_gemm_i8_swiglu(const int8_t* xq, int64_t ldx, const float* xs, const int8_t* wq_perm, int64_t ldw,
                       const float* ws_perm, uint16_t* out, int64_t ldo,
                       int64_t M, int64_t N, int64_t K, int32_t* ctr, hipStream_t stream);

/* Gated residual, in place: resid[m,n] = bf16_RNE(fma(bf16(y), gate[n], resid[m,n])); gate [N] bf16;
 * resid [M, N] row stride ldr.
 * replaces cutlass_fp8.int8_gemm_gated_residual (cutlass_fp8.py:49-52, fp8_rowwise.cu:587-608) */
int rh3_gemm_i8_gated(const int8_t* xq, int64_t ldx, const float* xs, const int8_t* wq, int64_t ldw,
                      const float* ws, const uint16_t* gate, uint16_t* resid, int64_t ldr,
                      int64_t M, int64_t N, int64_t K, int32_t* ctr, hipStream_t stream);

/* Gated residual with a gate row per output row (per-token modulation), in place:
 * resid[m,n] = bf16_RNE(fma(bf16(y), gate[gidx[m], n], resid[m,n])); gate [R, ldg] bf16 (16-byte aligned,
 * ldg >= N, ldg % 8 == 0), gidx [M] int32 rows of it.
 * replaces the per-token branch of _fused_block's gated residual, h3._mod_gate(x, gate, int8_gemm(...),
 * segments) for segments whose row is a tensor (__init__.py:242-245) */
int rh3_gemm_i8_gated_rows(const int8_t* xq, int64_t ldx, const float* xs, const int8_t* wq, int64_t ldw,
                           const float* ws, const uint16_t* gate, int64_t ldg, const int32_t* gidx,
                           uint16_t* resid, int64_t ldr, int64_t M, int64_t N, int64_t K, int32_t* ctr,
                           hipStream_t stream);

/* Verification: the raw int32 accumulators acc [M, N] (row stride ldc) of the same kernel.
 * No reference counterpart as an entry point: it exposes the s32 accumulator of
 * fp8_rowwise.cu:282-331 so tests can check it bit for bit. */
int rh3_gemm_i8_acc(const int8_t* xq, int64_t ldx, const int8_t* wq, int64_t ldw, int32_t* acc, int64_t ldc,
                    int64_t M, int64_t N, int64_t K, int32_t* ctr, hipStream_t stream);

/* The qkv projection with the attention pre-pass partly fused into its epilogue.
 * replaces cutlass_fp8.int8_gemm_qkv_prep -> run_qkv_prep / VisitorQkvPrep (cutlass_fp8.py:42-46,
 * fp8_rowwise.cu:108-272, :635-655): out [M, 3*H*128] = bf16((acc * xs) * ws [+ bias]) for the k and v columns
 * (the q columns are left unwritten); the q columns go, after the per-head RMSNorm + RoPE (tab [M, rot/2, 2, 2],
 * qw; tab NULL: none), straight to the Q operands of the attention workspace (rh3_attention_workspace_bytes /
 * rh3_attention_u8_workspace_bytes for Sq = Sk = M): numerics 0 one scale per (head, 128-token block),
 * numerics 1 per token after the H128 rotation (rotate); the per-256-token channel sums of RMSNorm + RoPE(k)
 * (kw) and, for numerics 1, the V sums / max / min go to the same workspace. H must be even. Continue with
 * rh3_attention_prepass_qkv (numerics 0) or rh3_attention_u8_prepass_qkv (numerics 1). */
int rh3_gemm_i8_qkv(const int8_t* xq, int64_t ldx, const float* xs, const int8_t* wq, int64_t ldw,
                    const float* ws, const uint16_t* bias, uint16_t* out, int64_t ldo,
                    int64_t M, int64_t H, int64_t K, const uint16_t* tab, int rot,
                    const uint16_t* qw, const uint16_t* kw, float eps, int numerics, int rotate,
                    void* workspace, int64_t workspace_bytes, hipStream_t stream);

/* FP8 (OCP e4m3fn) row-wise GEMM, fp32 accumulate, same epilogue as rh3_gemm_i8.
 * replaces cutlass_fp8.fp8_gemm -> fp8_rowwise_gemm (cutlass_fp8.py:32-34, fp8_rowwise.cu:512-544) */
int rh3_gemm_fp8(const uint8_t* xq, int64_t ldx, const float* xs, const uint8_t* wq, int64_t ldw,
                 const float* ws, const uint16_t* bias, uint16_t* out, int64_t ldo,
                 int64_t M, int64_t N, int64_t K, int32_t* ctr, hipStream_t stream);

/* The raw fp32 accumulators acc [M, N] (row stride ldc) of the FP8 GEMM, before any scale: the product
 * torch._scaled_mm forms before it applies its scales, for outputs other than bf16.
 * replaces the fp16 / fp32 out_dtype of torch._scaled_mm in kernels.linear's fp8_tensor mode
 * (kernels.py:124-127); the caller applies (acc * scale_a) * scale_b and rounds to its dtype. */
int rh3_gemm_fp8_acc(const uint8_t* xq, int64_t ldx, const uint8_t* wq, int64_t ldw, float* acc, int64_t ldc,
                     int64_t M, int64_t N, int64_t K, int32_t* ctr, hipStream_t stream);

/* ---------------------------------------------------------------------------------------------
 * INT8 flash attention, head_dim 128, non-causal. q [Sq, H, 128], k and v [Sk, H, 128] bf16 with any
 * token / head strides (elements; the 128 channels contiguous). Q and K are quantized per
 * (head, 128-token block); K is first mean-smoothed (kmean over all Sk tokens); Q.K^T runs on int8
 * MFMA, softmax in fp32 (exp2 domain), P.V on bf16 MFMA. out [Sq, H, 128] bf16 with its own strides.
 * ------------------------------------------------------------------------------------------- */

/* Bytes of workspace the attention entry points need for (Sq, Sk, H). */
int64_t rh3_attention_workspace_bytes(int64_t Sq, int64_t Sk, int64_t H);

/* replaces attn_int8.attention -> int8_attention (attn_int8.py:30-34, attn_int8.cu:2660-2665) with
 * per-128-block Q/K scales (attn_int8.cu:402-443) and bf16 P.V. Sq may differ from Sk
 * (cross-attention); smooth_k 0 skips the K mean. */
int rh3_int8_attention(const uint16_t* q, int64_t q_ss, int64_t q_sh,
                       const uint16_t* k, int64_t k_ss, int64_t k_sh,
                       const uint16_t* v, int64_t v_ss, int64_t v_sh,
                       int64_t Sq, int64_t Sk, int64_t H, float scale, int smooth_k,
                       uint16_t* out, int64_t o_ss, int64_t o_sh,
                       void* workspace, int64_t workspace_bytes, hipStream_t stream);

/* rh3_int8_attention without a workspace argument, for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference. The pre-pass operands live in a 16 MiB device array of the library, one per GPU, held until the
 * process ends (every process that loads the library holds it on each GPU where the module loads, called or not);
 * sizes whose operands need more (rh3_attention_workspace_bytes less the split partials, roughly 512 bytes per
 * token and head, so about 32k token-heads) fail with RH3_EINVAL. The call allocates no device memory and calls no
 * allocating routine, except that the first call on a device resolves the array's address (hipGetSymbolAddress),
 * which may load the code object: make one call per device before capturing it in a graph. All calls on one GPU
 * share the array: calls that overlap there (two streams, two host threads) race. */
int rh3_int8_attention_noalloc(const uint16_t* q, int64_t q_ss, int64_t q_sh,
                               const uint16_t* k, int64_t k_ss, int64_t k_sh,
                               const uint16_t* v, int64_t v_ss, int64_t v_sh,
                               int64_t Sq, int64_t Sk, int64_t H, float scale, int smooth_k,
                               uint16_t* out, int64_t o_ss, int64_t o_sh, hipStream_t stream);

/* Same, with the per-head RMSNorm (weights qw/kw [128] bf16, eps) and split-half RoPE (table
 * tab [S, rot/2, 2, 2] bf16 = (cos, -sin, sin, cos), rot 96 or 128) applied to raw q and k inside
 * the pre-pass. Self-attention only (Sq == Sk == S).
 * replaces attn_int8.attention_rr -> int8_attention_rr (attn_int8.py:42-48, attn_int8.cu:2669-2676) */
int rh3_int8_attention_rr(const uint16_t* q, int64_t q_ss, int64_t q_sh,
                          const uint16_t* k, int64_t k_ss, int64_t k_sh,
                          const uint16_t* v, int64_t v_ss, int64_t v_sh,
                          int64_t S, int64_t H, const uint16_t* tab, int rot,
                          const uint16_t* qw, const uint16_t* kw, float eps, float scale, int smooth_k,
                          uint16_t* out, int64_t o_ss, int64_t o_sh,
                          void* workspace, int64_t workspace_bytes, hipStream_t stream);

/* Per-head RMSNorm (qw / kw [128] bf16, eps) and split-half RoPE (tab as above, rot 96 or 128) of q and k
 * [S, H, 128] bf16 in place (token / head strides in elements, multiples of 8): the prologue the *_rr entry points
 * and the pre-passes apply, on its own and bit-identical to it, for a caller that hands the roped q / k to another
 * attention.
 * replaces comfy_kitchen's ck.rms_rope_split_half_(q, k, rope_freqs, qw, kw, epsilon, rot_dim) (comfy-kitchen
 * 0.2.39, not vendored), called by _fused_block and _rr_check (__init__.py:297, :340) */
int rh3_rms_rope_qk(uint16_t* q, int64_t q_ss, int64_t q_sh, uint16_t* k, int64_t k_ss, int64_t k_sh,
                    int64_t S, int64_t H, const uint16_t* tab, int rot, const uint16_t* qw, const uint16_t* kw,
                    float eps, hipStream_t stream);

/* Pre-pass operands for verification (int8_prepass, attn_int8.cu:2851-2879): writes into the
 * workspace and returns pointers to q8 [H, Sqpad, 128] int8, qs [H, Sqpad/128] fp32, k8, ks,
 * kmean [H, 128] fp32 and vt [H, 128, Skpad] bf16 (keys permuted within 32-key groups).
 * tab NULL: no RMSNorm/RoPE. */
int rh3_attention_prepass(const uint16_t* q, int64_t q_ss, int64_t q_sh,
                          const uint16_t* k, int64_t k_ss, int64_t k_sh,
                          const uint16_t* v, int64_t v_ss, int64_t v_sh,
                          int64_t Sq, int64_t Sk, int64_t H, const uint16_t* tab, int rot,
                          const uint16_t* qw, const uint16_t* kw, float eps, int smooth_k,
                          void* workspace, int64_t workspace_bytes, void** ptrs /* [6] */,
                          hipStream_t stream);

/* The rest of the pre-pass after rh3_gemm_i8_qkv (numerics 0) on the same workspace: kmean from the GEMM's
 * K sums, the K quantizer (RMSNorm + RoPE with kw when tab is given) and the V relayout, reading k and v
 * [S, H, 128] from the GEMM output. ptrs as rh3_attention_prepass. Self-attention (Sq = Sk = S).
 * replaces attn_int8.attention_pre -> int8_attention_pre's pre-pass (attn_int8.py:50-57,
 * attn_int8.cu:2595-2610) for the per-block numerics. */
int rh3_attention_prepass_qkv(const uint16_t* k, int64_t k_ss, int64_t k_sh,
                              const uint16_t* v, int64_t v_ss, int64_t v_sh, int64_t S, int64_t H,
                              const uint16_t* tab, int rot, const uint16_t* kw, float eps, int smooth_k,
                              void* workspace, int64_t workspace_bytes, void** ptrs /* [6] */,
                              hipStream_t stream);

/* The main kernel alone, on a workspace rh3_attention_prepass filled for the same (Sq, Sk, H): the
 * second half of int8_attention (attn_int8.cu:2749-2849 after prepass()). Lets a caller time or
 * schedule the pre-pass and the main kernel separately. */
int rh3_attention_forward(int64_t Sq, int64_t Sk, int64_t H, float scale,
                          uint16_t* out, int64_t o_ss, int64_t o_sh,
                          void* workspace, int64_t workspace_bytes, hipStream_t stream);

/* ---------------------------------------------------------------------------------------------
 * INT8 flash attention with the reference's production numerics (attn_int8.cu configs 80-99: attn_fwd8
 * :2250-2511, and the cake configs 90/94 that are bit-identical to it; configs 1xx add the q/k RMSNorm +
 * RoPE pre-pass). Q and K per (token, head) row: K mean-smoothed (smooth_k), both rotated by the
 * normalized H128 Walsh-Hadamard matrix (rotate), sc = max(amax, 1e-8) / 127, q = rint(x / sc). V per
 * channel: mean-smoothed (smooth_v), vscale = max(max(vmax - vmean, vmean - vmin), 1e-6) / 127, codes
 * rint((v - vmean) / vscale). Per 128-key tile: u8 P = rint(255 * 2^(t - tile max)), int32 P.V, fp32
 * fold with the running max; out = bf16(O / l * vscale + vmean).
 * ------------------------------------------------------------------------------------------- */

/* Byte offsets of the arrays inside an attention workspace for (Sq, Sk, H), with the workspace size last.
 * numerics 0 (rh3_attention_workspace_bytes): q8, qs, k8, ks, kmean, part, vt, kn, bytes (9 values; kn [H, Skpad/128]
 * fp32: per 128-key block, an upper bound of the largest L2 norm of a key's int8 codes);
 * numerics 1 (rh3_attention_u8_workspace_bytes): q8, qs, k8, ks, side, vt, kmean, vmean, vscale, kpart, vsum,
 * vmax, vmin, bytes (14 values). No device access. No counterpart in the reference, whose operands are
 * separate torch tensors (attn_int8.cu:2568-2644); callers use it to view what rh3_gemm_i8_qkv wrote. */
int rh3_attention_workspace_layout(int numerics, int64_t Sq, int64_t Sk, int64_t H, int64_t* offsets);

/* Bytes of workspace the production-numerics entry points need for (Sq, Sk, H). */
int64_t rh3_attention_u8_workspace_bytes(int64_t Sq, int64_t Sk, int64_t H);

/* replaces attn_int8.attention / attention_rr / attention_rr_bias -> int8_attention(_rr, _rr_bias)
 * (attn_int8.py:30-65, attn_int8.cu:2660-2689) with config 80-99 (or 180-199). tab NULL: no RMSNorm/RoPE
 * (then Sq may differ from Sk); otherwise tab [S, rot/2, 2, 2] bf16, qw / kw [128] bf16, self-attention
 * only. nbias > 0 adds bias (natural-log units) to every query's logits of keys [0, nbias) (the Jenga
 * text bias, attn_int8.cu:2763-2774, attn_cake.cuh:97-99). */
int rh3_int8_attention_u8(const uint16_t* q, int64_t q_ss, int64_t q_sh,
                          const uint16_t* k, int64_t k_ss, int64_t k_sh,
                          const uint16_t* v, int64_t v_ss, int64_t v_sh,
                          int64_t Sq, int64_t Sk, int64_t H, const uint16_t* tab, int rot,
                          const uint16_t* qw, const uint16_t* kw, float eps, float scale,
                          int nbias, double bias, int smooth_k, int smooth_v, int rotate,
                          uint16_t* out, int64_t o_ss, int64_t o_sh,
                          void* workspace, int64_t workspace_bytes, hipStream_t stream);

/* Pre-pass operands of the production numerics for verification (the reference's prepass(),
 * attn_int8.cu:2568-2644): returns pointers into the workspace to q8 [H, Sqpad, 128] int8,
 * qs [H, Sqpad] fp32, k8 [H, Skpad, 128], ks [H, Skpad], side [H, Skpad/128, 2048 B] (per key the pair
 * (ks, -1.5*2^23 * ks) as fp32, padded keys (0, -inf); then per channel the int32 accumulator start
 * 1.5*2^23 bits + 128 * sum of the tile's V codes), vt [H, 128, Skpad] int8 V codes (keys permuted within
 * 32-key blocks), kmean, vscale, vmean [H, 128] fp32. */
int rh3_attention_u8_prepass(const uint16_t* q, int64_t q_ss, int64_t q_sh,
                             const uint16_t* k, int64_t k_ss, int64_t k_sh,
                             const uint16_t* v, int64_t v_ss, int64_t v_sh,
                             int64_t Sq, int64_t Sk, int64_t H, const uint16_t* tab, int rot,
                             const uint16_t* qw, const uint16_t* kw, float eps,
                             int smooth_k, int smooth_v, int rotate,
                             void* workspace, int64_t workspace_bytes, void** ptrs /* [9] */,
                             hipStream_t stream);

/* The rest of the production pre-pass after rh3_gemm_i8_qkv (numerics 1): kmean and vmean / vscale from the
 * GEMM's statistics, the per-token K quantizer with its (scale, bias) pairs, the int8 V codes. ptrs as
 * rh3_attention_u8_prepass. replaces attn_int8.cu int8_attention_pre's pre-pass (:2595-2610: stats_final,
 * quant_k_rr, quant_v). */
int rh3_attention_u8_prepass_qkv(const uint16_t* k, int64_t k_ss, int64_t k_sh,
                                 const uint16_t* v, int64_t v_ss, int64_t v_sh, int64_t S, int64_t H,
                                 const uint16_t* tab, int rot, const uint16_t* kw, float eps,
                                 int smooth_k, int smooth_v, int rotate,
                                 void* workspace, int64_t workspace_bytes, void** ptrs /* [9] */,
                                 hipStream_t stream);

/* The production main kernel alone, on a workspace rh3_attention_u8_prepass filled for (Sq, Sk, H). */
int rh3_attention_u8_forward(int64_t Sq, int64_t Sk, int64_t H, float scale, int nbias, double bias,
                             uint16_t* out, int64_t o_ss, int64_t o_sh,
                             void* workspace, int64_t workspace_bytes, hipStream_t stream);

/* ---------------------------------------------------------------------------------------------
 * INT8 flash attention with one K scale per 128-key block (attn_int8.cu configs 60-61: attn_fwd6
 * :1786-1962 and quant_k_block :404-443). Q and V as the production numerics above (per-token H128-rotated
 * Q; per-channel smoothed int8 V). K: mean-smoothed, H128-rotated (rotate), then one scale per (head,
 * 128-key block) kb = max(amax, 1e-8) / 127, codes rint(x * (1 / kb)). Per tile: integer max ti of the
 * accumulators, cc = qs * scale * log2(e) * kb, u8 P = rint(2^(fma(acc, cc, log2 255 - ti cc))), int32 P.V and
 * the same fold. No RMSNorm + RoPE path and no text bias, as in the reference. Workspace as
 * rh3_attention_u8_workspace_bytes.
 * ------------------------------------------------------------------------------------------- */

/* replaces attn_int8.attention(..., config=60 or 61) -> int8_attention (attn_int8.py:30-33,
 * attn_int8.cu:2660-2667, :2812-2813). */
int rh3_int8_attention_bk(const uint16_t* q, int64_t q_ss, int64_t q_sh,
                          const uint16_t* k, int64_t k_ss, int64_t k_sh,
                          const uint16_t* v, int64_t v_ss, int64_t v_sh,
                          int64_t Sq, int64_t Sk, int64_t H, float scale,
                          int smooth_k, int smooth_v, int rotate,
                          uint16_t* out, int64_t o_ss, int64_t o_sh,
                          void* workspace, int64_t workspace_bytes, hipStream_t stream);

/* Pre-pass operands of configs 60-61 for verification (the reference's int8_prepass with config 60,
 * attn_int8.cu:2618-2641): ptrs as rh3_attention_u8_prepass, except that ks holds the block scales
 * [H, Skpad/128] and each side record holds its block scale in its first float (the pair area is otherwise
 * unused). */
int rh3_attention_bk_prepass(const uint16_t* q, int64_t q_ss, int64_t q_sh,
                             const uint16_t* k, int64_t k_ss, int64_t k_sh,
                             const uint16_t* v, int64_t v_ss, int64_t v_sh,
                             int64_t Sq, int64_t Sk, int64_t H, int smooth_k, int smooth_v, int rotate,
                             void* workspace, int64_t workspace_bytes, void** ptrs /* [9] */,
                             hipStream_t stream);

/* The configs 60-61 main kernel alone, on a workspace rh3_attention_bk_prepass filled for (Sq, Sk, H). */
int rh3_attention_bk_forward(int64_t Sq, int64_t Sk, int64_t H, float scale,
                             uint16_t* out, int64_t o_ss, int64_t o_sh,
                             void* workspace, int64_t workspace_bytes, hipStream_t stream);

/* ---------------------------------------------------------------------------------------------
 * INT8 flash attention with FP8 P.V (attn_int8.cu configs 50-56: attn_fwd5 :1563-1785, quant_v's fp8 branch
 * :467-473). Q and K as the production numerics (per-token H128-rotated codes, per-key (scale, bias) pairs);
 * V per channel as e4m3 codes of ((v - vmean) / vscale) * fp32(448 / 127). Per group of `tile` keys (64 or 128,
 * the reference's BN): the running max m grows to the group max (O and l scaled by 2^((m_old - m) c)),
 * P = e4m3(2^(fma(t, c, log2 448 - m c))), l += P unquantized, O += P . V on the FP8 MFMA in fp32; out =
 * bf16(O / l * vscale * fp32(127 / 448) + vmean). RMSNorm + RoPE as the production entry points (tab != NULL),
 * no text bias. Workspace as rh3_attention_u8_workspace_bytes.
 * ------------------------------------------------------------------------------------------- */

/* replaces attn_int8.attention / attention_rr with config 50-56 (or 150-156) -> int8_attention(_rr)
 * (attn_int8.py:30-47, attn_int8.cu:2660-2676, :2804-2810). tile: 64 for configs 50, 51, 54, 56, 128 for 52,
 * 53, 55. */
int rh3_int8_attention_f8(const uint16_t* q, int64_t q_ss, int64_t q_sh,
                          const uint16_t* k, int64_t k_ss, int64_t k_sh,
                          const uint16_t* v, int64_t v_ss, int64_t v_sh,
                          int64_t Sq, int64_t Sk, int64_t H, const uint16_t* tab, int rot,
                          const uint16_t* qw, const uint16_t* kw, float eps, float scale, int tile,
                          int smooth_k, int smooth_v, int rotate,
                          uint16_t* out, int64_t o_ss, int64_t o_sh,
                          void* workspace, int64_t workspace_bytes, hipStream_t stream);

/* Pre-pass operands of configs 50-56 for verification (the reference's int8_prepass with config 50): ptrs as
 * rh3_attention_u8_prepass, with vt [H, 128, Skpad] e4m3 codes (keys permuted within 64-key chunks) and the
 * side records' accumulator starts unused. */
int rh3_attention_f8_prepass(const uint16_t* q, int64_t q_ss, int64_t q_sh,
                             const uint16_t* k, int64_t k_ss, int64_t k_sh,
                             const uint16_t* v, int64_t v_ss, int64_t v_sh,
                             int64_t Sq, int64_t Sk, int64_t H, const uint16_t* tab, int rot,
                             const uint16_t* qw, const uint16_t* kw, float eps,
                             int smooth_k, int smooth_v, int rotate,
                             void* workspace, int64_t workspace_bytes, void** ptrs /* [9] */,
                             hipStream_t stream);

/* The FP8 P.V main kernel alone, on a workspace rh3_attention_f8_prepass filled for (Sq, Sk, H). */
int rh3_attention_f8_forward(int64_t Sq, int64_t Sk, int64_t H, float scale, int tile,
                             uint16_t* out, int64_t o_ss, int64_t o_sh,
                             void* workspace, int64_t workspace_bytes, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* RH3_H */
