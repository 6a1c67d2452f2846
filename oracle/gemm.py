"""CPU restatement of the reference's row-wise W8A8 / FP8 GEMMs and their epilogues.

TEST INFRASTRUCTURE ONLY (see oracle/numerics.py).

  * accumulator     acc[m, n] = sum_k int32(xq[m, k]) * int32(wq[n, k]), exact
                    (kernels.py:133-136 `torch._int_mm`; fp8_rowwise.cu:282-331 s8 x s8 -> s32)
  * plain / bias    y = bf16_RNE((fp32(acc) * xs[m]) * ws[n] [+ fp32(bias[n])])   fp8_rowwise.cu:294-304
  * SwiGLU          g, u = bf16(acc * xs * ws) over the swiglu_perm interleave; h = bf16((g*sigmoid(g))*u)
                    fp8_rowwise.cu:24-107 (VisitorSwigluStore), cutlass_fp8.py:55-62
  * gated residual  r = bf16_RNE(fma(fp32(bf16(acc * xs * ws)), gate[n], r))      fp8_rowwise.cu:333-389
                    (per-token gate rows: gate[rows[m], n], the _mod_gate branch of __init__.py:244-245)

The int8 product is computed as a float64 matrix product of the int8 codes: every partial sum is an
integer below K * 127^2 < 2^53, so float64 BLAS gives the exact int32 accumulator (and is fast).
"""
import numpy as np

from .numerics import F32, bf16_to_f32, f32_to_bf16, fp8_e4m3_to_f32


def int8_acc(xq, wq):
    """Exact int32 accumulators of xq [M, K] int8 times wq [N, K] int8 (transposed)."""
    a = np.asarray(xq, dtype=np.float64)
    b = np.asarray(wq, dtype=np.float64)
    acc = a @ b.T
    return acc.astype(np.int64).astype(np.int32)


def dequant(acc, xs, ws):
    """(fp32(acc) * xs[m]) * ws[n] in fp32; acc int32 (or fp32 for the FP8 GEMM)."""
    xs = np.asarray(xs, F32).reshape(-1, 1)
    ws = np.asarray(ws, F32).reshape(1, -1)
    return ((np.asarray(acc).astype(F32) * xs) * ws).astype(F32)


def int8_gemm(xq, xs, wq, ws, bias=None):
    """cutlass_fp8.int8_gemm (cutlass_fp8.py:37-39) -> bf16 bits [M, N]."""
    y = dequant(int8_acc(xq, wq), xs, ws)
    if bias is not None:
        y = (y + bf16_to_f32(bias).reshape(1, -1)).astype(F32)
    return f32_to_bf16(y)


def swiglu_perm(n2):
    """cutlass_fp8.swiglu_perm (cutlass_fp8.py:55-62): fc1 row order so each 8-row group is
    [gate 4j..4j+3 | up 4j..4j+3] for an fc1 weight [gate (F rows) | up (F rows)]."""
    f = n2 // 2
    j = np.arange(0, f, 4)
    blk = np.arange(4)
    return np.stack([j[:, None] + blk, f + j[:, None] + blk], axis=1).reshape(-1)


def swiglu_from_interleaved(y_bf16):
    """Epilogue of int8_gemm_swiglu on the bf16 GEMM output y [M, 2F] in swiglu_perm order -> h [M, F] bf16 bits."""
    y = bf16_to_f32(y_bf16)
    m, n2 = y.shape
    t = y.reshape(m, n2 // 8, 2, 4)               # [row, group, gate|up, 4]
    g = t[:, :, 0, :].reshape(m, n2 // 2)
    u = t[:, :, 1, :].reshape(m, n2 // 2)
    sig = (F32(1.0) / (F32(1.0) + np.exp(-g))).astype(F32)
    return f32_to_bf16((g * sig).astype(F32) * u)


def int8_gemm_swiglu(xq, xs, wq_perm, ws_perm):
    """cutlass_fp8.int8_gemm_swiglu (cutlass_fp8.py:65-67) -> h [M, N/2] bf16 bits."""
    return swiglu_from_interleaved(int8_gemm(xq, xs, wq_perm, ws_perm))


def fma_f32(a, b, c):
    """fp32 fused multiply-add, single rounding: a, b, c are fp32 whose a*b+c is exact in float64
    (true for bf16 a, b, c, the only use here)."""
    return (a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64)).astype(F32)


def int8_gemm_gated_residual(xq, xs, wq, ws, gate, resid):
    """cutlass_fp8.int8_gemm_gated_residual (cutlass_fp8.py:49-52): returns the new resid (bf16 bits);
    ComfyUI `resid.addcmul_(y, gate)` with y the bf16 GEMM output."""
    y = bf16_to_f32(int8_gemm(xq, xs, wq, ws))
    g = bf16_to_f32(gate).reshape(1, -1)
    r = bf16_to_f32(resid)
    return f32_to_bf16(fma_f32(y, np.broadcast_to(g, y.shape), r))


def int8_gemm_gated_residual_rows(xq, xs, wq, ws, gate, rows, resid):
    """The gated residual with a gate row per token (the per-token modulation branch of _fused_block,
    __init__.py:244-245, h3._mod_gate with _mod_row's bf16 rounding): r[m] = bf16(fma(y[m], gate[rows[m]], r[m]))."""
    y = bf16_to_f32(int8_gemm(xq, xs, wq, ws))
    g = bf16_to_f32(gate)[np.asarray(rows)]
    r = bf16_to_f32(resid)
    return f32_to_bf16(fma_f32(y, g, r))


def fp8_gemm(xq, xs, wq, ws, bias=None):
    """cutlass_fp8.fp8_gemm (cutlass_fp8.py:32-34) with an exact (float64) product of the e4m3 codes,
    rounded once to fp32 before the same epilogue. The GPU accumulates in fp32, so this is the
    tolerance reference (rel-L2), not a bit pattern."""
    a = fp8_e4m3_to_f32(xq).astype(np.float64)
    b = fp8_e4m3_to_f32(wq).astype(np.float64)
    acc = (a @ b.T).astype(F32)
    y = dequant(acc, xs, ws)
    if bias is not None:
        y = (y + bf16_to_f32(bias).reshape(1, -1)).astype(F32)
    return f32_to_bf16(y)


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))
