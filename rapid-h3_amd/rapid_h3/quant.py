"""Per-token activation quantizers on the HIP kernels (librh3: rh3_quant_*).

Each returns (q, s): q [M, K] int8 (or float8_e4m3fn), s [M, 1] fp32, like the reference's
triton_fp8 wrappers (/root/reference/custom_nodes/rapid_h3/triton_fp8.py:57-64, :424-455).
Semantics: s = max(amax / QMAX, 1e-12), q = round_half_even(v / s) with the IEEE quotient of the
reference's PyTorch path (kernels.py:75-82).
"""
import torch

from . import _native as nat

FP8 = torch.float8_e4m3fn


def _check_rows(x, name):
    if x.ndim != 2 or x.stride(1) != 1:
        raise AssertionError(f"{name}: x must be 2-D with a contiguous last dim, got shape "
                             f"{tuple(x.shape)} stride {tuple(x.stride())}")
    if x.dtype != torch.bfloat16:
        raise TypeError(f"{name}: x must be bf16, got {x.dtype}")
    if not x.is_cuda:
        raise RuntimeError(f"{name}: x must be on a GPU (no CPU path)")


def _out(x, m, k, dtype=torch.int8):
    q = torch.empty((m, k), device=x.device, dtype=dtype)
    s = torch.empty((m, 1), device=x.device, dtype=torch.float32)
    return q, s


def quant_rows_i8(x):
    """Per-row symmetric INT8 of x [M, K] bf16 (triton_fp8.quant_rows_i8)."""
    _check_rows(x, "quant_rows_i8")
    m, k = x.shape
    q, s = _out(x, m, k)
    nat.call("rh3_quant_rows_i8", nat.ptr(x), x.stride(0), m, k, nat.ptr(q), q.stride(0), nat.ptr(s),
             nat.stream(x.device))
    return q, s


def quant_rows(x):
    """Per-row FP8 e4m3fn of x [M, K] bf16 with s = amax / 448 (triton_fp8.quant_rows)."""
    _check_rows(x, "quant_rows")
    m, k = x.shape
    q, s = _out(x, m, k, FP8)
    nat.call("rh3_quant_rows_fp8", nat.ptr(x), x.stride(0), m, k, nat.ptr(q), q.stride(0), nat.ptr(s),
             nat.stream(x.device))
    return q, s


def norm_mod_quant_rows_i8(x, weight, eps, idx, shift, scale):
    """INT8 of rms_norm(x) * w * (1 + scale[idx]) + shift[idx] (triton_fp8.norm_mod_rot_quant_rows_i8
    prologue, without ConvRot): idx [M] int32 rows into shift/scale tables [R, K] (fp32 or bf16, shared
    row stride, unit column stride); weight [K] bf16 or None."""
    _check_rows(x, "norm_mod_quant_rows_i8")
    m, k = x.shape
    if shift.stride(1) != 1 or scale.stride(1) != 1 or shift.stride(0) != scale.stride(0):
        raise AssertionError("norm_mod_quant_rows_i8: shift/scale need unit column stride and a shared row stride")
    if shift.dtype != scale.dtype or shift.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError("norm_mod_quant_rows_i8: shift/scale must both be fp32 or both bf16")
    if idx.dtype != torch.int32 or idx.numel() != m:
        raise TypeError("norm_mod_quant_rows_i8: idx must be int32 [M]")
    if weight is not None:
        weight = weight.to(torch.bfloat16).contiguous()
        if weight.numel() != k:
            raise ValueError("norm_mod_quant_rows_i8: weight must have K elements")
    idx = idx.contiguous()
    q, s = _out(x, m, k)
    dt = nat.RH3_DTYPE_F32 if shift.dtype == torch.float32 else nat.RH3_DTYPE_BF16
    nat.call("rh3_quant_norm_mod_i8", nat.ptr(x), x.stride(0), m, k, nat.ptr(weight), float(eps), nat.ptr(idx),
             nat.ptr(shift), nat.ptr(scale), dt, shift.stride(0), nat.ptr(q), q.stride(0), nat.ptr(s),
             nat.stream(x.device))
    return q, s


def heads_quant_rows_i8(o):
    """INT8 of o.transpose(0, 1).reshape(M, H * 128) for a head-major attention output o [H, M, 128]
    (any head / token stride), without materializing the transpose (triton_fp8.rot_quant_heads_i8 gather)."""
    h, m, d = o.shape
    if d != 128 or o.stride(2) != 1:
        raise AssertionError("heads_quant_rows_i8: o must be [H, M, 128] with contiguous last dim")
    if o.dtype != torch.bfloat16 or not o.is_cuda:
        raise TypeError("heads_quant_rows_i8: o must be bf16 on a GPU")
    q, s = _out(o, m, h * d)
    nat.call("rh3_quant_heads_i8", nat.ptr(o), h, m, o.stride(0), o.stride(1), nat.ptr(q), q.stride(0),
             nat.ptr(s), nat.stream(o.device))
    return q, s


def swiglu_quant_rows_i8(x):
    """x [M, 2F] (gate | up) -> INT8 of silu(gate) * up (triton_fp8.swiglu_rot_quant_rows_i8 prologue)."""
    _check_rows(x, "swiglu_quant_rows_i8")
    m, k2 = x.shape
    f = k2 // 2
    q, s = _out(x, m, f)
    nat.call("rh3_quant_swiglu_i8", nat.ptr(x), x.stride(0), m, f, nat.ptr(q), q.stride(0), nat.ptr(s),
             nat.stream(x.device))
    return q, s
