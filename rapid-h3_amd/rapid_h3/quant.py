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


# ---------------------------------------------------------------- ConvRot (int8_rot) quantizers
# Same prologues as above, then x @ blockdiag(H256)^T before the per-row INT8 (librh3 rh3_*rot*):
# per 256-group bf16(v) in four 64-chunks, z_k = fp32(exact X_k H64^T), the reference's fp32 H4/2
# combine of the chunks, s = max(amax / 127, 1e-12), q = rint(clamp(y * (1 / s))) (triton_fp8.py:102-116,
# :277-351). K must be a multiple of 256 and at most 16384.

def _check_rot_width(k, name):
    if k % 256 != 0:
        raise AssertionError(f"{name}: K={k} must be a multiple of the rotation group 256")


def rot_quant_rows_i8(x):
    """INT8 of x [M, K] bf16 @ blockdiag(H256)^T (triton_fp8.rot_quant_rows_i8)."""
    _check_rows(x, "rot_quant_rows_i8")
    m, k = x.shape
    _check_rot_width(k, "rot_quant_rows_i8")
    q, s = _out(x, m, k)
    nat.call("rh3_rot_quant_rows_i8", nat.ptr(x), x.stride(0), m, k, nat.ptr(q), q.stride(0), nat.ptr(s),
             nat.stream(x.device))
    return q, s


def swiglu_rot_quant_rows_i8(x):
    """x [M, 2F] (gate | up) -> INT8 of rot(silu(gate) * up) (triton_fp8.swiglu_rot_quant_rows_i8)."""
    _check_rows(x, "swiglu_rot_quant_rows_i8")
    m, k2 = x.shape
    f = k2 // 2
    _check_rot_width(f, "swiglu_rot_quant_rows_i8")
    q, s = _out(x, m, f)
    nat.call("rh3_swiglu_rot_quant_rows_i8", nat.ptr(x), x.stride(0), m, f, nat.ptr(q), q.stride(0), nat.ptr(s),
             nat.stream(x.device))
    return q, s


def norm_mod_rot_quant_rows_i8(x, weight, eps, idx, shift, scale):
    """INT8 of rot(rms_norm(x) * w * (1 + scale[idx]) + shift[idx]) (triton_fp8.norm_mod_rot_quant_rows_i8);
    arguments as norm_mod_quant_rows_i8."""
    _check_rows(x, "norm_mod_rot_quant_rows_i8")
    m, k = x.shape
    _check_rot_width(k, "norm_mod_rot_quant_rows_i8")
    if shift.stride(1) != 1 or scale.stride(1) != 1 or shift.stride(0) != scale.stride(0):
        raise AssertionError("norm_mod_rot_quant_rows_i8: shift/scale need unit column stride and a shared row stride")
    if shift.dtype != scale.dtype or shift.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError("norm_mod_rot_quant_rows_i8: shift/scale must both be fp32 or both bf16")
    if idx.dtype != torch.int32 or idx.numel() != m:
        raise TypeError("norm_mod_rot_quant_rows_i8: idx must be int32 [M]")
    if weight is not None:
        weight = weight.to(torch.bfloat16).contiguous()
        if weight.numel() != k:
            raise ValueError("norm_mod_rot_quant_rows_i8: weight must have K elements")
    idx = idx.contiguous()
    q, s = _out(x, m, k)
    dt = nat.RH3_DTYPE_F32 if shift.dtype == torch.float32 else nat.RH3_DTYPE_BF16
    nat.call("rh3_norm_mod_rot_quant_i8", nat.ptr(x), x.stride(0), m, k, nat.ptr(weight), float(eps), nat.ptr(idx),
             nat.ptr(shift), nat.ptr(scale), dt, shift.stride(0), nat.ptr(q), q.stride(0), nat.ptr(s),
             nat.stream(x.device))
    return q, s


def rot_quant_heads_i8(o):
    """INT8 of rot(o.transpose(0, 1).reshape(M, H * 128)) for a head-major o [H, M, 128]
    (triton_fp8.rot_quant_heads_i8)."""
    h, m, d = o.shape
    if d != 128 or o.stride(2) != 1:
        raise AssertionError("rot_quant_heads_i8: o must be [H, M, 128] with contiguous last dim")
    if o.dtype != torch.bfloat16 or not o.is_cuda:
        raise TypeError("rot_quant_heads_i8: o must be bf16 on a GPU")
    _check_rot_width(h * d, "rot_quant_heads_i8")
    q, s = _out(o, m, h * d)
    nat.call("rh3_rot_quant_heads_i8", nat.ptr(o), h, m, o.stride(0), o.stride(1), nat.ptr(q), q.stride(0),
             nat.ptr(s), nat.stream(o.device))
    return q, s


def _dtype_code(t, name):
    if t.dtype == torch.bfloat16:
        return nat.RH3_DTYPE_BF16
    if t.dtype == torch.float32:
        return nat.RH3_DTYPE_F32
    raise TypeError(f"{name}: bf16 or fp32 input, got {t.dtype}")


def quant_any(x, mode):
    """Quantization of a 2-D GPU tensor of any float dtype (bf16, fp16, fp32) on rh3_quant_any, the reference's torch
    path semantics (kernels.py:57-82, :125-128): mode "int8" / "fp8" one scale per row -> (q, s [M, 1] fp32);
    "fp8_tensor" one scale for the tensor -> (q, s [] fp32). IEEE quotient; codes int8 or float8_e4m3fn."""
    if x.ndim != 2 or not x.is_cuda:
        raise AssertionError("quant_any: x must be a 2-D GPU tensor (no CPU path)")
    codes = {torch.bfloat16: nat.RH3_DTYPE_BF16, torch.float32: nat.RH3_DTYPE_F32, torch.float16: nat.RH3_DTYPE_F16}
    if x.dtype not in codes:
        raise TypeError(f"quant_any: float input (bf16, fp16, fp32), got {x.dtype}")
    if x.stride(1) != 1:
        x = x.contiguous()
    m, k = x.shape
    mo = {"int8": 0, "fp8": 1, "fp8_tensor": 2}[mode]
    q = torch.empty((m, k), device=x.device, dtype=torch.int8 if mo == 0 else torch.uint8)
    s = torch.empty((1, 1) if mo == 2 else (m, 1), device=x.device, dtype=torch.float32)
    amax = torch.empty(1, device=x.device, dtype=torch.float32) if mo == 2 else None
    nat.call("rh3_quant_any", nat.ptr(x), codes[x.dtype], x.stride(0), m, k, mo, nat.ptr(q), q.stride(0), nat.ptr(s),
             nat.ptr(amax), nat.stream(x.device))
    return (q if mo == 0 else q.view(FP8)), (s.reshape(()) if mo == 2 else s)


def convrot_f32(x):
    """x [M, K] (bf16 or fp32, GPU) @ blockdiag(H256)^T as fp32, the exact product rounded once."""
    if x.ndim != 2 or x.stride(1) != 1 or not x.is_cuda:
        raise AssertionError("convrot: x must be a 2-D GPU tensor with a contiguous last dim (no CPU path)")
    m, k = x.shape
    _check_rot_width(k, "convrot")
    dt = _dtype_code(x, "convrot")
    if x.data_ptr() % 16 or x.stride(0) % 8:
        x = x.contiguous()
    y = torch.empty((m, k), device=x.device, dtype=torch.float32)
    nat.call("rh3_convrot_f32", nat.ptr(x), dt, x.stride(0), m, k, nat.ptr(y), y.stride(0), nat.stream(x.device))
    return y


def fake_nvfp4_bf16(x):
    """kernels.fake_nvfp4(x).to(torch.bfloat16) (kernels.py:38-49, :56, :122): the NVFP4 round trip of a 2-D GPU
    tensor (bf16 or fp32, last dim a multiple of 16) on rh3_fake_nvfp4 -> bf16 of the same shape."""
    if x.ndim != 2 or x.stride(1) != 1 or not x.is_cuda:
        raise AssertionError("fake_nvfp4: x must be a 2-D GPU tensor with a contiguous last dim (no CPU path)")
    m, k = x.shape
    if k % 16:
        raise AssertionError("fake_nvfp4: the last dim must be a multiple of 16")
    dt = _dtype_code(x, "fake_nvfp4")
    out = torch.empty((m, k), device=x.device, dtype=torch.bfloat16)
    amax = torch.empty(1, device=x.device, dtype=torch.float32)
    nat.call("rh3_fake_nvfp4", nat.ptr(x), dt, x.stride(0), m, k, nat.ptr(out), out.stride(0), nat.ptr(amax),
             nat.stream(x.device))
    return out


def quantize_weight_rot(w):
    """kernels.quantize_weight(w, "int8_rot"): per-row INT8 of convrot(w) -> (q [N, K] int8, s [N, 1] fp32)."""
    if w.ndim != 2 or not w.is_cuda:
        raise AssertionError("quantize_weight_rot: w must be a 2-D GPU tensor")
    w = w.contiguous()
    n, k = w.shape
    _check_rot_width(k, "quantize_weight_rot")
    dt = _dtype_code(w, "quantize_weight_rot")
    q, s = _out(w, n, k)
    nat.call("rh3_quant_weight_rot_i8", nat.ptr(w), dt, w.stride(0), n, k, nat.ptr(q), q.stride(0), nat.ptr(s),
             nat.stream(w.device))
    return q, s
