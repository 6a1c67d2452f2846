"""Drop-in for the reference's kernels module (/root/reference/custom_nodes/rapid_h3/kernels.py:29-137):
QWeight, quantize_weight, quantize_rows, linear, gemm_config with the same modes and layouts, every
quantizer and GEMM running on librh3's gfx950 kernels.

Differences from the reference, all on purpose:
  * the reference's plain-PyTorch branches (int8_rowwise via torch._int_mm, fp8_rowwise_torch via
    _scaled_mm) run here on the same HIP kernels as the fast modes; results are bit-identical to the
    PyTorch semantics for int8 (exact int32 accumulators, the same (acc * xs) * ws rounding);
  * there is no silent fallback: if librh3 is missing, calls raise (the reference prints and drops to
    torch, kernels.py:88-98);
  * int8_rot weights are rotated exactly (float64 butterflies, rounded once to fp32) instead of by a
    torch fp32 matmul of unspecified order;
  * the nvfp4 verification modes run their fp32 round trip on a HIP kernel (rh3_fake_nvfp4) and the
    bf16 x bf16 product on torch.nn.functional.linear, as the reference does (kernels.py:53-56, :120-122).
"""
from dataclasses import dataclass

import torch

from . import cutlass_fp8 as _cf, triton_fp8 as _tq  # noqa: F401  (the reference's module handles)
from . import gemm as _gemm, quant as _quant

FP8 = torch.float8_e4m3fn
FP8_MAX = 448.0
MODES = ("bf16", "fp8_tensor", "fp8_rowwise", "fp8_rowwise_torch", "int8_rowwise", "int8_fast", "int8_rot",
         "nvfp4_fake", "nvfp4_rot_fake")


@dataclass
class QWeight:
    q: torch.Tensor        # [N, K] quantized
    scale: torch.Tensor    # [1, N] fp32 (row-wise) or [] fp32 (tensor-wise)


def _row_quant(w, fp8):
    """Per-output-channel quantization of a bf16 weight [N, K] on the per-row kernels (the reference's
    row-wise weight rule, kernels.py:62-71, is the per-token activation rule applied along K)."""
    w = w.to(torch.bfloat16).contiguous()
    q, s = (_quant.quant_rows(w) if fp8 else _quant.quant_rows_i8(w))
    return QWeight(q, s.t().contiguous())


def quantize_weight(w, mode):
    """kernels.quantize_weight (kernels.py:52-72) for bf16 weights [N, K]."""
    if mode == "int8_fast":
        mode = "int8_rowwise"
    if mode in ("nvfp4_fake", "nvfp4_rot_fake"):   # verification only: a bf16 weight after the round trip
        wf = _quant.convrot_f32(w) if mode == "nvfp4_rot_fake" else w.contiguous()
        return QWeight(_quant.fake_nvfp4_bf16(wf), None)
    if mode == "int8_rot":
        q, s = _quant.quantize_weight_rot(w)
        return QWeight(q, s.t().contiguous())
    if w.dtype != torch.bfloat16:
        raise TypeError("quantize_weight: bf16 weights only (the checkpoint dtype of the DiT linears)")
    if mode == "fp8_tensor":
        s = (w.abs().amax().float() / FP8_MAX).clamp_min(1e-12)
        return QWeight((w.float() / s).clamp(-FP8_MAX, FP8_MAX).to(FP8), s)
    if mode in ("fp8_rowwise", "fp8_rowwise_torch"):
        return _row_quant(w, fp8=True)
    if mode == "int8_rowwise":
        return _row_quant(w, fp8=False)
    raise ValueError(mode)


def adopt_convrot(qdata, scale, group=256, transposed=False):
    """QWeight of an already-quantized Comfy int8_convrot weight (H256, per-row scale), taken as is, the
    check of __init__.py:107-114: int8 [N, K] codes, group 256, not transposed; scale -> [1, N] fp32."""
    if group != _tq.ROT_GROUP or transposed or qdata.dtype != torch.int8 or qdata.ndim != 2:
        raise ValueError("adopt_convrot: needs int8 [N, K] codes rotated with group 256, not transposed")
    return QWeight(qdata.contiguous(), scale.float().reshape(1, -1).contiguous())


def quantize_rows(x, mode):
    """Per-token (row) dynamic quantization -> (q, scale [M, 1] fp32) (kernels.py:75-82)."""
    if mode == "int8_rowwise":
        return _quant.quant_rows_i8(x)
    if mode in ("fp8_rowwise", "fp8_rowwise_torch"):
        return _quant.quant_rows(x)
    raise ValueError(mode)


def gemm_config(k, n):
    """Tile id of the reference (kernels.py:101-104); this backend ignores it."""
    return 6


def linear(x, qw, mode):
    """y = x @ W^T for x [M, K] bf16 and a QWeight of W [N, K]; returns x.dtype (kernels.py:107-137)."""
    if mode in ("nvfp4_fake", "nvfp4_rot_fake"):   # verification only (kernels.py:120-122)
        x2 = x.reshape(-1, x.shape[-1]).contiguous()
        xr = _quant.convrot_f32(x2) if mode == "nvfp4_rot_fake" else x2
        y = torch.nn.functional.linear(_quant.fake_nvfp4_bf16(xr), qw.q)
        return y.reshape(*x.shape[:-1], qw.q.shape[0]).to(x.dtype)
    if x.dtype != torch.bfloat16:
        raise TypeError("linear: bf16 activations only")
    x = x.contiguous()
    if mode == "int8_rot":
        xq, xs = _quant.rot_quant_rows_i8(x)
        return _gemm.int8_gemm(xq, xs, qw.q, qw.scale, config=gemm_config(x.shape[1], qw.q.shape[0]))
    if mode in ("int8_rowwise", "int8_fast"):
        xq, xs = _quant.quant_rows_i8(x)
        return _gemm.int8_gemm(xq, xs, qw.q, qw.scale, config=gemm_config(x.shape[1], qw.q.shape[0]))
    if mode in ("fp8_rowwise", "fp8_rowwise_torch"):
        xq, xs = _quant.quant_rows(x)
        return _gemm.fp8_gemm(xq, xs, qw.q, qw.scale, config=2)
    if mode == "fp8_tensor":
        s = (x.abs().amax().float() / FP8_MAX).clamp_min(1e-12)
        xq = (x.float() / s).clamp(-FP8_MAX, FP8_MAX).to(FP8)
        m, n = x.shape[0], qw.q.shape[0]
        return _gemm.fp8_gemm(xq, s.reshape(1).expand(m).contiguous(), qw.q,
                              qw.scale.reshape(1).expand(n).contiguous())
    raise ValueError(mode)
