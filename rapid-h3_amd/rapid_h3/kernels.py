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
    bf16 x bf16 product on torch.nn.functional.linear, as the reference does (kernels.py:53-56, :120-122);
  * fp8_tensor: the tensor absmax and codes on rh3_quant_any, the product on the FP8 GEMM kernel: for bf16 x with the
    two scales in its epilogue, for fp16 / fp32 x as raw fp32 accumulators scaled by (acc * s_x) * s_w and rounded
    once to x.dtype, as the reference's _scaled_mm(out_dtype=x.dtype) does.
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
    """Per-output-channel quantization of a weight [N, K] (kernels.py:62-71, the per-token activation rule applied
    along K): bf16 weights on the fused per-row kernels, fp16 / fp32 ones on the any-dtype quantizer (the
    reference computes in w.float())."""
    if w.dtype == torch.bfloat16:
        w = w.contiguous()
        q, s = (_quant.quant_rows(w) if fp8 else _quant.quant_rows_i8(w))
    else:
        q, s = _quant.quant_any(w, "fp8" if fp8 else "int8")
    return QWeight(q, s.t().contiguous())


def quantize_weight(w, mode):
    """kernels.quantize_weight (kernels.py:52-72) for weights [N, K] of any float dtype (bf16, fp16, fp32)."""
    if mode == "int8_fast":
        mode = "int8_rowwise"
    if mode in ("nvfp4_fake", "nvfp4_rot_fake"):   # verification only: a bf16 weight after the round trip
        w = w if w.dtype in (torch.bfloat16, torch.float32) else w.float()
        wf = _quant.convrot_f32(w) if mode == "nvfp4_rot_fake" else w.contiguous()
        return QWeight(_quant.fake_nvfp4_bf16(wf), None)
    if mode == "int8_rot":
        q, s = _quant.quantize_weight_rot(w if w.dtype in (torch.bfloat16, torch.float32) else w.float())
        return QWeight(q, s.t().contiguous())
    if mode == "fp8_tensor":
        q, s = _quant.quant_any(w, "fp8_tensor")
        return QWeight(q, s)
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
    """Per-token (row) dynamic quantization -> (q, scale [M, 1] fp32) (kernels.py:75-82); bf16 rows on the fused
    kernels, other float dtypes on the any-dtype quantizer. A mode other than int8_rowwise quantizes to FP8, as in
    the reference."""
    if x.dtype == torch.bfloat16:
        return _quant.quant_rows_i8(x) if mode == "int8_rowwise" else _quant.quant_rows(x)
    return _quant.quant_any(x.reshape(-1, x.shape[-1]), "int8" if mode == "int8_rowwise" else "fp8")


def gemm_config(k, n):
    """Tile id of the reference (kernels.py:101-104); this backend ignores it."""
    return 6


def linear(x, qw, mode):
    """y = x @ W^T for x [M, K] and a QWeight of W [N, K]; returns x.dtype (kernels.py:107-137). bf16 x runs the fused
    quantizer + GEMM kernels of each mode. Other float dtypes take the reference's torch-path semantics (its fast
    paths are bf16-only): codes from the any-dtype quantizer, the exact int32 (or unit-scale FP8) product on the GEMM
    kernels, then (acc * sa * ws).to(x.dtype) (kernels.py:131-137); int8_rot / int8_fast have no such path there and
    raise ValueError, as in the reference."""
    if mode in ("nvfp4_fake", "nvfp4_rot_fake"):   # verification only (kernels.py:120-122)
        x2 = x.reshape(-1, x.shape[-1])
        x2 = (x2 if x2.dtype in (torch.bfloat16, torch.float32) else x2.float()).contiguous()
        xr = _quant.convrot_f32(x2) if mode == "nvfp4_rot_fake" else x2
        y = torch.nn.functional.linear(_quant.fake_nvfp4_bf16(xr), qw.q)
        return y.reshape(*x.shape[:-1], qw.q.shape[0]).to(x.dtype)
    if mode == "fp8_tensor":
        xq, s = _quant.quant_any(x, "fp8_tensor")
        m, n = x.shape[0], qw.q.shape[0]
        if x.dtype == torch.bfloat16:   # the two scales in the GEMM epilogue, rounded once to bf16
            return _gemm.fp8_gemm(xq, s.reshape(1).expand(m).contiguous(), qw.q,
                                  qw.scale.reshape(1).expand(n).contiguous())
        # fp16 / fp32 out: the raw fp32 product, then (acc * s_x) * s_w rounded once to x.dtype
        return ((_gemm.fp8_gemm_acc(xq, qw.q) * s.reshape(1)) * qw.scale.reshape(1)).to(x.dtype)
    if x.dtype != torch.bfloat16:
        if mode == "fp8_rowwise_torch":
            mode = "fp8_rowwise"
        if mode not in ("int8_rowwise", "fp8_rowwise"):
            raise ValueError(mode)
        xq, sa = quantize_rows(x, mode)
        if mode == "int8_rowwise":
            acc = _gemm.int8_gemm_acc(xq, qw.q).float()
        else:   # the reference's _scaled_mm with unit scales and a bf16 result (kernels.py:131-133)
            m, n = xq.shape[0], qw.q.shape[0]
            one = torch.ones(max(m, n), device=x.device, dtype=torch.float32)
            acc = _gemm.fp8_gemm(xq, one[:m], qw.q, one[:n]).float()
        return (acc * sa * qw.scale).to(x.dtype)
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
    raise ValueError(mode)
