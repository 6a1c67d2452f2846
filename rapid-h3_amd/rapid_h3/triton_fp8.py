"""Drop-in for the reference's triton_fp8 quantizer module (/root/reference/custom_nodes/rapid_h3/triton_fp8.py):
same names, arguments and return values ((q, s) with s [M, 1] fp32), backed by librh3's gfx950
quantizer kernels instead of Triton.

The rot_* entry points compute INT8 of the ConvRot-rotated activation (x @ blockdiag(H256)^T) on
librh3's rotation kernels (the H64 chunk products exact in float64 and rounded once, then the
reference's fp32 H4/2 combine); cfg (a Triton tile config) is accepted and ignored. convrot runs the
exact rotation on the GPU and returns x.dtype like the reference.
"""
import numpy as np
import torch

from . import quant as _q
from .quant import (heads_quant_rows_i8, norm_mod_quant_rows_i8, quant_rows, quant_rows_i8,  # noqa: F401
                    swiglu_quant_rows_i8)

FP8 = torch.float8_e4m3fn
FP8_MAX = 448.0
ROT_GROUP = 256

_RH = {}


def regular_hadamard(n, device, dtype=torch.float32):
    """ConvRot matrix: Kronecker powers of the 4x4 regular Hadamard, normalized (triton_fp8.py:70-80)."""
    key = (n, str(device), dtype)
    if key not in _RH:
        h4 = np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=np.float64)
        h = h4
        while h.shape[0] < n:
            h = np.kron(h, h4)
        _RH[key] = torch.from_numpy(h / np.sqrt(n)).to(device=device, dtype=dtype)
    return _RH[key]


def convrot(x, group=ROT_GROUP):
    """x @ blockdiag(H256)^T (triton_fp8.py:86-90), returned in x.dtype; computed on the GPU as the exact
    product rounded once to fp32 (the reference's torch fp32 matmul has no fixed summation order)."""
    if group != ROT_GROUP:
        raise ValueError(f"convrot: group {group} (only the int8_convrot group {ROT_GROUP} is built)")
    return _q.convrot_f32(x).to(x.dtype)


rotate = convrot


def rot_quant_rows_i8(x, cfg=None):
    """(q, s) of x @ blockdiag(H256)^T, per-row INT8 (triton_fp8.py:424-427)."""
    return _q.rot_quant_rows_i8(x)


def rot_quant_heads_i8(o, cfg=None):
    """Head-major attention output o [H, M, 128] -> (q, s) of the rotated per-token rows (:429-434)."""
    return _q.rot_quant_heads_i8(o)


def swiglu_rot_quant_rows_i8(x, cfg=None):
    """x [M, 2F] (gate | up) -> (q, s) of rot(silu(gate) * up) (:437-439)."""
    return _q.swiglu_rot_quant_rows_i8(x)


def norm_mod_rot_quant_rows_i8(x, weight, eps, idx, shift, scale, cfg=None):
    """RMSNorm + modulation prologue, rotation, per-row INT8 (:442-446)."""
    return _q.norm_mod_rot_quant_rows_i8(x, weight, eps, idx, shift, scale)
