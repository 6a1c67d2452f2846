"""Drop-in for the reference's triton_fp8 quantizer module (/root/reference/custom_nodes/rapid_h3/triton_fp8.py):
same names, arguments and return values ((q, s) with s [M, 1] fp32), backed by librh3's gfx950
quantizer kernels instead of Triton.

The rot_* entry points compute INT8 of the ConvRot-rotated activation (x @ blockdiag(H256)^T); the
rotation prologue is not built for gfx950 yet, so they raise NotImplementedError. The unrotated
recipe (int8_rowwise / int8_fast) uses quant_rows_i8 and the *_quant_rows_i8 prologue variants of
rapid_h3.quant.
"""
import numpy as np
import torch

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
    """x @ blockdiag(H)^T in fp32 (offline weight rotation, triton_fp8.py:86-90)."""
    m, k = x.shape
    h = regular_hadamard(group, x.device, torch.float32)
    return (x.float().reshape(-1, group) @ h.T).reshape(m, k).to(x.dtype)


rotate = convrot


def _no_rot(name):
    raise NotImplementedError(f"{name}: the ConvRot (H256) quantizer prologue is not built for gfx950 yet; "
                              "use the int8_rowwise / int8_fast recipe")


def rot_quant_rows_i8(x, cfg=None):
    _no_rot("rot_quant_rows_i8")


def rot_quant_heads_i8(o, cfg=None):
    _no_rot("rot_quant_heads_i8")


def swiglu_rot_quant_rows_i8(x, cfg=None):
    _no_rot("swiglu_rot_quant_rows_i8")


def norm_mod_rot_quant_rows_i8(x, weight, eps, idx, shift, scale, cfg=None):
    _no_rot("norm_mod_rot_quant_rows_i8")
