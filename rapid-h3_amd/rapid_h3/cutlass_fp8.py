"""Drop-in for the reference's cutlass_fp8 module (/root/reference/custom_nodes/rapid_h3/cutlass_fp8.py):
same names and signatures, backed by librh3's gfx950 GEMMs instead of a CUTLASS JIT build. `config`
arguments are accepted and ignored."""
from . import _native
from .gemm import fp8_gemm, int8_gemm, int8_gemm_gated_residual, int8_gemm_swiglu, swiglu_perm  # noqa: F401


def ext():
    """The loaded native library (the reference JIT-builds its extension here, cutlass_fp8.py:16-29)."""
    return _native.lib()


def int8_gemm_qkv_prep(xq, xs, wq, ws, tab, qw, kw, eps, heads, rotate=True):
    """qkv projection with the INT8 attention's pre-pass partly fused into the epilogue (config 3xx,
    cutlass_fp8.py:42-46): returns (qkv [M, 3*heads*128] bf16 with the q columns left unwritten, q8, qs, part)
    for attn_int8.attention_pre, with the reference's production numerics (per-token Q after the H128
    rotation). q8 / qs / part are views of one attention workspace that attention_pre continues on; part
    holds the float64 K and V statistics of this build (not the reference's fp32 [H, nchunk, 4, 128])."""
    from . import attention as _attn
    from .gemm import int8_gemm_qkv
    m = xq.shape[0]
    wsb = _attn.workspace_u8(m, m, heads, xq.device)
    out = int8_gemm_qkv(xq, xs, wq, ws, heads, wsb, 1, tab=tab, qw=qw, kw=kw, eps=eps, rotate=rotate)
    v = _attn.workspace_views_u8(wsb, m, m, heads)
    return out, v["q8"], v["qs"], v["part"]
