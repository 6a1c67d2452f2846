"""Drop-in for the reference's cutlass_fp8 module (/root/reference/custom_nodes/rapid_h3/cutlass_fp8.py):
same names and signatures, backed by librh3's gfx950 GEMMs instead of a CUTLASS JIT build. `config`
arguments are accepted and ignored."""
from . import _native
from .gemm import fp8_gemm, int8_gemm, int8_gemm_gated_residual, int8_gemm_swiglu, swiglu_perm  # noqa: F401


def ext():
    """The loaded native library (the reference JIT-builds its extension here, cutlass_fp8.py:16-29)."""
    return _native.lib()


def int8_gemm_qkv_prep(*args, **kwargs):
    """The reference's opt-in config-3xx qkv epilogue pre-pass (cutlass_fp8.py:42-46) is not part of this
    build (not wired into the reference's presets either)."""
    raise NotImplementedError("int8_gemm_qkv_prep (attention config 3xx) is not built in rapid_h3 for gfx950")
