"""rapid_h3 — MI355X (gfx950) HIP implementation of Rapid-H3's per-step DiT hot path.

Implementation modules: quant (per-token quantizers), gemm (W8A8 / FP8 GEMMs with fused epilogues),
attention (INT8 flash attention), block (the fused DiT block chain). Drop-in modules keep the
reference's import names and signatures (/root/reference/custom_nodes/rapid_h3/): kernels,
cutlass_fp8, triton_fp8, attn_int8. All compute goes through librh3.so (_native); there is no
fallback path.
"""
from . import _native  # noqa: F401

__all__ = ["quant", "gemm", "attention", "kernels", "cutlass_fp8", "triton_fp8", "attn_int8"]
