"""Bit-level number formats for the CPU oracle: bf16 and OCP FP8 e4m3fn, stored as integer arrays.

TEST INFRASTRUCTURE ONLY. Nothing under oracle/ is part of the product: only tests/, the smoke check
in __graft_entry__.py and bench.py's CPU-baseline leg may import it, and only as the checker.

numpy has no bf16 or fp8 dtype, so tensors of those types travel as uint16 / uint8 bit patterns.
Conversions follow IEEE round-to-nearest-even, the rounding torch uses for `.to(torch.bfloat16)` and
`.to(torch.float8_e4m3fn)` (the casts in /root/reference/custom_nodes/rapid_h3/kernels.py:66-82).
"""
import numpy as np

F32 = np.float32


def bf16_to_f32(u16):
    """bf16 bit patterns (uint16) -> float32 values (exact)."""
    u16 = np.asarray(u16, dtype=np.uint16)
    return (u16.astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_bf16(x):
    """float32 -> bf16 bit patterns, round to nearest even; NaN stays a quiet NaN."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = (u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    out = r.astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        out[nan] = ((u[nan] >> np.uint64(16)) | np.uint64(0x40)).astype(np.uint16)
    return out


def round_bf16(x):
    """float32 -> float32 value of its bf16 rounding."""
    return bf16_to_f32(f32_to_bf16(x))


def fp8_e4m3_to_f32(u8):
    """OCP e4m3fn bit patterns (uint8) -> float32 (0x7F / 0xFF are NaN; no infinities)."""
    u8 = np.asarray(u8, dtype=np.uint8)
    s = np.where(u8 & 0x80, -1.0, 1.0)
    e = (u8 >> 3) & 0xF
    m = (u8 & 7).astype(np.float64)
    v = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * 2.0 ** (e.astype(np.float64) - 7.0))
    v = np.where((u8 & 0x7F) == 0x7F, np.nan, v)
    return (s * v).astype(np.float32)


def f32_to_fp8_e4m3(x):
    """float32 in [-448, 448] -> e4m3fn bit patterns, round to nearest even (callers clamp first, as
    kernels.py:67-68 and :81-82 do before the cast, so no value saturates or becomes NaN)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if np.any(np.abs(x) > 448.0):
        raise ValueError("f32_to_fp8_e4m3: clamp to +-448 before the cast")
    a = np.abs(x)
    sign = np.where(np.signbit(x), 0x80, 0).astype(np.uint32)
    # subnormal range |x| < 2^-6: code = rint(|x| * 2^9) (0..8; 8 is the smallest normal, 0x08)
    sub = np.rint(a.astype(np.float64) * 512.0).astype(np.uint32)
    # normal range: round the 23-bit mantissa to 3 bits (RNE); a carry moves into the exponent
    u = a.view(np.uint32).astype(np.uint64)
    r = u + np.uint64(0x7FFFF) + ((u >> np.uint64(20)) & np.uint64(1))
    e = (r >> np.uint64(23)).astype(np.int64) - 127
    m3 = ((r >> np.uint64(20)) & np.uint64(7)).astype(np.uint32)
    nor = (((e + 7).clip(0, 15).astype(np.uint32)) << np.uint32(3)) | m3
    code = np.where(a < 2.0 ** -6, sub, nor)
    return (code | sign).astype(np.uint8)
