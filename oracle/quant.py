"""CPU restatement of the reference's activation and weight quantizers (numpy, float32 arithmetic).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's CPU baseline, as
the checker. The product path never calls it.

Semantics are the PyTorch path of the reference, which is the parity target:
  * per-token INT8   /root/reference/custom_nodes/rapid_h3/kernels.py:75-80
      s = max(amax/127, 1e-12) (fp32), q = clamp(round_half_even(fp32(x) / s), -127, 127)
  * per-token FP8    kernels.py:81-82
      s = max(amax/448, 1e-12), q = e4m3fn_RNE(clamp(x / s, -448, 448))
  * per-channel weights, int8 / fp8   kernels.py:52-72 (same, along K of each output row; scale [1, N])
  * fused prologues   triton_fp8.py:128-148 (KIND 1 SwiGLU, KIND 2 RMSNorm + modulation, KIND 3
    head-major gather), with IEEE x / s as in kernels.py rather than the Triton x * (1/s).

The RMSNorm sum of squares is order dependent. Its order here is the one the HIP kernel uses, stated
once so both sides agree (the reference pins its own Triton layout instead, triton_fp8.py:216-232):
one 64-lane wavefront per row; lane l owns columns 512*j + 8*l + e (j ascending, then e = 0..7) and
accumulates ss += x*x in fp32 from 0 (x is bf16, so x*x is exact and fma == mul+add); the 64 lane sums
are then added by a butterfly over lane distances 32, 16, 8, 4, 2, 1.
"""
import numpy as np

from .numerics import F32, bf16_to_f32, f32_to_bf16, f32_to_fp8_e4m3

I8_MAX = F32(127.0)
FP8_MAX = F32(448.0)
EPS_SCALE = F32(1e-12)


def _as_f32(x):
    x = np.asarray(x)
    return bf16_to_f32(x) if x.dtype == np.uint16 else x.astype(np.float32)


def _quant_i8(v, s):
    return np.clip(np.rint(v / s), -127, 127).astype(np.int8)


def quantize_rows(x, mode="int8_rowwise"):
    """kernels.quantize_rows (kernels.py:75-82): x [M, K] (bf16 bits or fp32) -> (q, s [M, 1] fp32).
    int8 q is np.int8; fp8 q is e4m3fn bits (np.uint8)."""
    v = _as_f32(x)
    amax = np.abs(v).max(axis=-1, keepdims=True) if v.shape[-1] else np.zeros(v.shape[:-1] + (1,), F32)
    if mode == "int8_rowwise":
        s = np.maximum(amax / I8_MAX, EPS_SCALE).astype(F32)
        return _quant_i8(v, s), s
    if mode in ("fp8_rowwise", "fp8_rowwise_torch"):
        s = np.maximum(amax / FP8_MAX, EPS_SCALE).astype(F32)
        return f32_to_fp8_e4m3(np.clip(v / s, -FP8_MAX, FP8_MAX)), s
    raise ValueError(mode)


def quantize_weight(w, mode="int8_rowwise"):
    """kernels.quantize_weight (kernels.py:52-72) for the row-wise modes: w [N, K] -> (q [N, K], scale [1, N]).
    int8_rot applies ConvRot (blockdiag H256, triton_fp8.py:86-90) before the row-wise quantization."""
    if mode == "int8_fast":
        mode = "int8_rowwise"
    v = _as_f32(w)
    if mode == "int8_rot":
        v = convrot(v)
        mode = "int8_rowwise"
    q, s = quantize_rows(v, mode)
    return q, np.ascontiguousarray(s.T)


def sumsq_rows(v):
    """Row sums of squares of v [M, K] fp32 in the wavefront order stated in the module docstring."""
    m, k = v.shape
    kp = -(-k // 512) * 512
    vp = np.zeros((m, kp), F32)
    vp[:, :k] = v
    t = vp.reshape(m, kp // 512, 64, 8)               # [row, j, lane, e]
    lane = np.zeros((m, 64), F32)
    for j in range(t.shape[1]):
        for e in range(8):
            x = t[:, j, :, e]
            lane = (lane + x * x).astype(F32)
    w = 32
    while w >= 1:
        lane = (lane[:, :w] + lane[:, w:2 * w]).astype(F32)
        w //= 2
    return lane[:, 0]


def norm_mod(x, weight, eps, idx, shift, scale):
    """RMSNorm + modulation prologue (triton_fp8.py:141-147, :165-172):
    v = ((x * rstd) * w) * (1 + scale[idx]) + shift[idx], rstd = 1 / sqrt(sumsq / K + eps), all fp32.
    weight [K] bf16 or None; idx [M] int32; shift / scale [R, K] (bf16 bits or fp32)."""
    v = _as_f32(x)
    k = v.shape[1]
    ss = sumsq_rows(v)
    rstd = (F32(1.0) / np.sqrt(ss / F32(k) + F32(eps))).astype(F32)
    y = v * rstd[:, None]
    if weight is not None:
        y = y * _as_f32(weight)[None, :]
    idx = np.asarray(idx, dtype=np.int64)
    sc = _as_f32(scale)[idx]
    sh = _as_f32(shift)[idx]
    return (y * (F32(1.0) + sc) + sh).astype(F32)


def norm_mod_quant_rows_i8(x, weight, eps, idx, shift, scale):
    """triton_fp8.norm_mod_rot_quant_rows_i8 without the rotation (the int8_rowwise recipe)."""
    return quantize_rows(norm_mod(x, weight, eps, idx, shift, scale), "int8_rowwise")


def heads_to_rows(o):
    """Head-major attention output o [H, M, 128] -> [M, H*128]: column k is head k // 128, dim k % 128
    (triton_fp8.py:133-135)."""
    h, m, d = o.shape
    return np.ascontiguousarray(np.transpose(o, (1, 0, 2)).reshape(m, h * d))


def heads_quant_rows_i8(o):
    """triton_fp8.rot_quant_heads_i8 without the rotation."""
    return quantize_rows(heads_to_rows(o), "int8_rowwise")


def silu_mul(g, u):
    """fp32 (g * sigmoid(g)) * u with sigmoid(g) = 1 / (1 + exp(-g)) (triton_fp8.py:138-139)."""
    g = g.astype(F32)
    sig = (F32(1.0) / (F32(1.0) + np.exp(-g))).astype(F32)
    return ((g * sig) * u.astype(F32)).astype(F32)


def swiglu_quant_rows_i8(x):
    """triton_fp8.swiglu_rot_quant_rows_i8 without the rotation: x [M, 2F] = [gate | up]."""
    v = _as_f32(x)
    f = v.shape[1] // 2
    return quantize_rows(silu_mul(v[:, :f], v[:, f:]), "int8_rowwise")


def regular_hadamard(n):
    """ConvRot matrix (triton_fp8.py:70-80): Kronecker powers of the 4x4 regular Hadamard, / sqrt(n)."""
    h4 = np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=np.float64)
    h = h4
    while h.shape[0] < n:
        h = np.kron(h, h4)
    return h / np.sqrt(n)


# ---------------------------------------------------------------- ConvRot (int8_rot)
# The regular H4 = J - 2P (P the anti-identity): H4 x = sum(x) - 2 reverse(x). H64 = H4 (x) H4 (x) H4 over
# the index i = 16a + 4b + c of a 64-chunk, applied as three radix-4 stages (c, then b, then a), each
# t = ((x0 + x1) + x2) + x3, y_j = t - 2 x_(3-j), in float64. With bf16 / fp32 inputs every product is
# exact and, for values within 2^38 of each other, so is every stage, which makes the result the exact
# dot product (pinned against rational arithmetic in tests/test_oracle.py); the stage order is the HIP
# kernel's (rapid-h3_amd/csrc/rot.hip), so both sides agree even where float64 would round.

def _h4_stage(d, s):
    """One radix-4 stage over indices (i, i+s, i+2s, i+3s) of the last axis (length 64), float64."""
    v = d.reshape(d.shape[:-1] + (64 // (4 * s), 4, s))
    x0, x1, x2, x3 = v[..., 0, :], v[..., 1, :], v[..., 2, :], v[..., 3, :]
    t = ((x0 + x1) + x2) + x3
    return np.stack([t - 2.0 * x3, t - 2.0 * x2, t - 2.0 * x1, t - 2.0 * x0], axis=-2).reshape(d.shape)


def h64_unnormalized(x):
    """(8 * H64) @ x over the last axis (length 64) in float64 staged butterflies."""
    d = np.asarray(x, dtype=np.float64)
    for s in (1, 4, 16):
        d = _h4_stage(d, s)
    return d


def rot_rows(v):
    """The activation rotation of triton_fp8._rot256 / _rot_wide (triton_fp8.py:102-116, :218-233) on the
    prologue values v [M, K] fp32: per 256-group, X_k = bf16(v) chunks, z_k = fp32(X_k H64^T) (the exact
    products rounded once), then y0 = ((z0 + z1) + z2 - z3) * 0.5, y1 = ((z0 + z1) - z2 + z3) * 0.5,
    y2 = ((z0 - z1) + z2 + z3) * 0.5, y3 = ((z1 + z2) + z3 - z0) * 0.5 in fp32. Returns y [M, K] fp32."""
    v = np.asarray(v, dtype=F32)
    m, k = v.shape
    assert k % 256 == 0, "ConvRot needs K % 256 == 0"
    xb = bf16_to_f32(f32_to_bf16(v)).reshape(m, k // 256, 4, 64)
    z = (h64_unnormalized(xb) * 0.125).astype(F32)
    z0, z1, z2, z3 = z[:, :, 0], z[:, :, 1], z[:, :, 2], z[:, :, 3]
    h = F32(0.5)
    y = np.stack([(((z0 + z1) + z2) - z3) * h, (((z0 + z1) - z2) + z3) * h,
                  (((z0 - z1) + z2) + z3) * h, (((z1 + z2) + z3) - z0) * h], axis=2)
    return y.astype(F32).reshape(m, k)


def rot_quantize(v):
    """Per-row INT8 of rot_rows(v) as the Triton rotation kernels quantize (triton_fp8.py:96-99, :341-351):
    s = max(amax / 127, 1e-12), q = rint(clamp(y * (1 / s), -127, 127)). -> (q [M, K] int8, s [M, 1])."""
    y = rot_rows(v)
    amax = np.abs(y).max(axis=1, keepdims=True)
    s = np.maximum(amax / I8_MAX, EPS_SCALE).astype(F32)
    inv = (F32(1.0) / s).astype(F32)
    q = np.rint(np.clip((y * inv).astype(F32), -127.0, 127.0)).astype(np.int8)
    return q, s


def rot_quant_rows_i8(x):
    """triton_fp8.rot_quant_rows_i8 (triton_fp8.py:424-427): x [M, K] bf16 bits."""
    return rot_quantize(_as_f32(x))


def norm_mod_rot_quant_rows_i8(x, weight, eps, idx, shift, scale):
    """triton_fp8.norm_mod_rot_quant_rows_i8 (triton_fp8.py:442-446)."""
    return rot_quantize(norm_mod(x, weight, eps, idx, shift, scale))


def rot_quant_heads_i8(o):
    """triton_fp8.rot_quant_heads_i8 (triton_fp8.py:429-434): o [H, M, 128] head-major."""
    return rot_quantize(_as_f32(heads_to_rows(o)))


def swiglu_rot_quant_rows_i8(x):
    """triton_fp8.swiglu_rot_quant_rows_i8 (triton_fp8.py:437-439): x [M, 2F] = [gate | up]."""
    v = _as_f32(x)
    f = v.shape[1] // 2
    return rot_quantize(silu_mul(v[:, :f], v[:, f:]))


def convrot(x, group=256):
    """x @ blockdiag(H256)^T (triton_fp8.py:86-90) as the exact product rounded once to fp32: H256 =
    (H4 (x) H64) / 16, the H64 stages of h64_unnormalized then the chunk stage t = ((d0 + d1) + d2) + d3,
    y_k = t - 2 d_(3-k), all float64 (the HIP kernel's order)."""
    assert group == 256
    v = _as_f32(x)
    m, k = v.shape
    d = h64_unnormalized(v.reshape(m, k // 256, 4, 64))
    d0, d1, d2, d3 = d[:, :, 0], d[:, :, 1], d[:, :, 2], d[:, :, 3]
    t = ((d0 + d1) + d2) + d3
    y = np.stack([t - 2.0 * d3, t - 2.0 * d2, t - 2.0 * d1, t - 2.0 * d0], axis=2) * 0.0625
    return y.astype(F32).reshape(m, k)


def convrot_matmul(x, group=256):
    """The closed form x @ blockdiag(H)^T in float64 (BLAS order), rounded once to fp32 (a checker)."""
    v = _as_f32(x).astype(np.float64)
    m, k = v.shape
    h = regular_hadamard(group)
    return (v.reshape(-1, group) @ h.T).reshape(m, k).astype(F32)


E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], F32)   # kernels.py:35


def fake_nvfp4(x):
    """kernels.fake_nvfp4 (kernels.py:38-49), the NVFP4 round trip of the verification modes nvfp4_fake /
    nvfp4_rot_fake: x fp32 (last dim a multiple of 16) -> fp32. One fp32 scale per tensor gs = max(amax / (448 *
    6), 1e-12); per 16-element block s = e4m3(min(fp32(fp32(block amax / 6) / gs), 448)) * gs (1 where that is 0);
    q = x / s rounded to the e2m1 grid {0, .5, 1, 1.5, 2, 3, 4, 6} by torch.bucketize over the midpoints
    (right=False: a tie goes to the lower value), result = grid * sign(q) * s."""
    from .numerics import fp8_e4m3_to_f32
    x = np.asarray(x, F32)
    t = x.reshape(-1, 16)
    gs = np.maximum((np.abs(t).max() / F32(448.0 * 6.0)).astype(F32), EPS_SCALE).astype(F32)
    bm = np.abs(t).max(axis=1, keepdims=True)
    sb = np.minimum(((bm / F32(6.0)).astype(F32) / gs).astype(F32), FP8_MAX).astype(F32)
    s = (fp8_e4m3_to_f32(f32_to_fp8_e4m3(sb)) * gs).astype(F32)
    s = np.where(s == 0, F32(1.0), s).astype(F32)
    q = (t / s).astype(F32)
    mid = ((E2M1[1:] + E2M1[:-1]) / F32(2.0)).astype(F32)
    idx = np.searchsorted(mid, np.minimum(np.abs(q), F32(6.0)), side="left")
    return ((E2M1[idx] * np.sign(q)).astype(F32) * s).astype(F32).reshape(x.shape)
