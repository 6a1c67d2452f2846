"""GPU parity of the ConvRot (int8_rot) quantizers (librh3 rh3_*rot*) against the CPU oracle
(oracle/quant.py rot_*): int8 codes and fp32 scales bit-exact for the plain, RMSNorm+modulation and
head-major prologues, the weight quantizer and convrot; the SwiGLU prologue within one code step (its
exp is not correctly rounded on either side). Then the drop-in surfaces (kernels.linear int8_rot,
triton_fp8.rot_*) and full-size properties."""
import numpy as np
import pytest

from conftest import to_dev, to_np
from oracle import quant as oq
from oracle.numerics import bf16_to_f32, f32_to_bf16

pytestmark = pytest.mark.gpu


def _eq(q, s, eq, es):
    qn, sn = to_np(q), to_np(s)
    assert np.array_equal(sn, es), f"scales differ in {(sn != es).sum()} rows"
    assert np.array_equal(qn, eq), f"codes differ in {(qn != eq).sum()} places"


def test_rot_quant_rows_golden(dev, golden):
    from rapid_h3 import quant
    g = golden("rot")
    for x, q, s in (("x", "q", "s"), ("x2", "q2", "s2"), ("x3", "q3", "s3")):   # K = 3072, 5376, 14336
        qq, ss = quant.rot_quant_rows_i8(to_dev(g[x], dev))
        _eq(qq, ss, g[q], g[s])


def test_rot_onehot_and_zero_rows(dev, golden):
    """Known answers: a zero row gives s = 1e-12 and q = 0; a one-hot row e_300 gives the column of
    blockdiag(H256) with |y| = 1/16 everywhere, so every code of its group is +-127 (signs of H256[:, 44])
    and the other groups are 0."""
    from rapid_h3 import quant
    g = golden("rot")
    q, s = quant.rot_quant_rows_i8(to_dev(g["x"], dev))
    q, s = to_np(q), to_np(s)
    assert s[2, 0] == np.float32(1e-12) and not q[2].any()
    h = oq.regular_hadamard(256)
    col = np.sign(h[:, 300 - 256])
    assert np.array_equal(q[4, 256:512], (127 * col).astype(np.int8))
    assert not q[4, :256].any() and not q[4, 512:].any()
    assert s[4, 0] == np.float32(np.float32(1 / 16) / np.float32(127))


def test_norm_mod_rot_golden(dev, golden):
    from rapid_h3 import quant
    g = golden("rot")
    x, w, idx = to_dev(g["xn"], dev), to_dev(g["w"], dev), to_dev(g["idx"], dev)
    q, s = quant.norm_mod_rot_quant_rows_i8(x, w, float(g["eps"]), idx, to_dev(g["shift"], dev),
                                            to_dev(g["scale"], dev))
    _eq(q, s, g["qn"], g["sn"])
    q, s = quant.norm_mod_rot_quant_rows_i8(x, w, float(g["eps"]), idx, to_dev(g["shift_bf"], dev),
                                            to_dev(g["scale_bf"], dev))
    _eq(q, s, g["qnb"], g["snb"])


def test_heads_rot_golden(dev, golden):
    from rapid_h3 import quant
    g = golden("rot")
    q, s = quant.rot_quant_heads_i8(to_dev(g["o"], dev))
    _eq(q, s, g["qh"], g["sh"])
    # a strided head-major view (token offset 3 inside a longer buffer)
    big = np.concatenate([g["o"], g["o"]], axis=1)
    q2, s2 = quant.rot_quant_heads_i8(to_dev(big, dev)[:, 3:3 + g["o"].shape[1]])
    eq, es = oq.rot_quant_heads_i8(big[:, 3:3 + g["o"].shape[1]])
    _eq(q2, s2, eq, es)


def test_swiglu_rot_golden(dev, golden):
    from rapid_h3 import quant
    g = golden("rot")
    q, s = quant.swiglu_rot_quant_rows_i8(to_dev(g["g"], dev))
    qn, sn = to_np(q), to_np(s)
    # exp is not correctly rounded on either side: scales within 1e-5, codes within one step on < 1 %
    assert np.allclose(sn, g["sg"], rtol=1e-5, atol=0)
    d = np.abs(qn.astype(np.int32) - g["qg"].astype(np.int32))
    assert d.max() <= 1 and (d > 0).mean() < 0.01


def test_weight_rot_golden(dev, golden):
    from rapid_h3 import kernels, quant
    g = golden("rot")
    q, s = quant.quantize_weight_rot(to_dev(g["wt"], dev))
    _eq(q, s.t().contiguous(), g["wq"], g["ws"])
    assert not to_np(q)[3].any() and to_np(s)[3, 0] == np.float32(1e-12)
    qw = kernels.quantize_weight(to_dev(g["wf"], dev), "int8_rot")      # fp32 weights
    _eq(qw.q, qw.scale, g["wfq"], g["wfs"])


def test_convrot_golden(dev, golden):
    import torch
    from rapid_h3 import quant, triton_fp8
    g = golden("rot")
    x = to_dev(g["cx"], dev)
    y = quant.convrot_f32(x)
    assert np.array_equal(to_np(y), g["cy"])
    yb = triton_fp8.convrot(x)                      # the reference returns x.dtype
    assert yb.dtype == torch.bfloat16 and np.array_equal(to_np(yb), f32_to_bf16(g["cy"]))
    # H256 is orthogonal: rotating twice with the transpose gives back x (through fp32 rounding)
    xf = bf16_to_f32(g["cx"])
    back = to_np(y).astype(np.float64) @ np.kron(np.eye(4), oq.regular_hadamard(256))
    assert np.abs(back - xf).max() < 1e-5


@pytest.mark.parametrize("m,k", [(1, 256), (5, 768), (130, 4096), (9, 4352), (3, 8192), (2, 8448), (4, 16384)])
def test_rot_shapes(dev, m, k):
    """Row counts around the 4-row workgroup and widths around the 64-chunk passes (1, 2 and 4 passes,
    partial last pass)."""
    from rapid_h3 import quant
    rng = np.random.default_rng(m * 131 + k)
    x = f32_to_bf16((rng.standard_normal((m, k)) * np.exp(rng.standard_normal((1, k)))).astype(np.float32))
    q, s = quant.rot_quant_rows_i8(to_dev(x, dev))
    eq, es = oq.rot_quant_rows_i8(x)
    _eq(q, s, eq, es)


def test_rot_extreme_magnitudes(dev):
    """Rows from bf16's subnormal range (2^-133) to 2^118, and a row mixing 2^-128 columns into normal ones, through
    the plain and head-major rotations: bit-exact against the oracle, which rounds each chunk value to fp32 after
    the 1/8 normalization (the kernel applies the 1/8 in the combine instead; the two agree wherever it matters:
    tiny rows sit at the 1e-12 scale floor with codes 0 and the large ones stay finite)."""
    from rapid_h3 import quant
    rng = np.random.default_rng(11)
    k = 768
    rows = [(rng.standard_normal(k) * 2.0 ** e).astype(np.float32)
            for e in (-133, -130, -126, -120, -100, -40, -36, 0, 60, 100, 118)]
    mixed = rng.standard_normal(k).astype(np.float32)
    mixed[::3] *= np.float32(2.0 ** -128)
    rows.append(mixed)
    x = f32_to_bf16(np.stack(rows))
    q, s = quant.rot_quant_rows_i8(to_dev(x, dev))
    eq, es = oq.rot_quant_rows_i8(x)
    _eq(q, s, eq, es)
    assert (np.abs(eq[5:7].astype(np.int32)).max(axis=1) > 0).all()   # the 1e-12 floor rows with nonzero codes
    o = np.ascontiguousarray(x.reshape(len(rows), k // 128, 128).transpose(1, 0, 2))
    q, s = quant.rot_quant_heads_i8(to_dev(o, dev))
    eq, es = oq.rot_quant_heads_i8(o)
    _eq(q, s, eq, es)


def test_rot_strided_rows(dev):
    from rapid_h3 import quant
    rng = np.random.default_rng(7)
    buf = f32_to_bf16(rng.standard_normal((33, 1536 + 64)).astype(np.float32))
    q, s = quant.rot_quant_rows_i8(to_dev(buf, dev)[:, 64:])
    eq, es = oq.rot_quant_rows_i8(buf[:, 64:])
    _eq(q, s, eq, es)


def test_rot_rejects(dev):
    import torch
    from rapid_h3 import quant
    x = torch.zeros(4, 300, dtype=torch.bfloat16, device=dev)
    with pytest.raises(AssertionError):
        quant.rot_quant_rows_i8(x)                  # K % 256 != 0
    with pytest.raises(RuntimeError, match="16384"):
        quant.rot_quant_rows_i8(torch.zeros(2, 16640, dtype=torch.bfloat16, device=dev))


def test_linear_int8_rot(dev):
    """kernels.linear(x, quantize_weight(w, "int8_rot"), "int8_rot") equals the oracle chain
    (rotated activation codes x rotated weight codes, the W8A8 epilogue) bit for bit, and stays within
    the rotation's quantization error of the bf16 product."""
    import torch
    from oracle import gemm as og
    from rapid_h3 import kernels
    rng = np.random.default_rng(3)
    m, n, k = 200, 264, 768
    x = np.asarray(rng.standard_normal((m, k)), np.float32)
    x[:, rng.permutation(k)[:8]] *= 20.0
    xb = f32_to_bf16(x)
    wb = f32_to_bf16((0.02 * rng.standard_normal((n, k))).astype(np.float32))
    qw = kernels.quantize_weight(to_dev(wb, dev), "int8_rot")
    y = kernels.linear(to_dev(xb, dev), qw, "int8_rot")
    assert y.dtype == torch.bfloat16 and tuple(y.shape) == (m, n)
    xq, xs = oq.rot_quant_rows_i8(xb)
    wq, ws = oq.quantize_weight(wb, "int8_rot")
    ref = og.int8_gemm(xq, xs, wq, ws)
    assert np.array_equal(to_np(y), ref)
    exact = bf16_to_f32(xb).astype(np.float64) @ bf16_to_f32(wb).astype(np.float64).T
    assert og.rel_l2(bf16_to_f32(to_np(y)), exact) < 0.02


def test_adopt_convrot(dev):
    import torch
    from rapid_h3 import kernels
    q = torch.zeros(8, 256, dtype=torch.int8, device=dev)
    s = torch.ones(8, dtype=torch.float32, device=dev)
    qw = kernels.adopt_convrot(q, s)
    assert tuple(qw.scale.shape) == (1, 8)
    with pytest.raises(ValueError):
        kernels.adopt_convrot(q, s, group=128)
    with pytest.raises(ValueError):
        kernels.adopt_convrot(q, s, transposed=True)


def test_rot_full_size_properties(dev):
    """C2 X [145152, 3072] through the RMSNorm-free plain rotation: 1024 sampled rows bit-exact, and on
    every row the code of the largest |y| is +-127 and the scale is positive."""
    import torch
    from rapid_h3 import quant
    m, k = 145152, 3072
    gen = torch.Generator(device="cpu").manual_seed(0)
    x = torch.randn(m, k, generator=gen, dtype=torch.float32)
    x[:, torch.randperm(k, generator=gen)[:31]] *= 20.0
    xb = x.to(torch.bfloat16)
    q, s = quant.rot_quant_rows_i8(xb.to(dev))
    rows = np.sort(np.random.default_rng(5).choice(m, 1024, replace=False))
    xs = xb[torch.from_numpy(rows)].view(torch.int16).numpy().view(np.uint16)
    eq, es = oq.rot_quant_rows_i8(xs)
    qn, sn = to_np(q), to_np(s)
    assert np.array_equal(qn[rows], eq) and np.array_equal(sn[rows], es)
    assert (np.abs(qn.astype(np.int32)).max(axis=1) == 127).all() and (sn > 0).all()
