"""CPU tests that pin the oracle (oracle/) independently of its own formulas.

The reference holds no golden tensors for this path (its tests are torch.equal checks between CUDA
kernels), so each oracle function is pinned by something it does not share code with:
  * torch's CPU kernels for the same operations (bf16 / e4m3fn casts, division + round, _int_mm,
    addcmul_, silu, scaled_dot_product_attention);
  * closed forms and invariants (absmax code 127, |x - q s| <= s/2, ties to even, zero rows, RoPE
    at angle 0, rotation preserves pair norms, softmax shift invariance under K smoothing);
  * brute-force scalar loops on tiny inputs (the stated reduction orders).
A planted mistake (dropped term, wrong index, transposed operand, wrong rounding) fails at least one.
"""
import math
import struct

import numpy as np
import pytest
import torch

from oracle import attn as oa
from oracle import gemm as og
from oracle import quant as oq
from oracle.numerics import bf16_to_f32, f32_to_bf16, f32_to_fp8_e4m3, fp8_e4m3_to_f32, round_bf16


def t_bf16(u16):
    return torch.from_numpy(np.ascontiguousarray(u16).view(np.int16)).view(torch.bfloat16)


def np_bf16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def f32(x):
    """Round a Python float to fp32 (double rounding is exact for +,-,*,/ of fp32 operands)."""
    return struct.unpack("f", struct.pack("f", x))[0]


def rb(x):
    """Round a Python float (an fp32 value) to bf16, as a Python float."""
    return float(round_bf16(np.array([x], np.float32))[0])


# ----------------------------------------------------------------------------- number formats
def test_bf16_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 10 ** rng.uniform(-30, 30, 100000),
                        np.array([0.0, -0.0, np.inf, -np.inf, 1e-45, 3.4e38], np.float32)]).astype(np.float32)
    ours = f32_to_bf16(x)
    theirs = np_bf16(torch.from_numpy(x).to(torch.bfloat16))
    assert np.array_equal(ours, theirs)
    assert np.array_equal(bf16_to_f32(ours), t_bf16(ours).float().numpy())


def test_fp8_matches_torch_exhaustive():
    # every bf16 value in [-448, 448] plus random fp32 values: RNE with subnormals, as torch casts
    allb = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    v = bf16_to_f32(allb)
    v = v[np.isfinite(v) & (np.abs(v) <= 448)]
    rng = np.random.default_rng(1)
    r = (rng.uniform(-448, 448, 200000) * 10 ** rng.uniform(-6, 0, 200000)).astype(np.float32)
    x = np.concatenate([v, r]).astype(np.float32)
    ours = f32_to_fp8_e4m3(x)
    theirs = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, theirs)
    codes = np.arange(256, dtype=np.uint8)
    dec = fp8_e4m3_to_f32(codes)
    tdec = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    ok = ~np.isnan(tdec)
    assert np.array_equal(dec[ok], tdec[ok]) and np.isnan(dec[~ok]).all()
    with pytest.raises(ValueError):
        f32_to_fp8_e4m3(np.array([449.0], np.float32))


# ----------------------------------------------------------------------------- quantizers
def _torch_quant_rows(xb, fp8):
    """kernels.quantize_rows (kernels.py:75-82) in torch CPU ops."""
    x = t_bf16(xb)
    amax = x.abs().amax(dim=-1, keepdim=True).float()
    if fp8:
        s = (amax / 448.0).clamp_min(1e-12)
        return (x.float() / s).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8).numpy(), s.numpy()
    s = (amax / 127.0).clamp_min(1e-12)
    return (x.float() / s).round().clamp(-127, 127).to(torch.int8).numpy(), s.numpy()


@pytest.mark.parametrize("fp8", [False, True])
def test_quantize_rows_matches_torch(fp8, golden):
    g = golden("quant_rows")
    q, s = oq.quantize_rows(g["x"], "fp8_rowwise" if fp8 else "int8_rowwise")
    tq, ts = _torch_quant_rows(g["x"], fp8)
    assert np.array_equal(q, tq) and np.array_equal(s, ts)
    assert np.array_equal(q, g["q_fp8" if fp8 else "q_i8"]) and np.array_equal(s, g["s_fp8" if fp8 else "s_i8"])


def test_quantize_rows_invariants(golden):
    x = bf16_to_f32(golden("quant_rows")["x"])
    q, s = oq.quantize_rows(f32_to_bf16(x))
    nz = np.abs(x).max(axis=1) > 0
    assert (np.abs(q[nz]).max(axis=1) == 127).all()
    assert np.all(np.abs(x - q * s) <= s * (0.5 + 2 ** -14))
    assert s[3, 0] == np.float32(1e-12) and not q[3].any()          # zero row
    # row 5: s = 127 / 127 = 1 exactly, so x / s = x and x.5 ties go to even
    assert s[5, 0] == 1.0
    assert list(q[5, 1:9]) == [0, 2, 2, 0, -2, -2, 126, -126]


def test_quantize_rows_bruteforce():
    rng = np.random.default_rng(2)
    x = f32_to_bf16(rng.standard_normal((3, 24)).astype(np.float32) * 5)
    q, s = oq.quantize_rows(x)
    for i in range(3):
        row = [float(v) for v in bf16_to_f32(x[i])]
        amax = max(abs(v) for v in row)
        si = max(f32(amax / 127.0), f32(1e-12))
        assert s[i, 0] == np.float32(si)
        for j, v in enumerate(row):
            t = f32(v / si)
            n = math.floor(t)
            r = n + 1 if (t - n > 0.5 or (t - n == 0.5 and n % 2)) else n
            assert q[i, j] == max(-127, min(127, r))


def test_quantize_weight_layout():
    rng = np.random.default_rng(3)
    w = f32_to_bf16((0.02 * rng.standard_normal((40, 64))).astype(np.float32))
    q, s = oq.quantize_weight(w, "int8_rowwise")
    assert q.shape == (40, 64) and s.shape == (1, 40)
    tw = t_bf16(w).float()
    ts = (tw.abs().amax(dim=1, keepdim=True) / 127.0).clamp_min(1e-12)
    assert np.array_equal(q, (tw / ts).round().clamp(-127, 127).to(torch.int8).numpy())
    assert np.array_equal(s, ts.t().contiguous().numpy())


def test_sumsq_order_and_value():
    rng = np.random.default_rng(4)
    v = round_bf16(rng.standard_normal((5, 1300)).astype(np.float32))
    ss = oq.sumsq_rows(v)
    exact = (v.astype(np.float64) ** 2).sum(axis=1)
    assert np.allclose(ss, exact, rtol=1e-6)
    # the stated order, as scalar loops: lane l owns 512 j + 8 l + e, then a butterfly 32..1
    for i in range(2):
        lane = [0.0] * 64
        for j in range(3):
            for ln in range(64):
                for e in range(8):
                    c = 512 * j + 8 * ln + e
                    xv = float(v[i, c]) if c < 1300 else 0.0
                    lane[ln] = f32(lane[ln] + f32(xv * xv))
        w = 32
        while w >= 1:
            lane = [f32(lane[a] + lane[a + w]) for a in range(w)]
            w //= 2
        assert np.float32(lane[0]) == ss[i]


def test_norm_mod_closed_forms():
    rng = np.random.default_rng(5)
    m, k = 6, 1024
    x = f32_to_bf16((rng.standard_normal((m, k)) * 3 + 1).astype(np.float32))
    idx = np.zeros(m, np.int32)
    zero = np.zeros((1, k), np.float32)
    v = oq.norm_mod(x, None, 0.0, idx, zero, zero)
    assert np.allclose(np.sqrt((v.astype(np.float64) ** 2).mean(axis=1)), 1.0, atol=1e-5)
    # modulation: (1 + scale) multiplies, shift adds, per table row idx[m]
    tabs = np.stack([np.full(k, 0.5, np.float32), np.full(k, -0.25, np.float32)])
    idx2 = np.array([0, 1, 0, 1, 1, 0], np.int32)
    v2 = oq.norm_mod(x, None, 0.0, idx2, tabs, tabs)
    sc = tabs[idx2, :1]
    assert np.allclose(v2, v * (1 + sc) + sc, rtol=1e-6, atol=1e-6)
    # against torch rms_norm-style ops (different sum order: tolerance)
    w = f32_to_bf16((1 + 0.3 * rng.standard_normal(k)).astype(np.float32))
    tx = t_bf16(x).float()
    ref = tx * torch.rsqrt(tx.pow(2).mean(-1, keepdim=True) + 1e-6) * t_bf16(w).float()
    v3 = oq.norm_mod(x, w, 1e-6, idx, zero, zero)
    assert np.allclose(v3, ref.numpy(), rtol=1e-5, atol=1e-5)


def test_heads_and_swiglu_layout():
    o = np.arange(3 * 5 * 128, dtype=np.float32).reshape(3, 5, 128)
    r = oq.heads_to_rows(o)
    for m in range(5):
        for c in (0, 127, 128, 300, 383):
            assert r[m, c] == o[c // 128, m, c % 128]
    rng = np.random.default_rng(6)
    g = f32_to_bf16((2 * rng.standard_normal((4, 64))).astype(np.float32))
    tg = t_bf16(g).float()
    ref = torch.nn.functional.silu(tg[:, :32]) * tg[:, 32:]
    v = oq.silu_mul(bf16_to_f32(g)[:, :32], bf16_to_f32(g)[:, 32:])
    assert np.allclose(v, ref.numpy(), rtol=1e-6, atol=1e-7)


def test_convrot_orthonormal():
    h = oq.regular_hadamard(256)
    assert np.allclose(h @ h.T, np.eye(256), atol=1e-12)
    assert np.allclose(np.abs(h), 1 / 16)
    x = np.random.default_rng(7).standard_normal((3, 512)).astype(np.float32)
    y = oq.convrot(x)
    assert np.allclose(np.linalg.norm(y.reshape(-1, 256), axis=1), np.linalg.norm(x.reshape(-1, 256), axis=1),
                       rtol=1e-5)


def _bf16_wide(rng, shape, lo=-20, hi=20):
    """bf16-representable values with exponents spread over 2^lo .. 2^hi (random signs)."""
    m = rng.integers(128, 256, size=shape).astype(np.float64) / 128.0
    e = rng.integers(lo, hi, size=shape)
    sg = rng.choice([-1.0, 1.0], size=shape)
    return (sg * m * np.exp2(e)).astype(np.float32)


def test_h64_is_the_exact_dot_product():
    """The staged float64 H64 equals the exact rational dot products with H64 (brute force in
    fractions.Fraction), for bf16 inputs spread over 2^40 of magnitude."""
    from fractions import Fraction
    rng = np.random.default_rng(11)
    x = _bf16_wide(rng, (6, 64))
    h = np.rint(oq.regular_hadamard(64) * 8).astype(np.int64)          # +-1 entries
    got = oq.h64_unnormalized(x)
    for r in range(x.shape[0]):
        xf = [Fraction(float(v)) for v in x[r]]
        for j in range(64):
            exact = sum((int(h[j, i]) * xf[i] for i in range(64)), Fraction(0))
            assert Fraction(float(got[r, j])) == exact


def test_rot_rows_bruteforce_and_closed_form():
    """rot_rows against (a) a scalar restatement of triton_fp8._rot256 from its parts -- bf16 rounding,
    z_k = fp32(exact dot with H64/8), the fp32 combine in the order of triton_fp8.py:109-113 -- built from
    Fraction sums and np.float32 scalar arithmetic, and (b) the float64 closed form bf16(v) @ blockdiag(H256)^T
    within fp32 rounding."""
    from fractions import Fraction
    rng = np.random.default_rng(12)
    v = (rng.standard_normal((3, 512)) * np.exp(rng.standard_normal((1, 512)))).astype(np.float32)
    y = oq.rot_rows(v)
    xb = bf16_to_f32(f32_to_bf16(v))
    h = np.rint(oq.regular_hadamard(64) * 8).astype(np.int64)
    f = np.float32
    for r in range(3):
        for g in range(2):
            z = np.zeros((4, 64), np.float32)
            for k in range(4):
                xs = [Fraction(float(t)) for t in xb[r, 256 * g + 64 * k: 256 * g + 64 * (k + 1)]]
                for j in range(64):
                    z[k, j] = f(float(sum((int(h[j, i]) * xs[i] for i in range(64)), Fraction(0)) / 8))
            for j in range(64):
                z0, z1, z2, z3 = (f(z[k, j]) for k in range(4))
                ref = [(((z0 + z1) + z2) - z3) * f(0.5), (((z0 + z1) - z2) + z3) * f(0.5),
                       (((z0 - z1) + z2) + z3) * f(0.5), (((z1 + z2) + z3) - z0) * f(0.5)]
                for k in range(4):
                    assert y[r, 256 * g + 64 * k + j] == ref[k]
    exact = xb.astype(np.float64).reshape(-1, 256) @ oq.regular_hadamard(256).T
    err = np.abs(y.reshape(-1, 256) - exact)
    assert (err <= 4 * 2.0 ** -24 * np.abs(exact).max(axis=1, keepdims=True)).all()


def test_rot_quant_known_answers():
    """Zero row -> s = 1e-12, q = 0; one-hot e_j -> y = column j of blockdiag(H256), all |y| = 1/16, codes
    +-127 with the column's signs; codes use the Triton form rint(clamp(y * (1/s))) (triton_fp8.py:96-99)."""
    x = np.zeros((2, 512), np.float32)
    x[1, 256 + 77] = 3.0
    q, s = oq.rot_quantize(x)
    assert s[0, 0] == np.float32(1e-12) and not q[0].any()
    col = np.sign(oq.regular_hadamard(256)[:, 77])
    assert np.array_equal(q[1, 256:], (127 * col).astype(np.int8)) and not q[1, :256].any()
    assert s[1, 0] == np.float32(np.float32(3.0 / 16) / np.float32(127))
    # invariants on random rows: |q| <= 127, the row max code is 127, s * 127 == amax(|y|) to fp32
    rng = np.random.default_rng(13)
    v = (rng.standard_normal((5, 1024)) * 4).astype(np.float32)
    q, s = oq.rot_quantize(v)
    y = oq.rot_rows(v)
    assert (np.abs(q.astype(np.int32)).max(axis=1) == 127).all()
    assert np.array_equal(s[:, 0], np.maximum(np.abs(y).max(axis=1) / np.float32(127), np.float32(1e-12)))
    assert (np.abs(y - q * s) <= s * 0.5000001).all()


def test_convrot_exact_and_weight_rot():
    """convrot (staged, exact, rounded once) equals the float64 matmul closed form for bf16 and fp32 inputs,
    and quantize_weight(int8_rot) is quantize_rows of it with the IEEE quotient (kernels.py:62-71)."""
    rng = np.random.default_rng(14)
    wb = f32_to_bf16(_bf16_wide(rng, (7, 768), -12, 4))
    assert np.array_equal(oq.convrot(wb), oq.convrot_matmul(wb))
    wf = (0.02 * rng.standard_normal((5, 512))).astype(np.float32)
    assert np.array_equal(oq.convrot(wf), oq.convrot_matmul(wf))
    q, s = oq.quantize_weight(wb, "int8_rot")
    q2, s2 = oq.quantize_rows(oq.convrot_matmul(wb), "int8_rowwise")
    assert np.array_equal(q, q2) and np.array_equal(s, s2.T)
    t = torch.from_numpy(oq.convrot(wb))
    st = (t.abs().amax(dim=1, keepdim=True) / 127.0).clamp_min(1e-12)
    qt = (t / st).round().clamp(-127, 127).to(torch.int8)             # kernels.py:69-71 in torch
    assert np.array_equal(q, qt.numpy())


# ----------------------------------------------------------------------------- GEMM
def test_int8_acc_matches_int_mm_and_bruteforce():
    rng = np.random.default_rng(8)
    a = rng.integers(-127, 128, (33, 128), dtype=np.int8)
    b = rng.integers(-127, 128, (40, 128), dtype=np.int8)
    acc = og.int8_acc(a, b)
    assert np.array_equal(acc, torch._int_mm(torch.from_numpy(a), torch.from_numpy(b).t().contiguous()).numpy())
    for i, j in ((0, 0), (32, 39), (5, 17)):
        assert acc[i, j] == sum(int(a[i, t]) * int(b[j, t]) for t in range(128))
    big = np.full((2, 8192), 127, np.int8)
    assert og.int8_acc(big, -big)[0, 0] == -8192 * 127 * 127


def test_gemm_epilogues_match_torch(golden):
    g = golden("gemm")
    acc = torch.from_numpy(g["acc"])
    xs, ws = torch.from_numpy(g["xs"]), torch.from_numpy(g["ws"])
    y = acc.float() * xs * ws                                   # kernels.py:137
    assert np.array_equal(og.int8_gemm(g["xq"], g["xs"], g["wq"], g["ws"]), np_bf16(y.to(torch.bfloat16)))
    yb = y + t_bf16(g["bias"]).float()
    assert np.array_equal(g["out_bias"], np_bf16(yb.to(torch.bfloat16)))
    r = t_bf16(g["resid"]).clone()
    r.addcmul_(y.to(torch.bfloat16), t_bf16(g["gate"]))          # ComfyUI _mod_gate semantics
    assert np.array_equal(g["gated"], np_bf16(r))


def test_gated_rows_matches_torch_gather(golden):
    """Per-token gate rows: torch's addcmul_ with the gate table gathered by row index (_mod_gate of tensor rows);
    a table whose rows are all the segment's row reduces to the per-segment epilogue."""
    g = golden("gemm")
    m, n = g["resid"].shape
    rng = np.random.default_rng(5)
    tab = f32_to_bf16(rng.standard_normal((5, n)).astype(np.float32))
    rows = rng.integers(0, 5, m)
    y = (torch.from_numpy(g["acc"]).float() * torch.from_numpy(g["xs"]) * torch.from_numpy(g["ws"])).to(torch.bfloat16)
    r = t_bf16(g["resid"]).clone()
    r.addcmul_(y, t_bf16(tab)[torch.from_numpy(rows)])
    got = og.int8_gemm_gated_residual_rows(g["xq"], g["xs"], g["wq"], g["ws"], tab, rows, g["resid"])
    assert np.array_equal(got, np_bf16(r))
    one = np.broadcast_to(g["gate"].reshape(1, -1), (3, n))
    assert np.array_equal(og.int8_gemm_gated_residual_rows(g["xq"], g["xs"], g["wq"], g["ws"], one, np.full(m, 1),
                                                           g["resid"]), g["gated"])


def test_swiglu_perm_and_epilogue(golden):
    p = og.swiglu_perm(32)
    assert sorted(p) == list(range(32))
    for j in range(4):
        assert list(p[8 * j:8 * j + 4]) == [4 * j + i for i in range(4)]
        assert list(p[8 * j + 4:8 * j + 8]) == [16 + 4 * j + i for i in range(4)]
    g = golden("gemm")
    perm = g["perm"]
    y = og.int8_gemm(g["xq"], g["xs"], g["w1q"], g["w1s"])      # unpermuted [gate | up]
    gt, ut = t_bf16(y).float().chunk(2, dim=1)
    ref = np_bf16((gt * torch.sigmoid(gt) * ut).to(torch.bfloat16))  # bench/swiglu_epi_test.py:28-35
    d = np.abs(bf16_to_f32(g["h"]).astype(np.float64) - bf16_to_f32(ref))
    assert (d > 0).mean() < 0.01 and np.all(d <= np.abs(bf16_to_f32(ref)) * 2 ** -7 + 1e-30)
    assert np.array_equal(og.swiglu_from_interleaved(y[:, perm]), g["h"])


def test_fp8_gemm_against_torch(golden):
    g = golden("gemm")
    a = torch.from_numpy(g["fq"]).view(torch.float8_e4m3fn).float()
    b = torch.from_numpy(g["fwq"]).view(torch.float8_e4m3fn).float()
    y = (a.double() @ b.double().t()).float() * torch.from_numpy(g["fs"]) * torch.from_numpy(g["fws"])
    assert np.array_equal(g["fout"], np_bf16(y.to(torch.bfloat16)))


# ----------------------------------------------------------------------------- attention
def test_block_quant_invariants():
    rng = np.random.default_rng(9)
    x = rng.standard_normal((300, 2, 128)).astype(np.float32)
    x[200:] *= 10
    codes, sc = oa.block_quant(x)
    assert codes.shape == (2, 384, 128) and sc.shape == (2, 3)
    assert not codes[:, 300:].any()                            # padding rows
    for h in range(2):
        for b in range(3):
            blk = x[b * 128:min(300, (b + 1) * 128), h]
            assert sc[h, b] == np.float32(np.float32(np.abs(blk).max()) / np.float32(127))
            assert np.abs(codes[h, b * 128:b * 128 + len(blk)]).max() == 127
            assert np.all(np.abs(blk - codes[h, b * 128:b * 128 + len(blk)] * sc[h, b]) <= sc[h, b] * 0.5001)
    # emulation form (bench/attn_emulate.py:10-18): q8(x, dim=1, group=128) on one head
    t = torch.from_numpy(x[:, 0])
    a = t.abs().amax(dim=1, keepdim=True)
    a = torch.nn.functional.pad(a, (0, 0, 0, (-a.shape[0]) % 128))
    a = a.view(-1, 128, 1).amax(1, keepdim=True).expand(-1, 128, 1).reshape(-1, 1)[:300]
    s2 = a.clamp_min(1e-8) / 127
    assert np.array_equal(codes[0, :300], (t / s2).round().clamp(-127, 127).to(torch.int8).numpy())


def test_kmean_closed_form():
    k = np.zeros((500, 2, 128), np.float32)
    k[:, 0] = 1.5
    k[:, 1, :] = np.arange(500, dtype=np.float32)[:, None]
    km = oa.kmean(f32_to_bf16(k))
    assert np.all(km[0] == 1.5) and np.all(km[1] == np.float32(249.5))


def test_rms_rope_pins():
    rng = np.random.default_rng(10)
    s, h = 7, 3
    x = f32_to_bf16(rng.standard_normal((s, h, 128)).astype(np.float32) * 4)
    w = f32_to_bf16((1 + 0.3 * rng.standard_normal(128)).astype(np.float32))
    eps = 1e-5
    # angle 0 -> plain RMSNorm (bf16((r x) w))
    tab0 = f32_to_bf16(oa.rope_table(np.zeros(s), rot=96))
    y0 = oa.rms_rope(x, tab0, w, eps)
    xf = t_bf16(x).float()
    ref = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)) * t_bf16(w).float()
    assert np.allclose(y0, ref.to(torch.bfloat16).float().numpy(), rtol=2 ** -7, atol=1e-6)
    # rotation preserves each (i, i + 48) pair norm and leaves channels >= 96 alone
    tab = f32_to_bf16(oa.rope_table(np.arange(s) * 3.7, rot=96))
    y = oa.rms_rope(x, tab, w, eps)
    assert np.array_equal(y[..., 96:], y0[..., 96:])
    n0 = np.hypot(y0[..., :48], y0[..., 48:96])
    n1 = np.hypot(y[..., :48], y[..., 48:96])
    assert np.allclose(n0, n1, rtol=0.02, atol=1e-3)
    # the stated order on one row, as scalar loops
    row = [float(v) for v in bf16_to_f32(x[2, 1])]
    lanes = []
    for ln in range(16):
        a = 0.0
        for e in range(8):
            a = f32(a + f32(row[8 * ln + e] * row[8 * ln + e]))
        lanes.append(a)
    for wd in (8, 4, 2, 1):
        lanes = [f32(lanes[i] + lanes[i + wd]) for i in range(wd)]
    r = f32(1.0 / f32(math.sqrt(f32(f32(lanes[0] / 128.0) + f32(eps)))))
    wf = [float(v) for v in bf16_to_f32(w)]
    yb = [rb(f32(f32(r * row[d]) * wf[d])) for d in range(128)]
    tb = bf16_to_f32(tab[2])
    for i in (0, 17, 47):
        a, b = yb[i], yb[i + 48]
        o1 = rb(f32(f32(a * float(tb[i, 0, 0])) + f32(b * float(tb[i, 0, 1]))))
        o2 = rb(f32(f32(a * float(tb[i, 1, 0])) + f32(b * float(tb[i, 1, 1]))))
        assert y[2, 1, i] == o1 and y[2, 1, i + 48] == o2


def test_attention_oracles_agree_with_sdpa():
    rng = np.random.default_rng(11)
    s, h = 200, 2
    q = f32_to_bf16(rng.standard_normal((s, h, 128)).astype(np.float32))
    k = f32_to_bf16((rng.standard_normal((s, h, 128)) + 2 * rng.standard_normal((1, h, 128))).astype(np.float32))
    v = f32_to_bf16(rng.standard_normal((s, h, 128)).astype(np.float32))
    ex = oa.attention_exact(q, k, v, 128 ** -0.5)
    tq, tk, tv = (t_bf16(a).double().permute(1, 0, 2) for a in (q, k, v))
    sd = torch.nn.functional.scaled_dot_product_attention(tq[None], tk[None], tv[None])[0].permute(1, 0, 2)
    assert np.allclose(ex, sd.numpy(), atol=1e-5)
    # K smoothing is exact for softmax: subtracting kmean shifts every logit of a query equally
    km = oa.kmean(k)
    ksm = (bf16_to_f32(k) - km[None]).astype(np.float32)
    assert np.allclose(oa.attention_exact(q, ksm, v, 128 ** -0.5), ex, atol=1e-5)
    # the int8 pipeline stays within the reference's observed error band of the exact result
    q8, qs, k8, ks, _ = oa.prepass(q, k)
    out = oa.attention_from_codes(q8, qs, k8, ks, v, 128 ** -0.5)[:s]
    assert og.rel_l2(out, ex) < 0.03
    # and smoothing matters: without it the per-block K scale spans the offset, error grows
    q8n, qsn, k8n, ksn, _ = oa.prepass(q, k, smooth_k=False)
    outn = oa.attention_from_codes(q8n, qsn, k8n, ksn, v, 128 ** -0.5)[:s]
    assert og.rel_l2(outn, ex) > og.rel_l2(out, ex)


def test_attention_from_codes_against_sdpa_on_dequantized_codes():
    """attention_from_codes pinned to 1e-10 (float64) against torch's SDPA in float64 on the dequantized operands
    q8 * qs[block], k8 * ks[block]: three query and three key blocks of 128 tokens whose scales differ by up to 40x,
    cross-attention with a ragged key count and sampled rows, so a wrong block index (a scale taken from a neighbour
    block), a transposed operand or a dropped scale moves the result far past the bound."""
    rng = np.random.default_rng(13)
    h, sq, sk = 2, 384, 300                                    # 3 query blocks; keys 300 of 384 padded
    q8 = rng.integers(-127, 128, (h, sq, 128)).astype(np.int8)
    k8 = rng.integers(-127, 128, (h, 384, 128)).astype(np.int8)
    k8[:, sk:] = 0
    qs = np.array([[0.002, 0.02, 0.08], [0.05, 0.004, 0.01]], np.float32)
    ks = np.array([[0.001, 0.04, 0.01], [0.03, 0.002, 0.02]], np.float32)
    v = rng.standard_normal((sk, h, 128)).astype(np.float32)
    scale = 128 ** -0.5
    rows = np.array([0, 5, 127, 128, 200, 255, 256, 383])
    got = oa.attention_from_codes(q8, qs, k8, ks, v, scale, rows=rows, out_dtype=np.float64)
    qd = torch.from_numpy(q8.astype(np.float64) * np.repeat(qs, 128, axis=1)[..., None])
    kd = torch.from_numpy(k8[:, :sk].astype(np.float64) * np.repeat(ks, 128, axis=1)[:, :sk, None])
    vd = torch.from_numpy(v.astype(np.float64)).transpose(0, 1)
    ref = torch.nn.functional.scaled_dot_product_attention(qd[None], kd[None], vd[None], scale=scale)[0]  # [H, Sq, D]
    ref = ref.numpy().transpose(1, 0, 2)[rows]
    assert np.abs(got - ref).max() <= 1e-10 * np.abs(ref).max()


def test_golden_fixtures_regenerate(golden):
    """The committed fixtures are what the oracle computes today (guards silent oracle drift)."""
    g = golden("attention")
    q8, qs, k8, ks, km = oa.prepass(g["q"], g["k"])
    assert np.array_equal(q8, g["q8"]) and np.array_equal(k8, g["k8"]) and np.array_equal(km, g["kmean"])
    n = golden("norm_mod")
    q, s = oq.norm_mod_quant_rows_i8(n["x"], n["w"], float(n["eps"]), n["idx"], n["shift"], n["scale"])
    assert np.array_equal(q, n["q_f32"]) and np.array_equal(s, n["s_f32"])
    h = golden("heads_swiglu")
    q, s = oq.heads_quant_rows_i8(h["o"])
    assert np.array_equal(q, h["q"]) and np.array_equal(s, h["s"])
    r = golden("rot")
    q, s = oq.rot_quant_rows_i8(r["x"])
    assert np.array_equal(q, r["q"]) and np.array_equal(s, r["s"])
    q, s = oq.norm_mod_rot_quant_rows_i8(r["xn"], r["w"], float(r["eps"]), r["idx"], r["shift"], r["scale"])
    assert np.array_equal(q, r["qn"]) and np.array_equal(s, r["sn"])
    assert np.array_equal(oq.convrot(r["cx"]), r["cy"])
    u = golden("attention_u8")
    pp = oa.prepass_u8(u["q"], u["k"], u["v"])
    for n in ("q8", "qs", "k8", "ksb", "vinit", "v8", "vscale", "vmean"):
        assert np.array_equal(pp[n], u[n]), n
    b = golden("attention_bk")
    pp = oa.prepass_blockk(b["q"], b["k"], b["v"])
    for n in ("q8", "qs", "k8", "kbs", "vinit", "v8", "vscale", "vmean"):
        assert np.array_equal(pp[n], b[n]), n
    f = golden("attention_f8")
    pp = oa.prepass_fp8v(f["q"], f["k"], f["v"])
    for n in ("q8", "qs", "k8", "ksb", "vf8", "vscale", "vmean"):
        assert np.array_equal(pp[n], f[n]), n


# ----------------------------------------------------------------------------- production attention numerics
def _u8_inputs(seed, s=300, h=2, sk=None):
    rng = np.random.default_rng(seed)
    sk = s if sk is None else sk
    q = f32_to_bf16(rng.standard_normal((s, h, 128)).astype(np.float32))
    k = f32_to_bf16((rng.standard_normal((sk, h, 128)) + 2 * rng.standard_normal((1, h, 128))).astype(np.float32))
    v = f32_to_bf16((rng.standard_normal((sk, h, 128)) + 0.5 * rng.standard_normal((1, h, 128))).astype(np.float32))
    return q, k, v


def test_hadamard128_sylvester_closed_form():
    """Small integers keep every fp32 stage exact, so the staged transform must equal scipy's Sylvester
    matrix times x, scaled once by fp32(1/sqrt(128)); a real row agrees with the float64 product to fp32
    rounding and the transform is its own inverse."""
    from scipy.linalg import hadamard
    hm = hadamard(128).astype(np.float64)
    rng = np.random.default_rng(3)
    xi = rng.integers(-8, 9, size=(5, 128)).astype(np.float32)
    exp = ((xi.astype(np.float64) @ hm.T) * np.float64(oa.INV_SQRT128)).astype(np.float32)
    assert np.array_equal(oa.hadamard128(xi), exp)
    xr = rng.standard_normal((7, 128)).astype(np.float32)
    y = oa.hadamard128(xr)
    assert np.allclose(y, xr.astype(np.float64) @ hm.T / np.sqrt(128), rtol=0, atol=2e-6)
    assert np.allclose(oa.hadamard128(y), xr, rtol=0, atol=4e-6)


def test_token_quant_known_answers():
    """One-hot rows rotate to +-1/sqrt(128) everywhere: every code is +-127 with the signs of Sylvester
    column i; zero rows give sc = 1e-8/127 and code 0; padded rows are zero; without rotation the codes
    are torch's round(x / sc) and the absmax code is 127."""
    from scipy.linalg import hadamard
    x = np.zeros((3, 2, 128), np.float32)
    x[0, 0, 5] = 1.0
    x[2, 1, 77] = -3.0
    x[1] = np.random.default_rng(4).standard_normal((2, 128)).astype(np.float32)
    codes, sc = oa.token_quant(x, rotate=True)
    hm = hadamard(128)
    assert np.array_equal(codes[0, 0], (127 * hm[:, 5]).astype(np.int8))
    assert np.array_equal(codes[1, 2], (-127 * hm[:, 77]).astype(np.int8))
    assert sc[0, 0] == np.float32(oa.INV_SQRT128 / np.float32(127))
    assert not codes[1, 0].any() and sc[1, 0] == np.float32(np.float32(1e-8) / np.float32(127))
    assert codes.shape == (2, 128, 128) and not codes[:, 3:].any() and not sc[:, 3:].any()
    c2, s2 = oa.token_quant(x, rotate=False)
    t = torch.from_numpy(x[1, 1]).double()
    ref = (t.float() * (1.0 / torch.tensor(s2[1, 1]))).round()
    assert np.array_equal(c2[1, 1].astype(np.float32), ref.numpy()) and np.abs(c2[1, 1]).max() == 127


def test_v_int8_matches_torch():
    _, _, v = _u8_inputs(5)
    codes, sc, vm = oa.v_int8(v)
    tv = t_bf16(v).float()
    ref = ((tv - torch.from_numpy(vm)) / torch.from_numpy(sc)).round()
    assert np.array_equal(codes.astype(np.float32), ref.numpy())
    assert (np.abs(codes.astype(np.int32)).max(axis=0) == 127).all()     # the extreme deviation is +-127
    assert np.allclose(vm, bf16_to_f32(v).astype(np.float64).mean(axis=0), atol=1e-6)
    codes0, sc0, vm0 = oa.v_int8(v, smooth_v=False)
    assert not vm0.any() and np.allclose(sc0 * 127, np.abs(bf16_to_f32(v)).max(axis=0), rtol=1e-6)


def test_prepass_u8_side_records():
    q, k, v = _u8_inputs(6, s=300)
    pp = oa.prepass_u8(q, k, v)
    assert np.array_equal(pp["ksb"][:, :300, 1], (np.float32(-oa.MAGIC) * pp["ks"][:, :300]).astype(np.float32))
    assert (pp["ksb"][:, 300:, 1] == -np.inf).all() and not pp["ksb"][:, 300:, 0].any()
    vs = np.zeros((384, 2, 128), np.int64)
    vs[:300] = pp["v8"]
    for t in range(3):
        assert np.array_equal(pp["vinit"][:, t], oa.MAGIC_I + 128 * vs[128 * t:128 * t + 128].sum(axis=0))
    # K smoothing removes the per-head channel offset before the rotation
    assert np.allclose(pp["kmean"], bf16_to_f32(k).astype(np.float64).mean(axis=0), atol=1e-6)


def test_attention_u8_single_key_and_closed_form():
    """One key: P = 255, so the output is that key's dequantized V. Three tiles: the online rescaling equals
    the closed form sum_t 2^((tm_t - M) c) sum_j P_tj v_j / (same with v = 1), P_tj = rint(2^(fma(t, c,
    log2 255 - tm_t c))) against each tile's own max tm_t; the P.V integer start values are consistent."""
    q, k, v = _u8_inputs(7, s=1)
    pp = oa.prepass_u8(q, k, v)
    out = oa.attention_u8_from_codes(pp, 128 ** -0.5)[:1]
    dq = (pp["v8"].astype(np.float64) * pp["vscale"][None] + pp["vmean"][None]).astype(np.float32)
    assert np.allclose(out, dq, rtol=0, atol=1e-6)
    q, k, v = _u8_inputs(8, s=5, sk=300)
    pp = oa.prepass_u8(q, k, v)
    sl2 = np.float32(np.float32(128 ** -0.5) * np.float32(1.4426950408889634))
    out = oa.attention_u8_from_codes(pp, 128 ** -0.5)[:5]
    for h in range(2):
        acc = pp["q8"][h, :5].astype(np.int64) @ pp["k8"][h].astype(np.int64).T
        t = (((oa.MAGIC + acc) * pp["ksb"][h, :, 0][None].astype(np.float64)
              + pp["ksb"][h, :, 1][None].astype(np.float64))).astype(np.float32)
        c = (pp["qs"][h, :5] * sl2).astype(np.float32)[:, None]
        tms = [t[:, j:j + 128].max(axis=1, keepdims=True) for j in (0, 128, 256)]
        mm = np.maximum.reduce(tms)
        num = np.zeros((5, 128))
        den = np.zeros((5, 1))
        vq = np.zeros((384, 128))
        vq[:300] = pp["v8"][:, h]
        for ti, j in enumerate((0, 128, 256)):
            bb = (np.float64(-1) * tms[ti] * c + np.float64(oa.LOG2_255)).astype(np.float32)
            with np.errstate(invalid="ignore"):
                p = np.nan_to_num(np.rint(np.exp2((t[:, j:j + 128].astype(np.float64) * c + bb).astype(np.float32))))
            w = np.exp2(((tms[ti] - mm) * c).astype(np.float32).astype(np.float64))
            num += w * (p @ vq[j:j + 128])
            den += w * p.sum(axis=1, keepdims=True)
        ref = num / den * pp["vscale"][h][None] + pp["vmean"][h][None]
        assert np.allclose(out[:, h], ref, rtol=0, atol=1e-5)


def test_attention_u8_accuracy_and_bias():
    """Within the reference's error band of exact attention (its production configs measure 0.7-1.2 % on
    real q/k/v); with a text bias the output follows exact attention with + bias on the biased keys."""
    q, k, v = _u8_inputs(9)
    ex = oa.attention_exact(q, k, v, 128 ** -0.5)
    pp = oa.prepass_u8(q, k, v)
    out = oa.attention_u8_from_codes(pp, 128 ** -0.5)[:300]
    assert og.rel_l2(out, ex) < 0.03
    nb, bias = 40, 2.0
    outb = oa.attention_u8_from_codes(pp, 128 ** -0.5, nbias=nb, bias=bias)[:300]
    qf, kf, vf = (bf16_to_f32(a).astype(np.float64) for a in (q, k, v))
    exb = np.zeros_like(ex)
    for h in range(2):
        lg = qf[:, h] @ kf[:, h].T * 128 ** -0.5
        lg[:, :nb] += bias
        p = np.exp(lg - lg.max(axis=1, keepdims=True))
        exb[:, h] = (p @ vf[:, h]) / p.sum(axis=1, keepdims=True)
    assert og.rel_l2(outb, exb) < 0.03 and og.rel_l2(outb, ex) > 0.1


def test_block_quant_rot_known_answers():
    """Configs 60-61's K quantizer: one scale per (head, 128-token block). A block whose only non-zero row is
    one-hot rotates to +-1/sqrt(128): that row's codes are +-127 with the signs of Sylvester column i and the
    block's other rows are code 0 under the same scale; without rotation the codes are torch's
    round(x * (1 / sc)) with sc the block absmax / 127, and a partial last block takes its scale from its own
    rows only."""
    from scipy.linalg import hadamard
    x = np.zeros((200, 2, 128), np.float32)
    x[3, 0, 5] = 1.0
    x[140:200, 1] = np.random.default_rng(9).standard_normal((60, 128)).astype(np.float32)
    x[10, 1, 7] = 50.0
    codes, kbs = oa.block_quant_rot(x, rotate=True)
    assert codes.shape == (2, 256, 128) and kbs.shape == (2, 2)
    assert np.array_equal(codes[0, 3], (127 * hadamard(128)[:, 5]).astype(np.int8))
    assert not np.delete(codes[0, :128], 3, axis=0).any()
    assert kbs[0, 0] == np.float32(oa.INV_SQRT128 / np.float32(127))
    assert kbs[0, 1] == np.float32(np.float32(1e-8) / np.float32(127)) and not codes[0, 128:].any()
    c2, s2 = oa.block_quant_rot(x, rotate=False)
    for blk in range(2):
        t = torch.from_numpy(x[128 * blk:128 * blk + 128, 1])
        sc = (t.abs().max() / 127).float()
        assert s2[1, blk] == sc.item()
        ref = (t * (1.0 / sc)).round()
        assert np.array_equal(c2[1, 128 * blk:128 * blk + t.shape[0]].astype(np.float32), ref.numpy())
    assert c2[1, 10, 7] == 127 and not c2[1, 200:].any()


def test_prepass_blockk_operands():
    """Q per token (as the production pre-pass), K per block on K - kmean, V as the production pre-pass."""
    q, k, v = _u8_inputs(11, s=300)
    pp = oa.prepass_blockk(q, k, v)
    pu = oa.prepass_u8(q, k, v)
    for name in ("q8", "qs", "kmean", "v8", "vscale", "vmean", "vinit"):
        assert np.array_equal(pp[name], pu[name]), name
    kc, ks = oa.block_quant_rot((bf16_to_f32(k) - pu["kmean"][None]).astype(np.float32))
    assert np.array_equal(pp["k8"], kc) and np.array_equal(pp["kbs"], ks) and pp["kbs"].shape == (2, 3)


def test_attention_blockk_single_key_and_closed_form():
    """One key: its P is 255, so the output is that key's dequantized V. Three tiles (300 keys): the online
    rescaling equals the closed form sum_t 2^(tv_t - M) sum_j P_tj v_j / (same with v = 1), P_tj =
    rint(2^(fma(acc_j, cc_t, fma(-ti_t, cc_t, log2 255)))), cc_t = c * kb_t, tv_t = ti_t cc_t, keys past Sk
    excluded; the output is within the reference's error band of exact attention (and a kernel that skips the
    block scale or the pad mask is not)."""
    q, k, v = _u8_inputs(12, s=1, sk=1)
    pp = oa.prepass_blockk(q, k, v)
    out = oa.attention_blockk_from_codes(pp, 128 ** -0.5)[:1]
    dq = (pp["v8"].astype(np.float64) * pp["vscale"][None] + pp["vmean"][None]).astype(np.float32)
    assert np.allclose(out, dq, rtol=0, atol=1e-6)
    q, k, v = _u8_inputs(13, s=5, sk=300)
    pp = oa.prepass_blockk(q, k, v)
    sl2 = np.float32(np.float32(128 ** -0.5) * np.float32(1.4426950408889634))
    out = oa.attention_blockk_from_codes(pp, 128 ** -0.5)[:5]
    for h in range(2):
        acc = (pp["q8"][h, :5].astype(np.int64) @ pp["k8"][h, :300].astype(np.int64).T).astype(np.float64)
        c = (pp["qs"][h, :5] * sl2).astype(np.float32)[:, None]
        vq = pp["v8"][:, h].astype(np.float64)
        parts = []
        for t, j in enumerate((0, 128, 256)):
            a = acc[:, j:min(j + 128, 300)]
            ti = a.max(axis=1, keepdims=True)
            cc = (c * pp["kbs"][h, t]).astype(np.float32).astype(np.float64)
            bb = (-(oa.MAGIC + ti) * cc + np.float64(oa.LOG2_255)).astype(np.float32).astype(np.float64)
            p = np.rint(np.exp2(((oa.MAGIC + a) * cc + bb).astype(np.float32).astype(np.float64)))
            parts.append(((ti * cc).astype(np.float32).astype(np.float64), p, vq[j:j + a.shape[1]]))
        mm = np.maximum.reduce([tv for tv, _, _ in parts])
        num = sum(np.exp2(tv - mm) * (p @ vv) for tv, p, vv in parts)
        den = sum(np.exp2(tv - mm) * p.sum(axis=1, keepdims=True) for tv, p, _ in parts)
        ref = num / den * pp["vscale"][h][None] + pp["vmean"][h][None]
        assert np.allclose(out[:, h], ref, rtol=0, atol=1e-5)
    q, k, v = _u8_inputs(14, s=300)
    pp = oa.prepass_blockk(q, k, v)
    ex = oa.attention_exact(q, k, v, 128 ** -0.5)
    good = oa.attention_blockk_from_codes(pp, 128 ** -0.5)[:300]
    assert og.rel_l2(good, ex) < 0.03
    bad = dict(pp, kbs=np.ones_like(pp["kbs"]))
    assert og.rel_l2(oa.attention_blockk_from_codes(bad, 128 ** -0.5)[:300], ex) > 0.1
    unmasked = dict(pp, v8=np.concatenate([pp["v8"], np.zeros((84, 2, 128), np.int8)]))
    assert og.rel_l2(oa.attention_blockk_from_codes(unmasked, 128 ** -0.5)[:300], good) > 0.01


# ----------------------------------------------------------------------------- FP8 P.V (configs 50-56)
def test_v_fp8_matches_torch():
    """e4m3 V codes: torch's float8_e4m3fn cast of ((v - vmean) / vscale) * fp32(448 / 127); the extreme deviation
    of each channel lands on +-448; vscale and vmean are the int8 path's."""
    _, _, v = _u8_inputs(21)
    codes, sc, vm = oa.v_fp8(v)
    tv = t_bf16(v).float()
    x = ((tv - torch.from_numpy(vm)) / torch.from_numpy(sc)) * torch.tensor(np.float32(448.0) / np.float32(127.0))
    ref = x.clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(codes, ref)
    dec = fp8_e4m3_to_f32(codes)
    assert (np.abs(dec).max(axis=0) == 448).all()
    _, s8, m8 = oa.v_int8(v)
    assert np.array_equal(sc, s8) and np.array_equal(vm, m8)


def test_attention_fp8pv_single_key_and_closed_form():
    """One key: p = 448, so the output is that key's decoded V times vscale * 127 / 448 plus vmean. Five 64-key
    tiles: the online rescaling equals the closed form O = sum_t 2^((m_t - M) c) P8_t . V, l = sum_t 2^((m_t - M) c)
    sum p_t with m_t the running max after tile t and P8_t = e4m3(2^(fma(t, c, fma(-m_t, c, log2 448)))); within
    the FP8 error band of exact attention for 64- and 128-key tiles, and a kernel that drops the 127 / 448 factor
    is not."""
    q, k, v = _u8_inputs(22, s=1, sk=1)
    pp = oa.prepass_fp8v(q, k, v)
    out = oa.attention_fp8pv_from_codes(pp, 128 ** -0.5)[:1]
    dq = fp8_e4m3_to_f32(pp["vf8"]).astype(np.float64) * (pp["vscale"] * oa.V_FP8_UNSTRETCH)[None] + pp["vmean"][None]
    assert np.allclose(out, dq, rtol=1e-5, atol=1e-6)
    q, k, v = _u8_inputs(23, s=5, sk=300)
    pp = oa.prepass_fp8v(q, k, v)
    sl2 = np.float32(np.float32(128 ** -0.5) * np.float32(1.4426950408889634))
    out = oa.attention_fp8pv_from_codes(pp, 128 ** -0.5, tile=64)[:5]
    for h in range(2):
        acc = pp["q8"][h, :5].astype(np.int64) @ pp["k8"][h, :300].astype(np.int64).T
        t = (((oa.MAGIC + acc) * pp["ksb"][h, :300, 0][None].astype(np.float64)
              + pp["ksb"][h, :300, 1][None].astype(np.float64))).astype(np.float32)
        c = (pp["qs"][h, :5] * sl2).astype(np.float32)[:, None]
        vq = fp8_e4m3_to_f32(pp["vf8"][:, h]).astype(np.float64)
        runs, parts = -np.inf, []
        for j in range(0, 300, 64):
            tt = t[:, j:j + 64]
            runs = np.maximum(runs, tt.max(axis=1, keepdims=True))
            bb = (-runs.astype(np.float64) * c + np.float64(oa.LOG2_448)).astype(np.float32)
            p = np.exp2((tt.astype(np.float64) * c + bb).astype(np.float32).astype(np.float64)).astype(np.float32)
            p8 = fp8_e4m3_to_f32(f32_to_fp8_e4m3(np.minimum(p, np.float32(448)))).astype(np.float64)
            parts.append((runs.copy(), p8 @ vq[j:j + 64], p.astype(np.float64).sum(axis=1, keepdims=True)))
        mm = parts[-1][0]
        w = [np.exp2((r - mm).astype(np.float64) * c) for r, _, _ in parts]
        num = sum(wi * pv for wi, (_, pv, _) in zip(w, parts))
        den = sum(wi * ps for wi, (_, _, ps) in zip(w, parts))
        ref = num / den * (pp["vscale"][h] * oa.V_FP8_UNSTRETCH)[None] + pp["vmean"][h][None]
        assert np.allclose(out[:, h], ref, rtol=1e-5, atol=1e-5)
    q, k, v = _u8_inputs(24, s=300)
    pp = oa.prepass_fp8v(q, k, v)
    ex = oa.attention_exact(q, k, v, 128 ** -0.5)
    for tile in (64, 128):
        assert og.rel_l2(oa.attention_fp8pv_from_codes(pp, 128 ** -0.5, tile=tile)[:300], ex) < 0.03
    bad = dict(pp, vscale=(pp["vscale"] / oa.V_FP8_UNSTRETCH).astype(np.float32))
    assert og.rel_l2(oa.attention_fp8pv_from_codes(bad, 128 ** -0.5)[:300], ex) > 0.1


# ----------------------------------------------------------------------------- NVFP4 verification modes
def test_fake_nvfp4_known_answers():
    """With the tensor amax 2.625 = 2688 * 2^-10 every scale is exact (gs = 2^-10, the max block's e4m3 scale
    448, s = 0.4375): values on the e2m1 grid times s come back unchanged, midpoints go to the lower grid value
    (torch.bucketize with right=False), magnitudes past 6 s clamp to 6 s, a zero block stays zero (its scale
    becomes 1), the map is odd, and the grid index agrees with torch.bucketize on random inputs."""
    s = np.float32(0.4375)
    blk = np.zeros((4, 16), np.float32)
    blk[0, :8] = oq.E2M1 * s
    blk[0, 8] = np.float32(2.625)
    blk[1, :7] = ((oq.E2M1[1:] + oq.E2M1[:-1]) / 2) * s                 # the seven midpoints
    blk[1, 7] = np.float32(2.625)
    blk[3, :4] = [0.1, -0.2, 0.3, -0.05]
    out = oq.fake_nvfp4(blk)
    assert np.array_equal(out[0], blk[0])
    assert np.array_equal(out[1, :7], oq.E2M1[:7] * s)
    assert not out[2].any()
    assert np.array_equal(oq.fake_nvfp4(-blk), -out)
    rng = np.random.default_rng(31)
    x = (rng.standard_normal((64, 64)) * np.exp(rng.standard_normal((64, 1)))).astype(np.float32)
    y = oq.fake_nvfp4(x)
    t = torch.from_numpy(x).reshape(-1, 16)
    gs = (t.abs().amax() / (448.0 * 6.0)).clamp_min(1e-12)
    sb = (t.abs().amax(dim=1, keepdim=True) / 6.0 / gs).clamp(max=448.0).to(torch.float8_e4m3fn).float() * gs
    sb = torch.where(sb == 0, torch.ones_like(sb), sb)
    grid = torch.tensor(oq.E2M1)
    idx = torch.bucketize((t / sb).abs().clamp(max=6.0), (grid[1:] + grid[:-1]) / 2)
    assert np.array_equal(np.abs(y.reshape(-1, 16)), (grid[idx] * sb).numpy())
    assert np.abs(y - x).max() <= np.abs(x).max() / 6 + 1e-6            # at most one grid gap (2 s <= amax / 3)
