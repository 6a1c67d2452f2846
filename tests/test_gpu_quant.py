"""GPU parity of the per-token quantizers (librh3 rh3_quant_*) against the CPU oracle: bit-exact int8 /
fp8 codes and fp32 scales (SwiGLU prologue: exp-dependent, within one code)."""
import numpy as np
import pytest

from conftest import to_dev, to_np
from oracle import quant as oq
from oracle.numerics import f32_to_bf16

pytestmark = pytest.mark.gpu


def _bf(a):
    return f32_to_bf16(np.asarray(a, np.float32))


def _quant(x_t, fp8=False):
    from rapid_h3 import quant
    return quant.quant_rows(x_t) if fp8 else quant.quant_rows_i8(x_t)


def test_quant_rows_golden(dev, golden):
    g = golden("quant_rows")
    x = to_dev(g["x"], dev)
    q, s = _quant(x)
    assert np.array_equal(to_np(q), g["q_i8"])
    assert np.array_equal(to_np(s), g["s_i8"])
    q, s = _quant(x, fp8=True)
    assert np.array_equal(to_np(q), g["q_fp8"])
    assert np.array_equal(to_np(s), g["s_fp8"])


@pytest.mark.parametrize("m,k", [(1, 8), (7, 520), (33, 1024), (5, 8192), (9, 9216), (130, 3072), (3, 4104), (2, 12296),
                                 (4, 16384)])
def test_quant_rows_shapes(dev, m, k):
    rng = np.random.default_rng(m * 131 + k)
    x = _bf(rng.standard_normal((m, k)) * np.exp(rng.standard_normal((1, k))))
    xt = to_dev(x, dev)
    for fp8 in (False, True):
        q, s = _quant(xt, fp8)
        eq, es = oq.quantize_rows(x, "fp8_rowwise" if fp8 else "int8_rowwise")
        assert np.array_equal(to_np(q), eq), (m, k, fp8)
        assert np.array_equal(to_np(s), es), (m, k, fp8)


def test_quant_rows_strided(dev):
    import torch
    rng = np.random.default_rng(5)
    x = _bf(rng.standard_normal((40, 1040)))
    xt = to_dev(x, dev)[:, 8:1032]          # row stride 1040, 16-byte aligned start
    assert xt.stride(0) == 1040
    q, s = _quant(xt)
    eq, es = oq.quantize_rows(x[:, 8:1032], "int8_rowwise")
    assert np.array_equal(to_np(q), eq) and np.array_equal(to_np(s), es)
    with pytest.raises(RuntimeError):
        _quant(to_dev(x, dev)[:, 4:1028])   # 8-byte aligned start is refused, not mis-read
    del torch


def test_norm_mod_golden(dev, golden):
    import torch
    from rapid_h3 import quant
    g = golden("norm_mod")
    x = to_dev(g["x"], dev)
    w = to_dev(g["w"], dev)
    idx = to_dev(g["idx"], dev)
    eps = float(g["eps"])
    for sh, sc, eq, es, wt in ((g["shift"], g["scale"], g["q_f32"], g["s_f32"], w),
                               (g["shift_bf"], g["scale_bf"], g["q_bf"], g["s_bf"], w),
                               (g["shift"], g["scale"], g["q_now"], g["s_now"], None)):
        q, s = quant.norm_mod_quant_rows_i8(x, wt, eps, idx, to_dev(sh, dev), to_dev(sc, dev))
        assert np.array_equal(to_np(q), eq)
        assert np.array_equal(to_np(s), es)
    del torch


@pytest.mark.parametrize("m,k", [(1, 8), (7, 520), (33, 1032), (5, 3080), (70, 3072), (3, 5000), (2, 6144), (9, 6152)])
def test_norm_mod_shapes(dev, m, k):
    """Ragged K (a partial last 512-column chunk), M not a multiple of the rows a workgroup takes, and a padded
    output whose padding bytes must stay untouched."""
    import torch
    from rapid_h3 import _native as nat
    rng = np.random.default_rng(m * 977 + k)
    x = _bf(rng.standard_normal((m, k)) * np.exp(rng.standard_normal((1, k))))
    w = _bf(1.0 + 0.1 * rng.standard_normal(k))
    idx = rng.integers(0, 3, m).astype(np.int32)
    sh = (0.2 * rng.standard_normal((3, k))).astype(np.float32)
    sc = (0.3 * rng.standard_normal((3, k))).astype(np.float32)
    xt, it = to_dev(x, dev), to_dev(idx, dev)
    for tab_bf in (False, True):
        shv, scv = (_bf(sh), _bf(sc)) if tab_bf else (sh, sc)
        st, ct = to_dev(shv, dev), to_dev(scv, dev)
        for wt in (w, None):
            eq, es = oq.norm_mod_quant_rows_i8(x, wt, 1e-6, idx, shv, scv)
            ldq = k + 24
            q = torch.full((m, ldq), 77, dtype=torch.int8, device=dev)
            s = torch.empty(m, 1, dtype=torch.float32, device=dev)
            wd = None if wt is None else to_dev(wt, dev)
            nat.call("rh3_quant_norm_mod_i8", nat.ptr(xt), k, m, k, nat.ptr(wd), 1e-6, nat.ptr(it), nat.ptr(st),
                     nat.ptr(ct), nat.RH3_DTYPE_BF16 if tab_bf else nat.RH3_DTYPE_F32, k, nat.ptr(q), ldq, nat.ptr(s),
                     nat.stream(xt.device))
            qn = to_np(q)
            assert np.array_equal(qn[:, :k], eq), (m, k, tab_bf, wt is None)
            assert np.array_equal(to_np(s), es), (m, k, tab_bf, wt is None)
            assert (qn[:, k:] == 77).all(), (m, k, tab_bf, wt is None)
    del torch


@pytest.mark.parametrize("k", [64, 3072])
def test_norm_mod_many_groups(dev, k):
    """Segments of 4099 tokens on alternating table rows (row groups straddle segment ends, so a workgroup's staged
    row is not every token's), scattered tokens of a fourth row, and more workgroups than the GPU holds at once."""
    from rapid_h3 import quant
    m = 90001 if k == 64 else 40003
    rng = np.random.default_rng(k)
    x = _bf(rng.standard_normal((m, k)))
    idx = ((np.arange(m) // 4099) % 3).astype(np.int32)
    idx[rng.integers(0, m, 200)] = 3
    sh = (0.2 * rng.standard_normal((4, k))).astype(np.float32)
    sc = (0.3 * rng.standard_normal((4, k))).astype(np.float32)
    w = _bf(1.0 + 0.1 * rng.standard_normal(k))
    q, s = quant.norm_mod_quant_rows_i8(to_dev(x, dev), to_dev(w, dev), 1e-6, to_dev(idx, dev), to_dev(sh, dev),
                                        to_dev(sc, dev))
    eq, es = oq.norm_mod_quant_rows_i8(x, w, 1e-6, idx, sh, sc)
    assert np.array_equal(to_np(q), eq)
    assert np.array_equal(to_np(s), es)


def test_heads_golden(dev, golden):
    from rapid_h3 import quant
    g = golden("heads_swiglu")
    o = to_dev(g["o"], dev)
    q, s = quant.heads_quant_rows_i8(o)
    assert np.array_equal(to_np(q), g["q"]) and np.array_equal(to_np(s), g["s"])
    # a strided head-major view: [1, H, S, D] buffer read through o[0]
    big = to_dev(np.concatenate([g["o"], g["o"]], axis=1), dev)[:, 5:5 + g["o"].shape[1]]
    q2, s2 = quant.heads_quant_rows_i8(big)
    eq, es = oq.heads_quant_rows_i8(np.concatenate([g["o"], g["o"]], axis=1)[:, 5:5 + g["o"].shape[1]])
    assert np.array_equal(to_np(q2), eq) and np.array_equal(to_np(s2), es)


def test_swiglu_quant_golden(dev, golden):
    from rapid_h3 import quant
    g = golden("heads_swiglu")
    q, s = quant.swiglu_quant_rows_i8(to_dev(g["g"], dev))
    qn, sn = to_np(q), to_np(s)
    # exp is not correctly rounded on either side: scales within 1e-6, codes within one step on < 1 %
    assert np.allclose(sn, g["s_sw"], rtol=1e-6, atol=0)
    d = np.abs(qn.astype(np.int32) - g["q_sw"].astype(np.int32))
    assert d.max() <= 1 and (d > 0).mean() < 0.01


def test_quant_full_size_properties(dev):
    """C2 activation X [145152, 3072]: oracle bit-exact on 2048 sampled rows, size-independent
    properties (row absmax code 127, |x - q s| <= s/2) on every row."""
    import torch
    m, k = 145152, 3072
    gen = torch.Generator(device="cpu").manual_seed(0)
    x = torch.randn(m, k, generator=gen, dtype=torch.float32)
    x[:, torch.randperm(k, generator=gen)[:31]] *= 20
    xb = x.to(torch.bfloat16)
    del x
    xt = xb.to(dev)
    q, s = _quant(xt)
    rows = np.sort(np.random.default_rng(1).choice(m, 2048, replace=False))
    xr = xb[rows].view(torch.int16).numpy().view(np.uint16)
    eq, es = oq.quantize_rows(xr, "int8_rowwise")
    assert np.array_equal(to_np(q[torch.from_numpy(rows).to(dev)]), eq)
    assert np.array_equal(to_np(s[torch.from_numpy(rows).to(dev)]), es)
    assert int(q.abs().amax(dim=1).min()) == 127
    # q * s and the difference each round once in fp32: allow s * 2^-14 over the exact s / 2 bound
    err = (xt.float() - q.float() * s).abs()
    assert bool((err <= s * (0.5 + 2 ** -14)).all())
