"""The qkv GEMM with the attention pre-pass fused into its epilogue (rh3_gemm_i8_qkv, the reference's config 3xx:
cutlass_fp8.int8_gemm_qkv_prep + attn_int8.attention_pre): every pre-pass operand and the attention output are
the same bits as the unfused path (plain GEMM, then the pre-pass from its q, k, v), for both numerics, with and
without the RMSNorm + RoPE prologue, at token counts around the 128-token padding and the 256-row tile."""
import numpy as np
import pytest

from conftest import to_dev, to_np
from oracle import attn as oa
from oracle.numerics import f32_to_bf16

pytestmark = pytest.mark.gpu


def _case(dev, m, h, k=256, seed=0):
    import torch
    from rapid_h3 import kernels, quant
    rng = np.random.default_rng(seed + m + 7 * h)
    x = f32_to_bf16((rng.standard_normal((m, k)) * np.exp(rng.standard_normal((1, k)))).astype(np.float32))
    wt = f32_to_bf16((0.05 * rng.standard_normal((3 * h * 128, k))).astype(np.float32))
    wt[h * 128:2 * h * 128] += f32_to_bf16(np.full((h * 128, k), 0.0, np.float32))
    xq, xs = quant.quant_rows_i8(to_dev(x, dev))
    qw = kernels.quantize_weight(to_dev(wt, dev), "int8_rowwise")
    tab = to_dev(f32_to_bf16(oa.rope_table(np.arange(m) % 29, rot=96)), dev).view(1, m, 1, 48, 2, 2)
    nq = to_dev(f32_to_bf16((1.0 + 0.3 * rng.standard_normal(128)).astype(np.float32)), dev)
    nk = to_dev(f32_to_bf16((1.0 + 0.3 * rng.standard_normal(128)).astype(np.float32)), dev)
    return xq, xs, qw, tab, nq, nk


@pytest.mark.parametrize("m,h,rr", [(77, 2, True), (300, 2, True), (1000, 4, True), (300, 2, False), (512, 2, True)])
@pytest.mark.parametrize("numerics", [0, 1])
def test_qkv_epilogue_matches_unfused(dev, m, h, rr, numerics):
    import torch
    from rapid_h3 import attention, gemm
    xq, xs, qw, tab, nq, nk = _case(dev, m, h)
    plain = gemm.int8_gemm(xq, xs, qw.q, qw.scale)
    q, k, v = (t.view(m, h, 128) for t in plain.split(h * 128, dim=-1))
    wsb = (attention.workspace if numerics == 0 else attention.workspace_u8)(m, m, h, dev)
    args = dict(tab=tab, qw=nq, kw=nk, eps=1e-6) if rr else {}
    out = gemm.int8_gemm_qkv(xq, xs, qw.q, qw.scale, h, wsb, numerics, **args)
    assert torch.equal(out[:, h * 128:], plain[:, h * 128:])            # k, v columns; q is not written
    _, kf, vf = (t.view(m, h, 128) for t in out.split(h * 128, dim=-1))
    pf = attention.prepass_qkv(kf, vf, wsb, numerics, tab if rr else None, nk if rr else None, 1e-6)
    if numerics == 0:
        pu = attention.prepass(q, k, v, *((tab, nq, nk, 1e-6) if rr else ()))
        names = ("q8", "qs", "k8", "ks", "kmean", "vt")
    else:
        pu = attention.prepass_u8(q, k, v, *((tab, nq, nk, 1e-6) if rr else ()))
        names = ("q8", "qs", "k8", "ks", "ksb", "vinit", "vt", "kmean", "vscale", "vmean")
    for n in names:
        assert torch.equal(pf[n], pu[n]), n
    fwd = attention.forward if numerics == 0 else attention.forward_u8
    assert torch.equal(fwd(pf, m), fwd(pu, m))


def test_qkv_prep_reference_signature(dev):
    """cutlass_fp8.int8_gemm_qkv_prep + attn_int8.attention_pre (config 394's route) equal attention_rr with
    config 94 on the same GEMM's q, k, v."""
    import torch
    from rapid_h3 import attn_int8, cutlass_fp8, gemm
    m, h = 600, 2
    xq, xs, qw, tab, nq, nk = _case(dev, m, h, seed=3)
    out, q8, qs, part = cutlass_fp8.int8_gemm_qkv_prep(xq, xs, qw.q, qw.scale, tab, nq, nk, 1e-6, h)
    assert q8.shape == (h, 640, 128) and qs.shape == (h, 640)
    _, k, v = (t.view(m, h, 128) for t in out.split(h * 128, dim=-1))
    got = attn_int8.attention_pre(k, v, q8, qs, part, tab, nk, 1e-6, config=94)
    plain = gemm.int8_gemm(xq, xs, qw.q, qw.scale)
    pq, pk, pv = (t.view(m, h, 128) for t in plain.split(h * 128, dim=-1))
    ref = attn_int8.attention_rr(pq, pk, pv, tab, nq, nk, 1e-6, config=94)
    assert torch.equal(got, ref)


def test_qkv_rejects_odd_heads(dev):
    import torch
    from rapid_h3 import attention, gemm
    xq, xs, qw, tab, nq, nk = _case(dev, 128, 3)
    wsb = attention.workspace(128, 128, 3, dev)
    with pytest.raises(RuntimeError, match="even"):
        gemm.int8_gemm_qkv(xq, xs, qw.q, qw.scale, 3, wsb, 0)
