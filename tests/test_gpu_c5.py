"""BASELINE config C5 at its real size: the draft-size DiT block chain (S = 36 x 34 x 59 = 72,216 tokens,
hidden 3072, 24 x 128 heads, FFN 8192, random-init weights; the reference's _fused_block,
__init__.py:207-321) and an INT8 cross-attention from those tokens to 512 bf16 text tokens.

Every stage is checked against the CPU oracle on sampled rows, fed the GPU's own output of the stage
before (as tests/test_gpu_block.py does for the whole tensor at a small size): quantizer codes and scales,
GEMM epilogues and the per-segment gated residuals bit for bit, the SwiGLU epilogue within one bf16 step,
attention within rel-L2 1e-2 of the oracle's float64 softmax on the same INT8 operands (the pre-pass
codes of the sampled query blocks bit for bit)."""
import numpy as np
import pytest

from conftest import to_dev, to_np
from oracle import attn as oa
from oracle import gemm as og
from oracle import quant as oq
from oracle.gemm import rel_l2
from oracle.numerics import bf16_to_f32, f32_to_bf16

pytestmark = pytest.mark.gpu

S, HID, HEADS, FFN, TEXT = 36 * 34 * 59, 3072, 24, 8192, 512
SEGMENTS = [(0, 30000, 0), (30000, S, 1)]


def _bf(a):
    return f32_to_bf16(np.asarray(a, np.float32))


def _weights(dev, g):
    import torch
    from rapid_h3 import gemm, kernels
    from rapid_h3.block import BlockWeights

    def randn(*shape, std=1.0):
        return (torch.randn(*shape, generator=g, device=dev) * std)

    qw = {}
    for name, n, k in (("qkv", 3 * HID, HID), ("out", HID, HID), ("fc1", 2 * FFN, HID), ("fc2", HID, FFN)):
        w = randn(n, k, std=0.02).to(torch.bfloat16)
        qw[name] = kernels.quantize_weight(w, "int8_rowwise")
        rows = torch.arange(0, n, 997, device=dev)
        eq, es = oq.quantize_weight(to_np(w[rows]))
        assert np.array_equal(to_np(qw[name].q[rows]), eq) and np.array_equal(to_np(qw[name].scale[:, rows]), es)
    perm = gemm.swiglu_perm(2 * FFN, dev)
    fc1 = kernels.QWeight(qw["fc1"].q[perm].contiguous(), qw["fc1"].scale[:, perm].contiguous())
    norms = {n: (1 + 0.3 * randn(k)).to(torch.bfloat16) for n, k in
             (("norm1", HID), ("norm2", HID), ("qn", 128), ("kn", 128))}
    w = BlockWeights(qkv=qw["qkv"], out=qw["out"], fc1_perm=fc1, fc2=qw["fc2"], norm1_w=norms["norm1"],
                     norm2_w=norms["norm2"], q_norm_w=norms["qn"], k_norm_w=norms["kn"], heads=HEADS)
    return w, qw, norms


def test_c5_draft_block_chain(dev):
    import torch
    from rapid_h3.block import fused_block
    g = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn(S, HID, generator=g, device=dev)
    x[:, torch.randperm(HID, generator=g, device=dev)[:HID // 100]] *= 20
    x = x.to(torch.bfloat16)
    x0 = to_np(x)
    w, qw, norms = _weights(dev, g)
    mod = tuple(torch.randn(2, HID, generator=g, device=dev) * 0.1 for _ in range(6))
    tab = _bf(oa.rope_table(np.arange(S) % 1999, rot=96))
    tr = {}
    out = fused_block(x, w, mod, SEGMENTS, to_dev(tab, dev).view(1, S, 1, 48, 2, 2), trace=tr, fuse_qkv=False)
    torch.cuda.synchronize()

    rows = np.sort(np.random.default_rng(5).choice(S, 256, replace=False))
    rt = torch.from_numpy(rows).to(dev)

    def T(name):
        return to_np(tr[name][rt])

    ow = {n: (to_np(q.q), to_np(q.scale)) for n, q in qw.items()}
    nn = {n: to_np(v) for n, v in norms.items()}
    md = [to_np(m) for m in mod]
    shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp = md
    idx = np.concatenate([np.full(b - a, r, np.int32) for a, b, r in SEGMENTS])
    ridx = idx[rows]

    def gated(xq, xs, wq, ws, gate, resid):
        out = resid.copy()
        for r in (0, 1):
            sel = ridx == r
            out[sel] = og.int8_gemm_gated_residual(xq[sel], xs[sel], wq, ws, _bf(gate[r]), resid[sel])
        return out

    # 1. RMSNorm + modulation quantizer
    q1, s1 = oq.norm_mod_quant_rows_i8(x0[rows], nn["norm1"], 1e-6, ridx, shift_msa, scale_msa)
    xq1, xs1 = T("xq1"), T("xs1")
    assert np.array_equal(xq1, q1) and np.array_equal(xs1, s1)
    # 2. QKV GEMM
    assert np.array_equal(T("qkv"), og.int8_gemm(xq1, xs1, *ow["qkv"]))
    # 3. attention on the GPU's qkv: the oracle pre-pass (oa.prepass's steps) for K over every token (its
    # mean and block scales span all of them) and for Q over the 128-token blocks of 64 sampled query rows,
    # whose codes and scales must match bit for bit; then those rows x 24 heads
    qkv = to_np(tr["qkv"]).reshape(S, 3, HEADS, 128)
    kf = oa.rms_rope(qkv[:, 1], tab, nn["kn"], 1e-6)
    km = (kf.astype(np.float64).sum(axis=0) / S).astype(np.float32)
    k8, ks = oa.block_quant((kf - km[None]).astype(np.float32))
    del kf
    ar = rows[::4]
    blocks = np.unique(ar // 128)
    qrows = (blocks[:, None] * 128 + np.arange(128)[None]).reshape(-1)
    qrows = qrows[qrows < S]
    q8, qs = oa.block_quant(oa.rms_rope(qkv[qrows, 0], tab[qrows], nn["qn"], 1e-6))
    g8 = to_np(tr["q8"]).reshape(HEADS, -1, 128, 128)[:, blocks].reshape(HEADS, -1, 128)
    assert np.array_equal(g8[:, :len(qrows)], q8[:, :len(qrows)])
    assert np.array_equal(to_np(tr["qs"])[:, blocks], qs)
    local = np.searchsorted(qrows, ar)                                                       # rows inside qrows
    att = oa.attention_from_codes(q8, qs, k8, ks, qkv[:, 2], 128 ** -0.5, rows=local)        # [64, H, D]
    o = to_np(tr["o"][0][:, torch.from_numpy(ar).to(dev)])                                   # [H, 64, D]
    assert rel_l2(bf16_to_f32(o).transpose(1, 0, 2), att) < 1e-2
    del qkv, q8, k8, g8
    # 4. head-major quantizer
    oq_, os_ = oq.heads_quant_rows_i8(to_np(tr["o"][0][:, rt]))
    assert np.array_equal(T("oq"), oq_) and np.array_equal(T("os"), os_)
    # 5. out-proj GEMM + gated residual per segment
    xa = T("x_attn")
    assert np.array_equal(xa, gated(T("oq"), T("os"), *ow["out"], gate_msa, x0[rows]))
    # 6. second quantizer
    q2, s2 = oq.norm_mod_quant_rows_i8(xa, nn["norm2"], 1e-6, ridx, shift_mlp, scale_mlp)
    assert np.array_equal(T("xq2"), q2) and np.array_equal(T("xs2"), s2)
    # 7. FFN-up GEMM + SwiGLU epilogue
    p = og.swiglu_perm(2 * FFN)
    h = og.int8_gemm_swiglu(q2, s2, ow["fc1"][0][p], ow["fc1"][1][:, p])
    d = np.abs(T("h").astype(np.int32) - h.astype(np.int32))
    assert d.max() <= 1 and (d > 0).mean() < 0.01
    # 8. quantizer of h
    hq, hs = oq.quantize_rows(T("h"), "int8_rowwise")
    assert np.array_equal(T("hq"), hq) and np.array_equal(T("hs"), hs)
    # 9. FFN-down GEMM + gated residual -> the block output (in place)
    assert np.array_equal(to_np(out[rt]), gated(hq, hs, *ow["fc2"], gate_mlp, xa))
    assert out.data_ptr() == x.data_ptr()


def test_c5_cross_attention_to_text(dev):
    """INT8 cross-attention of the 72,216 image tokens to 512 text tokens: the text goes through a W8A8
    K/V projection (quantizer + GEMM on the GPU), the per-block attention recipe runs with Sq != Sk."""
    import torch
    from rapid_h3 import attention, gemm, kernels, quant
    g = torch.Generator(device=dev).manual_seed(6)
    q = torch.randn(S, HEADS, 128, generator=g, device=dev).to(torch.bfloat16)
    text = torch.randn(TEXT, HID, generator=g, device=dev).to(torch.bfloat16)
    wkv = kernels.quantize_weight((torch.randn(2 * HID, HID, generator=g, device=dev) * 0.02).to(torch.bfloat16),
                                  "int8_rowwise")
    tq, ts = quant.quant_rows_i8(text)
    kv = gemm.int8_gemm(tq, ts, wkv.q, wkv.scale)
    assert np.array_equal(to_np(kv), og.int8_gemm(to_np(tq), to_np(ts), to_np(wkv.q), to_np(wkv.scale)))
    k, v = (t.view(TEXT, HEADS, 128) for t in kv.split(HID, dim=-1))
    o = attention.attention(q, k, v)
    rows = np.sort(np.random.default_rng(6).choice(S, 96, replace=False))
    qn, kn, vn = to_np(q), to_np(k), to_np(v)
    q8, qs, k8, ks, _ = oa.prepass(qn, kn)
    ref = oa.attention_from_codes(q8, qs, k8, ks, vn, 128 ** -0.5, rows=rows)
    got = bf16_to_f32(to_np(o[torch.from_numpy(rows).to(dev)]))
    assert rel_l2(got, ref) < 1e-2
    exact = oa.attention_exact(qn, kn, vn, 128 ** -0.5, rows=rows)
    assert rel_l2(got, exact) < 0.03
