"""The fused DiT block chain (rapid_h3.block.fused_block, the reference's _fused_block,
__init__.py:207-321) against the CPU oracle, stage by stage, for both recipes (int8_rowwise and the
reference's int8_rot). Each stage's oracle is fed the GPU's output of the stage before, so every
quantizer, GEMM epilogue and per-segment gated residual is checked bit for bit at its place in the
chain; attention (float64 softmax on the oracle side) is checked within rel-L2 1e-2 and the SwiGLU
epilogue within one bf16 step (exp is not correctly rounded on either side)."""
import numpy as np
import pytest

from conftest import to_dev, to_np
from oracle import attn as oa
from oracle import gemm as og
from oracle import quant as oq
from oracle.gemm import rel_l2
from oracle.numerics import bf16_to_f32, f32_to_bf16

pytestmark = pytest.mark.gpu

S, HID, HEADS, FFN, R = 600, 256, 2, 512, 2
SEGMENTS = [(0, 200, 0), (200, S, 1)]     # two modality segments with their own modulation rows


def _bf(a):
    return f32_to_bf16(np.asarray(a, np.float32))


def _setup(rng):
    x = rng.standard_normal((S, HID)).astype(np.float32)
    x[:, rng.permutation(HID)[:3]] *= 20.0
    ws = {name: _bf(0.02 * rng.standard_normal(shape)) for name, shape in
          (("qkv", (3 * HID, HID)), ("out", (HID, HID)), ("fc1", (2 * FFN, HID)), ("fc2", (HID, FFN)))}
    norms = {n: _bf(1.0 + 0.3 * rng.standard_normal(k)) for n, k in
             (("norm1", HID), ("norm2", HID), ("qn", 128), ("kn", 128))}
    mod = [(0.1 * rng.standard_normal((R, HID))).astype(np.float32) for _ in range(6)]
    tab = _bf(oa.rope_table(np.arange(S) % 53, rot=96).reshape(S, 48, 2, 2))
    return _bf(x), ws, norms, mod, tab


@pytest.mark.parametrize("recipe,fuse_qkv,tokrows", [("int8_rowwise", True, False), ("int8_rot", True, False),
                                                      ("int8_rowwise", False, False), ("int8_rowwise", False, True)])
def test_fused_block_chain(dev, recipe, fuse_qkv, tokrows):
    """tokrows: the second segment carries per-token modulation rows (a LongTensor row, the _mod_gate branch of
    __init__.py:244-245): its quantizers index the tables per token and its gated residuals run the per-row gate
    epilogue."""
    import torch
    from rapid_h3 import gemm, kernels
    from rapid_h3.block import BlockWeights, fused_block
    rng = np.random.default_rng(21 if recipe == "int8_rot" else 20)
    x0, ws, norms, mod, tab = _setup(rng)
    segments = SEGMENTS
    if tokrows:
        segments = [(0, 200, 0), (200, S, rng.integers(0, R, S - 200))]
    segs_dev = [(a, b, torch.from_numpy(r).to(dev) if isinstance(r, np.ndarray) else r) for a, b, r in segments]
    # weights: GPU quantization equals the oracle's
    qw, oqw = {}, {}
    for name, w in ws.items():
        qw[name] = kernels.quantize_weight(to_dev(w, dev), recipe)
        oqw[name] = oq.quantize_weight(w, recipe)
        assert np.array_equal(to_np(qw[name].q), oqw[name][0]) and np.array_equal(to_np(qw[name].scale),
                                                                                  oqw[name][1])
    perm = gemm.swiglu_perm(2 * FFN, dev)
    fc1 = kernels.QWeight(qw["fc1"].q[perm].contiguous(), qw["fc1"].scale[:, perm].contiguous())
    w = BlockWeights(qkv=qw["qkv"], out=qw["out"], fc1_perm=fc1, fc2=qw["fc2"], norm1_w=to_dev(norms["norm1"], dev),
                     norm2_w=to_dev(norms["norm2"], dev), q_norm_w=to_dev(norms["qn"], dev),
                     k_norm_w=to_dev(norms["kn"], dev), heads=HEADS, eps=1e-6, qk_eps=1e-6, recipe=recipe)
    modd = tuple(to_dev(m, dev) for m in mod)
    x = to_dev(x0, dev)
    tr = {}
    out = fused_block(x, w, modd, segs_dev, to_dev(tab, dev).view(1, S, 1, 48, 2, 2), trace=tr, fuse_qkv=fuse_qkv)
    T = {k: to_np(v) for k, v in tr.items()}

    rot = recipe == "int8_rot"
    norm_q = oq.norm_mod_rot_quant_rows_i8 if rot else oq.norm_mod_quant_rows_i8
    heads_q = oq.rot_quant_heads_i8 if rot else oq.heads_quant_rows_i8
    rows_q = oq.rot_quant_rows_i8 if rot else (lambda h: oq.quantize_rows(h, "int8_rowwise"))
    idx = np.concatenate([np.asarray(r, np.int32) if isinstance(r, np.ndarray) else np.full(b - a, r, np.int32)
                          for a, b, r in segments])

    def gated(xq, xs, wq, ws_, gate, resid):
        out_ = resid.copy()
        for a, b, r in segments:
            if isinstance(r, np.ndarray):
                out_[a:b] = og.int8_gemm_gated_residual_rows(xq[a:b], xs[a:b], wq, ws_, _bf(gate), r, resid[a:b])
            else:
                out_[a:b] = og.int8_gemm_gated_residual(xq[a:b], xs[a:b], wq, ws_, _bf(gate[r]), resid[a:b])
        return out_
    shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp = mod

    # 1. RMSNorm + modulation quantizer
    q1, s1 = norm_q(x0, norms["norm1"], 1e-6, idx, shift_msa, scale_msa)
    assert np.array_equal(T["xq1"], q1) and np.array_equal(T["xs1"], s1)
    # 2. QKV GEMM (the fused epilogue leaves the q columns unwritten: k and v are compared, Q via its codes)
    qkv_ref = og.int8_gemm(T["xq1"], T["xs1"], *oqw["qkv"])
    lo = HID if fuse_qkv else 0
    assert np.array_equal(T["qkv"][:, lo:], qkv_ref[:, lo:])
    # 3. q/k RMSNorm + RoPE + INT8 attention (head-major output)
    qkv = qkv_ref.reshape(S, 3, HEADS, 128)
    q8, qs, k8, ks, _ = oa.prepass(qkv[:, 0], qkv[:, 1], rr=(tab, norms["qn"], norms["kn"], 1e-6))
    assert np.array_equal(T["q8"], q8) and np.array_equal(T["qs"], qs)
    att = oa.attention_from_codes(q8, qs, k8, ks, qkv[:, 2], 128 ** -0.5)[:S]        # [S, H, D]
    o = T["o"][0]                                                                       # [H, S, D] bf16
    assert rel_l2(bf16_to_f32(o).transpose(1, 0, 2), att) < 1e-2
    # 4. head-major quantizer
    oq_, os_ = heads_q(o)
    assert np.array_equal(T["oq"], oq_) and np.array_equal(T["os"], os_)
    # 5. out-proj GEMM + gated residual per segment (gate row rounded to bf16, __init__.py:242-251)
    xa = gated(T["oq"], T["os"], *oqw["out"], gate_msa, x0)
    assert np.array_equal(T["x_attn"], xa)
    # 6. second RMSNorm + modulation quantizer
    q2, s2 = norm_q(T["x_attn"], norms["norm2"], 1e-6, idx, shift_mlp, scale_mlp)
    assert np.array_equal(T["xq2"], q2) and np.array_equal(T["xs2"], s2)
    # 7. FFN-up GEMM + SwiGLU epilogue on the permuted fc1
    p = og.swiglu_perm(2 * FFN)
    h = og.int8_gemm_swiglu(T["xq2"], T["xs2"], oqw["fc1"][0][p], oqw["fc1"][1][:, p])
    d = np.abs(T["h"].astype(np.int32) - h.astype(np.int32))
    assert d.max() <= 1 and (d > 0).mean() < 0.01
    # 8. quantizer of h
    hq, hs = rows_q(T["h"])
    assert np.array_equal(T["hq"], hq) and np.array_equal(T["hs"], hs)
    # 9. FFN-down GEMM + gated residual per segment -> the block output
    xf = gated(T["hq"], T["hs"], *oqw["fc2"], gate_mlp, T["x_attn"])
    assert np.array_equal(to_np(out), xf)
    assert out.data_ptr() == x.data_ptr()          # in place, like the reference's residual stream


@pytest.mark.parametrize("text_bias,fuse_qkv", [(None, False), ((150, 1.25), False), (None, True), ((150, 1.25), True)])
def test_fused_block_production_attention(dev, text_bias, fuse_qkv):
    """The block chain with the reference's production attention (attn_config 94, its 194 preset): the
    attention stage matches the oracle's tile-by-tile emulation on the GPU's own qkv (with and without the
    text bias), and the head-major quantizer that follows consumes it bit-exactly. fuse_qkv: the QKV GEMM's epilogue
    writes the per-token H128-rotated Q operands and the K / V statistics (the reference's config 3xx route); its
    Q codes and scales are checked bit for bit against the oracle's pre-pass of the same qkv, and its K / V columns
    against the oracle GEMM."""
    from rapid_h3 import gemm, kernels
    from rapid_h3.block import BlockWeights, fused_block
    rng = np.random.default_rng(22)
    x0, ws, norms, mod, tab = _setup(rng)
    qw = {n: kernels.quantize_weight(to_dev(w, dev), "int8_rowwise") for n, w in ws.items()}
    perm = gemm.swiglu_perm(2 * FFN, dev)
    fc1 = kernels.QWeight(qw["fc1"].q[perm].contiguous(), qw["fc1"].scale[:, perm].contiguous())
    w = BlockWeights(qkv=qw["qkv"], out=qw["out"], fc1_perm=fc1, fc2=qw["fc2"], norm1_w=to_dev(norms["norm1"], dev),
                     norm2_w=to_dev(norms["norm2"], dev), q_norm_w=to_dev(norms["qn"], dev),
                     k_norm_w=to_dev(norms["kn"], dev), heads=HEADS, eps=1e-6, qk_eps=1e-6)
    tr = {}
    fused_block(to_dev(x0, dev), w, tuple(to_dev(m, dev) for m in mod), SEGMENTS,
                to_dev(tab, dev).view(1, S, 1, 48, 2, 2), trace=tr, attn_config=94, text_bias=text_bias,
                fuse_qkv=fuse_qkv)
    T = {k: to_np(v) for k, v in tr.items()}
    qkv_ref = og.int8_gemm(T["xq1"], T["xs1"], *[o for o in (to_np(qw["qkv"].q), to_np(qw["qkv"].scale))])
    assert np.array_equal(T["qkv"][:, HID:], qkv_ref[:, HID:])
    qkv = qkv_ref.reshape(S, 3, HEADS, 128)
    pp = oa.prepass_u8(qkv[:, 0], qkv[:, 1], qkv[:, 2], rr=(tab, norms["qn"], norms["kn"], 1e-6))
    assert np.array_equal(T["q8"], pp["q8"]) and np.array_equal(T["qs"], pp["qs"])
    nb, bias = text_bias if text_bias is not None else (0, 0.0)
    att = oa.attention_u8_from_codes(pp, 128 ** -0.5, nbias=nb, bias=bias)[:S]
    o = T["o"][0]
    assert rel_l2(bf16_to_f32(o).transpose(1, 0, 2), att) < 2e-3
    oq_, os_ = oq.heads_quant_rows_i8(o)
    assert np.array_equal(T["oq"], oq_) and np.array_equal(T["os"], os_)
