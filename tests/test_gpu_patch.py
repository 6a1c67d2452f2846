"""The model patch (rapid_h3.patch) on a 2-block H3-shaped stub on the GPU: the patched blocks run the fused INT8
chain with the cached QWeights (bit-identical to block.fused_block on weights quantized with
kernels.quantize_weight(w, "int8_rot"), itself checked against the oracle stage by stage in test_gpu_block), and
the fused MLP (attention linears left in bf16) bit-exact against the oracle's int8_rot chain:
rot-quant + GEMM for fc1, the SwiGLU rot-quantizer, the fc2 GEMM."""
import numpy as np
import pytest
import torch
from torch import nn

from conftest import to_np
from oracle import gemm as og
from oracle import quant as oq
from oracle.numerics import bf16_to_f32, f32_to_bf16

pytestmark = pytest.mark.gpu

S, HID, HEADS, FFN, R = 600, 256, 2, 512, 2


class _Norm(nn.Module):
    def __init__(self, n, g):
        super().__init__()
        self.weight = nn.Parameter((1 + 0.3 * torch.randn(n, generator=g)).to(torch.bfloat16))
        self.eps = 1e-6


def _lin(i, o, g):
    lin = nn.Linear(i, o, bias=False)
    lin.weight = nn.Parameter((0.02 * torch.randn(o, i, generator=g)).to(torch.bfloat16))
    return lin


class _Attn(nn.Module):
    def __init__(self, g):
        super().__init__()
        self.heads, self.head_dim = HEADS, 128
        self.qkv_proj, self.out_proj = _lin(HID, 3 * HID, g), _lin(HID, HID, g)
        self.q_norm, self.k_norm = _Norm(128, g), _Norm(128, g)


class _MLP(nn.Module):
    def __init__(self, g):
        super().__init__()
        self.fc1, self.fc2 = _lin(HID, 2 * FFN, g), _lin(FFN, HID, g)


class _Block(nn.Module):
    def __init__(self, g):
        super().__init__()
        self.norm1, self.norm2 = _Norm(HID, g), _Norm(HID, g)
        self.attn, self.mlp = _Attn(g), _MLP(g)
        self.mods = nn.Parameter(0.1 * torch.randn(6, R, HID, generator=g))

    def adaln_proj(self, t_emb):
        return tuple(self.mods[i] for i in range(6))

    def forward(self, x, t_emb, mod_segments, rope_freqs, transformer_options={}, attention=None):  # noqa: B006
        raise AssertionError("the unfused block forward is not part of this test")


class _DiT(nn.Module):
    def __init__(self, g):
        super().__init__()
        self.blocks = nn.ModuleList(_Block(g) for _ in range(2))


def _rope(dev):
    import bench                                                     # the benchmark's H3-layout RoPE table
    return bench.rope_table(S, dev)


def test_patched_blocks_run_the_fused_chain(dev):
    from rapid_h3 import gemm, kernels, patch
    from rapid_h3.block import BlockWeights, fused_block
    g = torch.Generator().manual_seed(3)
    model = _DiT(g).to(dev)
    x0 = (torch.randn(S, HID, generator=g) * torch.where(torch.rand(HID, generator=g) < 0.02, 20.0, 1.0)).to(
        torch.bfloat16).to(dev)
    segs = [(0, 200, 0), (200, S, 1)]
    tab = _rope(dev)
    p = patch.patch(model, "int8_rot", patch_id=lambda: 7)

    def run(x):
        for b in model.blocks:
            x = b(x, None, segs, tab)
        return x

    got = p.wrapper(run, x0.clone())
    got2 = p.wrapper(run, x0.clone())                               # second call: cached weights, same bits
    ref = x0.clone()
    for b in model.blocks:
        qw = {n: kernels.quantize_weight(lin.weight, "int8_rot") for n, lin in
              (("qkv", b.attn.qkv_proj), ("out", b.attn.out_proj), ("fc1", b.mlp.fc1), ("fc2", b.mlp.fc2))}
        perm = gemm.swiglu_perm(2 * FFN, dev)
        w = BlockWeights(qkv=qw["qkv"], out=qw["out"],
                         fc1_perm=kernels.QWeight(qw["fc1"].q[perm].contiguous(), qw["fc1"].scale[:, perm].contiguous()),
                         fc2=qw["fc2"], norm1_w=b.norm1.weight, norm2_w=b.norm2.weight, q_norm_w=b.attn.q_norm.weight,
                         k_norm_w=b.attn.k_norm.weight, heads=HEADS, eps=1e-6, qk_eps=1e-6, recipe="int8_rot")
        ref = fused_block(ref, w, b.adaln_proj(None), segs, tab)
    assert torch.equal(got, ref) and torch.equal(got2, ref)
    assert all("forward" not in mod.__dict__ for mod, _ in p.wrappers)


def test_fused_mlp_against_oracle(dev):
    """fc1's output bit-exact, the SwiGLU rot-quantizer within its tolerance, the fc2 GEMM bit-exact on its codes.
    exp is not correctly rounded on either side, and the prologue rounds silu(g) * u to bf16 before the H256
    rotation, so an fp32 ulp can flip a bf16 rounding and move a rotated row's absmax by ~1e-4: scales within 2e-3,
    codes within one step on < 1 %."""
    from rapid_h3 import block, patch
    g = torch.Generator().manual_seed(4)
    model = _DiT(g).to(dev)
    x = torch.randn(S, HID, generator=g).to(torch.bfloat16).to(dev)
    p = patch.patch(model, "int8_rot", targets="fc1,fc2")
    mlp = model.blocks[1].mlp
    y = p.wrapper(lambda t: mlp(t), x)
    fc1, fc2 = p.by_name["blocks.1.mlp.fc1"], p.by_name["blocks.1.mlp.fc2"]
    tr = {}
    y2 = block.fused_mlp(x, fc1, fc2, trace=tr)                     # the forward the patch installed, traced
    assert torch.equal(y, y2)
    T = {k: to_np(v) for k, v in tr.items()}
    q1, s1 = oq.quantize_weight(to_np(mlp.fc1.weight), "int8_rot")
    q2, s2 = oq.quantize_weight(to_np(mlp.fc2.weight), "int8_rot")
    xq, xs = oq.rot_quant_rows_i8(to_np(x))
    assert np.array_equal(T["h"], og.int8_gemm(xq, xs, q1, s1))     # fc1 as QuantLinear (int8_rot)
    hq, hs = oq.swiglu_rot_quant_rows_i8(T["h"])
    assert np.allclose(T["hs"], hs, rtol=2e-3, atol=0)
    d = np.abs(T["hq"].astype(np.int32) - hq.astype(np.int32))
    assert d.max() <= 1 and (d > 0).mean() < 0.01
    assert np.array_equal(to_np(y), og.int8_gemm(T["hq"], T["hs"], q2, s2))


# ---------------------------------------------------------------------------------------------------------------
# The attention route of a fused block (__init__.py:277-306, :334-349, :1023-1041): an override tagged for the fused
# RMSNorm + RoPE path (configs >= 100) runs inside the block's pre-pass; an untagged override (configs < 100, or any
# exact_rows) gets q, k after a separate RMSNorm + RoPE and decides the numerics itself.

SL = 1100                                                          # >= 1024: the override's INT8 path


class _Layout:
    def __init__(self, segments):
        self.segments, self.seq_len = segments, SL


def _route_setup(dev, seed):
    g = torch.Generator().manual_seed(seed)
    model = _DiT(g).to(dev)
    x0 = (torch.randn(SL, HID, generator=g) * torch.where(torch.rand(HID, generator=g) < 0.02, 20.0, 1.0)).to(
        torch.bfloat16).to(dev)
    import bench
    return model, x0, bench.rope_table(SL, dev)


def _spy(ov, log):
    """An untagged wrapper of an override that records what the block hands it and what it returns."""
    def spy(func, *args, **kwargs):
        out = ov(func, *args, **kwargs)
        log.append(([a.clone() for a in args[:3]], args[3], dict(kwargs), out.clone()))
        return out
    return spy


def test_untagged_override_decides_the_numerics(dev):
    """make_override(94) (untagged): the block's q, k reach the override after RMSNorm + RoPE (bit-exact against the
    oracle's rms_rope of the qkv GEMM output), in ComfyUI's [1, H, S, 128] skip_reshape convention, and the block
    continues from the override's own output, which matches the oracle's config-94 emulation. The whole patched
    block is bit-identical to the tagged route make_override(194), whose RMSNorm + RoPE runs inside the pre-pass."""
    from oracle import attn as oa
    from rapid_h3 import override, patch
    model, x0, tab = _route_setup(dev, 21)
    segs = [(0, 300, 0), (300, SL, 1)]
    p = patch.patch(model, "int8_rot")
    blk = model.blocks[0]
    log = []
    opts = {"optimized_attention_override": _spy(override.make_override(94), log)}
    got = p.wrapper(lambda x: blk(x, None, segs, tab, transformer_options=opts), x0.clone())
    (q4, k4, v4), heads, kw, out = log[0]
    assert heads == HEADS and kw["skip_reshape"] and kw["skip_output_reshape"] and kw["mask"] is None
    assert tuple(q4.shape) == (1, HEADS, SL, 128) and kw["transformer_options"] is opts
    # q, k, v are what the oracle's chain gives: the int8_rot qkv GEMM, then rms_rope on q and k
    qkv_w = p.by_name["blocks.0.attn.qkv_proj"].qweight_for()
    xq, xs = oq.norm_mod_rot_quant_rows_i8(to_np(x0), to_np(blk.norm1.weight), 1e-6, np.repeat([0, 1], [300, SL - 300]),
                                          to_np(blk.mods[0]), to_np(blk.mods[1]))
    qkv = og.int8_gemm(xq, xs, to_np(qkv_w.q), to_np(qkv_w.scale)).reshape(SL, 3, HEADS, 128)
    tb = to_np(tab).reshape(SL, 48, 2, 2)
    rq = f32_to_bf16(oa.rms_rope(qkv[:, 0], tb, to_np(blk.attn.q_norm.weight), 1e-6))
    rk = f32_to_bf16(oa.rms_rope(qkv[:, 1], tb, to_np(blk.attn.k_norm.weight), 1e-6))
    assert np.array_equal(to_np(q4[0].transpose(0, 1)), rq)
    assert np.array_equal(to_np(k4[0].transpose(0, 1)), rk)
    assert np.array_equal(to_np(v4[0].transpose(0, 1)), qkv[:, 2])
    pp = oa.prepass_u8(rq, rk, qkv[:, 2])
    rows = np.arange(0, SL, 7)
    ref = oa.attention_u8_from_codes(pp, 128 ** -0.5, rows=rows)
    o = bf16_to_f32(to_np(out[0].transpose(0, 1)[rows]))
    assert og.rel_l2(o, ref) < 2e-3
    # the tagged route (fused RMSNorm + RoPE, same config) gives the same block output bit for bit
    opts2 = {"optimized_attention_override": override.make_override(194)}
    assert override.make_override(194).rapidh3_rmsrope == 94
    got2 = p.wrapper(lambda x: blk(x, None, segs, tab, transformer_options=opts2), x0.clone())
    assert torch.equal(got, got2)


def test_exact_rows_override_through_the_block(dev):
    """make_override(194, exact_rows="text") is untagged (exact_rows needs the unfused route): the text segment's
    query rows come out as exact attention of the roped q, k (fp32, rounded once), the others as config 94."""
    from oracle import attn as oa
    from rapid_h3 import override, patch
    model, x0, tab = _route_setup(dev, 22)
    segs = [(0, 64, 0), (64, SL, 1)]
    lay = _Layout([(0, 64, "text"), (64, SL, "video")])
    ov = override.make_override(194, exact_rows="text")
    assert getattr(ov, "rapidh3_rmsrope", None) is None
    p = patch.patch(model, "int8_rot")
    blk = model.blocks[1]
    log = []
    opts = {"optimized_attention_override": _spy(ov, log), "minimax_h3_layout": lay}
    p.wrapper(lambda x: blk(x, None, segs, tab, transformer_options=opts), x0.clone())
    (q4, k4, v4), _, _, out = log[0]
    qn, kn, vn = (to_np(t[0].transpose(0, 1)) for t in (q4, k4, v4))
    ex = oa.attention_exact(qn, kn, vn, 128 ** -0.5, rows=np.arange(64))
    o = bf16_to_f32(to_np(out[0].transpose(0, 1)[:64]))
    assert og.rel_l2(o, ex) < 4e-3                                 # bf16 rounding of the output only
    rows = np.arange(64, SL, 9)
    ref = oa.attention_u8_from_codes(oa.prepass_u8(qn, kn, vn), 128 ** -0.5, rows=rows)
    assert og.rel_l2(bf16_to_f32(to_np(out[0].transpose(0, 1)[rows])), ref) < 2e-3


def test_rrcheck_override_records_equality(dev, tmp_path, monkeypatch):
    """make_override(294): tagged for the fused path with the config-2xx check, which appends one JSON record per
    block: the fused RMSNorm + RoPE pre-pass and output equal the unfused ones bit for bit."""
    import json
    from rapid_h3 import override, patch
    model, x0, tab = _route_setup(dev, 23)
    rec = tmp_path / "rr.jsonl"
    monkeypatch.setenv("RAPIDH3_RRCHECK", str(rec))
    ov = override.make_override(294)
    assert ov.rapidh3_rmsrope == 94 and ov.rapidh3_rrcheck
    p = patch.patch(model, "int8_rot")
    segs = [(0, SL, 0)]

    def run(x):
        for i, b in enumerate(model.blocks):
            x = b(x, None, segs, tab, transformer_options={"optimized_attention_override": ov, "block_index": i})
        return x

    p.wrapper(run, x0.clone())
    lines = [json.loads(s) for s in rec.read_text().splitlines()]
    assert [r["block"] for r in lines] == [0, 1]
    assert all(r["out_equal"] and r["operands_equal"] and r["max_abs_diff"] == 0.0 and r["S"] == SL for r in lines)


def test_stock_attention_for_the_unfused_route(dev):
    """patch(attention=f) with no override: the block hands f the roped q, k, v; a short sequence under a tagged
    override (S < 1024) takes the same route and the override falls through to f, as in the reference."""
    from rapid_h3 import override, patch
    model, x0, tab = _route_setup(dev, 24)
    log = []

    def stock(q, k, v, heads, **kw):
        out = override.stock_attention(q, k, v, heads, **kw)
        log.append(out)
        return out

    p = patch.patch(model, "int8_rot", attention=stock)
    blk = model.blocks[0]
    p.wrapper(lambda x: blk(x, None, [(0, SL, 0)], tab), x0.clone())
    assert len(log) == 1 and tuple(log[0].shape) == (1, HEADS, SL, 128)
    short = x0[:500].clone()
    tab_s = tab[:, :500].contiguous()
    p2 = patch.patch(model, "int8_rot", attention=stock)
    p2.wrapper(lambda x: blk(x, None, [(0, 500, 0)], tab_s,
                             transformer_options={"optimized_attention_override": override.make_override(194)}),
               short)
    assert len(log) == 2 and tuple(log[1].shape) == (1, HEADS, 500, 128)
