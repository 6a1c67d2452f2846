"""GPU parity of the production-numerics INT8 attention (librh3 rh3_*attention_u8*, the reference's configs
80-99) against the CPU oracle (oracle/attn.py prepass_u8, attention_u8_from_codes): per-token Q/K codes and
scales, the per-key (scale, bias) pairs, V codes (transposed layout), P.V accumulator starts, kmean, vscale
and vmean bit-exact; the output within rel-L2 2e-3 of the oracle's tile-by-tile emulation (the kernels'
exp2 is a hardware approximation, so an integer P next to a .5 boundary can differ by one) and within
3 % of exact attention."""
import numpy as np
import pytest

from conftest import to_dev, to_np
from oracle import attn as oa
from oracle.gemm import rel_l2
from oracle.numerics import bf16_to_f32, f32_to_bf16

pytestmark = pytest.mark.gpu

TOL = 2e-3
SC = 128 ** -0.5


def _perm_keys_u8(skp):
    """Key held at each position of the int8 V^T layout: p = 16 g + r inside a 32-key block <-> key
    8 (r / 4) + 4 g + r % 4."""
    p = np.arange(skp)
    w = p & 31
    g, r = w >> 4, w & 15
    return (p & ~31) + 8 * (r >> 2) + 4 * g + (r & 3)


def _check_pp(pp, exp, pre, s_k):
    for n in ("q8", "qs", "k8", "ks", "kmean"):
        if pre + n in exp:
            assert np.array_equal(to_np(pp[n]), exp[pre + n]), pre + n
    assert np.array_equal(to_np(pp["ksb"]), exp[pre + "ksb"]), pre + "ksb"
    vpre = "" if pre == "r" else pre
    assert np.array_equal(to_np(pp["vinit"]), exp[vpre + "vinit"]), pre + "vinit"
    assert np.array_equal(to_np(pp["vscale"]), exp[vpre + "vscale"]), pre + "vscale"
    assert np.array_equal(to_np(pp["vmean"]), exp[vpre + "vmean"]), pre + "vmean"
    vt = to_np(pp["vt"])                                          # [H, 128, Skpad] int8
    keys = _perm_keys_u8(vt.shape[2])
    vpad = np.zeros((vt.shape[2],) + exp[vpre + "v8"].shape[1:], np.int8)
    vpad[:s_k] = exp[vpre + "v8"]
    assert np.array_equal(vt, vpad[keys].transpose(1, 2, 0)), pre + "vt"


def _rr(g, dev, s):
    return to_dev(g["tab"], dev).view(1, s, 1, 48, 2, 2), to_dev(g["qw"], dev), to_dev(g["kw"], dev)


def test_u8_prepass_golden(dev, golden):
    from rapid_h3 import attention
    g = golden("attention_u8")
    q, k, v = (to_dev(g[n], dev) for n in ("q", "k", "v"))
    s = g["q"].shape[0]
    tab, qw, kw = _rr(g, dev, s)
    _check_pp(attention.prepass_u8(q, k, v), g, "", s)
    _check_pp(attention.prepass_u8(q, k, v, tab, qw, kw, 1e-5), g, "r", s)
    _check_pp(attention.prepass_u8(q, k, v, rotate=False, smooth_v=False), g, "n", s)
    pc = attention.prepass_u8(q, k[:200], v[:200])
    _check_pp(pc, g, "c", 200)
    assert np.array_equal(to_np(pc["q8"]), g["q8"]) and np.array_equal(to_np(pc["qs"]), g["qs"])


def test_ext_int8_prepass_golden(dev, golden):
    """attn_int8.ext().int8_prepass, the reference extension's verification entry (attn_int8.cu:2692-2704, called
    by _rr_check, __init__.py:342-343): the operand list [q8, qs, k8, ks, ksb, vt, vscale, vmean] bit-exact against
    the oracle, with and without the fused RMSNorm + RoPE; the default config 0 of attn_int8.attention runs the
    same production numerics."""
    from rapid_h3 import attn_int8
    g = golden("attention_u8")
    q, k, v = (to_dev(g[n], dev) for n in ("q", "k", "v"))
    s = g["q"].shape[0]
    tab, qw, kw = _rr(g, dev, s)
    ext = attn_int8.ext()
    for pre, args in (("", ()), ("r", (tab, qw, kw, 1e-5))):
        ops = ext.int8_prepass(q, k, v, *args, config=94)
        assert len(ops) == 8
        pp = dict(zip(("q8", "qs", "k8", "ks", "ksb", "vt", "vscale", "vmean"), ops))
        pp["kmean"] = None
        for n in ("q8", "qs", "k8", "ks", "ksb"):
            assert np.array_equal(to_np(pp[n]), g[pre + n]), pre + n
        vpre = ""
        assert np.array_equal(to_np(pp["vscale"]), g[vpre + "vscale"]) and np.array_equal(to_np(pp["vmean"]),
                                                                                          g[vpre + "vmean"])
        vt = to_np(pp["vt"])
        keys = _perm_keys_u8(vt.shape[2])
        vpad = np.zeros((vt.shape[2],) + g["v8"].shape[1:], np.int8)
        vpad[:s] = g["v8"]
        assert np.array_equal(vt, vpad[keys].transpose(1, 2, 0))
    got = bf16_to_f32(to_np(attn_int8.attention(q, k, v)))                 # config None -> RAPIDH3_ATTN_CONFIG / 0
    assert attn_int8.CONFIG != 0 or rel_l2(got, bf16_to_f32(g["out"])) < TOL


def test_u8_forward_golden(dev, golden):
    """Every public route to the production kernel: attention(config), attention_rr (default config 94),
    cross-attention, no rotation / no V smoothing, and the text bias."""
    import torch
    from rapid_h3 import attention, attn_int8
    g = golden("attention_u8")
    q, k, v = (to_dev(g[n], dev) for n in ("q", "k", "v"))
    s = g["q"].shape[0]
    tab, qw, kw = _rr(g, dev, s)

    def check(out, name):
        got = bf16_to_f32(to_np(out))
        ref = bf16_to_f32(g[name])
        assert rel_l2(got, ref) < TOL, (name, rel_l2(got, ref))

    check(attention.attention(q, k, v, config=80), "out")
    check(attn_int8.attention(q, k, v, config=94), "out")
    q0, k0 = q.clone(), k.clone()
    check(attention.attention_rr(q, k, v, tab, qw, kw, 1e-5), "rout")
    assert torch.equal(q, q0) and torch.equal(k, k0)
    check(attention.attention(q, k, v, config=90, rotate=False, smooth_v=False), "nout")
    check(attention.attention(q, k[:200], v[:200], config=94), "cout")
    check(attention.attention_rr_bias(q, k, v, tab, qw, kw, 1e-5, 77, 1.5), "bout")
    check(attention.attention_rr_bias(q, k, v, tab, qw, kw, 1e-5, 77, 1.5, config=90), "bout")
    # the main kernel alone on the pre-pass operands gives the same bits as the one-call path
    pp = attention.prepass_u8(q, k, v)
    a = attention.forward_u8(pp, s)
    b = attention.attention(q, k, v, config=80)
    assert torch.equal(a, b)
    # exact attention is within the quantization error
    ex = oa.attention_exact(g["q"], g["k"], g["v"], SC)
    assert rel_l2(bf16_to_f32(to_np(b)), ex) < 0.03


@pytest.mark.parametrize("sq,sk,h", [(1, 1, 1), (127, 129, 2), (256, 256, 1), (257, 600, 3), (1000, 77, 2)])
def test_u8_shapes(dev, sq, sk, h):
    """Query blocks around the 256-query workgroup and 128-token padding, key tiles around the 128-key tile
    (one partial tile, several tiles), cross-attention in both directions."""
    from rapid_h3 import attention
    rng = np.random.default_rng(sq * 7 + sk * 3 + h)
    q = f32_to_bf16(rng.standard_normal((sq, h, 128)).astype(np.float32))
    k = f32_to_bf16((rng.standard_normal((sk, h, 128)) + 2 * rng.standard_normal((1, h, 128))).astype(np.float32))
    v = f32_to_bf16(rng.standard_normal((sk, h, 128)).astype(np.float32))
    out = attention.attention(to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), config=94)
    pp = oa.prepass_u8(q, k, v)
    ref = oa.attention_u8_from_codes(pp, SC)[:sq]
    got = bf16_to_f32(to_np(out))
    assert rel_l2(got, ref) < TOL


def test_u8_strided_out_and_inputs(dev):
    """q, k, v as strided views of one qkv buffer, head-major output through out= (the block's layout)."""
    import torch
    from rapid_h3 import attention
    rng = np.random.default_rng(12)
    s, h = 700, 3
    buf = f32_to_bf16(rng.standard_normal((s, 3 * h * 128)).astype(np.float32))
    bt = to_dev(buf, dev)
    q, k, v = (t.view(s, h, 128) for t in bt.split(h * 128, dim=-1))
    o = torch.empty(1, h, s, 128, dtype=torch.bfloat16, device=dev)
    attention.attention(q, k, v, config=94, out=o[0].transpose(0, 1))
    b = buf.reshape(s, 3, h, 128)
    ref = oa.attention_u8_from_codes(oa.prepass_u8(b[:, 0], b[:, 1], b[:, 2]), SC)[:s]
    assert rel_l2(bf16_to_f32(to_np(o[0].transpose(0, 1))), ref) < TOL


def test_u8_routing_and_errors(dev):
    import torch
    from rapid_h3 import attention
    x = torch.zeros(300, 1, 128, dtype=torch.bfloat16, device=dev)
    tab = torch.zeros(1, 300, 1, 48, 2, 2, dtype=torch.bfloat16, device=dev)
    w = torch.ones(128, dtype=torch.bfloat16, device=dev)
    for c in (57, 59, 62, 69, 361):    # not in the reference's kernel dispatch
        with pytest.raises(NotImplementedError):
            attention.attention(x, x, x, config=c)
    with pytest.raises(RuntimeError, match="config 94 or 90"):
        attention.attention_rr_bias(x, x, x, tab, w, w, 1e-5, 5, 1.0, config=80)
    with pytest.raises(RuntimeError, match="nbias"):
        attention.attention_rr_bias(x, x, x, tab, w, w, 1e-5, 301, 1.0)
    # all-zero inputs: uniform softmax over zero V
    for c in (94, 60, 50):
        out = attention.attention(x, x, x, config=c)
        assert not torch.isnan(out.float()).any() and not out.float().abs().max().item(), c


def test_u8_full_size_sampled(dev):
    """S = 145,152 (1134 key tiles) with 2 heads: codes, scales, pairs and V codes of head 1 bit-exact;
    output on 48 sampled query rows within tolerance of the emulation and within 3 % of exact attention."""
    import torch
    from rapid_h3 import attention
    s, h = 145152, 2
    gen = torch.Generator(device="cpu").manual_seed(1)
    q = torch.randn(s, h, 128, generator=gen).to(torch.bfloat16)
    k = (torch.randn(s, h, 128, generator=gen) + 2.0 * torch.randn(1, h, 128, generator=gen)).to(torch.bfloat16)
    v = torch.randn(s, h, 128, generator=gen).to(torch.bfloat16)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    pp = attention.prepass_u8(qd, kd, vd)
    out = attention.attention(qd, kd, vd, config=94)
    rows = np.sort(np.random.default_rng(3).choice(s, 48, replace=False))
    qn, kn, vn = (t[:, 1:2].contiguous().view(torch.int16).numpy().view(np.uint16) for t in (q, k, v))
    ep = oa.prepass_u8(qn, kn, vn)
    for n in ("q8", "qs", "k8", "ks", "ksb", "vinit", "kmean", "vscale", "vmean"):
        assert np.array_equal(to_np(pp[n][1:2]), ep[n]), n
    ref = oa.attention_u8_from_codes(ep, SC, rows=rows)[:, 0]
    got = bf16_to_f32(to_np(out[torch.from_numpy(rows).to(dev), 1]))
    assert rel_l2(got, ref) < TOL
    exact = oa.attention_exact(qn, kn, vn, SC, rows=rows)[:, 0]
    assert rel_l2(got, exact) < 0.03


# ----------------------------------------------------------------------------- configs 60-61 (per-block K)
def _check_bk(pp, exp, pre, s_k):
    for n in ("q8", "qs", "k8", "kbs", "kmean"):
        if pre + n in exp:
            assert np.array_equal(to_np(pp[n]), exp[pre + n]), pre + n
    kb = exp[pre + "kbs"]
    assert np.array_equal(to_np(pp["side_kb"]), kb), pre + "side kb"
    for n in ("vinit", "vscale", "vmean"):
        assert np.array_equal(to_np(pp[n]), exp[pre + n]), pre + n
    vt = to_np(pp["vt"])
    keys = _perm_keys_u8(vt.shape[2])
    vpad = np.zeros((vt.shape[2],) + exp[pre + "v8"].shape[1:], np.int8)
    vpad[:s_k] = exp[pre + "v8"]
    assert np.array_equal(vt, vpad[keys].transpose(1, 2, 0)), pre + "vt"


def test_bk_prepass_golden(dev, golden):
    """Configs 60-61's pre-pass: per-token Q codes and scales, per-block K codes and scales (also in the side
    records the main kernel reads), V codes, accumulator starts, kmean, vscale, vmean bit-exact."""
    from rapid_h3 import attention
    g = golden("attention_bk")
    q, k, v = (to_dev(g[n], dev) for n in ("q", "k", "v"))
    s = g["q"].shape[0]
    _check_bk(attention.prepass_bk(q, k, v), g, "", s)
    _check_bk(attention.prepass_bk(q, k, v, rotate=False, smooth_v=False), g, "n", s)
    _check_bk(attention.prepass_bk(q, k[:200], v[:200]), g, "c", 200)


def test_bk_forward_golden(dev, golden):
    """attention(config=60 / 61), the drop-in module, no rotation / no V smoothing, cross-attention, and the main
    kernel alone; within 3 % of exact attention; configs 60-69 refuse the fused RMSNorm + RoPE path."""
    import torch
    from rapid_h3 import attention, attn_int8
    g = golden("attention_bk")
    q, k, v = (to_dev(g[n], dev) for n in ("q", "k", "v"))
    s = g["q"].shape[0]

    def check(out, name):
        got = bf16_to_f32(to_np(out))
        ref = bf16_to_f32(g[name])
        assert rel_l2(got, ref) < TOL, (name, rel_l2(got, ref))

    check(attention.attention(q, k, v, config=60), "out")
    check(attn_int8.attention(q, k, v, config=61), "out")
    check(attention.attention(q, k, v, config=60, rotate=False, smooth_v=False), "nout")
    check(attention.attention(q, k[:200], v[:200], config=61), "cout")
    pp = attention.prepass_bk(q, k, v)
    assert torch.equal(attention.forward_bk(pp, s), attention.attention(q, k, v, config=60))
    ex = oa.attention_exact(g["q"], g["k"], g["v"], SC)
    assert rel_l2(bf16_to_f32(to_np(attention.attention(q, k, v, config=60))), ex) < 0.03
    tab = torch.zeros(1, s, 1, 48, 2, 2, dtype=torch.bfloat16, device=dev)
    w = torch.ones(128, dtype=torch.bfloat16, device=dev)
    with pytest.raises(RuntimeError, match="no fused rms/rope"):
        attention.attention_rr(q, k, v, tab, w, w, 1e-5, config=60)
    with pytest.raises(NotImplementedError):
        attention.attention(q, k, v, config=62)


@pytest.mark.parametrize("sq,sk,h", [(1, 1, 1), (127, 129, 2), (256, 256, 1), (257, 600, 3), (1000, 77, 2)])
def test_bk_shapes(dev, sq, sk, h):
    """Query blocks around the 256-query workgroup, key tiles around the 128-key tile (the in-kernel pad mask of
    a ragged last tile), cross-attention in both directions."""
    from rapid_h3 import attention
    rng = np.random.default_rng(sq * 5 + sk * 11 + h)
    q = f32_to_bf16(rng.standard_normal((sq, h, 128)).astype(np.float32))
    k = f32_to_bf16((rng.standard_normal((sk, h, 128)) + 2 * rng.standard_normal((1, h, 128))).astype(np.float32))
    v = f32_to_bf16(rng.standard_normal((sk, h, 128)).astype(np.float32))
    out = attention.attention(to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), config=60)
    ref = oa.attention_blockk_from_codes(oa.prepass_blockk(q, k, v), SC)[:sq]
    assert rel_l2(bf16_to_f32(to_np(out)), ref) < TOL


# ----------------------------------------------------------------------------- configs 50-56 (FP8 P.V)
def _perm_keys_f8(skp):
    """Key held at each position of the e4m3 V^T layout: p = 32 g + 16 h + r inside a 64-key chunk <-> key
    32 h + 8 (r / 4) + 4 g + r % 4."""
    p = np.arange(skp)
    w = p & 63
    g, hh, r = w >> 5, (w >> 4) & 1, w & 15
    return (p & ~63) + 32 * hh + 8 * (r >> 2) + 4 * g + (r & 3)


def _check_f8(pp, exp, pre, s_k):
    for n in ("q8", "qs", "k8", "ks", "kmean"):
        if pre + n in exp:
            assert np.array_equal(to_np(pp[n]), exp[pre + n]), pre + n
    assert np.array_equal(to_np(pp["ksb"]), exp[pre + "ksb"]), pre + "ksb"
    for n in ("vscale", "vmean"):
        assert np.array_equal(to_np(pp[n]), exp[pre + n]), pre + n
    vt = to_np(pp["vt"])                                           # [H, 128, Skpad] e4m3 codes
    keys = _perm_keys_f8(vt.shape[2])
    vpad = np.zeros((vt.shape[2],) + exp[pre + "vf8"].shape[1:], np.uint8)
    vpad[:s_k] = exp[pre + "vf8"]
    assert np.array_equal(vt, vpad[keys].transpose(1, 2, 0)), pre + "vt"


def test_f8_prepass_golden(dev, golden):
    """Configs 50-56's pre-pass: Q / K codes, scales and per-key pairs as the production numerics, e4m3 V codes
    (on the hardware's v_cvt_pk_fp8_f32) in the 64-key-chunk layout, vscale, vmean, kmean bit-exact."""
    from rapid_h3 import attention
    g = golden("attention_f8")
    q, k, v = (to_dev(g[n], dev) for n in ("q", "k", "v"))
    s = g["q"].shape[0]
    tab, qw, kw = _rr(g, dev, s)
    _check_f8(attention.prepass_f8(q, k, v), g, "", s)
    _check_f8(attention.prepass_f8(q, k, v, tab, qw, kw, 1e-5), g, "r", s)
    _check_f8(attention.prepass_f8(q, k, v, rotate=False, smooth_v=False), g, "n", s)
    _check_f8(attention.prepass_f8(q, k[:200], v[:200]), g, "c", 200)


def test_f8_forward_golden(dev, golden):
    """Every route to the FP8 P.V kernel: configs 50 / 54 / 56 (64-key running-max groups) and 52 / 53 / 55
    (128), attention_rr (1xx presets), no rotation / no V smoothing, cross-attention, the main kernel alone and
    the drop-in module; within the FP8 error band of exact attention; no text bias (as in the reference)."""
    import torch
    from rapid_h3 import attention, attn_int8
    g = golden("attention_f8")
    q, k, v = (to_dev(g[n], dev) for n in ("q", "k", "v"))
    s = g["q"].shape[0]
    tab, qw, kw = _rr(g, dev, s)

    def check(out, name):
        got = bf16_to_f32(to_np(out))
        ref = bf16_to_f32(g[name])
        assert rel_l2(got, ref) < TOL, (name, rel_l2(got, ref))

    for c in (50, 54, 56, 150):
        check(attention.attention(q, k, v, config=c), "out64")
    for c in (52, 53, 55):
        check(attn_int8.attention(q, k, v, config=c), "out128")
    check(attention.attention_rr(q, k, v, tab, qw, kw, 1e-5, config=150), "rout64")
    check(attention.attention_rr(q, k, v, tab, qw, kw, 1e-5, config=52), "rout128")
    check(attention.attention(q, k, v, config=51, rotate=False, smooth_v=False), "nout64")
    check(attention.attention(q, k[:200], v[:200], config=50), "cout64")
    pp = attention.prepass_f8(q, k, v)
    assert torch.equal(attention.forward_f8(pp, s, tile=64), attention.attention(q, k, v, config=50))
    ex = oa.attention_exact(g["q"], g["k"], g["v"], SC)
    assert rel_l2(bf16_to_f32(to_np(attention.attention(q, k, v, config=52))), ex) < 0.03
    with pytest.raises(RuntimeError, match="config 94 or 90"):
        attention.attention_rr_bias(q, k, v, tab, qw, kw, 1e-5, 10, 1.0, config=50)
    with pytest.raises(NotImplementedError):
        attention.attention(q, k, v, config=57)


@pytest.mark.parametrize("sq,sk,h,c", [(1, 1, 1, 50), (127, 129, 2, 52), (256, 256, 1, 50), (257, 600, 3, 55),
                                       (1000, 77, 2, 56), (300, 192, 1, 54)])
def test_f8_shapes(dev, sq, sk, h, c):
    """Query blocks around the 256-query workgroup, key tiles around the 128-key tile, a last tile whose second
    64-key chunk is all padding (sk = 192, 77), cross-attention in both directions."""
    from rapid_h3 import attention
    rng = np.random.default_rng(sq * 3 + sk * 7 + h + c)
    q = f32_to_bf16(rng.standard_normal((sq, h, 128)).astype(np.float32))
    k = f32_to_bf16((rng.standard_normal((sk, h, 128)) + 2 * rng.standard_normal((1, h, 128))).astype(np.float32))
    v = f32_to_bf16(rng.standard_normal((sk, h, 128)).astype(np.float32))
    out = attention.attention(to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), config=c)
    tile = 128 if c in (52, 53, 55) else 64
    ref = oa.attention_fp8pv_from_codes(oa.prepass_fp8v(q, k, v), SC, tile=tile)[:sq]
    assert rel_l2(bf16_to_f32(to_np(out)), ref) < TOL


@pytest.mark.parametrize("c", [60, 52, 50])
def test_bk_f8_full_size_sampled(dev, c):
    """C4's S = 145,152 (1134 key tiles) with 2 heads through configs 60 (per-block K) and 52 / 50 (FP8 P.V, 128-
    and 64-key groups): every pre-pass operand of head 1 bit-exact, 48 sampled query rows within tolerance of the
    oracle's emulation (the parity bar), and near exact attention: 5 % for config 60, whose single K scale per
    128 x 128 block is coarser (the emulation itself is 3.2 % away here), 15 % for FP8 P.V, whose e4m3 P and V
    carry 3-bit mantissas (the emulation itself is 9.5 % away on this zero-mean V, where the output is a small
    average of 145,152 terms)."""
    import torch
    from rapid_h3 import attention
    s, h = 145152, 2
    gen = torch.Generator(device="cpu").manual_seed(2)
    q = torch.randn(s, h, 128, generator=gen).to(torch.bfloat16)
    k = (torch.randn(s, h, 128, generator=gen) + 2.0 * torch.randn(1, h, 128, generator=gen)).to(torch.bfloat16)
    v = torch.randn(s, h, 128, generator=gen).to(torch.bfloat16)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    out = attention.attention(qd, kd, vd, config=c)
    rows = np.sort(np.random.default_rng(4).choice(s, 48, replace=False))
    qn, kn, vn = (t[:, 1:2].contiguous().view(torch.int16).numpy().view(np.uint16) for t in (q, k, v))
    if c == 60:
        pp, ep = attention.prepass_bk(qd, kd, vd), oa.prepass_blockk(qn, kn, vn)
        names = ("q8", "qs", "k8", "kbs", "vinit", "kmean", "vscale", "vmean")
        ref = oa.attention_blockk_from_codes(ep, SC, rows=rows)[:, 0]
    else:
        pp, ep = attention.prepass_f8(qd, kd, vd), oa.prepass_fp8v(qn, kn, vn)
        names = ("q8", "qs", "k8", "ks", "ksb", "kmean", "vscale", "vmean")
        ref = oa.attention_fp8pv_from_codes(ep, SC, rows=rows, tile=128 if c == 52 else 64)[:, 0]
        vt = to_np(pp["vt"][1])
        keys = _perm_keys_f8(vt.shape[1])
        assert np.array_equal(vt[:, :s], ep["vf8"][:, 0][keys[:s]].T)
    for n in names:
        assert np.array_equal(to_np(pp[n][1:2]), ep[n]), n
    got = bf16_to_f32(to_np(out[torch.from_numpy(rows).to(dev), 1]))
    assert rel_l2(got, ref) < TOL
    exact = oa.attention_exact(qn, kn, vn, SC, rows=rows)[:, 0]
    assert rel_l2(got, exact) < (0.05 if c == 60 else 0.15)
