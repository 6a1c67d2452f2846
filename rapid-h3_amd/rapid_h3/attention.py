"""INT8 flash attention on the HIP kernels (librh3: rh3_int8_attention*, rh3_attention_prepass,
rh3_*attention_u8*).

Signatures follow /root/reference/custom_nodes/rapid_h3/attn_int8.py:30-65. Two numerics, picked by config:
  * config=None: the per-block recipe of this build's benchmark: Q and K int8 with one scale per (head,
    128-token block), K mean-smoothed over all tokens, Q.K^T on int8 MFMA, fp32 online softmax, P.V on
    bf16 MFMA with V in bf16;
  * config=c (an int): the reference's production numerics, configs 80-99 (attn_int8.cu attn_fwd8 :2250-2511
    and the cake kernels bit-identical to it): per-token H128-rotated Q/K (rotate), K mean-smoothed
    (smooth_k), per-channel int8 V (smooth_v), u8 P against each 128-key tile's max, int32 P.V, fp32 fold.
    1xx / 2xx select the same math (the reference's node-level fused-pre-pass and checked variants).
    The reference's other kernel configs run this same arithmetic here; the 64-key-tile configs (0, 1, 4-8,
    10-12, 20-29) and those with the acc * ks dequant (0-12) differ from their own outputs by the tile-max
    granularity and the rounding of t;
  * config 60 or 61 (attn_int8.cu attn_fwd6 :1786-1962, quant_k_block :404-443): as the production numerics but
    with one K scale per 128-key block (after the smoothing and the H128 rotation), an integer tile max over
    the raw accumulators and no per-key dequantization. No RMSNorm + RoPE path and no text bias (the
    reference's own limits, attn_int8.cu:2606, :2764).
  * configs 50-56 (attn_int8.cu attn_fwd5 :1563-1785): the production Q / K numerics with e4m3 V (per channel,
    stretched to 448) and P in e4m3 against the running max (scaled to 448), P.V on the FP8 MFMA straight into fp32,
    the running max updated per 64 keys (configs 50, 51, 54, 56) or 128 keys (52, 53, 55); the reference's
    two-level accumulation of 51 / 53 is the same sum with another fp32 rounding order. RMSNorm + RoPE path yes,
    text bias no (as in the reference).
Configs 57-59 and 62-69 do not exist in the reference's dispatch (attn_int8.cu:2776-2830) and raise
NotImplementedError. The reference's "config 3xx" is attention_pre (Q operands and K / V statistics from the qkv
GEMM epilogue) with a kernel config 80-99.
"""
import torch

from . import _native as nat

D = 128


def _check_qkv(q, k, v, name, self_only=False):
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        if t.ndim != 3 or t.shape[2] != D:
            raise RuntimeError(f"{name}: {n} must be [S, H, 128], got {tuple(t.shape)}")
        if t.dtype != torch.bfloat16:
            raise RuntimeError(f"{name}: {n} must be bf16")
        if t.stride(2) != 1:
            raise RuntimeError(f"{name}: {n} last dim must be contiguous")
        if not t.is_cuda:
            raise RuntimeError(f"{name}: {n} must be on a GPU (no CPU path)")
    if k.shape != v.shape or q.shape[1] != k.shape[1]:
        raise RuntimeError(f"{name}: k/v shapes {tuple(k.shape)} / {tuple(v.shape)} and q heads must match")
    if self_only and q.shape != k.shape:
        raise RuntimeError(f"{name}: self-attention shapes only")


def _out(q, out):
    sq, h, _ = q.shape
    if out is None:
        return torch.empty((sq, h, D), device=q.device, dtype=torch.bfloat16)
    if out.shape != (sq, h, D) or out.stride(2) != 1 or out.dtype != torch.bfloat16:
        raise RuntimeError("out must be bf16 [Sq, H, 128] with contiguous last dim")
    return out


def workspace(sq, sk, h, device):
    n = nat.lib().rh3_attention_workspace_bytes(sq, sk, h)
    return torch.empty(n, device=device, dtype=torch.uint8)


def _production(config, name):
    """True when config selects the reference's production numerics (see the module docstring)."""
    if config is None:
        return False
    c = int(config)
    if c < 0 or c >= 300:
        raise NotImplementedError(f"{name}: config {c} is not built for gfx950 (3xx needs the qkv-GEMM epilogue "
                                  "pre-pass)")
    if c % 100 in (57, 58, 59) or 62 <= c % 100 < 70:
        raise NotImplementedError(f"{name}: config {c} does not exist in the reference's kernel dispatch")
    return True


def _fp8_tile(config):
    """Keys per running-max update of the FP8 P.V configs 50-56 (the reference's BN, attn_int8.cu:2804-2810), or
    None for any other config."""
    if config is None or not 50 <= int(config) % 100 < 60:
        return None
    c = int(config) % 100
    if c > 56:
        raise NotImplementedError(f"config {int(config)}: the FP8 P.V kernel is configs 50-56 only")
    return 128 if c in (52, 53, 55) else 64


def _attention_f8(name, q, k, v, rr, scale, tile, smooth_k, smooth_v, rotate, out):
    sq, h, _ = q.shape
    sk = k.shape[0]
    out = _out(q, out)
    tab, qw, kw, eps, rot = rr if rr is not None else (None, None, None, 0.0, 0)
    ws = workspace_u8(sq, sk, h, q.device)
    nat.call("rh3_int8_attention_f8", nat.ptr(q), q.stride(0), q.stride(1), nat.ptr(k), k.stride(0), k.stride(1),
             nat.ptr(v), v.stride(0), v.stride(1), sq, sk, h, nat.ptr(tab), rot, nat.ptr(qw), nat.ptr(kw),
             float(eps), float(scale), int(tile), int(bool(smooth_k)), int(bool(smooth_v)), int(bool(rotate)),
             nat.ptr(out), out.stride(0), out.stride(1), nat.ptr(ws), ws.numel(), nat.stream(q.device))
    return out


def _block_k(config):
    """True for configs 60 and 61 (one K scale per 128-key block, attn_fwd6); 62-69 do not exist in the
    reference's dispatch (attn_int8.cu:2812-2813) and raise."""
    if config is None or not 60 <= int(config) % 100 < 70:
        return False
    if int(config) not in (60, 61):
        raise NotImplementedError(f"config {int(config)}: the per-block-K kernel is configs 60 and 61 only")
    return True


def _attention_bk(q, k, v, scale, smooth_k, smooth_v, rotate, out):
    sq, h, _ = q.shape
    sk = k.shape[0]
    out = _out(q, out)
    ws = workspace_u8(sq, sk, h, q.device)
    nat.call("rh3_int8_attention_bk", nat.ptr(q), q.stride(0), q.stride(1), nat.ptr(k), k.stride(0), k.stride(1),
             nat.ptr(v), v.stride(0), v.stride(1), sq, sk, h, float(scale), int(bool(smooth_k)),
             int(bool(smooth_v)), int(bool(rotate)), nat.ptr(out), out.stride(0), out.stride(1), nat.ptr(ws),
             ws.numel(), nat.stream(q.device))
    return out


def workspace_u8(sq, sk, h, device):
    n = nat.lib().rh3_attention_u8_workspace_bytes(sq, sk, h)
    return torch.empty(n, device=device, dtype=torch.uint8)


def _attention_u8(name, q, k, v, rr, scale, nbias, bias, smooth_k, smooth_v, rotate, out):
    sq, h, _ = q.shape
    sk = k.shape[0]
    out = _out(q, out)
    tab, qw, kw, eps, rot = rr if rr is not None else (None, None, None, 0.0, 0)
    ws = workspace_u8(sq, sk, h, q.device)
    nat.call("rh3_int8_attention_u8", nat.ptr(q), q.stride(0), q.stride(1), nat.ptr(k), k.stride(0), k.stride(1),
             nat.ptr(v), v.stride(0), v.stride(1), sq, sk, h, nat.ptr(tab), rot, nat.ptr(qw), nat.ptr(kw),
             float(eps), float(scale), int(nbias), float(bias), int(bool(smooth_k)), int(bool(smooth_v)),
             int(bool(rotate)), nat.ptr(out), out.stride(0), out.stride(1), nat.ptr(ws), ws.numel(),
             nat.stream(q.device))
    return out


def attention(q, k, v, scale=None, config=None, smooth_k=True, smooth_v=True, rotate=True, out=None):
    """q [Sq, H, 128], k / v [Sk, H, 128] bf16 (strided ok, last dim contiguous) -> [Sq, H, 128] bf16.
    Sq may differ from Sk (cross-attention). config None: the per-block bf16 P.V recipe (smooth_v and
    rotate do not apply to it); an int config: the production numerics with smooth_v / rotate."""
    _check_qkv(q, k, v, "attention")
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    if _block_k(config):
        return _attention_bk(q, k, v, scale, smooth_k, smooth_v, rotate, out)
    tile = _fp8_tile(config)
    if tile:
        return _attention_f8("attention", q, k, v, None, scale, tile, smooth_k, smooth_v, rotate, out)
    if _production(config, "attention"):
        return _attention_u8("attention", q, k, v, None, scale, 0, 0.0, smooth_k, smooth_v, rotate, out)
    out = _out(q, out)
    sq, h, _ = q.shape
    sk = k.shape[0]
    ws = workspace(sq, sk, h, q.device)
    nat.call("rh3_int8_attention", nat.ptr(q), q.stride(0), q.stride(1), nat.ptr(k), k.stride(0), k.stride(1),
             nat.ptr(v), v.stride(0), v.stride(1), sq, sk, h, float(scale), int(bool(smooth_k)), nat.ptr(out),
             out.stride(0), out.stride(1), nat.ptr(ws), ws.numel(), nat.stream(q.device))
    return out


def attention_bhsd(q, k, v, scale=None, **kw):
    """[1, H, S, 128] layout (comfy's skip_reshape convention) -> [1, H, S, 128]."""
    o = attention(q[0].transpose(0, 1), k[0].transpose(0, 1), v[0].transpose(0, 1), scale, **kw)
    return o.transpose(0, 1).unsqueeze(0)


def _check_rr(q, tab, qw, kw):
    s = q.shape[0]
    if not (tab.dim() == 6 and tab.shape[0] == 1 and tab.shape[1] == s and tab.shape[2] == 1
            and tab.shape[4] == 2 and tab.shape[5] == 2):
        raise RuntimeError("rope table must be [1, S, 1, rot/2, 2, 2]")
    if tab.dtype != torch.bfloat16 or qw.dtype != torch.bfloat16 or kw.dtype != torch.bfloat16:
        raise RuntimeError("rope table and norm weights must be bf16")
    if qw.numel() != D or kw.numel() != D:
        raise RuntimeError("norm weights must have 128 elements")
    rot = tab.shape[3] * 2
    if rot not in (96, 128):
        raise RuntimeError("rot_dim 96 or 128 supported")
    return tab.contiguous(), qw.contiguous(), kw.contiguous(), rot


def rms_rope_(q, k, tab, qw, kw, eps):
    """Per-head RMSNorm (qw / kw [128] bf16, eps) and split-half RoPE (tab [1, S, 1, rot/2, 2, 2] bf16) of q and k
    ([S, H, 128] bf16, strided ok) in place, bit-identical to the prologue the *_rr pre-passes fuse (rh3_rms_rope_qk).
    The stand-in for comfy_kitchen's ck.rms_rope_split_half_(q, k, rope_freqs, qw, kw, epsilon, rot_dim) that
    _fused_block calls before handing q, k to another attention (__init__.py:297)."""
    for t, n in ((q, "q"), (k, "k")):
        if t.ndim != 3 or t.shape[2] != D or t.dtype != torch.bfloat16 or t.stride(2) != 1 or not t.is_cuda:
            raise RuntimeError(f"rms_rope_: {n} must be a bf16 [S, H, 128] GPU tensor with contiguous last dim")
    if q.shape != k.shape:
        raise RuntimeError("rms_rope_: q and k shapes must match")
    tab, qw, kw, rot = _check_rr(q, tab, qw, kw)
    nat.call("rh3_rms_rope_qk", nat.ptr(q), q.stride(0), q.stride(1), nat.ptr(k), k.stride(0), k.stride(1),
             q.shape[0], q.shape[1], nat.ptr(tab), rot, nat.ptr(qw), nat.ptr(kw), float(eps), nat.stream(q.device))
    return q, k


def attention_rr(q, k, v, tab, qw, kw, eps, scale=None, config=94, smooth_k=True, smooth_v=True, rotate=True,
                 out=None):
    """attention() on the raw qkv-projection q, k ([S, H, 128] bf16, strided ok) with the per-head
    RMSNorm (qw / kw, eps) and split-half RoPE (tab [1, S, 1, rot/2, 2, 2] bf16) fused into the
    pre-pass; q, k untouched. Self-attention only. The default config 94 is the production numerics, as in
    the reference; config=None runs the per-block bf16 P.V recipe."""
    _check_qkv(q, k, v, "attention_rr", self_only=True)
    if config is not None and 60 <= int(config) % 100 < 70:
        raise RuntimeError("configs 60-69 have no fused rms/rope path")    # attn_int8.cu:2606
    tab, qw, kw, rot = _check_rr(q, tab, qw, kw)
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    tile = _fp8_tile(config)
    if tile:
        return _attention_f8("attention_rr", q, k, v, (tab, qw, kw, eps, rot), scale, tile, smooth_k, smooth_v, rotate,
                             out)
    if _production(config, "attention_rr"):
        return _attention_u8("attention_rr", q, k, v, (tab, qw, kw, eps, rot), scale, 0, 0.0, smooth_k, smooth_v,
                             rotate, out)
    out = _out(q, out)
    s, h, _ = q.shape
    ws = workspace(s, s, h, q.device)
    nat.call("rh3_int8_attention_rr", nat.ptr(q), q.stride(0), q.stride(1), nat.ptr(k), k.stride(0), k.stride(1),
             nat.ptr(v), v.stride(0), v.stride(1), s, h, nat.ptr(tab), rot, nat.ptr(qw), nat.ptr(kw), float(eps),
             float(scale), int(bool(smooth_k)), nat.ptr(out), out.stride(0), out.stride(1), nat.ptr(ws), ws.numel(),
             nat.stream(q.device))
    return out


def prepass(q, k, v, tab=None, qw=None, kw=None, eps=1e-5, smooth_k=True):
    """Pre-pass operands (the reference's int8_prepass, for verification): dict of
    q8 [H, Sqpad, 128] int8, qs [H, Sqpad/128] fp32, k8, ks, kmean [H, 128] fp32, vt [H, 128, Skpad] bf16."""
    import ctypes
    _check_qkv(q, k, v, "prepass")
    sq, h, _ = q.shape
    sk = k.shape[0]
    rot = 0
    if tab is not None:
        tab, qw, kw, rot = _check_rr(q, tab, qw, kw)
    ws = workspace(sq, sk, h, q.device)
    ptrs = (ctypes.c_void_p * 6)()
    nat.call("rh3_attention_prepass", nat.ptr(q), q.stride(0), q.stride(1), nat.ptr(k), k.stride(0), k.stride(1),
             nat.ptr(v), v.stride(0), v.stride(1), sq, sk, h, nat.ptr(tab), rot, nat.ptr(qw), nat.ptr(kw),
             float(eps), int(bool(smooth_k)), nat.ptr(ws), ws.numel(), ptrs, nat.stream(q.device))
    sqp, skp = (sq + 127) // 128 * 128, (sk + 127) // 128 * 128
    base = ws.data_ptr()

    def view(i, shape, dtype):
        off = ptrs[i] - base
        n = 1
        for d in shape:
            n *= d
        return ws[off:off + n * torch.tensor([], dtype=dtype).element_size()].view(dtype).view(shape)

    return {
        "q8": view(0, (h, sqp, D), torch.int8), "qs": view(1, (h, sqp // 128), torch.float32),
        "k8": view(2, (h, skp, D), torch.int8), "ks": view(3, (h, skp // 128), torch.float32),
        "kmean": view(4, (h, D), torch.float32), "vt": view(5, (h, D, skp), torch.bfloat16),
        "_ws": ws, "_sk": sk,
    }


def forward(pp, sq, out=None, scale=None):
    """The main kernel alone on operands prepass() produced (same workspace): out [Sq, H, 128] bf16."""
    h = pp["q8"].shape[0]
    sk = pp["_sk"]
    scale = D ** -0.5 if scale is None else scale
    if out is None:
        out = torch.empty((sq, h, D), device=pp["q8"].device, dtype=torch.bfloat16)
    ws = pp["_ws"]
    nat.call("rh3_attention_forward", sq, sk, h, float(scale), nat.ptr(out), out.stride(0), out.stride(1),
             nat.ptr(ws), ws.numel(), nat.stream(out.device))
    return out


def attention_rr_bias(q, k, v, tab, qw, kw, eps, nbias, bias, scale=None, config=94, smooth_k=True, smooth_v=True,
                      rotate=True, out=None):
    """attention_rr with the Jenga text-attention bias (attn_int8.py:60-65, attn_int8.cu:2680-2689): every
    query's logits on keys [0, nbias) get + bias (natural-log units). Config 94 or 90 only (the reference's
    check, attn_int8.cu:2764); nbias 0 is attention_rr."""
    nbias = int(nbias)
    if nbias == 0:
        return attention_rr(q, k, v, tab, qw, kw, eps, scale=scale, config=config, smooth_k=smooth_k,
                            smooth_v=smooth_v, rotate=rotate, out=out)
    if config is None or int(config) % 100 not in (90, 94):
        raise RuntimeError("text bias: config 94 or 90 only")
    _check_qkv(q, k, v, "attention_rr_bias", self_only=True)
    if nbias < 0 or nbias > q.shape[0]:
        raise RuntimeError("text bias: nbias > S")
    tab, qw, kw, rot = _check_rr(q, tab, qw, kw)
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    return _attention_u8("attention_rr_bias", q, k, v, (tab, qw, kw, eps, rot), scale, nbias, float(bias), smooth_k,
                         smooth_v, rotate, out)


def _ptr_views(ws, ptrs, spec):
    """Views into the workspace tensor ws at the device pointers the library returned."""
    base = ws.data_ptr()
    out = {}
    for name, (i, shape, dtype) in spec.items():
        off = ptrs[i] - base
        n = 1
        for d in shape:
            n *= d
        out[name] = ws[off:off + n * torch.tensor([], dtype=dtype).element_size()].view(dtype).view(shape)
    return out


def _u8_views(ws, ptrs, sq, sk, h):
    sqp, skp = (sq + 127) // 128 * 128, (sk + 127) // 128 * 128
    v = _ptr_views(ws, ptrs, {
        "q8": (0, (h, sqp, D), torch.int8), "qs": (1, (h, sqp), torch.float32),
        "k8": (2, (h, skp, D), torch.int8), "ks": (3, (h, skp), torch.float32),
        "_side": (4, (h, skp // 128, 2048), torch.uint8), "vt": (5, (h, D, skp), torch.int8),
        "kmean": (6, (h, D), torch.float32), "vscale": (7, (h, D), torch.float32),
        "vmean": (8, (h, D), torch.float32)})
    side = v.pop("_side")
    v["ksb"] = side[:, :, :1024].contiguous().view(torch.float32).view(h, skp, 2)
    v["vinit"] = side[:, :, 1024:1536].contiguous().view(torch.int32).view(h, skp // 128, D)
    v["_ws"], v["_sk"] = ws, sk
    return v


def _blk_views(ws, ptrs, sq, sk, h):
    sqp, skp = (sq + 127) // 128 * 128, (sk + 127) // 128 * 128
    v = _ptr_views(ws, ptrs, {
        "q8": (0, (h, sqp, D), torch.int8), "qs": (1, (h, sqp // 128), torch.float32),
        "k8": (2, (h, skp, D), torch.int8), "ks": (3, (h, skp // 128), torch.float32),
        "kmean": (4, (h, D), torch.float32), "vt": (5, (h, D, skp), torch.bfloat16)})
    v["_ws"], v["_sk"] = ws, sk
    return v


def workspace_offsets(numerics, sq, sk, h):
    """Byte offsets of the workspace arrays (rh3_attention_workspace_layout), as a dict."""
    import ctypes
    names = (("q8", "qs", "k8", "ks", "kmean", "part", "vt", "kn", "bytes") if numerics == 0 else
             ("q8", "qs", "k8", "ks", "side", "vt", "kmean", "vmean", "vscale", "kpart", "vsum", "vmax", "vmin",
              "bytes"))
    offs = (ctypes.c_int64 * len(names))()
    nat.call("rh3_attention_workspace_layout", int(numerics), sq, sk, h, offs)
    return dict(zip(names, offs))


def workspace_views_u8(ws, sq, sk, h):
    """q8, qs and the statistics block ("part": the float64 K and V sums and the V max / min, to the end of the
    workspace) of a production workspace, as views (what int8_gemm_qkv_prep returns)."""
    o = workspace_offsets(1, sq, sk, h)
    sqp = (sq + 127) // 128 * 128
    return {"q8": ws[o["q8"]:o["q8"] + h * sqp * D].view(torch.int8).view(h, sqp, D),
            "qs": ws[o["qs"]:o["qs"] + h * sqp * 4].view(torch.float32).view(h, sqp),
            "part": ws[o["kpart"]:o["bytes"]]}


def prepass_qkv(k, v, workspace, numerics, tab=None, kw=None, eps=1e-5, smooth_k=True, smooth_v=True, rotate=True):
    """The rest of the pre-pass after gemm.int8_gemm_qkv on the same workspace (k, v [S, H, 128] bf16 views of
    its output): dict as prepass() (numerics 0) or prepass_u8() (numerics 1)."""
    import ctypes
    _check_qkv(k, k, v, "prepass_qkv", self_only=True)
    s, h, _ = k.shape
    rot = 0
    if tab is not None:
        if tab.dim() != 6 or tab.shape[1] != s or tab.dtype != torch.bfloat16 or kw is None:
            raise RuntimeError("prepass_qkv: tab [1, S, 1, rot/2, 2, 2] bf16 and kw required together")
        rot = tab.shape[3] * 2
        tab, kw = tab.contiguous(), kw.contiguous()
    if numerics == 0:
        ptrs = (ctypes.c_void_p * 6)()
        nat.call("rh3_attention_prepass_qkv", nat.ptr(k), k.stride(0), k.stride(1), nat.ptr(v), v.stride(0),
                 v.stride(1), s, h, nat.ptr(tab), rot, nat.ptr(kw), float(eps), int(bool(smooth_k)),
                 nat.ptr(workspace), workspace.numel(), ptrs, nat.stream(k.device))
        return _blk_views(workspace, ptrs, s, s, h)
    ptrs = (ctypes.c_void_p * 9)()
    nat.call("rh3_attention_u8_prepass_qkv", nat.ptr(k), k.stride(0), k.stride(1), nat.ptr(v), v.stride(0),
             v.stride(1), s, h, nat.ptr(tab), rot, nat.ptr(kw), float(eps), int(bool(smooth_k)), int(bool(smooth_v)),
             int(bool(rotate)), nat.ptr(workspace), workspace.numel(), ptrs, nat.stream(k.device))
    return _u8_views(workspace, ptrs, s, s, h)


def attention_pre(k, v, q8, qs, part, tab, kw, eps, scale=None, config=94, smooth_k=True, smooth_v=True,
                  rotate=True, out=None):
    """Config 3xx (attn_int8.py:50-57): attention_rr whose Q operands and K / V statistics come from
    cutlass_fp8.int8_gemm_qkv_prep (q8, qs, part: views of its workspace); k, v are that GEMM's k and v columns
    ([S, H, 128] bf16 views). The same result as attention_rr with config on that GEMM's q, k, v. The rotate
    flag must match the one int8_gemm_qkv_prep used."""
    _production(config, "attention_pre")
    if 50 <= int(config) % 100 < 70:
        raise RuntimeError("config 3xx: configs 80-99")    # attn_int8.cu:2592
    if q8.untyped_storage().data_ptr() != part.untyped_storage().data_ptr():
        raise RuntimeError("attention_pre: q8 / qs / part must be the views int8_gemm_qkv_prep returned")
    ws = torch.empty(0, dtype=torch.uint8, device=q8.device).set_(q8.untyped_storage())
    scale = k.shape[-1] ** -0.5 if scale is None else scale
    pp = prepass_qkv(k, v, ws, 1, tab, kw, eps, smooth_k, smooth_v, rotate)
    return forward_u8(pp, k.shape[0], out=_out(k, out), scale=scale)


def prepass_u8(q, k, v, tab=None, qw=None, kw=None, eps=1e-5, smooth_k=True, smooth_v=True, rotate=True):
    """Production pre-pass operands (the reference's int8_prepass, attn_int8.cu:2691-2704, for verification):
    dict of q8 [H, Sqpad, 128] int8, qs [H, Sqpad] fp32, k8, ks, ksb [H, Skpad, 2] fp32, vinit
    [H, Skpad/128, 128] int32 (P.V accumulator starts), vt [H, 128, Skpad] int8 (keys permuted within 32-key
    blocks), kmean, vscale, vmean [H, 128] fp32."""
    import ctypes
    _check_qkv(q, k, v, "prepass_u8")
    sq, h, _ = q.shape
    sk = k.shape[0]
    rot = 0
    if tab is not None:
        tab, qw, kw, rot = _check_rr(q, tab, qw, kw)
    ws = workspace_u8(sq, sk, h, q.device)
    ptrs = (ctypes.c_void_p * 9)()
    nat.call("rh3_attention_u8_prepass", nat.ptr(q), q.stride(0), q.stride(1), nat.ptr(k), k.stride(0), k.stride(1),
             nat.ptr(v), v.stride(0), v.stride(1), sq, sk, h, nat.ptr(tab), rot, nat.ptr(qw), nat.ptr(kw),
             float(eps), int(bool(smooth_k)), int(bool(smooth_v)), int(bool(rotate)), nat.ptr(ws), ws.numel(), ptrs,
             nat.stream(q.device))
    return _u8_views(ws, ptrs, sq, sk, h)


def forward_u8(pp, sq, out=None, scale=None, nbias=0, bias=0.0):
    """The production main kernel alone on operands prepass_u8() produced: out [Sq, H, 128] bf16."""
    h = pp["q8"].shape[0]
    sk = pp["_sk"]
    scale = D ** -0.5 if scale is None else scale
    if out is None:
        out = torch.empty((sq, h, D), device=pp["q8"].device, dtype=torch.bfloat16)
    ws = pp["_ws"]
    nat.call("rh3_attention_u8_forward", sq, sk, h, float(scale), int(nbias), float(bias), nat.ptr(out),
             out.stride(0), out.stride(1), nat.ptr(ws), ws.numel(), nat.stream(out.device))
    return out


def prepass_bk(q, k, v, smooth_k=True, smooth_v=True, rotate=True):
    """Pre-pass operands of configs 60-61 (for verification): dict as prepass_u8() with kbs [H, Skpad/128] fp32
    (one K scale per 128-key block) in place of ks / ksb."""
    import ctypes
    _check_qkv(q, k, v, "prepass_bk")
    sq, h, _ = q.shape
    sk = k.shape[0]
    ws = workspace_u8(sq, sk, h, q.device)
    ptrs = (ctypes.c_void_p * 9)()
    nat.call("rh3_attention_bk_prepass", nat.ptr(q), q.stride(0), q.stride(1), nat.ptr(k), k.stride(0), k.stride(1),
             nat.ptr(v), v.stride(0), v.stride(1), sq, sk, h, int(bool(smooth_k)), int(bool(smooth_v)),
             int(bool(rotate)), nat.ptr(ws), ws.numel(), ptrs, nat.stream(q.device))
    vw = _u8_views(ws, ptrs, sq, sk, h)
    skp = (sk + 127) // 128 * 128
    vw["kbs"] = vw.pop("ks").reshape(-1)[:h * (skp // 128)].view(h, skp // 128)
    side = _ptr_views(ws, ptrs, {"s": (4, (h, skp // 128, 512), torch.float32)})["s"]
    vw["side_kb"] = side[:, :, 0]
    del vw["ksb"]
    return vw


def forward_bk(pp, sq, out=None, scale=None):
    """The configs 60-61 main kernel alone on operands prepass_bk() produced: out [Sq, H, 128] bf16."""
    h = pp["q8"].shape[0]
    sk = pp["_sk"]
    scale = D ** -0.5 if scale is None else scale
    if out is None:
        out = torch.empty((sq, h, D), device=pp["q8"].device, dtype=torch.bfloat16)
    ws = pp["_ws"]
    nat.call("rh3_attention_bk_forward", sq, sk, h, float(scale), nat.ptr(out), out.stride(0), out.stride(1),
             nat.ptr(ws), ws.numel(), nat.stream(out.device))
    return out


def prepass_f8(q, k, v, tab=None, qw=None, kw=None, eps=1e-5, smooth_k=True, smooth_v=True, rotate=True):
    """Pre-pass operands of the FP8 P.V configs 50-56 (for verification): dict as prepass_u8() with vt
    [H, 128, Skpad] uint8 e4m3 codes (keys permuted within 64-key chunks) and without vinit."""
    import ctypes
    _check_qkv(q, k, v, "prepass_f8")
    sq, h, _ = q.shape
    sk = k.shape[0]
    rot = 0
    if tab is not None:
        tab, qw, kw, rot = _check_rr(q, tab, qw, kw)
    ws = workspace_u8(sq, sk, h, q.device)
    ptrs = (ctypes.c_void_p * 9)()
    nat.call("rh3_attention_f8_prepass", nat.ptr(q), q.stride(0), q.stride(1), nat.ptr(k), k.stride(0), k.stride(1),
             nat.ptr(v), v.stride(0), v.stride(1), sq, sk, h, nat.ptr(tab), rot, nat.ptr(qw), nat.ptr(kw),
             float(eps), int(bool(smooth_k)), int(bool(smooth_v)), int(bool(rotate)), nat.ptr(ws), ws.numel(), ptrs,
             nat.stream(q.device))
    vw = _u8_views(ws, ptrs, sq, sk, h)
    vw["vt"] = vw["vt"].view(torch.uint8)
    del vw["vinit"]
    return vw


def forward_f8(pp, sq, out=None, scale=None, tile=64):
    """The FP8 P.V main kernel alone on operands prepass_f8() produced: out [Sq, H, 128] bf16."""
    h = pp["q8"].shape[0]
    sk = pp["_sk"]
    scale = D ** -0.5 if scale is None else scale
    if out is None:
        out = torch.empty((sq, h, D), device=pp["q8"].device, dtype=torch.bfloat16)
    ws = pp["_ws"]
    nat.call("rh3_attention_f8_forward", sq, sk, h, float(scale), int(tile), nat.ptr(out), out.stride(0),
             out.stride(1), nat.ptr(ws), ws.numel(), nat.stream(out.device))
    return out
