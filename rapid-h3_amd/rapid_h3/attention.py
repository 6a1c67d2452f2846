"""INT8 flash attention on the HIP kernels (librh3: rh3_int8_attention*, rh3_attention_prepass).

Signatures follow /root/reference/custom_nodes/rapid_h3/attn_int8.py:30-65. Numerics of this build
(the BASELINE recipe): Q and K int8 with one scale per (head, 128-token block), K mean-smoothed over
all tokens, Q.K^T on int8 MFMA, fp32 online softmax, P.V on bf16 MFMA. Arguments the reference uses
to pick its own variants are accepted for signature parity and mapped as documented per function.
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


def attention(q, k, v, scale=None, config=None, smooth_k=True, smooth_v=True, rotate=True, out=None):
    """q [Sq, H, 128], k / v [Sk, H, 128] bf16 (strided ok, last dim contiguous) -> [Sq, H, 128] bf16.
    Sq may differ from Sk (cross-attention). config / smooth_v / rotate select reference-only variants
    (its kernel configs, int8 V, H128 rotation) and are accepted without effect: V stays bf16 and Q/K
    are not rotated in this recipe."""
    _check_qkv(q, k, v, "attention")
    scale = q.shape[-1] ** -0.5 if scale is None else scale
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


def attention_rr(q, k, v, tab, qw, kw, eps, scale=None, config=94, smooth_k=True, smooth_v=True, rotate=True,
                 out=None):
    """attention() on the raw qkv-projection q, k ([S, H, 128] bf16, strided ok) with the per-head
    RMSNorm (qw / kw, eps) and split-half RoPE (tab [1, S, 1, rot/2, 2, 2] bf16) fused into the
    pre-pass; q, k untouched. Self-attention only."""
    _check_qkv(q, k, v, "attention_rr", self_only=True)
    tab, qw, kw, rot = _check_rr(q, tab, qw, kw)
    scale = q.shape[-1] ** -0.5 if scale is None else scale
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
