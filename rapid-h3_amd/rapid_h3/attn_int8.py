"""Drop-in for the reference's attn_int8 module (/root/reference/custom_nodes/rapid_h3/attn_int8.py),
backed by librh3's gfx950 INT8 attention.

attention(config=None) takes RAPIDH3_ATTN_CONFIG, default 0, as the reference does (attn_int8.py:14, :30-33):
an int config runs the reference's numerics for it (rapid_h3.attention documents the mapping). This build's
per-block bf16 P.V recipe (the benchmark's) is rapid_h3.attention.attention(config=None).

ext() returns the object the reference's JIT-built extension is (attn_int8.cu:2851-2879): int8_attention,
int8_attention_rr, int8_attention_rr_bias, int8_prepass, int8_attention_pre and int8_prepass_pre with the
reference's argument names and defaults. int8_prepass returns the reference's operand list [q8, qs, k8, ks, ksb, vt,
vscale, vmean] (attn_int8.cu:2692-2704), in this build's layouts: vt keys are permuted within 32-key blocks for
the gfx950 MFMA operand order (the reference's perm32 is for its mma.sync layout), and for configs 60-61 ks holds
the per-128-key-block scales with ksb None (the reference's own ks / ksb there are the per-token ones its
quant_k_block codes no longer use)."""
import os

from . import _native
from . import attention as _attention
from .attention import attention_pre, attention_rr, attention_rr_bias, prepass, prepass_u8  # noqa: F401

CONFIG = int(os.environ.get("RAPIDH3_ATTN_CONFIG", "0"))


def attention(q, k, v, scale=None, config=None, smooth_k=True, smooth_v=True, rotate=True, out=None):
    """q, k, v: [S, H, 128] bf16 (strided ok, last dim contiguous) -> [S, H, 128] bf16 (attn_int8.py:30-33)."""
    return _attention.attention(q, k, v, scale, CONFIG if config is None else config, smooth_k, smooth_v, rotate,
                                out)


def attention_bhsd(q, k, v, scale=None, **kw):
    """[1, H, S, 128] layout (comfy's skip_reshape convention) -> [1, H, S, 128] (attn_int8.py:36-39)."""
    o = attention(q[0].transpose(0, 1), k[0].transpose(0, 1), v[0].transpose(0, 1), scale, **kw)
    return o.transpose(0, 1).unsqueeze(0)


def _operands(pp, config):
    """The reference's prepass operand list from one of this build's pre-pass dicts."""
    if 60 <= int(config) % 100 < 70:
        return [pp["q8"], pp["qs"], pp["k8"], pp["kbs"], None, pp["vt"], pp["vscale"], pp["vmean"]]
    return [pp["q8"], pp["qs"], pp["k8"], pp["ks"], pp["ksb"], pp["vt"], pp["vscale"], pp["vmean"]]


class _Ext:
    """The reference extension's functions (PYBIND11_MODULE, attn_int8.cu:2851-2879) on librh3."""

    lib = property(lambda self: _native.lib())

    @staticmethod
    def int8_attention(q, k, v, scale, config=0, smooth_k=True, smooth_v=True, rotate=True, out=None):
        return _attention.attention(q, k, v, scale, config, smooth_k, smooth_v, rotate, out)

    @staticmethod
    def int8_attention_rr(q, k, v, tab, qw, kw, eps, scale, config=94, smooth_k=True, smooth_v=True, rotate=True,
                          out=None):
        return _attention.attention_rr(q, k, v, tab, qw, kw, eps, scale, config, smooth_k, smooth_v, rotate, out)

    @staticmethod
    def int8_attention_rr_bias(q, k, v, tab, qw, kw, eps, scale, config=94, nbias=0, bias=0.0, smooth_k=True,
                               smooth_v=True, rotate=True, out=None):
        return _attention.attention_rr_bias(q, k, v, tab, qw, kw, eps, nbias, bias, scale, config, smooth_k,
                                            smooth_v, rotate, out)

    @staticmethod
    def int8_prepass(q, k, v, tab=None, qw=None, kw=None, eps=1e-5, config=94, smooth_k=True, smooth_v=True,
                     rotate=True):
        """Pre-pass operands (verification), attn_int8.cu:2692-2704."""
        _attention._production(config, "int8_prepass")
        c = int(config) % 100
        rr = dict(tab=tab, qw=qw, kw=kw, eps=eps) if tab is not None else {}
        if 60 <= c < 70:
            if tab is not None:
                raise RuntimeError("configs 60-69 have no fused rms/rope path")    # attn_int8.cu:2606
            pp = _attention.prepass_bk(q, k, v, smooth_k, smooth_v, rotate)
        elif 50 <= c < 60:
            pp = _attention.prepass_f8(q, k, v, smooth_k=smooth_k, smooth_v=smooth_v, rotate=rotate, **rr)
        else:
            pp = _attention.prepass_u8(q, k, v, smooth_k=smooth_k, smooth_v=smooth_v, rotate=rotate, **rr)
        return _operands(pp, config)

    @staticmethod
    def int8_attention_pre(k, v, q8, qs, part, tab, kw, eps, scale, config=94, smooth_k=True, smooth_v=True,
                           rotate=True, out=None):
        return _attention.attention_pre(k, v, q8, qs, part, tab, kw, eps, scale, config, smooth_k, smooth_v, rotate,
                                        out)

    @staticmethod
    def int8_prepass_pre(k, v, q8, qs, part, tab, kw, eps, config=94, smooth_k=True, smooth_v=True, rotate=True):
        """Config 3xx pre-pass operands (verification), attn_int8.cu:2719-2730: the rest of the pre-pass on the
        workspace int8_gemm_qkv_prep filled (q8 / qs / part are its views)."""
        import torch
        _attention._production(config, "int8_prepass_pre")
        if 50 <= int(config) % 100 < 70:
            raise RuntimeError("config 3xx: configs 80-99")    # attn_int8.cu:2592
        ws = torch.empty(0, dtype=torch.uint8, device=q8.device).set_(q8.untyped_storage())
        pp = _attention.prepass_qkv(k, v, ws, 1, tab, kw, eps, smooth_k, smooth_v, rotate)
        return _operands(pp, config)


_EXT = _Ext()


def ext():
    """The extension object (the reference JIT-builds attn_int8.cu here, attn_int8.py:17-27)."""
    _native.lib()
    return _EXT
