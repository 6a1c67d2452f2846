"""Drop-in for the reference's attn_int8 module (/root/reference/custom_nodes/rapid_h3/attn_int8.py),
backed by librh3's gfx950 INT8 attention.

attention(config=None) takes RAPIDH3_ATTN_CONFIG when it is set (attn_int8.py:13, :30-33); unset, it runs
the per-block bf16 P.V recipe instead of the reference's config 0 (rapid_h3.attention documents both)."""
import os

from . import _native
from . import attention as _attention
from .attention import attention_pre, attention_rr, attention_rr_bias, prepass, prepass_u8  # noqa: F401

_ENV_CONFIG = os.environ.get("RAPIDH3_ATTN_CONFIG")
CONFIG = None if _ENV_CONFIG is None else int(_ENV_CONFIG)


def attention(q, k, v, scale=None, config=None, smooth_k=True, smooth_v=True, rotate=True, out=None):
    """q, k, v: [S, H, 128] bf16 (strided ok, last dim contiguous) -> [S, H, 128] bf16 (attn_int8.py:30-33)."""
    return _attention.attention(q, k, v, scale, CONFIG if config is None else config, smooth_k, smooth_v, rotate,
                                out)


def attention_bhsd(q, k, v, scale=None, **kw):
    """[1, H, S, 128] layout (comfy's skip_reshape convention) -> [1, H, S, 128] (attn_int8.py:36-39)."""
    o = attention(q[0].transpose(0, 1), k[0].transpose(0, 1), v[0].transpose(0, 1), scale, **kw)
    return o.transpose(0, 1).unsqueeze(0)


def ext():
    return _native.lib()
