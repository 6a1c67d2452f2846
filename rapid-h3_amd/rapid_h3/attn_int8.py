"""Drop-in for the reference's attn_int8 module (/root/reference/custom_nodes/rapid_h3/attn_int8.py),
backed by librh3's gfx950 INT8 attention."""
import os

from . import _native
from .attention import attention, attention_bhsd, attention_rr, prepass  # noqa: F401

CONFIG = int(os.environ.get("RAPIDH3_ATTN_CONFIG", "0"))


def ext():
    return _native.lib()


def attention_pre(*args, **kwargs):
    """Config 3xx (q8/qs from the qkv GEMM epilogue, attn_int8.py:51-57) is not built for gfx950."""
    raise NotImplementedError("attention_pre (config 3xx) is not built in rapid_h3 for gfx950")


def attention_rr_bias(q, k, v, tab, qw, kw, eps, nbias, bias, scale=None, config=94, smooth_k=True, smooth_v=True,
                      rotate=True, out=None):
    """attention_rr with the Jenga text bias (attn_int8.py:60-65): nbias 0 is attention_rr; a bias on
    keys [0, nbias) is not built for gfx950 yet."""
    if int(nbias) == 0:
        return attention_rr(q, k, v, tab, qw, kw, eps, scale=scale, config=config, smooth_k=smooth_k,
                            smooth_v=smooth_v, rotate=rotate, out=out)
    raise NotImplementedError("attention_rr_bias with nbias > 0 (text bias) is not built in rapid_h3 for gfx950")
