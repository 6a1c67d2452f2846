"""CPU restatement of the INT8 attention path: pre-pass (RMSNorm + split-half RoPE, K mean-smoothing,
per-128-token-block INT8 Q/K) and the attention it feeds.

TEST INFRASTRUCTURE ONLY (see oracle/numerics.py).

Reference semantics followed:
  * K/V statistics and smoothing   attn_int8.cu:80-109 (stats_partial / stats_final: kmean = sum_s k / S)
  * per-128-key-block K scale      attn_int8.cu:402-443 (quant_k_block), bench/attn_emulate.py:10-18
                                   (q8(x, 1, group=128): sc = max(amax, 1e-8) / 127, q = round(x / sc))
  * per-head RMSNorm + RoPE        attn_int8.cu:173-185 / :217-260 (rms_rope_row), table layout
                                   [S, rot/2, 2, 2] = (cos, -sin, sin, cos) from bench/rmsrope_fuse.py:22-33
  * attention                      attn_int8.cu:602-709: softmax(scale * q.k) v, non-causal, D = 128

Orders fixed by this build (both sides use them, so Q/K codes and scales are bit-exact):
  * kmean: float64 sum over all S tokens, divided by S in float64, rounded once to fp32;
  * RMSNorm sum of squares over D = 128: 16 lanes own channels 8*l + e, accumulate x*x in fp32 for
    e = 0..7 from 0, then a butterfly over lane distances 8, 4, 2, 1;
  * r = 1 / sqrt(ss / 128 + eps), y = bf16((r * x) * w), RoPE pair (a, b) = (y_i, y_{i+rot/2}):
    out_i = bf16(a*t00 + b*t01), out_{i+rot/2} = bf16(a*t10 + b*t11) (bf16 products are exact in fp32).
"""
import numpy as np

from .numerics import F32, bf16_to_f32, round_bf16

D = 128
BLOCK = 128


def spad(s):
    return (s + BLOCK - 1) // BLOCK * BLOCK


def _as_f32(x):
    x = np.asarray(x)
    return bf16_to_f32(x) if x.dtype == np.uint16 else x.astype(np.float32)


def kmean(k):
    """k [S, H, D] (bf16 bits) -> [H, D] fp32 per-head channel mean."""
    kf = _as_f32(k).astype(np.float64)
    return (kf.sum(axis=0) / kf.shape[0]).astype(F32)


def rms_rope(x, tab, w, eps):
    """Per-head RMSNorm + split-half partial RoPE of x [S, H, D] (bf16 bits) -> fp32 values of the bf16 result.
    tab [S, rot/2, 2, 2] bf16 bits; w [D] bf16 bits."""
    xf = _as_f32(x)
    s, h, d = xf.shape
    t = xf.reshape(s, h, 16, 8)
    acc = np.zeros((s, h, 16), F32)
    for e in range(8):
        acc = (acc + t[..., e] * t[..., e]).astype(F32)
    for wdt in (8, 4, 2, 1):
        acc = (acc[..., :wdt] + acc[..., wdt:2 * wdt]).astype(F32)
    ss = acc[..., 0]
    r = (F32(1.0) / np.sqrt(ss / F32(D) + F32(eps))).astype(F32)
    y = round_bf16((r[..., None] * xf) * _as_f32(w)[None, None, :])
    tb = _as_f32(tab)
    hr = tb.shape[1]
    rot = 2 * hr
    out = y.copy()
    a = y[..., :hr]
    b = y[..., hr:rot]
    t00 = tb[:, None, :, 0, 0]
    t01 = tb[:, None, :, 0, 1]
    t10 = tb[:, None, :, 1, 0]
    t11 = tb[:, None, :, 1, 1]
    out[..., :hr] = round_bf16((a * t00) + (b * t01))
    out[..., hr:rot] = round_bf16((a * t10) + (b * t11))
    return out


def block_quant(x, block=BLOCK):
    """x [S, H, D] fp32 -> (codes [H, Spad, D] int8, scales [H, Spad/block] fp32), one scale per
    (head, 128-token block): sc = max(amax, 1e-8) / 127, q = clamp(rint(x / sc), +-127); rows S..Spad are 0."""
    s, h, d = x.shape
    sp = spad(s)
    xp = np.zeros((sp, h, d), F32)
    xp[:s] = x
    xb = xp.reshape(sp // block, block, h, d)
    amax = np.abs(xb).max(axis=(1, 3))                        # [nblk, H]
    sc = (np.maximum(amax, F32(1e-8)) / F32(127.0)).astype(F32)
    q = np.clip(np.rint(xb / sc[:, None, :, None]), -127, 127).astype(np.int8)
    codes = np.ascontiguousarray(q.reshape(sp, h, d).transpose(1, 0, 2))
    return codes, np.ascontiguousarray(sc.T)


def prepass(q, k, rr=None, smooth_k=True):
    """Pre-pass operands: (q8 [H,Spad,D], qs [H,Spad/128], k8, ks, kmean [H,D]).
    q, k [S, H, D] bf16 bits; rr = (tab, qw, kw, eps) applies the per-head RMSNorm + RoPE first."""
    if rr is not None:
        tab, qw, kw, eps = rr
        qf = rms_rope(q, tab, qw, eps)
        kf = rms_rope(k, tab, kw, eps)
        km = (kf.astype(np.float64).sum(axis=0) / kf.shape[0]).astype(F32)
    else:
        qf = _as_f32(q)
        kf = _as_f32(k)
        km = kmean(k)
    if not smooth_k:
        km = np.zeros_like(km)
    q8, qs = block_quant(qf)
    k8, ks = block_quant((kf - km[None]).astype(F32))
    return q8, qs, k8, ks, km


def attention_from_codes(q8, qs, k8, ks, v, scale, rows=None, heads=None):
    """Attention on the INT8 operands, float64 softmax: out[s, h] = softmax_j(scale * qs*ks * q8.k8) v.
    q8/k8 [H, Spad, D] int8; qs/ks [H, Spad/128]; v [S, H, D] bf16 bits (or fp32). Sk is v's S
    (cross-attention: q8 may have another length). rows: query indices to evaluate (default all).
    Returns fp32 [len(rows), len(heads), D]."""
    vf = _as_f32(v).astype(np.float64)
    sk = vf.shape[0]
    hh = range(q8.shape[0]) if heads is None else heads
    sq = q8.shape[1] if rows is None else None
    rows = np.arange(sq) if rows is None else np.asarray(rows)
    out = np.zeros((len(rows), len(hh), D), F32)
    for hi, h in enumerate(hh):
        qd = q8[h, rows].astype(np.float64) * np.repeat(qs[h], BLOCK)[rows][:, None]
        kd = k8[h, :sk].astype(np.float64) * np.repeat(ks[h], BLOCK)[:sk][:, None]
        lg = (qd @ kd.T) * scale
        lg -= lg.max(axis=1, keepdims=True)
        p = np.exp(lg)
        out[:, hi] = ((p @ vf[:, h]) / p.sum(axis=1, keepdims=True)).astype(F32)
    return out


def attention_exact(q, k, v, scale, rows=None, heads=None):
    """Unquantized float64 attention on q, k, v [S, H, D] (bf16 bits or fp32) for the error report."""
    qf = _as_f32(q).astype(np.float64)
    kf = _as_f32(k).astype(np.float64)
    vf = _as_f32(v).astype(np.float64)
    hh = range(qf.shape[1]) if heads is None else heads
    rows = np.arange(qf.shape[0]) if rows is None else np.asarray(rows)
    out = np.zeros((len(rows), len(hh), D), F32)
    for hi, h in enumerate(hh):
        lg = (qf[rows, h] @ kf[:, h].T) * scale
        lg -= lg.max(axis=1, keepdims=True)
        p = np.exp(lg)
        out[:, hi] = ((p @ vf[:, h]) / p.sum(axis=1, keepdims=True)).astype(F32)
    return out


def rope_table(positions, rot=96, theta=10000.0):
    """A split-half RoPE table [S, rot/2, 2, 2] fp32 = (cos, -sin, sin, cos) for integer positions [S]
    (the layout of bench/rmsrope_fuse.py:22-33; the caller rounds it to bf16)."""
    hr = rot // 2
    inv = theta ** (-np.arange(hr, dtype=np.float64) / hr)
    ang = np.asarray(positions, np.float64)[:, None] * inv[None, :]
    c, s = np.cos(ang), np.sin(ang)
    return np.stack([np.stack([c, -s], -1), np.stack([s, c], -1)], -2).astype(F32)
