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


def attention_from_codes(q8, qs, k8, ks, v, scale, rows=None, heads=None, out_dtype=F32):
    """Attention on the INT8 operands, float64 softmax: out[s, h] = softmax_j(scale * qs*ks * q8.k8) v.
    q8/k8 [H, Spad, D] int8; qs/ks [H, Spad/128]; v [S, H, D] bf16 bits (or fp32). Sk is v's S
    (cross-attention: q8 may have another length). rows: query indices to evaluate (default all).
    Returns [len(rows), len(heads), D] in out_dtype (fp32; np.float64 keeps the float64 result)."""
    vf = _as_f32(v).astype(np.float64)
    sk = vf.shape[0]
    hh = range(q8.shape[0]) if heads is None else heads
    sq = q8.shape[1] if rows is None else None
    rows = np.arange(sq) if rows is None else np.asarray(rows)
    out = np.zeros((len(rows), len(hh), D), out_dtype)
    for hi, h in enumerate(hh):
        qd = q8[h, rows].astype(np.float64) * np.repeat(qs[h], BLOCK)[rows][:, None]
        kd = k8[h, :sk].astype(np.float64) * np.repeat(ks[h], BLOCK)[:sk][:, None]
        lg = (qd @ kd.T) * scale
        lg -= lg.max(axis=1, keepdims=True)
        p = np.exp(lg)
        out[:, hi] = ((p @ vf[:, h]) / p.sum(axis=1, keepdims=True)).astype(out_dtype)
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



# ---------------------------------------------------------------- production numerics (configs 80-99)
# The reference's production attention (attn_int8.cu config 80 = attn_fwd8 :2250-2511; configs 90/94 run the
# same math on a persistent schedule, csrc/attn_cake/DESIGN.md in the reference: "bit-identical to config 80"):
#   pre-pass  (attn_int8.cu:2568-2644)
#     * kmean, vmean: per-head channel means over all S tokens (K after the optional RMSNorm + RoPE);
#       vscale = max(max(vmax - vm, vm - vmin), 1e-6) / 127                                (:97-109)
#     * Q, K per (token, head) row: [RMSNorm + RoPE], K - kmean, the normalized Walsh-Hadamard H128 when
#       rotate, sc = max(amax, 1e-8) / 127, q = rint(x * (1 / sc)); padded rows 0 with scale 0  (:130-170)
#     * ksb = (sc, fp32(-1.5*2^23 * sc)) per key; padded keys (0, -inf)                    (:138, :168)
#     * V per channel: code = rint((v - vm) / vscale)                                        (:452-475)
#   main kernel, per 128-key tile (:2400-2470)
#     * t = fma(float(1.5*2^23 + acc), s_j, b_j) (the integer accumulator starts at the bits of 1.5*2^23)
#     * tm = tile row max, n = max(m, tm), a = 2^((m - n) c), ts = 2^((tm - n) c), m = n, with
#       c = qs * scale * log2(e)
#     * P = sat_u8(rint(2^(fma(t, c, fma(-tm, c, log2 255))))), rs = sum P, l = fma(ts, rs, l a)
#     * O = a O + ts * sum_j P_j v8_j; out = bf16(fma(O (1 / l), vscale, vmean))
#   text bias (attn_cake.cuh:97-99, :210-240): t += bias*log2(e) / c on keys [0, nbias) after the dequant.
# Orders fixed by this build: kmean / vmean are float64 sums divided by S in float64 and rounded once (the
# reference sums in fp32 per 256-token chunk); the Walsh-Hadamard stages are the reference's own (strides
# 1, 2, ..., 64, each stage rounded to fp32), so codes and scales are bit-exact.

MAGIC = F32(12582912.0)               # 1.5 * 2^23 (attn_int8.cu:22-23)
MAGIC_I = 0x4B400000
LOG2_255 = F32(7.99435343685886)      # attn_int8.cu:24
INV_SQRT128 = F32(0.08838834764831845)
TILE = 128


def hadamard128(x):
    """Normalized Walsh-Hadamard transform over the last axis (attn_int8.cu:113-128): radix-2 stages at
    strides 1, 2, 4, ..., 64, (a, b) -> (a + b, a - b) in fp32, then * fp32(1 / sqrt(128))."""
    y = np.asarray(x, F32)
    shp = y.shape
    for s in (1, 2, 4, 8, 16, 32, 64):
        v = y.reshape(shp[:-1] + (D // (2 * s), 2, s))
        a, b = v[..., 0, :], v[..., 1, :]
        y = np.stack([a + b, a - b], axis=-2).reshape(shp)
    return (y * INV_SQRT128).astype(F32)


def token_quant(x, rotate=True):
    """x [S, H, D] fp32 -> (codes [H, Spad, D] int8, scales [H, Spad] fp32), one scale per (token, head)
    (attn_int8.cu:130-170); rows S..Spad are code 0, scale 0."""
    s, h, _ = x.shape
    y = hadamard128(x) if rotate else np.asarray(x, F32)
    amax = np.abs(y).max(axis=2)
    sc = (np.maximum(amax, F32(1e-8)) / F32(127.0)).astype(F32)
    inv = (F32(1.0) / sc).astype(F32)
    q = np.rint((y * inv[..., None]).astype(F32))
    assert np.abs(q).max() <= 127
    sp = spad(s)
    codes = np.zeros((h, sp, D), np.int8)
    codes[:, :s] = q.astype(np.int8).transpose(1, 0, 2)
    scales = np.zeros((h, sp), F32)
    scales[:, :s] = sc.T
    return codes, scales


def v_int8(v, smooth_v=True):
    """V [S, H, D] (bf16 bits) -> (codes [S, H, D] int8, vscale [H, D], vmean [H, D]) per channel
    (attn_int8.cu:97-109, :452-475)."""
    vf = _as_f32(v)
    s = vf.shape[0]
    vm = ((vf.astype(np.float64).sum(axis=0) / s).astype(F32) if smooth_v
          else np.zeros(vf.shape[1:], F32))
    rng = np.maximum((vf.max(axis=0) - vm).astype(F32), (vm - vf.min(axis=0)).astype(F32))
    sc = (np.maximum(rng, F32(1e-6)) / F32(127.0)).astype(F32)
    codes = np.rint(((vf - vm[None]).astype(F32) / sc[None]).astype(F32))
    assert np.abs(codes).max() <= 127
    return codes.astype(np.int8), sc, vm


def prepass_u8(q, k, v, rr=None, smooth_k=True, smooth_v=True, rotate=True):
    """Production pre-pass operands: dict q8, qs [H, Sqpad], k8, ks, ksb [H, Skpad, 2] fp32, kmean [H, D],
    v8 [S, H, D] int8 codes, vscale, vmean [H, D], vinit [H, Skpad/128, D] int32 = 1.5*2^23 bits + 128 *
    (sum of the tile's V codes per channel) (the start value of the kernel's P.V accumulator). q [Sq, H, D],
    k, v [Sk, H, D] bf16 bits; rr = (tab, qw, kw, eps) applies the per-head RMSNorm + RoPE to q and k."""
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
    q8, qs = token_quant(qf, rotate)
    k8, ks = token_quant((kf - km[None]).astype(F32), rotate)
    sk = kf.shape[0]
    ksb = np.stack([ks, (F32(-MAGIC) * ks).astype(F32)], axis=-1)
    ksb[:, sk:, 1] = -np.inf
    v8, vs, vm = v_int8(v, smooth_v)
    skp = spad(sk)
    vpad = np.zeros((skp, v8.shape[1], D), np.int64)
    vpad[:sk] = v8
    vsum = vpad.reshape(skp // TILE, TILE, -1, D).sum(axis=1).transpose(1, 0, 2)     # [H, ntiles, D]
    vinit = (MAGIC_I + 128 * vsum).astype(np.int32)
    return dict(q8=q8, qs=qs, k8=k8, ks=ks, ksb=ksb, kmean=km, v8=v8, vscale=vs, vmean=vm, vinit=vinit)


def _fma32(a, b, c):
    """fp32 fma(a, b, c) for fp32 operands: the float64 product is exact, the sum is rounded once more
    (a double rounding only when the float64 sum is inexact, which these magnitudes make rare)."""
    return (np.asarray(a, np.float64) * np.asarray(b, np.float64) + np.asarray(c, np.float64)).astype(F32)


def attention_u8_from_codes(pp, scale, rows=None, heads=None, sk=None, nbias=0, bias=0.0):
    """The production main kernel's arithmetic on the pre-pass operands, tile by tile (128 keys): fp32 t, tile
    max, u8 P = rint(2^x) with 2^x evaluated in float64 from the fp32 argument (the kernels' exp2 is a
    hardware approximation, so a P next to a .5 boundary may differ by one), exact integer P.V per tile and a
    float64 fold. Returns fp32 [len(rows), len(heads), D] before the bf16 rounding of the output."""
    q8, qs, k8, ksb, v8 = pp["q8"], pp["qs"], pp["k8"], pp["ksb"], pp["v8"]
    sk = v8.shape[0] if sk is None else sk
    skp = spad(sk)
    hh = range(q8.shape[0]) if heads is None else heads
    rows = np.arange(q8.shape[1]) if rows is None else np.asarray(rows)
    sl2 = F32(F32(scale) * F32(1.4426950408889634))
    bl2 = F32(bias * 1.4426950408889634)
    out = np.zeros((len(rows), len(hh), D), F32)
    for hi, h in enumerate(hh):
        vp = np.zeros((skp, D), np.int64)
        vp[:sk] = v8[:, h]
        # |acc| <= 128 * 127^2 < 2^53: the float64 product is the exact integer
        acc = q8[h, rows].astype(np.float64) @ k8[h, :skp].astype(np.float64).T
        with np.errstate(invalid="ignore"):
            t = _fma32((MAGIC + acc).astype(F32), ksb[h, :skp, 0][None], ksb[h, :skp, 1][None])
        c = (qs[h, rows] * sl2).astype(F32)[:, None]
        if nbias > 0:
            ib = np.where(c > 0, (bl2 / np.where(c > 0, c, 1)).astype(F32), F32(0)).astype(F32)
            t[:, :nbias] = (t[:, :nbias] + ib).astype(F32)
        m = np.full((len(rows), 1), -np.inf, F32)
        l = np.zeros((len(rows), 1))
        o = np.zeros((len(rows), D))
        for j0 in range(0, skp, TILE):
            tt = t[:, j0:j0 + TILE]
            tm = tt.max(axis=1, keepdims=True)
            n = np.maximum(m, tm)
            with np.errstate(invalid="ignore"):
                a = np.exp2(((m - n) * c).astype(F32).astype(np.float64))
                ts = np.exp2(((tm - n) * c).astype(F32).astype(np.float64))
            a = np.nan_to_num(a, nan=0.0)
            m = n
            b = _fma32(-tm, c, LOG2_255)
            with np.errstate(invalid="ignore"):
                e = np.exp2(_fma32(tt, c, b).astype(np.float64))
            p = np.clip(np.rint(np.nan_to_num(e, nan=0.0)), 0, 255)
            l = l * a + ts * p.sum(axis=1, keepdims=True)
            o = o * a + ts * (p @ vp[j0:j0 + TILE].astype(np.float64))
        out[:, hi] = (o / l * pp["vscale"][h][None].astype(np.float64) + pp["vmean"][h][None]).astype(F32)
    return out


def block_quant_rot(x, rotate=True):
    """Per-128-key-block K quantizer of configs 60-61 (attn_int8.cu:404-443, quant_k_block): x [S, H, D] fp32
    (K - kmean) -> [normalized H128] -> one scale per (head, 128-token block) sc = max(amax, 1e-8) / 127 and
    q = rint(x * fp32(1 / sc)) (the reference kernel multiplies by the reciprocal) -> (codes [H, Spad, D] int8,
    kbs [H, Spad / 128] fp32). Rows S..Spad are zero, inside the block max and as codes."""
    s, h, _ = x.shape
    y = hadamard128(x) if rotate else np.asarray(x, F32)
    sp = spad(s)
    yp = np.zeros((sp, h, D), F32)
    yp[:s] = y
    blk = yp.reshape(sp // BLOCK, BLOCK, h, D)
    amax = np.abs(blk).max(axis=(1, 3))                                   # [nblk, H]
    sc = (np.maximum(amax, F32(1e-8)) / F32(127.0)).astype(F32)
    inv = (F32(1.0) / sc).astype(F32)
    q = np.rint((blk * inv[:, None, :, None]).astype(F32))
    assert np.abs(q).max() <= 127
    codes = np.ascontiguousarray(q.reshape(sp, h, D).astype(np.int8).transpose(1, 0, 2))
    return codes, np.ascontiguousarray(sc.T)


def prepass_blockk(q, k, v, smooth_k=True, smooth_v=True, rotate=True):
    """Pre-pass operands of configs 60-61 (attn_int8.cu:2618-2641 without the RMSNorm + RoPE path, which those
    configs do not have): dict q8, qs [H, Sqpad] (per token, as prepass_u8), k8 [H, Skpad, D] and kbs
    [H, Skpad / 128] (one K scale per 128-key block after the smoothing and the H128 rotation), kmean, v8,
    vscale, vmean, vinit (as prepass_u8)."""
    qf, kf = _as_f32(q), _as_f32(k)
    km = kmean(k) if smooth_k else np.zeros((kf.shape[1], D), F32)
    q8, qs = token_quant(qf, rotate)
    k8, kbs = block_quant_rot((kf - km[None]).astype(F32), rotate)
    v8, vs, vm = v_int8(v, smooth_v)
    sk = kf.shape[0]
    skp = spad(sk)
    vpad = np.zeros((skp, v8.shape[1], D), np.int64)
    vpad[:sk] = v8
    vsum = vpad.reshape(skp // TILE, TILE, -1, D).sum(axis=1).transpose(1, 0, 2)
    vinit = (MAGIC_I + 128 * vsum).astype(np.int32)
    return dict(q8=q8, qs=qs, k8=k8, kbs=kbs, kmean=km, v8=v8, vscale=vs, vmean=vm, vinit=vinit)


def attention_blockk_from_codes(pp, scale, rows=None, heads=None, sk=None):
    """The main kernel of configs 60-61 (attn_fwd6, attn_int8.cu:1786-1962) on prepass_blockk's operands, tile by
    tile (128 keys). Per query and tile: the accumulator read as the float 1.5*2^23 + acc (keys past Sk forced to
    1.5*2^23 - 2^22), integer tile max ti, cc = fp32(c * kb) with c = qs * scale * log2(e), tv = (ti - 1.5*2^23) cc,
    n = max(m, tv), a = 2^(m - n), ts = 2^(tv - n), b = fma(-ti, cc, log2 255), P = rint(2^(fma(acc, cc, b))) in
    [0, 255], l = l a + ts sum P, O = O a + ts (P . V8) (exact integers per tile), out = O / l * vscale + vmean.
    2^x in float64 from the fp32 argument (the kernels' exp2 is a hardware approximation); the reference's
    P = 256 wrap (possible only when cc * 2^23 is large) is a saturation at 255 here. Returns fp32
    [len(rows), len(heads), D] before the bf16 rounding of the output."""
    q8, qs, k8, kbs, v8 = pp["q8"], pp["qs"], pp["k8"], pp["kbs"], pp["v8"]
    sk = v8.shape[0] if sk is None else sk
    skp = spad(sk)
    hh = range(q8.shape[0]) if heads is None else heads
    rows = np.arange(q8.shape[1]) if rows is None else np.asarray(rows)
    sl2 = F32(F32(scale) * F32(1.4426950408889634))
    out = np.zeros((len(rows), len(hh), D), F32)
    for hi, h in enumerate(hh):
        vp = np.zeros((skp, D), np.int64)
        vp[:sk] = v8[:, h]
        acc = q8[h, rows].astype(np.float64) @ k8[h, :skp].astype(np.float64).T
        bits = (MAGIC + acc).astype(F32)                       # exact: |acc| < 2^21
        bits[:, sk:] = MAGIC - F32(2 ** 22)
        c = (qs[h, rows] * sl2).astype(F32)[:, None]
        m = np.full((len(rows), 1), -np.inf, F32)
        l = np.zeros((len(rows), 1))
        o = np.zeros((len(rows), D))
        for j0 in range(0, skp, TILE):
            bt = bits[:, j0:j0 + TILE]
            ti = bt.max(axis=1, keepdims=True)
            cc = (c * kbs[h, j0 // TILE]).astype(F32)
            tv = ((ti - MAGIC).astype(F32) * cc).astype(F32)
            n = np.maximum(m, tv)
            with np.errstate(invalid="ignore"):
                a = np.nan_to_num(np.exp2((m - n).astype(F32).astype(np.float64)), nan=0.0)
            ts = np.exp2((tv - n).astype(F32).astype(np.float64))
            m = n
            b = _fma32(-ti, cc, LOG2_255)
            p = np.clip(np.rint(np.exp2(_fma32(bt, cc, b).astype(np.float64))), 0, 255)
            l = l * a + ts * p.sum(axis=1, keepdims=True)
            o = o * a + ts * (p @ vp[j0:j0 + TILE].astype(np.float64))
        out[:, hi] = (o / l * pp["vscale"][h][None].astype(np.float64) + pp["vmean"][h][None]).astype(F32)
    return out


LOG2_448 = F32(8.807354922057604)      # attn_int8.cu:1557
V_FP8_STRETCH = F32(F32(448.0) / F32(127.0))   # attn_int8.cu:468 (r = 448.f / 127.f)
V_FP8_UNSTRETCH = F32(F32(127.0) / F32(448.0))  # attn_int8.cu:2642 (vscale *= 127.f / 448.f)


def v_fp8(v, smooth_v=True):
    """V [S, H, D] (bf16 bits) -> (e4m3fn codes [S, H, D] uint8, vscale [H, D], vmean [H, D]) for the FP8 P.V
    configs (attn_int8.cu:467-473): code = e4m3(satfinite(((v - vmean) / vscale) * fp32(448 / 127))), vscale and
    vmean as v_int8 (the kernel's epilogue multiplies vscale by fp32(127 / 448), :2642)."""
    from .numerics import f32_to_fp8_e4m3
    vf = _as_f32(v)
    _, sc, vm = v_int8(v, smooth_v)
    x = (((vf - vm[None]).astype(F32) / sc[None]).astype(F32) * V_FP8_STRETCH).astype(F32)
    return f32_to_fp8_e4m3(np.clip(x, F32(-448.0), F32(448.0))), sc, vm


def prepass_fp8v(q, k, v, rr=None, smooth_k=True, smooth_v=True, rotate=True):
    """Pre-pass operands of the FP8 P.V configs 50-56 (attn_int8.cu:2568-2644 with fp8v): Q / K as prepass_u8
    (per-token codes and scales, per-key (scale, bias) pairs), V as e4m3 codes (v_fp8)."""
    pp = prepass_u8(q, k, v, rr, smooth_k, smooth_v, rotate)
    vf8, vs, vm = v_fp8(v, smooth_v)
    pp.update(vf8=vf8, vscale=vs, vmean=vm)
    for n in ("v8", "vinit"):
        pp.pop(n)
    return pp


def attention_fp8pv_from_codes(pp, scale, rows=None, heads=None, sk=None, tile=64):
    """The FP8 P.V main kernel (attn_fwd5, attn_int8.cu:1563-1785) on prepass_fp8v's operands, tile by tile (tile =
    64 keys for configs 50, 51, 54, 56, 128 for 52, 53, 55): t = fma(1.5*2^23 + acc, s_key, b_key), tile max tm;
    where tm exceeds the running max m: n = max(m, tm), O and l scaled by 2^((m - n) c), m = n; then
    p = 2^(fma(t, c, fma(-m, c, log2 448))) (0 < p <= 448), l += p (unquantized), O += e4m3(p) . e4m3 V;
    out = O / l * (vscale * fp32(127 / 448)) + vmean. 2^x in float64 from the fp32 argument, the sums in float64
    (the kernels' exp2 is a hardware approximation and their sums are fp32). Returns fp32 [rows, heads, D]."""
    from .numerics import f32_to_fp8_e4m3, fp8_e4m3_to_f32
    q8, qs, k8, ksb, vf8 = pp["q8"], pp["qs"], pp["k8"], pp["ksb"], pp["vf8"]
    sk = vf8.shape[0] if sk is None else sk
    skp = spad(sk)
    hh = range(q8.shape[0]) if heads is None else heads
    rows = np.arange(q8.shape[1]) if rows is None else np.asarray(rows)
    sl2 = F32(F32(scale) * F32(1.4426950408889634))
    out = np.zeros((len(rows), len(hh), D), F32)
    for hi, h in enumerate(hh):
        vp = np.zeros((skp, D), np.float64)
        vp[:sk] = fp8_e4m3_to_f32(vf8[:, h])
        acc = q8[h, rows].astype(np.float64) @ k8[h, :skp].astype(np.float64).T
        with np.errstate(invalid="ignore"):
            t = _fma32((MAGIC + acc).astype(F32), ksb[h, :skp, 0][None], ksb[h, :skp, 1][None])
        c = (qs[h, rows] * sl2).astype(F32)[:, None]
        m = np.full((len(rows), 1), -np.inf, F32)
        l = np.zeros((len(rows), 1))
        o = np.zeros((len(rows), D))
        for j0 in range(0, skp, tile):
            tt = t[:, j0:j0 + tile]
            tm = tt.max(axis=1, keepdims=True)
            n = np.maximum(m, tm)
            with np.errstate(invalid="ignore"):
                a = np.nan_to_num(np.exp2(((m - n).astype(F32) * c).astype(F32).astype(np.float64)), nan=0.0)
            o, l, m = o * a, l * a, n
            b = _fma32(-m, c, LOG2_448)
            with np.errstate(invalid="ignore"):
                p = np.nan_to_num(np.exp2(_fma32(tt, c, b).astype(np.float64)), nan=0.0).astype(F32)
            l = l + p.astype(np.float64).sum(axis=1, keepdims=True)
            p8 = fp8_e4m3_to_f32(f32_to_fp8_e4m3(np.minimum(p, F32(448.0)))).astype(np.float64)
            o = o + p8 @ vp[j0:j0 + tile]
        vs = (pp["vscale"][h] * V_FP8_UNSTRETCH).astype(F32).astype(np.float64)
        out[:, hi] = (o / l * vs[None] + pp["vmean"][h][None]).astype(F32)
    return out
