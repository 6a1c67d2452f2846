"""The attention override of the reference's RapidH3Int8Attention node (__init__.py:994-1046) without
ComfyUI's model objects: make_override(config, exact_rows) returns the callable ComfyUI installs as
transformer_options["optimized_attention_override"].

Behaviour kept from the reference:
  * calls with mask None, skip_reshape, q/k/v [1, H, S, 128] bf16 of one shape and S >= 1024 run the INT8
    kernel with config % 100 (attn_int8.attention); anything else goes to the previous override or to func;
  * exact_rows: a comma-separated list of segment kinds; after the INT8 call the query rows of those
    segments (merged [a, b) spans of transformer_options["minimax_h3_layout"].segments, cached per layout)
    are recomputed exactly (:1006-1022, :1035-1037). The reference uses bf16 scaled_dot_product_attention
    there; this build computes those rows in fp32 and rounds them to bf16;
  * config >= 100 (and no exact_rows) tags the override with rapidh3_rmsrope = config % 100 for the fused
    block, config >= 200 with rapidh3_rrcheck (:1000, :1043-1045);
  * a call carrying transformer_options["rapidh3_text_bias"] with S >= 1024 raises (the bias needs the fused
    block path, :1025-1027).
stock_attention stands in for ComfyUI's optimized_attention, the function an override receives as func and falls
through to. rr_check is the reference's config-2xx check of the fused RMSNorm + RoPE path (_rr_check, :334-349).
"""
import json
import os

import torch

from . import attention as _attention
from . import attn_int8


def merge_spans(segments, kinds):
    """Merged [a, b) row spans of the segments (a, b, kind) whose kind is in kinds (__init__.py:1006-1022)."""
    spans = []
    for a, b, kind in segments:
        if kind in kinds and b > a:
            if spans and spans[-1][1] == a:
                spans[-1][1] = b
            else:
                spans.append([a, b])
    return [tuple(x) for x in spans]


def exact_attention_rows(q, k, v, out, spans, scale=None):
    """Overwrite query rows [a, b) of out with exact attention (q, k, v, out in [1, H, S, 128]); fp32 math."""
    for a, b in spans:
        ref = torch.nn.functional.scaled_dot_product_attention(q[:, :, a:b].float(), k.float(), v.float(),
                                                               scale=scale)
        out[:, :, a:b] = ref.to(out.dtype)
    return out


def stock_attention(q, k, v, heads, mask=None, attn_precision=None, skip_reshape=False, skip_output_reshape=False,
                    transformer_options=None, scale=None, **kwargs):
    """The stock attention an override falls through to, in ComfyUI's optimized_attention calling convention: q, k, v
    [B, H, S, D] with skip_reshape, else [B, S, H * D]; the output [B, H, Sq, D] with skip_output_reshape, else
    [B, Sq, H * D], in q.dtype. Computed in fp32 (torch's scaled_dot_product_attention on fp32 copies, 1024 query rows
    at a time) and rounded once; mask is added to the scores (bool: True keeps)."""
    if not skip_reshape:
        b, _, hd = q.shape
        d = hd // heads
        q, k, v = (t.reshape(b, -1, heads, d).transpose(1, 2) for t in (q, k, v))
    b, h, sq, d = q.shape
    out = torch.empty(b, h, sq, d, dtype=q.dtype, device=q.device)
    kf, vf = k.float().contiguous(), v.float().contiguous()
    for a in range(0, sq, 1024):
        m = mask
        if m is not None and m.dim() >= 2 and m.shape[-2] == sq:
            m = m[..., a:a + 1024, :]
        out[:, :, a:a + 1024] = torch.nn.functional.scaled_dot_product_attention(
            q[:, :, a:a + 1024].float().contiguous(), kf, vf, attn_mask=m, scale=scale).to(q.dtype)
    if skip_output_reshape:
        return out
    return out.transpose(1, 2).reshape(b, sq, h * d)


def rr_check(q, k, v, o, tab, qw, kw, eps, cfg, transformer_options):
    """The config-2xx check (the reference's _rr_check, __init__.py:334-349) on the real q, k, v of one fused block:
    the fused RMSNorm + RoPE path's output o [1, H, S, 128] and its pre-pass operands against the unfused path
    (attention.rms_rope_ on copies of q, k, then attn_int8.attention with the same config). One JSON line per call,
    appended to $RAPIDH3_RRCHECK (default /data/output/rapidh3_rrcheck.jsonl, as in the reference). q, k, v:
    the raw [S, H, 128] qkv-projection views."""
    qc, kc = q.clone(), k.clone()
    _attention.rms_rope_(qc, kc, tab, qw, kw, eps)
    ref = attn_int8.attention(qc, kc, v, config=cfg)
    pu = attn_int8.ext().int8_prepass(qc, kc, v, config=cfg)
    pf = attn_int8.ext().int8_prepass(q, k, v, tab, qw, kw, eps, config=cfg)
    got = o[0].transpose(0, 1)
    rec = {"block": transformer_options.get("block_index"), "S": q.shape[0],
           "out_equal": torch.equal(ref, got),
           "operands_equal": all(a is None and b is None or torch.equal(a, b) for a, b in zip(pu, pf)),
           "max_abs_diff": float((ref.float() - got.float()).abs().max())}
    path = os.environ.get("RAPIDH3_RRCHECK", "/data/output/rapidh3_rrcheck.jsonl")
    with open(path, "a") as f:
        f.write(json.dumps(rec) + "\n")
    return rec


def make_override(config, exact_rows="", prev=None):
    exact = {s.strip() for s in exact_rows.split(",") if s.strip()}
    rmsrope, rrcheck = config >= 100 and not exact, config >= 200
    cfg = config % 100
    cache = {}

    def exact_spans(opts, s):
        lay = opts.get("minimax_h3_layout")
        if lay is None or getattr(lay, "seq_len", None) != s:
            return ()
        hit = cache.get(id(lay))
        if hit is not None and hit[0] is lay:
            return hit[1]
        cache.clear()
        cache[id(lay)] = (lay, merge_spans(lay.segments, exact))
        return cache[id(lay)][1]

    def override(func, *args, **kwargs):
        q, k, v = args[:3]
        mask = kwargs.get("mask", args[4] if len(args) > 4 else None)
        opts = kwargs.get("transformer_options") or {}
        if opts.get("rapidh3_text_bias") is not None and q.shape[-2] >= 1024:
            raise RuntimeError("RapidH3TextAttnBias: DiT attention left the fused INT8 path (fused block with "
                               "attention config 190 or 194 needed)")
        if (mask is None and kwargs.get("skip_reshape") and q.dim() == 4 and q.shape[0] == 1
                and q.shape == k.shape == v.shape and q.shape[-1] == 128 and q.shape[2] >= 1024
                and q.dtype == torch.bfloat16):
            out = torch.empty_like(q)
            attn_int8.attention(q[0].transpose(0, 1), k[0].transpose(0, 1), v[0].transpose(0, 1),
                                kwargs.get("scale"), config=cfg, out=out[0].transpose(0, 1))
            if exact:
                exact_attention_rows(q, k, v, out, exact_spans(opts, q.shape[2]), kwargs.get("scale"))
            if kwargs.get("skip_output_reshape"):
                return out
            return out.transpose(1, 2).reshape(1, q.shape[2], -1)
        return prev(func, *args, **kwargs) if prev else func(*args, **kwargs)

    if rmsrope:
        override.rapidh3_rmsrope = cfg
        override.rapidh3_rrcheck = rrcheck
    return override
