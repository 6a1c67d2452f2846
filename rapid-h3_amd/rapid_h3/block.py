"""The fused INT8 DiT block chain on the HIP kernels: the call sequence of the reference's
_fused_block (/root/reference/custom_nodes/rapid_h3/__init__.py:207-321), plus _row_index (:189-200)
and the per-segment gated residual (:242-251). Two recipes: int8_rot (the reference's, every quantizer
with the ConvRot H256 rotation and weights quantized with quantize_weight(w, "int8_rot")) and
int8_rowwise (the same chain without rotation, the configuration the benchmark names).

    x [S, hidden] bf16 residual stream (updated in place and returned)
    RMSNorm + modulation -> INT8 (one pass)        rh3_quant_norm_mod_i8      / rh3_norm_mod_rot_quant_i8
    QKV GEMM                                       rh3_gemm_i8 (fuse_qkv: rh3_gemm_i8_qkv, + Q operands, K/V stats)
    q/k RMSNorm + RoPE + INT8 attention            rh3_attention_prepass_qkv + rh3_attention_forward (head-major
                                                   out; production numerics: the *_u8 entry points)
    head-major gather -> INT8                      rh3_quant_heads_i8         / rh3_rot_quant_heads_i8
    out-proj GEMM + gated residual, per segment    rh3_gemm_i8_gated
    RMSNorm + modulation -> INT8                   rh3_quant_norm_mod_i8      / rh3_norm_mod_rot_quant_i8
    FFN-up GEMM + SwiGLU epilogue                  rh3_gemm_i8_swiglu
    INT8 of h                                      rh3_quant_rows_i8          / rh3_rot_quant_rows_i8
    FFN-down GEMM + gated residual, per segment    rh3_gemm_i8_gated

ComfyUI objects (the block module, adaln_proj, model management) are outside this build: the caller
passes the weights and the modulation tables as tensors.
"""
from dataclasses import dataclass

import torch

from . import attention as _attn
from . import gemm as _gemm
from . import quant as _quant
from .kernels import QWeight

D = 128


@dataclass
class BlockWeights:
    """Quantized weights of one DiT block (each QWeight: q [N, K] int8, scale [1, N] fp32).
    fc1 holds [gate | up] rows already permuted with swiglu_perm (the reference caches that order,
    __init__.py:231-240)."""
    qkv: QWeight
    out: QWeight
    fc1_perm: QWeight
    fc2: QWeight
    norm1_w: torch.Tensor
    norm2_w: torch.Tensor
    q_norm_w: torch.Tensor
    k_norm_w: torch.Tensor
    heads: int
    eps: float = 1e-6
    qk_eps: float = 1e-6
    recipe: str = "int8_rowwise"      # or "int8_rot": the weights above must be quantized the same way


_ROW_INDEX = {}


def row_index(segments, s, device):
    """Per-token modulation-row index (int32 [S]) from [(start, stop, row)] (__init__.py:189-200). Like the
    reference, the last index built is kept for the same segments object (identity, S and device), so the blocks of
    one model call build it once; a caller that edits a segments list in place passes a new list instead."""
    key = (id(segments), s, str(device))
    hit = _ROW_INDEX.get(key)
    if hit is not None and hit[0] is segments:
        return hit[1]
    idx = torch.empty(s, dtype=torch.int32, device=device)
    for a, b, row in segments:
        idx[a:b] = row.to(device=device, dtype=torch.int32) if torch.is_tensor(row) else int(row)
    _ROW_INDEX.clear()
    _ROW_INDEX[key] = (segments, idx)
    return idx


def gemm_gated(xq, xs, qw, x, gate, segments):
    """x += gate[row] * (xq @ W^T) per modality segment, in the GEMM epilogue (__init__.py:242-251).
    gate: [R, N] table (bf16 or fp32), rounded to bf16 like _mod_row. A segment's row is an int (one gate row for
    the segment) or a tensor of per-token rows (the reference's _mod_gate branch, __init__.py:244-245), which runs
    the per-row gate epilogue."""
    gate2 = gate.reshape(-1, gate.shape[-1])
    for a, b, row in segments:
        if torch.is_tensor(row):
            _gemm.int8_gemm_gated_residual_rows(xq[a:b], xs[a:b], qw.q, qw.scale, gate2, row, x[a:b])
            continue
        g = gate2[int(row)].to(torch.bfloat16).reshape(-1).contiguous()
        _gemm.int8_gemm_gated_residual(xq[a:b], xs[a:b], qw.q, qw.scale, g, x[a:b])
    return x


PHASES = ("quant_norm1", "gemm_qkv", "attn_prepass", "attn_main", "quant_heads", "gemm_out_gated", "quant_norm2",
          "gemm_up_swiglu", "quant_h", "gemm_down_gated")


_QUANTIZERS = {
    "int8_rowwise": (_quant.norm_mod_quant_rows_i8, _quant.heads_quant_rows_i8, _quant.quant_rows_i8),
    "int8_rot": (_quant.norm_mod_rot_quant_rows_i8, _quant.rot_quant_heads_i8, _quant.rot_quant_rows_i8),
}


def fused_block(x, w: BlockWeights, mod, segments, rope_tab, idx=None, mark=None, trace=None, attn_config=None,
                text_bias=None, fuse_qkv=False, attn_fn=None, attn_check=None):
    """One DiT block forward on x [S, hidden] bf16 (modified in place). mod = (shift_msa, scale_msa,
    gate_msa, shift_mlp, scale_mlp, gate_mlp), each [R, hidden]; rope_tab [1, S, 1, rot/2, 2, 2] bf16.
    mark: optional callable, called with each name of PHASES after that phase is enqueued (a timer
    records a stream event there); the kernels and their order are the same with or without it.
    trace: optional dict that receives every intermediate (a checker's view of each stage).
    attn_config: None runs the per-block bf16 P.V attention; an int runs the reference's production
    numerics with that config (its 1xx presets, __init__.py:274-291), 50-56 its FP8 P.V kernel. text_bias = (nbias, bias) adds the
    Jenga text bias (configs 90 / 94 only). fuse_qkv (even head counts): the QKV GEMM's epilogue writes the
    attention's Q operands and K / V statistics itself (gemm.int8_gemm_qkv, the reference's config 3xx
    path), so the pre-pass skips its Q pass and statistics passes; the result is the same bit for bit. Off by
    default: at the benchmark shape the longer GEMM epilogue costs 0.4-0.6 ms more than the pre-pass passes it
    removes.
    attn_fn(q, k, v) -> o [1, H, S, 128] bf16: the unfused attention route of the reference (__init__.py:295-305): q and
    k ([S, H, 128] views of the qkv output) get the per-head RMSNorm + RoPE in place (attention.rms_rope_), then attn_fn
    computes the attention (an installed override, or the stock attention); attn_config and text_bias do not apply.
    attn_check(q, k, v, o): called after the fused attention with the raw q, k, v views and o (the reference's
    config-2xx check, __init__.py:303-304)."""
    shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp = mod
    tick = mark or (lambda name: None)
    keep = trace.__setitem__ if trace is not None else (lambda k, v: None)
    if w.recipe not in _QUANTIZERS:
        raise ValueError(f"fused_block: recipe {w.recipe!r} (int8_rowwise or int8_rot)")
    norm_mod_q, heads_q, rows_q = _QUANTIZERS[w.recipe]
    s = x.shape[0]
    if idx is None:
        idx = row_index(segments, s, x.device)
    xq, xs = norm_mod_q(x, w.norm1_w, w.eps, idx, shift_msa, scale_msa)
    keep("xq1", xq), keep("xs1", xs)
    tick("quant_norm1")
    if attn_fn is not None:
        if attn_config is not None or text_bias is not None or fuse_qkv:
            raise RuntimeError("fused_block: attn_fn runs the unfused attention route (no attn_config, text_bias or "
                               "fuse_qkv)")
        o = _unfused_attention(xq, xs, w, rope_tab, s, tick, keep, attn_fn)
    else:
        o = _fused_attention(xq, xs, w, rope_tab, s, tick, keep, attn_config, text_bias, fuse_qkv, attn_check)
    oq, os_ = heads_q(o[0])
    keep("oq", oq), keep("os", os_)
    tick("quant_heads")
    del o
    x = gemm_gated(oq, os_, w.out, x, gate_msa, segments)
    if trace is not None:
        keep("x_attn", x.clone())
    tick("gemm_out_gated")
    xq, xs = norm_mod_q(x, w.norm2_w, w.eps, idx, shift_mlp, scale_mlp)
    keep("xq2", xq), keep("xs2", xs)
    tick("quant_norm2")
    hh = _gemm.int8_gemm_swiglu(xq, xs, w.fc1_perm.q, w.fc1_perm.scale)
    keep("h", hh)
    tick("gemm_up_swiglu")
    hq, hs = rows_q(hh)
    keep("hq", hq), keep("hs", hs)
    tick("quant_h")
    del hh
    x = gemm_gated(hq, hs, w.fc2, x, gate_mlp, segments)
    tick("gemm_down_gated")
    return x


def _unfused_attention(xq, xs, w, rope_tab, s, tick, keep, attn_fn):
    """QKV GEMM, RMSNorm + RoPE of q, k in place, then attn_fn (the reference's route when the installed attention
    override carries no fused-path tag, __init__.py:295-305)."""
    h = w.heads
    qkv = _gemm.int8_gemm(xq, xs, w.qkv.q, w.qkv.scale)
    keep("qkv", qkv)
    tick("gemm_qkv")
    q, k, v = (t.view(s, h, D) for t in qkv.split(h * D, dim=-1))
    _attn.rms_rope_(q, k, rope_tab, w.q_norm_w, w.k_norm_w, w.qk_eps)
    tick("attn_prepass")
    o = attn_fn(q, k, v)
    if tuple(o.shape) != (1, h, s, D) or o.dtype != torch.bfloat16 or o.stride(-1) != 1:
        raise RuntimeError(f"fused_block: attn_fn must return bf16 [1, {h}, {s}, {D}], got {o.dtype} "
                           f"{tuple(o.shape)}")
    keep("o", o)
    tick("attn_main")
    return o


def _fused_attention(xq, xs, w, rope_tab, s, tick, keep, attn_config, text_bias, fuse_qkv, attn_check):
    """QKV GEMM and this build's INT8 attention with the RMSNorm + RoPE in its pre-pass (attention_rr's two calls)."""
    h = w.heads
    x_dev = xq.device
    numerics = 0 if attn_config is None else 1
    if attn_config is None:
        if text_bias is not None:
            raise RuntimeError("text bias: needs the production attention (attn_config 90 or 94)")
    else:
        _attn._production(attn_config, "fused_block")
        if 60 <= int(attn_config) % 100 < 70:
            raise RuntimeError("configs 60-69 have no fused rms/rope path")    # attn_int8.cu:2606
        if text_bias is not None and text_bias[0] and int(attn_config) % 100 not in (90, 94):
            raise RuntimeError("text bias: config 94 or 90 only")
    f8_tile = _attn._fp8_tile(attn_config)     # configs 50-56: the FP8 P.V kernel
    fused = fuse_qkv and h % 2 == 0 and not f8_tile
    if fused:
        wsb = (_attn.workspace if numerics == 0 else _attn.workspace_u8)(s, s, h, x_dev)
        qkv = _gemm.int8_gemm_qkv(xq, xs, w.qkv.q, w.qkv.scale, h, wsb, numerics, tab=rope_tab, qw=w.q_norm_w,
                                  kw=w.k_norm_w, eps=w.qk_eps)
    else:
        qkv = _gemm.int8_gemm(xq, xs, w.qkv.q, w.qkv.scale)
    keep("qkv", qkv)
    tick("gemm_qkv")
    q, k, v = (t.view(s, h, D) for t in qkv.split(h * D, dim=-1))
    o = torch.empty(1, h, s, D, dtype=torch.bfloat16, device=x_dev)
    # attention_rr = pre-pass (RMSNorm + RoPE + stats + INT8) then the main kernel, as two calls
    if fused:
        pp = _attn.prepass_qkv(k, v, wsb, numerics, rope_tab, w.k_norm_w, w.qk_eps)
    elif numerics == 0:
        pp = _attn.prepass(q, k, v, rope_tab, w.q_norm_w, w.k_norm_w, w.qk_eps)
    elif f8_tile:
        pp = _attn.prepass_f8(q, k, v, rope_tab, w.q_norm_w, w.k_norm_w, w.qk_eps)
    else:
        pp = _attn.prepass_u8(q, k, v, rope_tab, w.q_norm_w, w.k_norm_w, w.qk_eps)
    keep("q8", pp["q8"]), keep("qs", pp["qs"])
    tick("attn_prepass")
    if numerics == 0:
        _attn.forward(pp, s, out=o[0].transpose(0, 1))
    elif f8_tile:
        _attn.forward_f8(pp, s, out=o[0].transpose(0, 1), tile=f8_tile)
    else:
        nbias, bias = text_bias if text_bias is not None else (0, 0.0)
        _attn.forward_u8(pp, s, out=o[0].transpose(0, 1), nbias=nbias, bias=bias)
    keep("o", o)
    tick("attn_main")
    if attn_check is not None:
        attn_check(q, k, v, o)
    return o


def fused_mlp(x, fc1, fc2, recipe="int8_rot", trace=None):
    """The reference's _fused_mlp (__init__.py:170-183) for a block whose attention linears are not all quantized:
    h = fc1(x) ([.., 2F] bf16, gate | up), then the SwiGLU-prologue quantizer (silu(gate) * up, rotated for int8_rot)
    straight into the fc2 GEMM, so silu(gate) * up is never written in bf16. fc1: a QuantLinear or any callable;
    fc2: a QuantLinear (its cached QWeight) or a QWeight. Like the reference, fc2's bias is not applied here.
    trace: optional dict that receives the intermediates h, hq, hs."""
    hdn = fc1(x)
    shape = hdn.shape
    q = _quant.swiglu_rot_quant_rows_i8 if recipe == "int8_rot" else _quant.swiglu_quant_rows_i8
    xq, xs = q(hdn.reshape(-1, shape[-1]).contiguous())
    if trace is not None:
        trace.update(h=hdn, hq=xq, hs=xs)
    qw = fc2.qweight_for() if hasattr(fc2, "qweight_for") else fc2
    y = _gemm.int8_gemm(xq, xs, qw.q, qw.scale)
    return y.reshape(*shape[:-1], y.shape[-1])
