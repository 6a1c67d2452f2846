"""Row-wise W8A8 / FP8 GEMMs with fused epilogues on the HIP kernels (librh3: rh3_gemm_*).

Signatures follow the reference's cutlass_fp8 wrappers (/root/reference/custom_nodes/rapid_h3/
cutlass_fp8.py:32-67): scales may be [M, 1] / [1, N] or 1-D; the `config` tile id is accepted and
ignored (this backend has one gfx950 schedule per epilogue).
"""
import torch

from . import _native as nat

FP8 = torch.float8_e4m3fn


def _check(xq, wq, dtype, name):
    if xq.ndim != 2 or wq.ndim != 2 or xq.shape[1] != wq.shape[1]:
        raise RuntimeError(f"{name}: shapes {tuple(xq.shape)} x {tuple(wq.shape)} do not match ([M,K] x [N,K])")
    if xq.dtype != dtype or wq.dtype != dtype:
        raise RuntimeError(f"{name}: operands must be {dtype}, got {xq.dtype} / {wq.dtype}")
    if xq.stride(1) != 1 or wq.stride(1) != 1:
        raise RuntimeError(f"{name}: operands must be K-contiguous")
    if not (xq.is_cuda and wq.is_cuda):
        raise RuntimeError(f"{name}: operands must be on a GPU (no CPU path)")


def _vec(t, n, name):
    t = t.reshape(-1)
    if t.numel() != n or t.dtype != torch.float32:
        raise RuntimeError(f"{name}: expected {n} fp32 values, got {t.numel()} {t.dtype}")
    return t.contiguous()


def int8_gemm(xq, xs, wq, ws, bias=None, config=2):
    """xq [M,K] int8, xs [M,1] fp32, wq [N,K] int8, ws [1,N] fp32 -> bf16 [M,N] (cutlass_fp8.int8_gemm)."""
    _check(xq, wq, torch.int8, "int8_gemm")
    m, k = xq.shape
    n = wq.shape[0]
    xs, ws = _vec(xs, m, "int8_gemm xs"), _vec(ws, n, "int8_gemm ws")
    if bias is not None:
        bias = bias.to(torch.bfloat16).contiguous()
    out = torch.empty((m, n), device=xq.device, dtype=torch.bfloat16)
    ctr = nat.gemm_ctr(xq.device)     # held until the launch is enqueued
    nat.call("rh3_gemm_i8", nat.ptr(xq), xq.stride(0), nat.ptr(xs), nat.ptr(wq), wq.stride(0), nat.ptr(ws),
             nat.ptr(bias), nat.ptr(out), out.stride(0), m, n, k, nat.ptr(ctr),
             nat.stream(xq.device))
    return out


def int8_gemm_acc(xq, wq):
    """Raw int32 accumulators xq @ wq^T [M, N] of the same kernel (verification)."""
    _check(xq, wq, torch.int8, "int8_gemm_acc")
    m, k = xq.shape
    n = wq.shape[0]
    acc = torch.empty((m, n), device=xq.device, dtype=torch.int32)
    ctr = nat.gemm_ctr(xq.device)     # held until the launch is enqueued
    nat.call("rh3_gemm_i8_acc", nat.ptr(xq), xq.stride(0), nat.ptr(wq), wq.stride(0), nat.ptr(acc), acc.stride(0),
             m, n, k, nat.ptr(ctr),
             nat.stream(xq.device))
    return acc


def fp8_gemm(xq, xs, wq, ws, bias=None, config=2, fast_accum=True):
    """xq [M,K] e4m3fn, xs [M,1] fp32, wq [N,K] e4m3fn, ws [1,N] fp32 -> bf16 [M,N] (cutlass_fp8.fp8_gemm).
    fast_accum is accepted for signature parity; MFMA accumulates in fp32 either way."""
    _check(xq, wq, FP8, "fp8_gemm")
    m, k = xq.shape
    n = wq.shape[0]
    xs, ws = _vec(xs, m, "fp8_gemm xs"), _vec(ws, n, "fp8_gemm ws")
    if bias is not None:
        bias = bias.to(torch.bfloat16).contiguous()
    out = torch.empty((m, n), device=xq.device, dtype=torch.bfloat16)
    ctr = nat.gemm_ctr(xq.device)     # held until the launch is enqueued
    nat.call("rh3_gemm_fp8", nat.ptr(xq), xq.stride(0), nat.ptr(xs), nat.ptr(wq), wq.stride(0), nat.ptr(ws),
             nat.ptr(bias), nat.ptr(out), out.stride(0), m, n, k, nat.ptr(ctr),
             nat.stream(xq.device))
    return out


def fp8_gemm_acc(xq, wq):
    """Raw fp32 accumulators xq @ wq^T [M, N] of the FP8 GEMM, no scales applied (the product torch._scaled_mm
    scales for a non-bf16 out_dtype)."""
    _check(xq, wq, FP8, "fp8_gemm_acc")
    m, k = xq.shape
    n = wq.shape[0]
    acc = torch.empty((m, n), device=xq.device, dtype=torch.float32)
    ctr = nat.gemm_ctr(xq.device)     # held until the launch is enqueued
    nat.call("rh3_gemm_fp8_acc", nat.ptr(xq), xq.stride(0), nat.ptr(wq), wq.stride(0), nat.ptr(acc), acc.stride(0),
             m, n, k, nat.ptr(ctr), nat.stream(xq.device))
    return acc


def int8_gemm_gated_residual(xq, xs, wq, ws, gate, resid, config=6):
    """resid[M,N] += bf16(xq @ wq^T * xs * ws) * gate[N], in place (cutlass_fp8.int8_gemm_gated_residual)."""
    _check(xq, wq, torch.int8, "int8_gemm_gated_residual")
    m, k = xq.shape
    n = wq.shape[0]
    if resid.shape != (m, n) or resid.dtype != torch.bfloat16 or resid.stride(1) != 1:
        raise RuntimeError("int8_gemm_gated_residual: resid must be bf16 [M, N] with unit column stride")
    xs, ws = _vec(xs, m, "gated xs"), _vec(ws, n, "gated ws")
    gate = gate.reshape(-1).to(torch.bfloat16).contiguous()
    if gate.numel() != n:
        raise RuntimeError("int8_gemm_gated_residual: gate must have N elements")
    ctr = nat.gemm_ctr(xq.device)     # held until the launch is enqueued
    nat.call("rh3_gemm_i8_gated", nat.ptr(xq), xq.stride(0), nat.ptr(xs), nat.ptr(wq), wq.stride(0), nat.ptr(ws),
             nat.ptr(gate), nat.ptr(resid), resid.stride(0), m, n, k, nat.ptr(ctr),
             nat.stream(xq.device))
    return resid


_ROWS_OK = {}


def _check_rows(rows, r):
    """Raise IndexError unless every gate row index is in [0, r), as torch's gather does. The kernel reads the table
    unchecked, so the check runs here, once per index tensor (identity, storage, version) and table height: the blocks
    of one model call share their segments' index tensors and pay for each once."""
    key = (id(rows), rows.data_ptr(), rows._version, r)
    hit = _ROWS_OK.get(key)
    if hit is not None and hit is rows:
        return
    if rows.numel():
        lo, hi = int(rows.min()), int(rows.max())
        if lo < 0 or hi >= r:
            raise IndexError(f"int8_gemm_gated_residual_rows: gate row index out of range [{lo}, {hi}] for a table "
                             f"of {r} rows")
    if len(_ROWS_OK) >= 64:
        _ROWS_OK.clear()
    _ROWS_OK[key] = rows


def int8_gemm_gated_residual_rows(xq, xs, wq, ws, gate, rows, resid):
    """resid[m, :] += bf16(xq @ wq^T * xs * ws)[m, :] * gate[rows[m], :], in place: the gated residual with one gate
    table row per token (per-token modulation, _fused_block's tensor-row segments, __init__.py:242-245). gate [R, N]
    (rounded to bf16 like _mod_row), rows [M] integer indices into it."""
    _check(xq, wq, torch.int8, "int8_gemm_gated_residual_rows")
    m, k = xq.shape
    n = wq.shape[0]
    if resid.shape != (m, n) or resid.dtype != torch.bfloat16 or resid.stride(1) != 1:
        raise RuntimeError("int8_gemm_gated_residual_rows: resid must be bf16 [M, N] with unit column stride")
    xs, ws = _vec(xs, m, "gated xs"), _vec(ws, n, "gated ws")
    gate = gate.to(torch.bfloat16).reshape(-1, n).contiguous()
    if rows.numel() != m:
        raise RuntimeError("int8_gemm_gated_residual_rows: one gate row index per token required")
    _check_rows(rows, gate.shape[0])
    rows = rows.reshape(-1).to(device=xq.device, dtype=torch.int32).contiguous()
    ctr = nat.gemm_ctr(xq.device)     # held until the launch is enqueued
    nat.call("rh3_gemm_i8_gated_rows", nat.ptr(xq), xq.stride(0), nat.ptr(xs), nat.ptr(wq), wq.stride(0),
             nat.ptr(ws), nat.ptr(gate), gate.stride(0), nat.ptr(rows), nat.ptr(resid), resid.stride(0), m, n, k,
             nat.ptr(ctr), nat.stream(xq.device))
    return resid


def swiglu_perm(n2, device):
    """Row order for an fc1 weight [gate (F rows) | up (F rows)] so each 8-row group is
    [gate 4j..4j+3 | up 4j..4j+3] (cutlass_fp8.swiglu_perm, cutlass_fp8.py:55-62)."""
    f = n2 // 2
    j = torch.arange(0, f, 4, device=device)
    blk = torch.arange(4, device=device)
    return torch.stack([j[:, None] + blk, f + j[:, None] + blk], dim=1).reshape(-1)


def int8_gemm_swiglu(xq, xs, wq_perm, ws_perm, config=6):
    """h [M, F] = bf16(silu(g) * u) for an fc1 whose rows were permuted with swiglu_perm
    (cutlass_fp8.int8_gemm_swiglu)."""
    _check(xq, wq_perm, torch.int8, "int8_gemm_swiglu")
    m, k = xq.shape
    n = wq_perm.shape[0]
    if n % 8:
        raise RuntimeError("int8_gemm_swiglu: N must be a multiple of 8")
    xs, ws = _vec(xs, m, "swiglu xs"), _vec(ws_perm, n, "swiglu ws")
    out = torch.empty((m, n // 2), device=xq.device, dtype=torch.bfloat16)
    ctr = nat.gemm_ctr(xq.device)     # held until the launch is enqueued
    nat.call("rh3_gemm_i8_swiglu", nat.ptr(xq), xq.stride(0), nat.ptr(xs), nat.ptr(wq_perm), wq_perm.stride(0),
             nat.ptr(ws), nat.ptr(out), out.stride(0), m, n, k, nat.ptr(ctr),
             nat.stream(xq.device))
    return out


def int8_gemm_qkv(xq, xs, wq, ws, heads, workspace, numerics, tab=None, qw=None, kw=None, eps=1e-6, rotate=True,
                  bias=None):
    """The qkv projection with the attention pre-pass fused into its epilogue (rh3_gemm_i8_qkv; the
    reference's config-3xx visitor, fp8_rowwise.cu:108-272): returns out [M, 3*heads*128] bf16 whose k and v
    columns hold bf16((acc * xs) * ws [+ bias]) and whose q columns are left unwritten; the Q operands and the
    K (and, numerics 1, V) statistics are written into workspace, the attention workspace of
    attention.workspace (numerics 0, per-block) or attention.workspace_u8 (numerics 1, production) for
    Sq = Sk = M. tab [1, M, 1, rot/2, 2, 2] bf16 with qw / kw [128] bf16 applies the per-head RMSNorm + RoPE."""
    _check(xq, wq, torch.int8, "int8_gemm_qkv")
    m, k = xq.shape
    n = wq.shape[0]
    if n != 3 * heads * 128:
        raise RuntimeError(f"int8_gemm_qkv: wq has {n} rows, expected 3 * {heads} * 128")
    xs, ws = _vec(xs, m, "int8_gemm_qkv xs"), _vec(ws, n, "int8_gemm_qkv ws")
    if bias is not None:
        bias = bias.to(torch.bfloat16).contiguous()
    rot = 0
    if tab is not None:
        rot = tab.shape[-3] * 2
        tab, qw, kw = tab.contiguous(), qw.contiguous(), kw.contiguous()
    out = torch.empty((m, n), device=xq.device, dtype=torch.bfloat16)
    nat.call("rh3_gemm_i8_qkv", nat.ptr(xq), xq.stride(0), nat.ptr(xs), nat.ptr(wq), wq.stride(0), nat.ptr(ws),
             nat.ptr(bias), nat.ptr(out), out.stride(0), m, heads, k, nat.ptr(tab), rot, nat.ptr(qw), nat.ptr(kw),
             float(eps), int(numerics), int(bool(rotate)), nat.ptr(workspace), workspace.numel(),
             nat.stream(xq.device))
    return out
