"""The model patch of the reference's RapidH3LinearQuant node (/root/reference/custom_nodes/rapid_h3/__init__.py:352-417)
without ComfyUI: select the block linears of a MiniMax-H3 DiT by name, replace their forwards with QuantLinear, and in
int8_rot mode replace whole blocks with the fused INT8 chain (block.fused_block) or, where only the MLP linears are
quantized, the MLP with block.fused_mlp. The forwards are swapped only for the duration of one call of the diffusion
model (wrapper(executor, ...), ComfyUI's DIFFUSION_MODEL wrapper contract) and restored afterwards.

Kept from the reference:
  * NAME_RE (:65): blocks.N.(attn|mlp).(qkv_proj|out_proj|fc1|fc2); `targets` (comma-separated leaf names) and
    `keep_bf16_blocks` ("a-b,c" block numbers, _parse_blocks :72-80) filter it; mode "bf16" patches nothing;
  * the fused paths only in int8_rot mode with measure_every 0 (:385-394): a block whose four linears are all
    selected gets the fused block forward when fuse_block is set, else a block with fc1 and fc2 selected gets the
    fused MLP forward;
  * the weight cache of each QuantLinear follows the caller's patch id (patches_uuid, :119-130) when given;
  * after the call, the per-linear error stats (measure_every) are written as JSON to stats_path.
The fused block forward reads the block duck-typed, with the attribute names of ComfyUI's H3 block that the reference
uses (:253-320): adaln_proj(t_emb) -> the six modulation tables, norm1 / norm2 (.weight, .eps), attn (.heads,
.head_dim, .q_norm, .k_norm), and takes forward(x, t_emb, mod_segments, rope_freqs, transformer_options={},
attention=None). Its attention follows the reference (:277-306):
  * an override tagged rapidh3_rmsrope (override.make_override, configs >= 100 without exact_rows) and S >= 1024: the
    INT8 attention with that config and the RMSNorm + RoPE in its pre-pass, with the text bias of
    transformer_options["rapidh3_text_bias"]; a rapidh3_rrcheck tag (configs >= 200) adds override.rr_check;
  * otherwise, when an override is installed (or patch() was given the stock attention): q, k get the RMSNorm + RoPE
    in place and the override is called in ComfyUI's convention, override(func, q, k, v, heads, mask=None,
    skip_reshape=True, skip_output_reshape=True, transformer_options=...), func being the stock attention
    (`attention`, default override.stock_attention), so the override's own config and exact_rows decide the
    numerics; with no override, func itself runs;
  * with neither an override nor a stock attention given, this build's per-block INT8 recipe (RMSNorm + RoPE fused
    in its pre-pass), the attention the benchmark measures.
Inputs the fused path does not take (not bf16, not 2-D, on the CPU, an attention argument, no rope table) go to the
block's own forward, as in the reference (:255-258).
"""
import json
import os
import re

import torch

from . import block as _block
from . import override as _override
from .linear import QuantLinear

NAME_RE = re.compile(r"^blocks\.(\d+)\.(attn|mlp)\.(qkv_proj|out_proj|fc1|fc2)$")
BLOCK_RE = re.compile(r"^blocks\.\d+$")
PARTS = ("attn.qkv_proj", "attn.out_proj", "mlp.fc1", "mlp.fc2")


def parse_blocks(spec):
    """Block numbers of a "0-3,7" spec (the reference's _parse_blocks, __init__.py:72-80)."""
    out = set()
    for part in filter(None, (p.strip() for p in spec.split(","))):
        if "-" in part:
            a, b = part.split("-")
            out.update(range(int(a), int(b) + 1))
        else:
            out.add(int(part))
    return out


class _ModuleLinear:
    """QuantLinear bound to a torch Linear module: the quantized weight follows the module's current weight."""

    def __init__(self, module, name, mode, measure_every, stats, patch_id):
        self.module = module
        self.q = QuantLinear(module.weight, module.bias, mode, name, measure_every, stats, patch_id)

    def qweight_for(self, x=None):
        self.q.weight, self.q.bias = self.module.weight, self.module.bias
        return self.q.qweight_for()

    def __call__(self, x):
        self.q.weight, self.q.bias = self.module.weight, self.module.bias
        return self.q(x)


def _text_rows(opts):
    """Text rows at the start of the packed sequence (the reference's _text_rows, __init__.py:323-330)."""
    lay = opts.get("minimax_h3_layout")
    seg = lay.segments[0] if lay is not None and lay.segments else None
    if seg is None or seg[2] != "text" or seg[0] != 0:
        raise RuntimeError("RapidH3TextAttnBias: no leading text segment in minimax_h3_layout")
    return seg[1]


def fused_block_forward(blk, qkv, out, fc1, fc2, recipe="int8_rot", stock_attention=None):
    """The forward that replaces a DiT block (the reference's _fused_block, __init__.py:207-321). stock_attention:
    the attention ComfyUI's dispatcher would run (override.stock_attention's convention), or None."""
    orig = type(blk).forward
    state = {}

    def norm_w(norm, x):
        w = getattr(norm, "weight", None)
        return None if w is None else w.to(device=x.device, dtype=torch.bfloat16).contiguous()

    def eps_of(norm):
        e = getattr(norm, "eps", None)
        return torch.finfo(torch.bfloat16).eps if e is None else e

    def weights(x):
        """BlockWeights over the cached QWeights; fc1 in SwiGLU-epilogue order, permuted once per cached weight."""
        from .gemm import swiglu_perm
        from .kernels import QWeight
        q1 = fc1.qweight_for(x)
        if state.get("fc1_src") is not q1:
            perm = swiglu_perm(q1.q.shape[0], q1.q.device)
            state["fc1_perm"] = QWeight(q1.q[perm].contiguous(), q1.scale[:, perm].contiguous())
            state["fc1_src"] = q1
        a = blk.attn
        return _block.BlockWeights(qkv=qkv.qweight_for(x), out=out.qweight_for(x), fc1_perm=state["fc1_perm"],
                                   fc2=fc2.qweight_for(x), norm1_w=norm_w(blk.norm1, x), norm2_w=norm_w(blk.norm2, x),
                                   q_norm_w=norm_w(a.q_norm, x), k_norm_w=norm_w(a.k_norm, x), heads=a.heads,
                                   eps=eps_of(blk.norm1), qk_eps=eps_of(a.q_norm), recipe=recipe)

    def forward(x, t_emb, mod_segments, rope_freqs, transformer_options={}, attention=None):  # noqa: B006
        if (attention is not None or rope_freqs is None or x.dtype != torch.bfloat16 or not x.is_cuda
                or x.ndim != 2):
            return orig(blk, x, t_emb, mod_segments, rope_freqs, transformer_options=transformer_options,
                        attention=attention)
        mod = blk.adaln_proj(t_emb)
        a = blk.attn
        ov = transformer_options.get("optimized_attention_override")
        cfg = getattr(ov, "rapidh3_rmsrope", None)
        if cfg is not None and not (x.shape[0] >= 1024 and a.head_dim == 128 and rope_freqs.dtype == torch.bfloat16):
            cfg = None                                  # the reference's fused-path condition (:284-285)
        tb = transformer_options.get("rapidh3_text_bias")
        w = weights(x)
        if cfg is None and (ov is not None or stock_attention is not None):
            if tb is not None:
                raise RuntimeError("RapidH3TextAttnBias: needs the fused INT8 attention path (RapidH3Int8Attention "
                                   "190 or 194)")
            func = stock_attention or _override.stock_attention

            def attn_fn(q, k, v):
                q4, k4, v4 = (t.unsqueeze(0).transpose(1, 2) for t in (q, k, v))     # [1, H, S, 128] views
                kw = dict(mask=None, skip_reshape=True, skip_output_reshape=True,
                          transformer_options=transformer_options)
                return ov(func, q4, k4, v4, a.heads, **kw) if ov is not None else func(q4, k4, v4, a.heads, **kw)

            return _block.fused_block(x, w, mod, mod_segments, rope_freqs, attn_fn=attn_fn)
        text_bias = None
        if tb is not None:
            if cfg is None:
                raise RuntimeError("RapidH3TextAttnBias: needs the fused INT8 attention path (RapidH3Int8Attention "
                                   "190 or 194)")
            text_bias = (_text_rows(transformer_options), tb)
        check = None
        if cfg is not None and getattr(ov, "rapidh3_rrcheck", False):
            def check(q, k, v, o):
                _override.rr_check(q, k, v, o, rope_freqs, w.q_norm_w, w.k_norm_w, w.qk_eps, cfg,
                                   transformer_options)
        return _block.fused_block(x, w, mod, mod_segments, rope_freqs, attn_config=cfg, text_bias=text_bias,
                                  attn_check=check)

    return forward


def fused_mlp_forward(mlp, fc2, recipe="int8_rot"):
    """The forward that replaces a block's MLP (the reference's _fused_mlp, __init__.py:170-183): mlp.fc1 is called
    as patched, its [gate | up] output feeds the SwiGLU-prologue quantizer and the fc2 GEMM."""
    orig = type(mlp).forward

    def forward(x):
        if x.dtype != torch.bfloat16 or not x.is_cuda:
            return orig(mlp, x)
        return _block.fused_mlp(x, mlp.fc1, fc2, recipe)

    return forward


class LinearQuantPatch:
    """RapidH3LinearQuant.patch (__init__.py:368-417) on a diffusion model's module tree. wrapper(executor, *args,
    **kwargs) runs executor with the replacement forwards installed and restores the previous ones afterwards."""

    def __init__(self, diffusion_model, mode, targets="qkv_proj,out_proj,fc1,fc2", keep_bf16_blocks="",
                 measure_every=0, fuse_block=True, patch_id=None, stats_path=None, attention=None):
        self.mode, self.stats, self.stats_path = mode, {}, stats_path
        self.wrappers, self.by_name = [], {}
        if mode == "bf16":
            return
        want = {t.strip() for t in targets.split(",") if t.strip()}
        keep = parse_blocks(keep_bf16_blocks)
        for name, mod in diffusion_model.named_modules():
            hit = NAME_RE.match(name)
            if not hit or hit.group(3) not in want or int(hit.group(1)) in keep:
                continue
            q = _ModuleLinear(mod, name, mode, measure_every, self.stats, patch_id)
            self.by_name[name] = q
            self.wrappers.append((mod, q))
        if mode == "int8_rot" and not measure_every:
            for name, mod in diffusion_model.named_modules():
                if not BLOCK_RE.match(name):
                    continue
                parts = [self.by_name.get(f"{name}.{p}") for p in PARTS]
                if all(parts) and fuse_block:
                    self.wrappers.append((mod, fused_block_forward(mod, *parts, stock_attention=attention)))
                elif parts[2] and parts[3]:
                    self.wrappers.append((mod.mlp, fused_mlp_forward(mod.mlp, parts[3])))

    def wrapper(self, executor, *args, **kwargs):
        saved = []
        for mod, fwd in self.wrappers:
            saved.append((mod, mod.__dict__.get("forward")))
            mod.forward = fwd
        try:
            return executor(*args, **kwargs)
        finally:
            for mod, prev in saved:
                if prev is None:
                    mod.__dict__.pop("forward", None)
                else:
                    mod.forward = prev
            if self.stats_path and self.stats:
                with open(self.stats_path, "w") as f:
                    json.dump({"mode": self.mode, "errors": self.stats}, f)

    def __call__(self, model, *args, **kwargs):
        """Run model(*args, **kwargs) with the patch installed."""
        return self.wrapper(model, *args, **kwargs)


def patch(diffusion_model, mode, targets="qkv_proj,out_proj,fc1,fc2", keep_bf16_blocks="", measure_every=0,
          fuse_block=True, patch_id=None, stats_path=None, attention=None):
    """LinearQuantPatch for a model; stats_path defaults to $RAPIDH3_STATS as in the reference (:396). attention: the
    stock attention of the fused blocks' unfused route (ComfyUI's optimized_attention in the reference; the
    calling convention of override.stock_attention)."""
    if stats_path is None:
        stats_path = os.environ.get("RAPIDH3_STATS")
    return LinearQuantPatch(diffusion_model, mode, targets, keep_bf16_blocks, measure_every, fuse_block, patch_id,
                            stats_path, attention)
