"""CPU tests of the model patch (rapid_h3.patch, the reference's RapidH3LinearQuant.patch,
__init__.py:352-417) on a stub module tree: which linears are selected (NAME_RE, targets, keep_bf16_blocks),
where the fused block / fused MLP forwards go, and that forwards are swapped only inside the wrapper call."""
import pytest
import torch
from torch import nn

from rapid_h3 import patch as P


class _Attn(nn.Module):
    def __init__(self):
        super().__init__()
        self.qkv_proj, self.out_proj = nn.Linear(8, 24, bias=False), nn.Linear(8, 8, bias=False)


class _MLP(nn.Module):
    def __init__(self):
        super().__init__()
        self.fc1, self.fc2 = nn.Linear(8, 16, bias=False), nn.Linear(8, 8, bias=False)


class _Block(nn.Module):
    def __init__(self):
        super().__init__()
        self.attn, self.mlp = _Attn(), _MLP()


class _DiT(nn.Module):
    def __init__(self, n=3):
        super().__init__()
        self.blocks = nn.ModuleList(_Block() for _ in range(n))
        self.proj_out = nn.Linear(8, 8)        # not a block linear: never selected


def test_parse_blocks():
    assert P.parse_blocks("") == set()
    assert P.parse_blocks("0-2, 5,7-7") == {0, 1, 2, 5, 7}


def test_selection_and_fused_paths():
    m = _DiT()
    p = P.patch(m, "int8_rot", keep_bf16_blocks="1")
    assert sorted(p.by_name) == sorted(f"blocks.{b}.{q}" for b in (0, 2) for q in P.PARTS)
    kinds = [(mod, type(f).__name__, getattr(f, "__name__", "")) for mod, f in p.wrappers]
    fused = [mod for mod, _, n in kinds if n == "forward" and isinstance(mod, _Block)]
    assert fused == [m.blocks[0], m.blocks[2]]                     # fused blocks where all four are quantized
    p = P.patch(m, "int8_rot", fuse_block=False)
    assert [mod for mod, f in p.wrappers if isinstance(mod, _MLP)] == [b.mlp for b in m.blocks]
    p = P.patch(m, "int8_rot", targets="fc1,fc2")                  # attention linears stay bf16: fused MLP only
    assert sorted(p.by_name) == sorted(f"blocks.{b}.mlp.{q}" for b in range(3) for q in ("fc1", "fc2"))
    assert [mod for mod, f in p.wrappers if isinstance(mod, _MLP)] == [b.mlp for b in m.blocks]
    assert not [mod for mod, f in p.wrappers if isinstance(mod, _Block)]
    p = P.patch(m, "int8_rot", targets="qkv_proj,out_proj,fc1")    # no fc2: neither fused path
    assert all(isinstance(mod, nn.Linear) for mod, _ in p.wrappers) and len(p.wrappers) == 9
    for mode in ("int8_rowwise", "fp8_rowwise"):                   # fused paths are int8_rot only (:385)
        assert all(isinstance(mod, nn.Linear) for mod, _ in P.patch(m, mode).wrappers)
    assert all(isinstance(mod, nn.Linear) for mod, _ in P.patch(m, "int8_rot", measure_every=4).wrappers)
    assert P.patch(m, "bf16").wrappers == []


def test_forwards_swapped_only_inside_the_call():
    m = _DiT(2)
    p = P.patch(m, "int8_rot")
    seen = {}

    def executor(tag):
        seen[tag] = {mod: mod.__dict__.get("forward") for mod, _ in p.wrappers}
        return tag

    assert p.wrapper(executor, "run") == "run"
    assert all(seen["run"][mod] is f for mod, f in p.wrappers)
    assert all("forward" not in mod.__dict__ for mod, _ in p.wrappers)

    def boom():
        raise ValueError("x")

    with pytest.raises(ValueError):
        p.wrapper(boom)
    assert all("forward" not in mod.__dict__ for mod, _ in p.wrappers)
    own = lambda x: x                                               # noqa: E731  a forward set by someone else
    m.blocks[0].mlp.fc1.forward = own
    p.wrapper(lambda: None)
    assert m.blocks[0].mlp.fc1.forward is own


def test_weight_cache_follows_patch_id():
    lin = nn.Linear(8, 8, bias=False)
    uuid = {"v": 1}
    q = P._ModuleLinear(lin, "blocks.0.attn.out_proj", "int8_rot", 0, {}, lambda: uuid["v"])
    assert q.q._key() == ("patch", 1, "cpu")
    uuid["v"] = 2
    assert q.q._key() == ("patch", 2, "cpu")
    assert P._ModuleLinear(lin, "n", "int8_rot", 0, {}, None).q._key()[1] == lin.weight.data_ptr()


def test_weight_cache_key_default_tracks_tensor():
    q = P._ModuleLinear(nn.Linear(4, 4, bias=False), "n", "int8_rowwise", 0, {}, None)
    k0 = q.q._key()
    with torch.no_grad():
        q.module.weight.add_(1)                                     # in-place update bumps the version counter
    assert q.q._key() != k0


def test_cpu_and_fp32_activations_take_f_linear():
    """Activations off the GPU or not bf16 / fp16 take torch's F.linear with the weight in x.dtype, as the reference's
    _QuantLinear does (__init__.py:147-148): an fp32 CPU forward through a patched stub returns F.linear exactly, and
    the quantized weight is never made."""
    import torch.nn.functional as F
    m = _DiT(2)
    with torch.no_grad():
        m.blocks[1].attn.qkv_proj.bias = nn.Parameter(torch.randn(24))
    p = P.patch(m, "int8_rot", targets="qkv_proj,out_proj")       # no fused paths
    x = torch.randn(3, 5, 8)
    for lin in (m.blocks[0].attn.qkv_proj, m.blocks[1].attn.qkv_proj, m.blocks[1].attn.out_proj):
        got = p.wrapper(lambda t: lin(t), x)
        assert torch.equal(got, F.linear(x, lin.weight, lin.bias))
        got16 = p.wrapper(lambda t: lin(t), x.to(torch.float64))
        assert got16.dtype == torch.float64
    assert all(q.q.qweight is None for q in p.by_name.values())


def test_adopted_convrot_weight_dequantizes_for_f_linear():
    """An adopted int8_convrot weight (codes of W @ blockdiag(H256)^T and a per-row scale, from the oracle) on the
    F.linear route: dequantized and rotated back, it reproduces W within the int8 quantization error."""
    import numpy as np
    from oracle import quant as oq
    from oracle.numerics import bf16_to_f32, f32_to_bf16
    from rapid_h3.linear import QuantLinear
    rng = np.random.default_rng(8)
    w = f32_to_bf16((0.02 * rng.standard_normal((48, 512))).astype(np.float32))
    q, s = oq.quantize_weight(w, "int8_rot")
    lin = QuantLinear.from_quantized(torch.from_numpy(q), torch.from_numpy(s).reshape(-1))
    x = torch.from_numpy(rng.standard_normal((7, 512)).astype(np.float32))
    y = lin(x)
    ref = x.double() @ torch.from_numpy(bf16_to_f32(w)).double().t()
    assert y.dtype == torch.float32 and float((y.double() - ref).norm() / ref.norm()) < 0.01
    wd = lin.dense_weight("cpu", torch.float64)
    assert float((wd - torch.from_numpy(bf16_to_f32(w)).double()).abs().max()) < 0.02 * 4 / 127
