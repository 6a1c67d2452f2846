"""rapid_h3.linear.QuantLinear, the _QuantLinear drop-in (__init__.py:83-167): output equal to
kernels.linear + bias, the weight cache and its invalidation, adoption of int8_convrot weights, the
measured-error diagnostics, and no CPU path."""
import numpy as np
import pytest

from conftest import to_np

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("mode", ["int8_rot", "int8_rowwise", "fp8_rowwise"])
def test_quant_linear_matches_kernels_linear(dev, mode):
    import torch
    from rapid_h3 import kernels
    from rapid_h3.linear import QuantLinear
    g = torch.Generator(device="cpu").manual_seed(5)
    w = (0.02 * torch.randn(264, 512, generator=g)).to(torch.bfloat16).to(dev)
    b = torch.randn(264, generator=g).to(torch.bfloat16).to(dev)
    x = torch.randn(3, 70, 512, generator=g).to(torch.bfloat16).to(dev)
    stats = {}
    lin = QuantLinear(w, b, mode, name="proj", measure_every=2, stats=stats)
    y = lin(x)
    assert tuple(y.shape) == (3, 70, 264) and y.dtype == torch.bfloat16
    ref = kernels.linear(x.reshape(-1, 512), kernels.quantize_weight(w, mode), mode) + b
    assert np.array_equal(to_np(y.reshape(-1, 264)), to_np(ref))
    q0 = lin.qweight
    lin(x)
    assert lin.qweight is q0                                   # cached
    assert len(stats["proj"]) == 1 and stats["proj"][0] < 0.05  # error sampled every 2nd call
    with torch.no_grad():
        w.mul_(2)                                              # in-place update bumps the version
    lin(x)
    assert lin.qweight is not q0


def test_quant_linear_adopts_convrot_and_refuses_cpu(dev):
    import torch
    from rapid_h3 import kernels
    from rapid_h3.linear import QuantLinear
    g = torch.Generator(device="cpu").manual_seed(6)
    w = (0.02 * torch.randn(128, 256, generator=g)).to(torch.bfloat16).to(dev)
    qw = kernels.quantize_weight(w, "int8_rot")
    lin = QuantLinear.from_quantized(qw.q, qw.scale.reshape(-1))
    x = torch.randn(33, 256, generator=g).to(torch.bfloat16).to(dev)
    assert np.array_equal(to_np(lin(x)), to_np(kernels.linear(x, qw, "int8_rot")))
    with pytest.raises(TypeError):
        lin(x.cpu())
    with pytest.raises(ValueError):
        QuantLinear(w, mode="bf16")
