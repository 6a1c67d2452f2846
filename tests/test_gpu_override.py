"""The RapidH3Int8Attention override (rapid_h3.override, the reference's __init__.py:994-1046): dispatch to the
INT8 kernel for the calls it accepts, fall-through for the others, and exact_rows recomputing the rows of
the named segment kinds."""
import types

import numpy as np
import pytest

from oracle import attn as oa
from oracle.gemm import rel_l2

pytestmark = pytest.mark.gpu


def test_override_dispatch_and_exact_rows(dev):
    import torch
    from rapid_h3 import attention, override
    s, h = 1100, 2
    g = torch.Generator(device="cpu").manual_seed(4)
    q, k, v = (torch.randn(1, h, s, 128, generator=g).to(torch.bfloat16).to(dev) for _ in range(3))
    lay = types.SimpleNamespace(seq_len=s, segments=[(0, 100, "text"), (100, 140, "text"), (140, 1000, "video"),
                                                     (1000, 1100, "text")])
    opts = {"minimax_h3_layout": lay}
    calls = []

    def func(*a, **kw):
        calls.append(1)
        return "fallback"

    ov = override.make_override(94, exact_rows="text")
    out = ov(func, q, k, v, h, skip_reshape=True, skip_output_reshape=True, transformer_options=opts)
    assert not calls and out.shape == q.shape
    base = attention.attention(q[0].transpose(0, 1), k[0].transpose(0, 1), v[0].transpose(0, 1), config=94)
    base = base.transpose(0, 1).unsqueeze(0)
    assert torch.equal(out[:, :, 140:1000], base[:, :, 140:1000])          # INT8 rows untouched
    qn, kn, vn = (t[0].transpose(0, 1).float().cpu().numpy() for t in (q, k, v))
    for a, b in ((0, 140), (1000, 1100)):
        ex = oa.attention_exact(qn, kn, vn, 128 ** -0.5, rows=np.arange(a, b))
        got = out[0, :, a:b].transpose(0, 1).float().cpu().numpy()
        assert rel_l2(got, ex) < 4e-3                                      # bf16 rounding of exact rows
    flat = ov(func, q, k, v, h, skip_reshape=True, transformer_options=opts)
    assert flat.shape == (1, s, h * 128)
    # rejected calls fall through: a mask, a short sequence
    assert ov(func, q, k, v, h, mask=torch.zeros(1), skip_reshape=True) == "fallback"
    assert ov(func, q[:, :, :512], k[:, :, :512], v[:, :, :512], h, skip_reshape=True) == "fallback"
    assert len(calls) == 2
    with pytest.raises(RuntimeError, match="TextAttnBias"):
        ov(func, q, k, v, h, skip_reshape=True, transformer_options={"rapidh3_text_bias": 1.0})
