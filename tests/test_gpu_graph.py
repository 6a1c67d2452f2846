"""The hot path inside a captured HIP graph (torch.cuda.CUDAGraph): the work counters and tile counters are cleared
by fill kernels on the call's stream (no hipMemsetAsync), so a captured call replays correctly. Each graph is
replayed three times, with other eager work of the library and synchronisations between the replays, and every
replay must reproduce the eager result bit for bit (same kernels on the same inputs; the tile and item claiming
changes which workgroup computes a tile, not what it computes)."""
import numpy as np
import pytest

from conftest import to_dev

pytestmark = pytest.mark.gpu


def _bf(a):
    from oracle.numerics import f32_to_bf16
    return f32_to_bf16(np.asarray(a, np.float32))


def _capture(fn):
    """fn() run twice on a side stream (lazy library state), then captured on torch's default capture stream. The
    GEMMs inside the capture take new tile-counter buffers from the graph's private pool, so no two graphs share
    one."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    torch.cuda.synchronize()
    return g, out


def _replays(g, out, want, reset=None, between=None):
    """reset() restores in-place inputs; every output is zeroed before a replay, so a replay that did not run
    (work executed once at capture time instead of recorded) fails the comparison."""
    import torch
    for i in range(3):
        if between is not None:
            between()                  # the program's own eager work between the replays
        torch.cuda.synchronize()
        for o in out:
            o.zero_()
        if reset is not None:
            reset()
        g.replay()
        torch.cuda.synchronize()
        for o, w in zip(out, want):
            assert torch.equal(o.view(torch.int16) if o.dtype == torch.bfloat16 else o,
                               w.view(torch.int16) if w.dtype == torch.bfloat16 else w), f"replay {i}"


def test_graph_gemms(dev):
    """Persistent-kernel shapes (K 512: tiles claimed from the per-XCD counters): plain, SwiGLU and the in-place gated
    residual, captured together."""
    import torch
    from rapid_h3 import gemm
    rng = np.random.default_rng(5)
    m, n, k = 4500, 4112, 512
    xq = to_dev(np.clip(np.rint(rng.standard_normal((m, k)) * 30), -127, 127).astype(np.int8), dev)
    wq = to_dev(np.clip(np.rint(rng.standard_normal((n, k)) * 30), -127, 127).astype(np.int8), dev)
    xs = to_dev((rng.random((m, 1)) * 1e-3 + 1e-4).astype(np.float32), dev)
    ws = to_dev((rng.random((1, n)) * 1e-3 + 1e-4).astype(np.float32), dev)
    gate = to_dev(_bf(rng.standard_normal(n)), dev)
    r0 = to_dev(_bf(rng.standard_normal((m, n))), dev)
    resid = r0.clone()

    def fn():
        y = gemm.int8_gemm(xq, xs, wq, ws)
        h = gemm.int8_gemm_swiglu(xq, xs, wq, ws)
        gemm.int8_gemm_gated_residual(xq, xs, wq, ws, gate, resid)
        return y, h

    resid.copy_(r0)
    y_e, h_e = fn()
    r_e = resid.clone()
    g, (y, h) = _capture(fn)
    xq2 = torch.randint(-127, 128, (1000, k), device=dev, dtype=torch.int8)
    _replays(g, (y, h, resid), (y_e, h_e, r_e), reset=lambda: resid.copy_(r0),
             between=lambda: gemm.int8_gemm(xq2, xs[:1000], wq, ws))


def test_graph_gemms_two_graphs_at_once(dev):
    """Two graphs captured on the same (default) capture stream, replayed at once on two streams: each holds its own
    tile counters, so neither skips a tile nor applies the in-place gated residual twice; each replay matches its
    eager result bit for bit."""
    import torch
    from rapid_h3 import gemm
    rng = np.random.default_rng(15)
    m, n, k = 6000, 4096, 1024
    sets = []
    for _ in range(2):
        xq = to_dev(np.clip(np.rint(rng.standard_normal((m, k)) * 30), -127, 127).astype(np.int8), dev)
        wq = to_dev(np.clip(np.rint(rng.standard_normal((n, k)) * 30), -127, 127).astype(np.int8), dev)
        xs = to_dev((rng.random((m, 1)) * 1e-3 + 1e-4).astype(np.float32), dev)
        ws = to_dev((rng.random((1, n)) * 1e-3 + 1e-4).astype(np.float32), dev)
        gate = to_dev(_bf(rng.standard_normal(n)), dev)
        r0 = to_dev(_bf(rng.standard_normal((m, n))), dev)
        sets.append((xq, wq, xs, ws, gate, r0, r0.clone()))

    def make(i):
        xq, wq, xs, ws, gate, r0, resid = sets[i]

        def fn():
            gemm.int8_gemm_gated_residual(xq, xs, wq, ws, gate, resid)
            return (gemm.int8_gemm(xq, xs, wq, ws),)
        return fn

    fns = [make(0), make(1)]
    want = []
    for i in range(2):
        sets[i][6].copy_(sets[i][5])
        y = fns[i]()[0]
        want.append((y, sets[i][6].clone()))
    graphs = []
    for i in range(2):
        sets[i][6].copy_(sets[i][5])
        graphs.append(_capture(fns[i]))
    streams = [torch.cuda.Stream(device=dev) for _ in range(2)]
    for rep in range(3):
        for i in range(2):
            graphs[i][1][0].zero_()
            sets[i][6].copy_(sets[i][5])
        torch.cuda.synchronize()
        for i in range(2):
            with torch.cuda.stream(streams[i]):
                graphs[i][0].replay()
        torch.cuda.synchronize()
        for i in range(2):
            y_w, r_w = want[i]
            assert torch.equal(graphs[i][1][0].view(torch.int16), y_w.view(torch.int16)), f"graph {i} replay {rep}"
            assert torch.equal(sets[i][6].view(torch.int16), r_w.view(torch.int16)), f"graph {i} resid {rep}"


@pytest.mark.parametrize("config", [None, 94])
def test_graph_attention(dev, config):
    """The per-block recipe (pre-pass, main kernel with its work counter, split last round when the grid has one) and
    the production numerics (config 94), each captured as one call."""
    import torch
    from rapid_h3 import attention
    rng = np.random.default_rng(6)
    s, h = 2600, 3
    q = to_dev(_bf(rng.standard_normal((s, h, 128))), dev)
    k = to_dev(_bf(rng.standard_normal((s, h, 128)) + 2.0 * rng.standard_normal((1, h, 128))), dev)
    v = to_dev(_bf(rng.standard_normal((s, h, 128))), dev)

    def fn():
        return (attention.attention(q, k, v, config=config),)

    want = fn()
    g, out = _capture(fn)
    q2 = q[:700].clone()
    _replays(g, out, want, between=lambda: attention.attention(q2, k, v, config=config))


def test_graph_fused_block(dev):
    """One whole fused DiT block (quantizers, four GEMMs, attention), in place on x, captured; x is reset before
    each replay."""
    import torch
    from rapid_h3 import gemm, kernels
    from rapid_h3.block import BlockWeights, fused_block
    rng = np.random.default_rng(7)
    s, hid, heads, ffn = 1200, 256, 2, 512
    x0 = to_dev(_bf(rng.standard_normal((s, hid))), dev)
    qw = {name: kernels.quantize_weight(to_dev(_bf(0.02 * rng.standard_normal(shape)), dev), "int8_rowwise")
          for name, shape in (("qkv", (3 * hid, hid)), ("out", (hid, hid)), ("fc1", (2 * ffn, hid)),
                              ("fc2", (hid, ffn)))}
    perm = gemm.swiglu_perm(2 * ffn, dev)
    fc1 = kernels.QWeight(qw["fc1"].q[perm].contiguous(), qw["fc1"].scale[:, perm].contiguous())
    ones = torch.ones(hid, dtype=torch.bfloat16, device=dev)
    ones128 = torch.ones(128, dtype=torch.bfloat16, device=dev)
    w = BlockWeights(qkv=qw["qkv"], out=qw["out"], fc1_perm=fc1, fc2=qw["fc2"], norm1_w=ones, norm2_w=ones,
                     q_norm_w=ones128, k_norm_w=ones128, heads=heads, eps=1e-6, qk_eps=1e-6, recipe="int8_rowwise")
    mod = tuple(to_dev((0.1 * rng.standard_normal((2, hid))).astype(np.float32), dev) for _ in range(6))
    from oracle import attn as oa
    tab = to_dev(_bf(oa.rope_table(np.arange(s) % 53, rot=128).reshape(s, 64, 2, 2)), dev).view(1, s, 1, 64, 2, 2)
    segments = [(0, 300, 0), (300, s, 1)]
    x = x0.clone()

    def fn():
        return (fused_block(x, w, mod, segments, tab),)

    want = (fn()[0].clone(),)
    x.copy_(x0)
    g, out = _capture(fn)
    _replays(g, out, want, reset=lambda: x.copy_(x0), between=lambda: fused_block(x0.clone(), w, mod, segments, tab))
