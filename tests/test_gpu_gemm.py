"""GPU parity of the W8A8 / FP8 GEMMs (librh3 rh3_gemm_*) against the CPU oracle: bit-exact int32
accumulators and bf16 epilogue outputs for int8 (SwiGLU: exp-dependent, within one bf16 ulp);
FP8 within rel-L2 1e-2 of the exact-product emulation."""
import numpy as np
import pytest

from conftest import to_dev, to_np
from oracle import gemm as og
from oracle import quant as oq
from oracle.numerics import bf16_to_f32, f32_to_bf16

pytestmark = pytest.mark.gpu


def _bf(a):
    return f32_to_bf16(np.asarray(a, np.float32))


def _bf16_ulps(a, b):
    """Distance in bf16 ulps between two bf16 bit arrays of finite values."""
    def key(u):
        u = u.astype(np.int32)
        return np.where(u & 0x8000, -(u & 0x7FFF), u)
    return np.abs(key(a) - key(b))


def test_gemm_golden(dev, golden):
    from rapid_h3 import gemm
    g = golden("gemm")
    xq, xs = to_dev(g["xq"], dev), to_dev(g["xs"], dev)
    wq, ws = to_dev(g["wq"], dev), to_dev(g["ws"], dev)
    assert np.array_equal(to_np(gemm.int8_gemm_acc(xq, wq)), g["acc"])
    assert np.array_equal(to_np(gemm.int8_gemm(xq, xs, wq, ws)), g["out"])
    assert np.array_equal(to_np(gemm.int8_gemm(xq, xs, wq, ws, bias=to_dev(g["bias"], dev))), g["out_bias"])
    resid = to_dev(g["resid"], dev)
    r = gemm.int8_gemm_gated_residual(xq, xs, wq, ws, to_dev(g["gate"], dev), resid)
    assert r is resid
    assert np.array_equal(to_np(resid), g["gated"])


def test_swiglu_golden(dev, golden):
    from rapid_h3 import gemm
    g = golden("gemm")
    xq, xs = to_dev(g["xq"], dev), to_dev(g["xs"], dev)
    perm = to_dev(g["perm"].astype(np.int64), dev)
    assert np.array_equal(to_np(gemm.swiglu_perm(512, dev)), g["perm"])
    w1q, w1s = to_dev(g["w1q"], dev), to_dev(g["w1s"], dev)
    h = to_np(gemm.int8_gemm_swiglu(xq, xs, w1q[perm].contiguous(), w1s[:, perm].contiguous()))
    d = _bf16_ulps(h, g["h"])
    assert d.max() <= 1 and (d > 0).mean() < 0.01


def test_fp8_golden(dev, golden):
    from rapid_h3 import gemm
    g = golden("gemm")
    out = gemm.fp8_gemm(to_dev(g["fq"], dev, "fp8"), to_dev(g["fs"], dev), to_dev(g["fwq"], dev, "fp8"),
                        to_dev(g["fws"], dev))
    got = bf16_to_f32(to_np(out))
    assert og.rel_l2(got, bf16_to_f32(g["fout"])) < 1e-2
    # and against the bf16 product of the unquantized operands (the reference's error metric)
    ref = bf16_to_f32(g["x"]).astype(np.float64) @ bf16_to_f32(g["w"]).astype(np.float64).T
    assert og.rel_l2(got, ref) < 0.08


@pytest.mark.parametrize("m,n,k", [(1, 8, 64), (17, 40, 128), (256, 256, 64), (513, 264, 1024), (64, 520, 8192),
                                   (1000, 3072, 3072)])
def test_gemm_shapes(dev, m, n, k):
    from rapid_h3 import gemm
    rng = np.random.default_rng(m + 7 * n + 13 * k)
    xq = rng.integers(-127, 128, size=(m, k), dtype=np.int8)
    wq = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    xs = (rng.random((m, 1)) * 1e-3).astype(np.float32)
    ws = (rng.random((1, n)) * 1e-3).astype(np.float32)
    xt, wt = to_dev(xq, dev), to_dev(wq, dev)
    assert np.array_equal(to_np(gemm.int8_gemm_acc(xt, wt)), og.int8_acc(xq, wq))
    out = gemm.int8_gemm(xt, to_dev(xs, dev), wt, to_dev(ws, dev))
    assert np.array_equal(to_np(out), og.int8_gemm(xq, xs, wq, ws))


@pytest.mark.parametrize("m,n,k", [(4500, 4112, 512), (700, 784, 1024)])
def test_gemm_persistent_epilogues(dev, m, n, k):
    """Shapes on the persistent kernel (K a multiple of 256, at least 512): 18 x 17 = 306 tiles give some
    workgroups two tiles, so a tile boundary falls inside the cross-tile k-loop; ragged last tile row and
    column. Every epilogue against the oracle: int32 accumulators, plain and bias outputs, the gated residual
    bit-exact, SwiGLU within one bf16 ulp, FP8 within rel-L2 1e-2."""
    from rapid_h3 import gemm
    rng = np.random.default_rng(m + n + k)
    xq = np.clip(np.rint(rng.standard_normal((m, k)) * 30), -127, 127).astype(np.int8)
    wq = np.clip(np.rint(rng.standard_normal((n, k)) * 30), -127, 127).astype(np.int8)
    xs = (rng.random((m, 1)) * 1e-3 + 1e-4).astype(np.float32)
    ws = (rng.random((1, n)) * 1e-3 + 1e-4).astype(np.float32)
    bias = _bf(rng.standard_normal(n))
    gate = _bf(rng.standard_normal(n))
    resid = _bf(rng.standard_normal((m, n)))
    xt, wt, xst, wst = to_dev(xq, dev), to_dev(wq, dev), to_dev(xs, dev), to_dev(ws, dev)
    acc = og.int8_acc(xq, wq)
    assert np.array_equal(to_np(gemm.int8_gemm_acc(xt, wt)), acc)
    y = og.dequant(acc, xs, ws)
    assert np.array_equal(to_np(gemm.int8_gemm(xt, xst, wt, wst)), f32_to_bf16(y))
    yb = (y + bf16_to_f32(bias).reshape(1, -1)).astype(np.float32)
    assert np.array_equal(to_np(gemm.int8_gemm(xt, xst, wt, wst, bias=to_dev(bias, dev))), f32_to_bf16(yb))
    rt = to_dev(resid, dev)
    gemm.int8_gemm_gated_residual(xt, xst, wt, wst, to_dev(gate, dev), rt)
    want = f32_to_bf16(og.fma_f32(bf16_to_f32(f32_to_bf16(y)), np.broadcast_to(bf16_to_f32(gate).reshape(1, -1), y.shape),
                                  bf16_to_f32(resid)))
    assert np.array_equal(to_np(rt), want)
    h = to_np(gemm.int8_gemm_swiglu(xt, xst, wt, wst))
    d = _bf16_ulps(h, og.swiglu_from_interleaved(f32_to_bf16(y)))
    assert d.max() <= 1 and (d > 0).mean() < 0.01
    fq = rng.integers(0, 256, size=(m, k), dtype=np.uint8)
    fwq = rng.integers(0, 256, size=(n, k), dtype=np.uint8)
    fq[(fq & 0x7F) == 0x7F] = 0  # no NaN codes
    fwq[(fwq & 0x7F) == 0x7F] = 0
    got = bf16_to_f32(to_np(gemm.fp8_gemm(to_dev(fq, dev, "fp8"), xst, to_dev(fwq, dev, "fp8"), wst)))
    assert og.rel_l2(got, bf16_to_f32(og.fp8_gemm(fq, xs, fwq, ws))) < 1e-2


@pytest.mark.parametrize("m,n,k", [(4500, 4112, 512), (9000, 8200, 256), (700, 784, 1024), (300, 264, 512)])
def test_gemm_tile_counters(dev, m, n, k):
    """The persistent kernel with per-XCD tile counters (ctr, the Python layer's default) and with the fixed tile
    shares (ctr NULL) against the oracle's int32 accumulators, bit-exact; two calls in a row on one counter buffer
    (each call clears it). 306 and 1155 tiles (more than one per CU, so workgroups claim and steal), 12 tiles
    (fewer than the CUs: every workgroup's first tile is its last) and 4 tiles (fewer than the 8 XCDs: some XCD
    ranges are empty and every claim returns none)."""
    import ctypes
    import torch
    from rapid_h3 import _native as nat
    rng = np.random.default_rng(m + n + k)
    xq = np.clip(np.rint(rng.standard_normal((m, k)) * 30), -127, 127).astype(np.int8)
    wq = np.clip(np.rint(rng.standard_normal((n, k)) * 30), -127, 127).astype(np.int8)
    want = og.int8_acc(xq, wq)
    xt, wt = to_dev(xq, dev), to_dev(wq, dev)
    ctr = torch.full((8,), 12345, dtype=torch.int32, device=dev)  # stale contents: the call must clear them
    for c in (None, ctypes.c_void_p(ctr.data_ptr()), ctypes.c_void_p(ctr.data_ptr())):
        acc = torch.full((m, n), -1, dtype=torch.int32, device=dev)
        nat.call("rh3_gemm_i8_acc", nat.ptr(xt), k, nat.ptr(wt), k, nat.ptr(acc), n, m, n, k, c, nat.stream(dev))
        assert np.array_equal(to_np(acc), want)


@pytest.mark.parametrize("m,n,k", [(4500, 4112, 512), (300, 264, 128)])
def test_gemm_gated_rows(dev, m, n, k):
    """The gated residual with a gate row per token (per-token modulation) bit-exact against the oracle, on the
    persistent kernel (K 512) and on the one-tile-per-workgroup kernel (K 128); rows index a 7-row table."""
    import torch
    from rapid_h3 import gemm
    rng = np.random.default_rng(m + k)
    xq = np.clip(np.rint(rng.standard_normal((m, k)) * 30), -127, 127).astype(np.int8)
    wq = np.clip(np.rint(rng.standard_normal((n, k)) * 30), -127, 127).astype(np.int8)
    xs = (rng.random((m, 1)) * 1e-3 + 1e-4).astype(np.float32)
    ws = (rng.random((1, n)) * 1e-3 + 1e-4).astype(np.float32)
    tab = _bf(rng.standard_normal((7, n)))
    rows = rng.integers(0, 7, m)
    resid = _bf(rng.standard_normal((m, n)))
    rt = to_dev(resid, dev)
    r = gemm.int8_gemm_gated_residual_rows(to_dev(xq, dev), to_dev(xs, dev), to_dev(wq, dev), to_dev(ws, dev),
                                           to_dev(tab, dev), torch.from_numpy(rows).to(dev), rt)
    assert r is rt
    assert np.array_equal(to_np(rt), og.int8_gemm_gated_residual_rows(xq, xs, wq, ws, tab, rows, resid))


def test_gemm_rejects_bad_shapes(dev):
    import torch
    from rapid_h3 import gemm
    xq = torch.zeros(4, 96, dtype=torch.int8, device=dev)
    wq = torch.zeros(8, 96, dtype=torch.int8, device=dev)
    with pytest.raises(RuntimeError, match="multiple of 64"):
        gemm.int8_gemm(xq, torch.ones(4, 1, device=dev), wq, torch.ones(1, 8, device=dev))
    with pytest.raises(RuntimeError):
        gemm.int8_gemm(xq[:, :64], torch.ones(4, 1, device=dev), wq[:7, :64], torch.ones(1, 7, device=dev))


def test_gemm_full_size_qkv(dev):
    """C2 QKV at M = 145,152, N = 9216, K = 3072: int32 accumulators bit-exact on 256 sampled rows, the
    bf16 output on the same rows, and an exact checksum of checksums over every accumulator:
    sum_m acc[m, n] == sum_k (sum_m xq[m, k]) * wq[n, k]."""
    import torch
    from rapid_h3 import gemm, quant
    m, n, k = 145152, 9216, 3072
    gen = torch.Generator(device="cpu").manual_seed(0)
    x = torch.randn(m, k, generator=gen)
    x[:, torch.randperm(k, generator=gen)[:31]] *= 20
    xt = x.to(torch.bfloat16).to(dev)
    del x
    w = (torch.randn(n, k, generator=gen) * 0.02).to(torch.bfloat16).to(dev)
    xq, xs = quant.quant_rows_i8(xt)
    wq, ws = quant.quant_rows_i8(w)
    acc = gemm.int8_gemm_acc(xq, wq)
    out = gemm.int8_gemm(xq, xs, wq, ws.t())
    rows = torch.from_numpy(np.sort(np.random.default_rng(2).choice(m, 256, replace=False))).to(dev)
    xr = to_np(xq[rows])
    wn = to_np(wq)
    assert np.array_equal(to_np(acc[rows]), og.int8_acc(xr, wn))
    assert np.array_equal(to_np(out[rows]), og.int8_gemm(xr, to_np(xs[rows]), wn, to_np(ws).T))
    lhs = acc.double().sum(dim=0)
    rhs = wq.double() @ xq.double().sum(dim=0)
    assert bool(torch.equal(lhs, rhs))


@pytest.mark.parametrize("epi", ["swiglu", "gated"])
def test_gemm_full_size_ffn(dev, epi):
    """The other two C2 GEMMs at M = 145,152 with their fused epilogues, on 256 sampled rows against the oracle:
    FFN-up (N = 16,384, K = 3072) with the SwiGLU epilogue over the swiglu_perm interleave (within 1 bf16 ulp on
    < 1 % of elements: the exp is approximate on both sides), FFN-down (N = 3072, K = 8192) with the in-place
    gated residual (bit-exact), and the rows outside the sample untouched by the sampling."""
    import torch
    from rapid_h3 import gemm, quant
    m = 145152
    n, k = (16384, 3072) if epi == "swiglu" else (3072, 8192)
    g = torch.Generator(device=dev).manual_seed(7)
    x = torch.randn(m, k, generator=g, device=dev)
    x[:, torch.randperm(k, generator=g, device=dev)[:k // 100]] *= 20
    xb = x.to(torch.bfloat16)
    del x
    w = (0.02 * torch.randn(n, k, generator=g, device=dev)).to(torch.bfloat16)
    xq, xs = quant.quant_rows_i8(xb)
    wq, ws = quant.quant_rows_i8(w)
    rows = torch.from_numpy(np.sort(np.random.default_rng(8).choice(m, 256, replace=False))).to(dev)
    xr, xsr = to_np(xq[rows]), to_np(xs[rows])
    if epi == "swiglu":
        perm = gemm.swiglu_perm(n, dev)
        wp, wsp = wq[perm].contiguous(), ws[perm].t().contiguous()
        h = gemm.int8_gemm_swiglu(xq, xs, wp, wsp)
        assert tuple(h.shape) == (m, n // 2)
        ref = og.int8_gemm_swiglu(xr, xsr, to_np(wp), to_np(wsp))
        d = _bf16_ulps(to_np(h[rows]), ref)
        assert d.max() <= 1 and (d > 0).mean() < 0.01
    else:
        gate = (0.5 * torch.randn(n, generator=g, device=dev)).to(torch.bfloat16)
        resid = torch.randn(m, n, generator=g, device=dev).to(torch.bfloat16)
        r0 = to_np(resid[rows])
        out = gemm.int8_gemm_gated_residual(xq, xs, wq, ws.t(), gate, resid)
        assert out.data_ptr() == resid.data_ptr()
        ref = og.int8_gemm_gated_residual(xr, xsr, to_np(wq), to_np(ws).T, to_np(gate), r0)
        assert np.array_equal(to_np(resid[rows]), ref)


@pytest.mark.parametrize("n,k", [(9216, 3072), (16384, 3072), (3072, 8192)])
def test_fp8_full_size_c3(dev, n, k):
    """the FP8 (OCP e4m3) row-wise GEMM on the three C2 shapes at M = 145,152, bf16
    activations N(0, 1) with 1 % of channels x20, weights N(0, 0.02): per-token and per-channel scales with
    the row absmax at 448, codes and scales bit-exact on 256 sampled rows (and sampled weight rows), the bf16
    output on those rows within rel-L2 1e-2 of the exact-product emulation, and against the unquantized
    product within the e4m3 error (rel-L2 < 0.08)."""
    import torch
    from rapid_h3 import gemm, kernels, quant
    m = 145152
    g = torch.Generator(device=dev).manual_seed(n + k)
    x = torch.randn(m, k, generator=g, device=dev)
    x[:, torch.randperm(k, generator=g, device=dev)[:k // 100]] *= 20
    x = x.to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    xq, xs = quant.quant_rows(x)
    qw = kernels.quantize_weight(w, "fp8_rowwise")
    out = gemm.fp8_gemm(xq, xs, qw.q, qw.scale)
    rows = torch.from_numpy(np.sort(np.random.default_rng(n).choice(m, 256, replace=False))).to(dev)
    xr = to_np(x[rows])
    eq, es = oq.quantize_rows(xr, "fp8_rowwise")
    assert np.array_equal(to_np(xq[rows]), eq) and np.array_equal(to_np(xs[rows]), es)
    wr = torch.arange(0, n, 509, device=dev)
    weq, wes = oq.quantize_weight(to_np(w[wr]), "fp8_rowwise")
    assert np.array_equal(to_np(qw.q[wr]), weq) and np.array_equal(to_np(qw.scale[:, wr]), wes)
    got = bf16_to_f32(to_np(out[rows]))
    ref = bf16_to_f32(og.fp8_gemm(eq, es, to_np(qw.q), to_np(qw.scale)))
    assert og.rel_l2(got, ref) < 1e-2
    exact = bf16_to_f32(xr).astype(np.float64) @ bf16_to_f32(to_np(w)).astype(np.float64).T
    assert og.rel_l2(got, exact) < 0.08


def test_gemm_counter_buffers_per_stream(dev):
    """The Python layer's tile-counter buffers: one per (device, stream), reused on its stream, never shared between
    streams (calls on different streams may run at once); a GEMM on a second stream matches the first bit for bit."""
    import torch
    from rapid_h3 import _native as nat
    from rapid_h3 import gemm
    a = nat.gemm_ctr(dev).data_ptr()
    assert nat.gemm_ctr(dev).data_ptr() == a
    s = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(s):
        b = nat.gemm_ctr(dev).data_ptr()
        assert nat.gemm_ctr(dev).data_ptr() == b
    assert a != b
    rng = np.random.default_rng(3)
    xq = to_dev(np.clip(np.rint(rng.standard_normal((2000, 512)) * 30), -127, 127).astype(np.int8), dev)
    wq = to_dev(np.clip(np.rint(rng.standard_normal((2048, 512)) * 30), -127, 127).astype(np.int8), dev)
    xs = to_dev((rng.random((2000, 1)) * 1e-3 + 1e-4).astype(np.float32), dev)
    ws = to_dev((rng.random((1, 2048)) * 1e-3 + 1e-4).astype(np.float32), dev)
    y0 = gemm.int8_gemm(xq, xs, wq, ws)
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        y1 = gemm.int8_gemm(xq, xs, wq, ws)
    torch.cuda.synchronize()
    assert torch.equal(y0.view(torch.int16), y1.view(torch.int16))


def test_gated_rows_index_out_of_range(dev):
    """A per-token gate row index outside the table raises on the host (torch's gather raises there too); the kernel
    is never launched with it."""
    import torch
    from rapid_h3 import gemm
    m, n, k = 64, 256, 256
    xq = torch.ones(m, k, dtype=torch.int8, device=dev)
    wq = torch.ones(n, k, dtype=torch.int8, device=dev)
    xs = torch.ones(m, 1, device=dev)
    ws = torch.ones(1, n, device=dev)
    gate = torch.ones(3, n, dtype=torch.bfloat16, device=dev)
    resid = torch.zeros(m, n, dtype=torch.bfloat16, device=dev)
    for bad in (3, -1):
        rows = torch.zeros(m, dtype=torch.long, device=dev)
        rows[17] = bad
        with pytest.raises(IndexError):
            gemm.int8_gemm_gated_residual_rows(xq, xs, wq, ws, gate, rows, resid)
    assert int(resid.abs().max()) == 0
    rows = torch.full((m,), 2, dtype=torch.long, device=dev)
    gemm.int8_gemm_gated_residual_rows(xq, xs, wq, ws, gate, rows, resid)
    assert float(resid.float().min()) == float(k)
