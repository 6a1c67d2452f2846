"""rapid_h3.linear.QuantLinear, the _QuantLinear drop-in (__init__.py:83-167): output equal to
kernels.linear + bias, the weight cache and its invalidation, adoption of int8_convrot weights, the
measured-error diagnostics, and F.linear for CPU / fp32 activations."""
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


def test_quant_linear_adopts_convrot_and_cpu_takes_f_linear(dev):
    """An adopted int8_convrot weight runs the quantized path on bf16 GPU activations; CPU and fp32 activations take
    F.linear with the weight dequantized (the reference's route for them, __init__.py:147-148)."""
    import torch
    from rapid_h3 import kernels
    from rapid_h3.linear import QuantLinear
    g = torch.Generator(device="cpu").manual_seed(6)
    w = (0.02 * torch.randn(128, 256, generator=g)).to(torch.bfloat16).to(dev)
    qw = kernels.quantize_weight(w, "int8_rot")
    lin = QuantLinear.from_quantized(qw.q, qw.scale.reshape(-1))
    x = torch.randn(33, 256, generator=g).to(torch.bfloat16).to(dev)
    assert np.array_equal(to_np(lin(x)), to_np(kernels.linear(x, qw, "int8_rot")))
    y = lin(x.cpu())
    assert y.device.type == "cpu" and torch.equal(y, torch.nn.functional.linear(x.cpu(), lin.dense_weight("cpu", x.dtype)))
    y32 = lin(x.float())
    ref = x.float() @ w.float().t()
    assert y32.dtype == torch.float32 and float((y32 - ref).norm() / ref.norm()) < 0.01
    with pytest.raises(ValueError):
        QuantLinear(w, mode="bf16")


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
def test_quantize_any_dtype_against_torch(dev, dtype):
    """quantize_weight / quantize_rows / linear for weights and activations of any float dtype, against the
    reference's own torch formulas run on the CPU (kernels.py:57-82, :125-137): int8 and FP8 row-wise codes and
    scales bit-exact, fp8_tensor codes and its scalar scale bit-exact, and for non-bf16 x the int8_rowwise output
    (acc * sa * ws).to(x.dtype) bit-exact (fp8_rowwise within rel-L2 1e-2: its product is fp32-accumulated)."""
    import torch
    from rapid_h3 import kernels
    dt = getattr(torch, dtype)
    g = torch.Generator(device="cpu").manual_seed(9)
    w = (0.02 * torch.randn(136, 320, generator=g)).to(dt)
    x = torch.randn(77, 320, generator=g).to(dt)
    wf = w.float()
    for mode in ("int8_rowwise", "fp8_rowwise"):
        qw = kernels.quantize_weight(w.to(dev), mode)
        qmax = 127.0 if mode == "int8_rowwise" else 448.0
        s = (wf.abs().amax(dim=1, keepdim=True) / qmax).clamp_min(1e-12)
        ref = ((wf / s).round().clamp(-127, 127).to(torch.int8) if mode == "int8_rowwise"
               else (wf / s).clamp(-448, 448).to(torch.float8_e4m3fn))
        assert torch.equal(qw.q.cpu().view(torch.int8), ref.view(torch.int8)) and torch.equal(qw.scale.cpu(), s.t())
    qt = kernels.quantize_weight(w.to(dev), "fp8_tensor")
    st = (wf.abs().amax() / 448.0).clamp_min(1e-12)
    assert qt.scale.shape == () and qt.scale.item() == st.item()
    assert torch.equal(qt.q.cpu().view(torch.int8), (wf / st).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.int8))
    xq, sa = kernels.quantize_rows(x.to(dev), "int8_rowwise")
    sx = (x.abs().amax(dim=-1, keepdim=True).float() / 127.0).clamp_min(1e-12)
    assert torch.equal(sa.cpu(), sx)
    assert torch.equal(xq.cpu(), (x.float() / sx).round().clamp(-127, 127).to(torch.int8))
    if dt != torch.bfloat16:
        qw = kernels.quantize_weight(w.to(dev), "int8_rowwise")
        y = kernels.linear(x.to(dev), qw, "int8_rowwise")
        ref = (torch._int_mm(xq.cpu(), qw.q.cpu().t().contiguous()).float() * sx * qw.scale.cpu()).to(dt)
        assert y.dtype == dt and torch.equal(y.cpu(), ref)
        qf = kernels.quantize_weight(w.to(dev), "fp8_rowwise")
        yf = kernels.linear(x.to(dev), qf, "fp8_rowwise")
        exact = x.float() @ w.float().t()
        assert yf.dtype == dt and float((yf.cpu().float() - exact).norm() / exact.norm()) < 0.05
        with pytest.raises(ValueError):
            kernels.linear(x.to(dev), qw, "int8_rot")            # the reference's torch path has no int8_rot


@pytest.mark.parametrize("dtype", ["float32", "float16"])
def test_fp8_tensor_linear_non_bf16_out(dev, dtype):
    """fp8_tensor with fp32 / fp16 activations returns x.dtype rounded once from fp32, as the reference's
    torch._scaled_mm(out_dtype=x.dtype) does (kernels.py:124-127): the raw fp32 accumulators of the FP8 GEMM
    (rh3_gemm_fp8_acc) within 1e-4 rel-L2 of the exact product of the codes (oracle; measured 3e-5, the MFMA's own
    fp32 accumulation), and the output within 1e-4 (fp32) or the fp16 rounding (1e-3) of torch._scaled_mm run on the
    CPU with the same codes and scales. A bf16-rounded epilogue would miss every bound (its rounding alone is about
    2e-3)."""
    import torch
    from oracle import gemm as og
    from oracle.numerics import fp8_e4m3_to_f32
    from rapid_h3 import gemm, kernels, quant
    dt = getattr(torch, dtype)
    g = torch.Generator(device="cpu").manual_seed(12)
    w = (0.02 * torch.randn(264, 512, generator=g)).to(dt)
    x = torch.randn(130, 512, generator=g)
    x[:, :5] *= 20
    x = x.to(dt)
    qw = kernels.quantize_weight(w.to(dev), "fp8_tensor")
    y = kernels.linear(x.to(dev), qw, "fp8_tensor")
    assert y.dtype == dt and tuple(y.shape) == (130, 264)
    xq, s = quant.quant_any(x.to(dev), "fp8_tensor")
    acc = gemm.fp8_gemm_acc(xq, qw.q)
    a64 = fp8_e4m3_to_f32(to_np(xq.view(torch.uint8))).astype(np.float64)
    b64 = fp8_e4m3_to_f32(to_np(qw.q.view(torch.uint8))).astype(np.float64)
    assert og.rel_l2(to_np(acc), a64 @ b64.T) < 1e-4
    ref = torch._scaled_mm(xq.cpu(), qw.q.cpu().t(), s.cpu().reshape(()), qw.scale.cpu().reshape(()), out_dtype=dt)
    err = float((y.cpu().double() - ref.double()).norm() / ref.double().norm())
    assert err < (1e-4 if dt == torch.float32 else 1e-3), err


def test_c1_linear_full_size(dev):
    """BASELINE config C1, the reference's CPU-runnable case (bench/int8_bench.py:37-47): X [4096, 3072]
    ~ N(0, 1) with 31 of its channels (1 %) x20, W [3072, 3072] ~ N(0, 0.02), seed 0, generated on the CPU.
    kernels.linear bit-exact against the oracle (quantize_rows + exact int32 product + (acc*xs)*ws to bf16;
    with int8_rot the H256-rotated quantizer and weights), and the output error against the unquantized
    float64 product: int8_rowwise about 4.9 %, int8_rot about 1.2 % rel-L2 (the reference reports 6.6 % and
    1.4 % for 16 outlier channels)."""
    import torch
    from oracle import gemm as og
    from oracle import quant as oq
    from oracle.numerics import bf16_to_f32
    from rapid_h3 import kernels
    g = torch.Generator(device="cpu").manual_seed(0)
    x = torch.randn(4096, 3072, generator=g)
    x[:, torch.randperm(3072, generator=g)[:31]] *= 20
    w = torch.randn(3072, 3072, generator=g) * 0.02
    xb, wb = x.to(torch.bfloat16), w.to(torch.bfloat16)
    xn, wn = to_np(xb), to_np(wb)
    exact = bf16_to_f32(xn).astype(np.float64) @ bf16_to_f32(wn).astype(np.float64).T
    for mode, quant_x, bound in (("int8_rowwise", lambda a: oq.quantize_rows(a, "int8_rowwise"), 0.06),
                                 ("int8_rot", oq.rot_quant_rows_i8, 0.015)):
        y = to_np(kernels.linear(xb.to(dev), kernels.quantize_weight(wb.to(dev), mode), mode))
        xq, xs = quant_x(xn)
        assert np.array_equal(y, og.int8_gemm(xq, xs, *oq.quantize_weight(wn, mode))), mode
        assert og.rel_l2(bf16_to_f32(y), exact) < bound, mode


def test_nvfp4_verification_modes(dev):
    """The NVFP4 round trip (kernels.fake_nvfp4 + bf16 cast) on the GPU equals the oracle's bit for bit, on bf16
    and fp32 rows with outlier and all-zero blocks; quantize_weight / linear in nvfp4_fake and nvfp4_rot_fake give
    torch's bf16 linear of those round trips (the reference's F.linear, kernels.py:120-122), with QuantLinear too."""
    import torch
    from oracle import quant as oq
    from oracle.numerics import f32_to_bf16
    from rapid_h3 import kernels, quant
    from rapid_h3.linear import QuantLinear
    rng = np.random.default_rng(41)
    x = (rng.standard_normal((96, 512)) * np.exp(rng.standard_normal((96, 1)))).astype(np.float32)
    x[:, rng.choice(512, 5, replace=False)] *= 30.0
    x[7, 32:48] = 0.0
    xb = f32_to_bf16(x)
    got = to_np(quant.fake_nvfp4_bf16(torch.from_numpy(xb.view(np.int16)).to(dev).view(torch.bfloat16)))
    assert np.array_equal(got, f32_to_bf16(oq.fake_nvfp4(bf16_f32(xb))))
    got32 = to_np(quant.fake_nvfp4_bf16(torch.from_numpy(x).to(dev)))
    assert np.array_equal(got32, f32_to_bf16(oq.fake_nvfp4(x)))
    g = torch.Generator(device="cpu").manual_seed(6)
    w = (0.02 * torch.randn(264, 512, generator=g)).to(torch.bfloat16).to(dev)
    xt = torch.randn(3, 40, 512, generator=g).to(torch.bfloat16).to(dev)
    for mode in ("nvfp4_fake", "nvfp4_rot_fake"):
        qw = kernels.quantize_weight(w, mode)
        assert qw.scale is None and qw.q.dtype == torch.bfloat16 and tuple(qw.q.shape) == (264, 512)
        wn = bf16_f32(to_np(w))
        xn = bf16_f32(to_np(xt.reshape(-1, 512)))
        if mode == "nvfp4_rot_fake":
            wn, xn = oq.convrot(wn), oq.convrot(xn)
        assert np.array_equal(to_np(qw.q), f32_to_bf16(oq.fake_nvfp4(wn)))
        y = kernels.linear(xt, qw, mode)
        assert tuple(y.shape) == (3, 40, 264) and y.dtype == torch.bfloat16
        xf = torch.from_numpy(f32_to_bf16(oq.fake_nvfp4(xn)).view(np.int16)).to(dev).view(torch.bfloat16)
        ref = torch.nn.functional.linear(xf, qw.q)
        assert torch.equal(y.reshape(-1, 264), ref)
        lin = QuantLinear(w, None, mode)
        assert torch.equal(lin(xt), y)


def bf16_f32(u16):
    from oracle.numerics import bf16_to_f32
    return bf16_to_f32(u16)
