"""Benchmark of the MI355X DiT hot path: one step = one full-size DiT block through the fused INT8 chain
(rapid_h3.block.fused_block) at M = S = 145,152 tokens, hidden 3072, 24 x 128 heads, FFN 8192:

  RMSNorm+modulation INT8 quantizer -> QKV W8A8 GEMM -> q/k RMSNorm+RoPE INT8 attention pre-pass ->
  INT8 attention (int8 Q.K^T, bf16 P.V) -> head-major INT8 quantizer -> out-proj GEMM + gated residual ->
  RMSNorm+modulation quantizer -> FFN-up GEMM + SwiGLU -> INT8 quantizer -> FFN-down GEMM + gated residual

value = algorithmic int8-MFMA work of the block (4 GEMMs 2*M*N*K + attention 4*S^2*D*H) / time, in
TOPS, inputs and weights resident in HBM before the timed region. Synthetic data: activations N(0,1)
with 1 % of channels x20, weights N(0, 0.02) random init, modulation and norm weights random.

    python bench.py [--gpus 1] [--steps 3] [--warmup 1] [--tokens 145152] [--no-cpu] [--no-side]
                    [--recipe int8_rot] [--attn-config 94] [--model h3]

After the timed block (outside the timed region): the C3 FP8 GEMMs at the three C2 shapes and hipBLASLt's int8
GEMM (torch._int_mm) beside this build's at the four block shapes (fp8_gemm_c3, int8_gemm_vs_hipblaslt), one block
at MiniMax-H3's shapes (h3_shapes), one block in the reference's preset numerics (reference_preset: int8_rot
quantizers, attention config 94), and the CPU baseline (cpu_baseline) on the same block's inputs.

--model h3 runs the same block at MiniMax-H3's own shapes (hidden 5376, 56 x 128 heads, FFN 14336,
S = 44,992 by default), the shapes of the reference's published GB10 numbers; the default (c2) is the
configuration the metric names.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "rapid-h3_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "INT8 attn + W8A8 GEMM TOPS (frac of MFMA peak) at 145k tokens; ms/DiT block"
PEAK_INT8_TOPS = 5033.0        # MI355X dense int8 MFMA
PEAK_BF16_TFLOPS = 2517.0      # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E
PEAK_FP8_TFLOPS = 5033.0       # MI355X dense OCP-FP8 MFMA
D = 128
MODELS = {  # hidden, heads, FFN width, default tokens
    "c2": (3072, 24, 8192, 145152),    # BASELINE.json configs C2 / C4: 36 x 48 x 84 latent patches
    "h3": (5376, 56, 14336, 44992),    # MiniMax-H3 (the reference's bench/microbench.py:15, docs/kernels.md:405)
}
HIDDEN, HEADS, FFN, _ = MODELS["c2"]
GRID = (36, 48, 84)            # latent frames x patch rows x patch columns = 145,152 tokens


def rope_table(s, device):
    """Split-half RoPE table [1, S, 1, 48, 2, 2] bf16 = (cos, -sin, sin, cos) over (t, h, w) positions of
    the latent grid, 16 frequencies per axis (the H3 layout of bench/rmsrope_fuse.py:22-33)."""
    import torch
    t, hh, ww = GRID
    idx = torch.arange(s, device=device)
    pos = torch.stack([(idx // (hh * ww)) % t, (idx // ww) % hh, idx % ww], 1).float()
    inv = 1.0 / (10000.0 ** (torch.arange(16, dtype=torch.float32, device=device) / 16))
    a = torch.cat((pos.unsqueeze(-1) * inv.view(1, 1, -1)).unbind(1), -1)      # [S, 48]
    c, sn = torch.cos(a), torch.sin(a)
    return torch.stack([c, -sn, sn, c], -1).reshape(1, s, 1, 48, 2, 2).to(torch.bfloat16)


def block_ops(m):
    gemms = {"gemm_qkv": 2 * m * 3 * HEADS * D * HIDDEN, "gemm_out_gated": 2 * m * HIDDEN * HEADS * D,
             "gemm_up_swiglu": 2 * m * 2 * FFN * HIDDEN, "gemm_down_gated": 2 * m * HIDDEN * FFN}
    return gemms, 4 * m * m * D * HEADS


def quant_bytes(m):
    """Algorithmic HBM bytes of each quantizer phase: input read once, int8 codes + fp32 scale written."""
    k_in = {"quant_norm1": HIDDEN, "quant_heads": HEADS * D, "quant_norm2": HIDDEN, "quant_h": FFN}
    return {n: m * k * 2 + m * k + 4 * m for n, k in k_in.items()}


def setup(m, device, recipe="int8_rowwise"):
    import torch
    from rapid_h3 import gemm, kernels
    from rapid_h3.block import BlockWeights
    g = torch.Generator(device=device).manual_seed(0)

    def randn(*shape, std=1.0):
        return torch.randn(*shape, generator=g, device=device) * std

    x = randn(m, HIDDEN)
    x[:, torch.randperm(HIDDEN, generator=g, device=device)[:HIDDEN // 100]] *= 20
    x = x.to(torch.bfloat16)
    qw = {}
    for name, n, k in (("qkv", 3 * HEADS * D, HIDDEN), ("out", HIDDEN, HEADS * D), ("fc1", 2 * FFN, HIDDEN),
                       ("fc2", HIDDEN, FFN)):
        qw[name] = kernels.quantize_weight(randn(n, k, std=0.02).to(torch.bfloat16), recipe)
    perm = gemm.swiglu_perm(2 * FFN, device)
    fc1 = kernels.QWeight(qw["fc1"].q[perm].contiguous(), qw["fc1"].scale[:, perm].contiguous())

    def nw(n):
        return (1 + 0.3 * randn(n)).to(torch.bfloat16)

    w = BlockWeights(qkv=qw["qkv"], out=qw["out"], fc1_perm=fc1, fc2=qw["fc2"], norm1_w=nw(HIDDEN),
                     norm2_w=nw(HIDDEN), q_norm_w=nw(D), k_norm_w=nw(D), heads=HEADS, recipe=recipe)
    mod = tuple(randn(1, HIDDEN, std=0.1) for _ in range(6))
    segments = [(0, m, 0)]
    tab = rope_table(m, device)
    torch.cuda.synchronize()
    return x, w, mod, segments, tab


def _cpu_threads():
    """Threads for the CPU baseline: every core this process may run on (os.sched_getaffinity; on the GPU box that
    is the job's share, where os.cpu_count() counts the whole host), set for torch and numpy's BLAS alike."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    import torch
    torch.set_num_threads(n)
    try:
        from threadpoolctl import threadpool_limits
        threadpool_limits(n)
    except Exception:  # noqa: BLE001
        pass
    return n


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_time(fn, runs=5, warmup=1):
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return ts[len(ts) // 2]


def cpu_baseline(m, x, w, mod, segments, tab, trace, ms=4096, rows=1024):
    """The CPU baseline: the build's CPU restatement of the reference's PyTorch path (oracle/, a numpy port:
    kernels.quantize_rows / quantize_weight, the exact int32 product, the (acc * xs) * ws epilogues, the per-block
    attention emulation), on the host cores of the GPU box, each part the median of 5 runs after 1 warm-up, sampled
    as follows:
      * C1 (X [4096, 3072] with 1 % outlier channels, W [3072, 3072] ~ N(0, 0.02), seed 0): measured in full;
      * C2: each of the block's four GEMMs with the quantizer that feeds it, on the first `ms` = 4,096 tokens of the
        GPU leg's own inputs (x, the block's int8 weights, its modulation, and the o / h / x of a traced run of the
        same block), scaled by M / ms;
      * C4: the attention of head 0 for the first `rows` = 1,024 query rows against all keys, scaled by
        (S / rows) x H, and that head's pre-pass over all keys, scaled by H.
    Each part's time and factor are reported; the block's time is their sum."""
    import numpy as np
    import torch
    from oracle import attn as oa
    from oracle import gemm as og
    from oracle import quant as oq
    from oracle.numerics import f32_to_bf16
    threads = _cpu_threads()

    def host(t):
        t = t.detach().cpu()
        return t.view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.numpy()

    # C1 in full, generated on the CPU as BASELINE.json's config C1 (seed 0)
    g = torch.Generator().manual_seed(0)
    x1 = torch.randn(4096, 3072, generator=g)
    x1[:, torch.randperm(3072, generator=g)[:31]] *= 20
    w1 = 0.02 * torch.randn(3072, 3072, generator=g)
    x1b, w1b = host(x1.to(torch.bfloat16)), host(w1.to(torch.bfloat16))

    def c1():
        xq, xs = oq.quantize_rows(x1b)
        wq, ws = oq.quantize_weight(w1b)
        og.int8_gemm(xq, xs, wq, ws)
    t_c1 = _median_time(c1)
    ops_c1 = 2 * 4096 * 3072 * 3072

    # the block sample on the GPU leg's inputs
    ms = min(ms, m)
    T = {k: v for k, v in trace.items()}
    idx = np.zeros(ms, np.int32)
    for a, b, r in segments:
        lo, hi = max(a, 0), min(b, ms)
        if lo < hi:
            idx[lo:hi] = int(r)
    mods = [host(t.float()) for t in mod]
    xs_ = host(x[:ms])
    xa = host(T["x_attn"][:ms])
    nw1, nw2 = host(w.norm1_w), host(w.norm2_w)
    wts = {n: (host(getattr(w, n).q), host(getattr(w, n).scale)) for n in ("qkv", "out", "fc1_perm", "fc2")}
    o_h = host(T["o"][0][:, :ms])                                          # [H, ms, 128] head-major
    h_ = host(T["h"][:ms])
    s = x.shape[0]
    rows = min(rows, s)
    qkv0 = T["qkv"].view(s, 3, HEADS, D)[:, :, 0]                           # head 0 of the raw projection
    q0, k0, v0 = host(qkv0[:rows, 0]).reshape(rows, 1, D), host(qkv0[:, 1]).reshape(s, 1, D), host(qkv0[:, 2])
    v0 = v0.reshape(s, 1, D)
    tabh = host(tab.reshape(s, 48, 2, 2))
    rr = (tabh, host(w.q_norm_w), host(w.k_norm_w), w.qk_eps)
    gate_a, gate_m = f32_to_bf16(mods[2][0]), f32_to_bf16(mods[5][0])

    def qkv_part():
        xq, xs = oq.norm_mod_quant_rows_i8(xs_, nw1, w.eps, idx, mods[0], mods[1])
        og.int8_gemm(xq, xs, *wts["qkv"])

    def out_part():
        oq_, os_ = oq.heads_quant_rows_i8(o_h)
        og.int8_gemm_gated_residual(oq_, os_, *wts["out"], gate_a, xa)

    def up_part():
        xq, xs = oq.norm_mod_quant_rows_i8(xa, nw2, w.eps, idx, mods[3], mods[4])
        og.int8_gemm_swiglu(xq, xs, *wts["fc1_perm"])

    def down_part():
        hq, hs = oq.quantize_rows(h_, "int8_rowwise")
        og.int8_gemm_gated_residual(hq, hs, *wts["fc2"], gate_m, xa)

    pre = {}

    def prepass():
        pre["ops"] = oa.prepass(np.concatenate([q0, np.zeros((s - rows, 1, D), np.uint16)]), k0, rr=rr)

    def attn_rows():
        q8, qs, k8, ks, _ = pre["ops"]
        oa.attention_from_codes(q8, qs, k8, ks, v0, D ** -0.5, rows=np.arange(rows))

    gemms, attn_ops = block_ops(m)
    parts = {}
    for name, fn, factor in (("quant_norm1+gemm_qkv", qkv_part, m / ms), ("quant_heads+gemm_out_gated", out_part, m / ms),
                             ("quant_norm2+gemm_up_swiglu", up_part, m / ms),
                             ("quant_h+gemm_down_gated", down_part, m / ms),
                             ("attn_prepass", prepass, HEADS), ("attn_main", attn_rows, (s / rows) * HEADS)):
        t = _median_time(fn)
        parts[name] = {"s": round(t, 3), "factor": round(factor, 1), "s_per_block": round(t * factor, 1)}
    t_block = sum(p_["s_per_block"] for p_ in parts.values())
    total = sum(gemms.values()) + attn_ops
    return {"value": round(total / t_block / 1e12, 4), "unit": "TOPS", "cores": int(threads), "kind": "port",
            "cpu_model": _cpu_model(), "os_cpu_count": os.cpu_count(), "runs": "median of 5 after 1 warm-up",
            "c1_measured": {"ms": round(t_c1 * 1e3, 1), "tops": round(ops_c1 / t_c1 / 1e12, 4),
                            "workload": "C1 W8A8 linear, 4096 x 3072 x 3072, in full"},
            "sample": (f"oracle (numpy) on the GPU leg's inputs: each block GEMM with its quantizer on the first {ms} "
                       f"tokens (x{m / ms:.1f}), head 0's pre-pass over all {s} keys (x{HEADS}) and its attention for "
                       f"{rows} query rows (x{s / rows * HEADS:.0f}); extrapolated to the block; C1 measured in full"),
            "parts": parts, "seconds_per_block": round(t_block, 1)}


def gemm_side_measurements(m, device, reps=5):
    """C3 FP8 (OCP e4m3) row-wise GEMMs at the three C2 shapes (rh3_gemm_fp8, bf16 out) and hipBLASLt's int8 GEMM
    (torch._int_mm, int32 out, no epilogue) at the four C2 block shapes, each the mean of reps launches timed
    with events on torch's current stream, codes uniform random (the GEMMs' speed does not depend on values)."""
    import torch
    from rapid_h3 import gemm
    g = torch.Generator(device=device).manual_seed(1)
    shapes = {"qkv": (3 * HEADS * D, HIDDEN), "up": (2 * FFN, HIDDEN), "down": (HIDDEN, FFN), "out": (HIDDEN, HEADS * D)}

    def timeit(fn):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    fp8, vendor = {}, {}
    xs = torch.rand(m, 1, device=device, generator=g) * 1e-3
    for name, (n, k) in shapes.items():
        ws = torch.rand(1, n, device=device, generator=g) * 1e-3
        ops = 2 * m * n * k
        if name != "out":
            xq = torch.randint(0, 256, (m, k), device=device, dtype=torch.uint8, generator=g)
            xq[(xq & 0x7F) == 0x7F] = 0
            wq = torch.randint(0, 256, (n, k), device=device, dtype=torch.uint8, generator=g)
            wq[(wq & 0x7F) == 0x7F] = 0
            xf, wf = xq.view(torch.float8_e4m3fn), wq.view(torch.float8_e4m3fn)
            t = timeit(lambda: gemm.fp8_gemm(xf, xs, wf, ws))
            fp8[name] = {"ms": round(t, 3), "tflops": round(ops / t / 1e9, 1), "frac_fp8_peak": round(ops / t / 1e9 / PEAK_FP8_TFLOPS, 4),
                         "shape": [m, n, k]}
            del xq, wq, xf, wf
        xi = torch.randint(-127, 128, (m, k), device=device, dtype=torch.int8, generator=g)
        wi = torch.randint(-127, 128, (n, k), device=device, dtype=torch.int8, generator=g)
        wt = wi.t()
        tv = timeit(lambda: torch._int_mm(xi, wt))
        to = timeit(lambda: gemm.int8_gemm(xi, xs, wi, ws))
        vendor[name] = {"int_mm_ms": round(tv, 3), "int_mm_tops": round(ops / tv / 1e9, 1),
                        "rh3_plain_ms": round(to, 3), "rh3_plain_tops": round(ops / to / 1e9, 1), "shape": [m, n, k]}
        del xi, wi, wt
        torch.cuda.empty_cache()
    return fp8, vendor


def lead_in():
    """A few milliseconds of GPU spin (torch's bounded clock-count sleep kernel), enqueued untimed right before a
    timed region: while it runs, the host enqueues the region's first launches, so the GPU does not sit idle inside
    the first phase waiting for Python (that wait would be charged to quant_norm1)."""
    import torch
    torch.cuda._sleep(10_000_000)  # clock cycles at the shader clock: ~5 ms


def h3_side_measurements(device, recipe, tokens=(22332, 44992)):
    """One DiT block at MiniMax-H3's own shapes (hidden 5376, 56 x 128 heads, FFN 14336; the shapes of the
    reference's published numbers) for each token count: 1 untimed block, then 1 block timed per phase with
    events on torch's current stream. Runs after the metric's timed region, on fresh synthetic inputs."""
    import torch
    from rapid_h3.block import PHASES, fused_block
    global HIDDEN, HEADS, FFN
    saved = (HIDDEN, HEADS, FFN)
    HIDDEN, HEADS, FFN, _ = MODELS["h3"]
    res = {}
    try:
        for m in tokens:
            x, w, mod, segments, tab = setup(m, device, recipe)
            fused_block(x, w, mod, segments, tab)
            torch.cuda.synchronize()
            ev = []

            def mark(name):
                e = torch.cuda.Event(enable_timing=True)
                e.record()
                ev.append((name, e))
            lead_in()
            b = torch.cuda.Event(enable_timing=True)
            b.record()
            ev.append(("begin", b))
            fused_block(x, w, mod, segments, tab, mark=mark)
            torch.cuda.synchronize()
            ph = {name: round(e0.elapsed_time(e1), 3) for (_, e0), (name, e1) in zip(ev[:-1], ev[1:])}
            gemms, attn_ops = block_ops(m)
            gms = sum(ph[k] for k in gemms)
            res[str(m)] = {"ms_per_block": round(sum(ph.values()), 3), "phases_ms": ph,
                           "gemm_tops": round(sum(gemms.values()) / (gms * 1e-3) / 1e12, 1),
                           "attn_tops": round(attn_ops / (ph["attn_main"] * 1e-3) / 1e12, 1)}
            del x, w, mod, tab
            torch.cuda.empty_cache()
    finally:
        HIDDEN, HEADS, FFN = saved
    return res


def preset_side_measurement(m, device, steps=2):
    """The reference's preset numerics at the metric's shape (its RapidH3 presets 190 / 194): every quantizer with the
    ConvRot H256 rotation (int8_rot weights and activations) and the production attention, config 94 (per-token
    H128-rotated Q/K, per-channel int8 V, u8 P against each 128-key tile's max, int8 P.V). 1 untimed block, then
    `steps` blocks timed per phase with events on torch's current stream; runs after the metric's timed region, on
    fresh synthetic inputs."""
    import torch
    from rapid_h3.block import PHASES, fused_block
    x, w, mod, segments, tab = setup(m, device, "int8_rot")
    fused_block(x, w, mod, segments, tab, attn_config=94)
    torch.cuda.synchronize()
    phase_ms = {p: 0.0 for p in PHASES}
    lead_in()
    for _ in range(steps):
        ev = []

        def mark(name):
            e = torch.cuda.Event(enable_timing=True)
            e.record()
            ev.append((name, e))
        b = torch.cuda.Event(enable_timing=True)
        b.record()
        ev.append(("begin", b))
        fused_block(x, w, mod, segments, tab, attn_config=94, mark=mark)
        torch.cuda.synchronize()
        for (_, e0), (name, e1) in zip(ev[:-1], ev[1:]):
            phase_ms[name] += e0.elapsed_time(e1) / steps
    gemms, attn_ops = block_ops(m)
    qbytes = quant_bytes(m)
    parts = {}
    for p_, t in phase_ms.items():
        parts[p_] = {"ms": round(t, 3)}
        if p_ in qbytes:
            parts[p_]["frac_hbm"] = round(qbytes[p_] / (t * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)
        elif p_ in gemms:
            parts[p_]["frac_int8_peak"] = round(gemms[p_] / (t * 1e-3) / 1e12 / PEAK_INT8_TOPS, 4)
    tops = attn_ops / (phase_ms["attn_main"] * 1e-3) / 1e12
    del x, w, mod, tab
    torch.cuda.empty_cache()
    return {"recipe": "int8_rot quantizers and weights + attention config 94 (attn_u8_kernel), the reference's "
                      "preset numerics", "steps": steps, "ms_per_block": round(sum(phase_ms.values()), 3),
            "attn_u8_tops": round(tops, 1), "attn_u8_frac_int8_peak": round(tops / PEAK_INT8_TOPS, 4),
            "parts": parts}


def traffic_from_profile():
    """HBM bytes per launch of the attention main kernel from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE, calibrated against a copy kernel), or None if there is none."""
    p = os.path.join(ROOT, "profiles", "attn_main_traffic.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f).get("bytes_per_launch")


def traffic_probe(m):
    """Workload of the rocprofv3 --pmc passes behind profiles/attn_main_traffic.json: one attention main
    kernel launch at the bench shape (S = m, H = 24, D = 128; pre-pass outside), then a plain device copy
    of exactly 2^30 bytes whose FETCH_SIZE / WRITE_SIZE readings calibrate the counters."""
    import torch
    from rapid_h3 import attention
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    q, k, v = (torch.randn(m, HEADS, D, device=dev, generator=g).to(torch.bfloat16) for _ in range(3))
    pp = attention.prepass(q, k, v)
    out = torch.empty(m, HEADS, D, dtype=torch.bfloat16, device=dev)
    torch.cuda.synchronize()
    attention.forward(pp, m, out=out)
    src = torch.ones(2 ** 29, dtype=torch.bfloat16, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    print(f"traffic probe: attn_fwd_kernel S={m} H={HEADS} D={D}; copy 1073741824 B", flush=True)


def quant_probe(m, recipe):
    """Workload of the rocprofv3 passes behind profiles/quant_traffic.md: each activation quantizer of one block
    three times at the bench shape (RMSNorm + modulation of x [m, hidden], the head-major attention output [H, m, 128],
    the FFN hidden h [m, FFN]), then the plain 2^30-byte device copy that calibrates FETCH_SIZE / WRITE_SIZE."""
    import torch
    from rapid_h3.block import _QUANTIZERS, row_index
    dev = torch.device("cuda:0")
    x, w, mod, segments, _ = setup(m, dev, recipe)
    norm_mod_q, heads_q, rows_q = _QUANTIZERS[recipe]
    idx = row_index(segments, m, dev)
    g = torch.Generator(device=dev).manual_seed(1)
    o = torch.randn(HEADS, m, D, generator=g, device=dev).to(torch.bfloat16)
    hh = torch.randn(m, FFN, generator=g, device=dev).to(torch.bfloat16)
    src = torch.ones(2 ** 29, dtype=torch.bfloat16, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        norm_mod_q(x, w.norm1_w, w.eps, idx, mod[0], mod[1])
        heads_q(o)
        rows_q(hh)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    print(f"quant probe: norm+mod [{m}, {HIDDEN}], heads [{HEADS}, {m}, {D}], rows [{m}, {FFN}] ({recipe}); "
          "copy 1073741824 B", flush=True)


def pmc_summary(path):
    """Per-kernel table of a rocprofv3 --pmc counter CSV (pmc_counter_collection.csv) holding GRBM_GUI_ACTIVE and
    SQ_VALU_MFMA_BUSY_CYCLES: average duration, the shader clock the kernel ran at (GRBM_GUI_ACTIVE sums one
    busy-cycle count per XCD, so clock = GRBM / 8 / duration) and the MFMA pipe's busy share of the SIMD cycles
    (SQ_VALU_MFMA_BUSY_CYCLES / (1024 SIMDs x GRBM / 8)), the utilisation at the clock actually run."""
    import collections
    import csv
    import re
    per = collections.defaultdict(dict)
    meta = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            d = int(r["Dispatch_Id"])
            per[d][r["Counter_Name"]] = float(r["Counter_Value"])
            meta[d] = (r["Kernel_Name"], int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    rows = collections.OrderedDict()
    for d in sorted(per):
        name, dur = meta[d]
        name = name.replace("(anonymous namespace)::", "")
        name = name[5:] if name.startswith("void ") else name
        if not name.startswith("rh3::") or dur <= 0:
            continue
        short = re.sub(r"\(.*", "", name)
        grbm = per[d].get("GRBM_GUI_ACTIVE", 0.0) / 8
        busy = per[d].get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) / 1024
        rows.setdefault(short, []).append((dur * 1e-6, grbm / dur, busy / grbm if grbm else 0.0))
    print("| kernel | launches | ms / launch | clock GHz | MFMA busy at that clock |")
    print("|---|---:|---:|---:|---:|")
    for k, v in rows.items():
        n = len(v)
        print(f"| `{k}` | {n} | {sum(x[0] for x in v) / n:.3f} | {sum(x[1] for x in v) / n:.2f} | "
              f"{sum(x[2] for x in v) / n:.1%} |")


def main():
    if len(sys.argv) == 3 and sys.argv[1] == "--pmc-summary":
        pmc_summary(sys.argv[2])
        return
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--tokens", type=int, default=None, help="default: the model's (145,152 for c2)")
    ap.add_argument("--model", default="c2", choices=tuple(MODELS),
                    help="c2: hidden 3072, 24 heads, FFN 8192 (the metric's); h3: 5376, 56, 14336")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-side", action="store_true",
                    help="skip the C3 FP8 GEMMs, the hipBLASLt int8 GEMM comparison and the MiniMax-H3-shape blocks after "
                         "the timed block")
    ap.add_argument("--recipe", default="int8_rowwise", choices=("int8_rowwise", "int8_rot"),
                    help="int8_rowwise (the configuration the metric names) or the reference's int8_rot")
    ap.add_argument("--attn-config", type=int, default=None,
                    help="run the attention with the reference's production numerics (config 80-99, e.g. 94) "
                         "instead of the per-block bf16 P.V recipe the metric names")
    ap.add_argument("--fuse-qkv", type=int, default=None, choices=(0, 1),
                    help="1: the QKV GEMM epilogue writes the attention's Q operands and K/V statistics "
                         "(gemm.int8_gemm_qkv); 0: plain QKV GEMM + the full pre-pass; default: the block's")
    ap.add_argument("--quant-probe", action="store_true",
                    help="run only the block's three activation quantizers + a 1 GiB copy (workload of the --pmc passes)")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="run only the attention kernel + a 1 GiB copy (workload of the --pmc passes)")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {a.gpus} is not supported (no multi-GPU path)",
              file=sys.stderr)
        sys.exit(2)
    global HIDDEN, HEADS, FFN
    HIDDEN, HEADS, FFN, m_default = MODELS[a.model]
    if a.tokens is None:
        a.tokens = m_default
    if a.traffic_probe:
        traffic_probe(a.tokens)
        return
    if a.quant_probe:
        quant_probe(a.tokens, a.recipe)
        return
    import torch
    from rapid_h3.block import PHASES, fused_block
    dev = torch.device("cuda:0")
    m = a.tokens
    x, w, mod, segments, tab = setup(m, dev, a.recipe)

    ac = a.attn_config
    fq = {} if a.fuse_qkv is None else {"fuse_qkv": bool(a.fuse_qkv)}
    for _ in range(a.warmup):
        fused_block(x, w, mod, segments, tab, attn_config=ac, **fq)
    torch.cuda.synchronize()

    events = []

    def mark(name):
        e = torch.cuda.Event(enable_timing=True)
        e.record()                      # torch's current stream: the stream every rh3 launch uses
        events[-1].append((name, e))

    t0 = time.perf_counter()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    lead_in()
    start.record()
    for _ in range(a.steps):
        b = torch.cuda.Event(enable_timing=True)
        b.record()
        events.append([("begin", b)])
        fused_block(x, w, mod, segments, tab, mark=mark, attn_config=ac, **fq)
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = start.elapsed_time(end) / a.steps

    phase_ms = {p: 0.0 for p in PHASES}
    for ev in events:
        for (_, e0), (name, e1) in zip(ev[:-1], ev[1:]):
            phase_ms[name] += e0.elapsed_time(e1) / a.steps
    gemms, attn_ops = block_ops(m)
    qbytes = quant_bytes(m)
    total_ops = sum(gemms.values()) + attn_ops
    value = total_ops / (ms_step * 1e-3) / 1e12
    parts = {}
    for p in PHASES:
        t = phase_ms[p]
        if p in gemms:
            tops = gemms[p] / (t * 1e-3) / 1e12
            parts[p] = {"ms": round(t, 3), "tops": round(tops, 1), "frac_int8_peak": round(tops / PEAK_INT8_TOPS, 4)}
        elif p == "attn_main":
            tops = attn_ops / (t * 1e-3) / 1e12
            mixed = 1.0 / (0.5 / PEAK_INT8_TOPS + 0.5 / PEAK_BF16_TFLOPS)
            parts[p] = {"ms": round(t, 3), "tops": round(tops, 1), "frac_int8_peak": round(tops / PEAK_INT8_TOPS, 4),
                        "frac_mixed_roofline": round(tops / mixed, 4)}
        elif p in qbytes:
            gbs = qbytes[p] / (t * 1e-3) / 1e9
            parts[p] = {"ms": round(t, 3), "gbs": round(gbs, 0), "frac_hbm": round(gbs / PEAK_HBM_GBS, 4)}
        else:
            parts[p] = {"ms": round(t, 3)}
    t_attn = phase_ms["attn_main"]
    achieved = attn_ops / (t_attn * 1e-3) / 1e12
    # the committed counter summary is of the attention at the metric's shape only
    traffic = traffic_from_profile() if ac is None and a.model == "c2" and m == MODELS["c2"][3] else None
    kname = "attn_fwd_kernel" if ac is None else "attn_u8_kernel"
    attn_recipe = ("per-128-block Q/K, K smoothing, bf16 P.V" if ac is None else
                   f"production attention config {ac}: per-token H128-rotated Q/K, K/V smoothing, int8 V, "
                   "u8 P vs the 128-key tile max, int8 P.V")
    gemm_ms = sum(phase_ms[p] for p in gemms)
    out = {
        "metric": METRIC, "value": round(value, 2), "unit": "TOPS", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms_step, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": ("full-size DiT block: fused quantizers + 4 W8A8 GEMMs (C2) + INT8 attention (C4)"
                                if a.model == "c2" else
                                "DiT block at MiniMax-H3's own shapes: fused quantizers + 4 W8A8 GEMMs + INT8 attention"),
                   "tokens": m, "hidden": HIDDEN, "heads": HEADS, "head_dim": D, "ffn": FFN,
                   "recipe": f"{a.recipe}, {attn_recipe}", "parallelism": "none"},
        "ms_per_block": round(ms_step, 3),
        "gemm_tops": round(sum(gemms.values()) / (gemm_ms * 1e-3) / 1e12, 1),
        "gemm_frac_int8_peak": round(sum(gemms.values()) / (gemm_ms * 1e-3) / 1e12 / PEAK_INT8_TOPS, 4),
        "attn_tops": round(achieved, 1), "attn_frac_int8_peak": round(achieved / PEAK_INT8_TOPS, 4),
        "parts": parts,
        "roofline": {"kernel": kname, "bound": "mfma", "achieved": round(achieved, 1),
                     "peak": PEAK_INT8_TOPS, "unit": "TFLOP/s", "frac": round(achieved / PEAK_INT8_TOPS, 4),
                     "traffic": traffic,
                     "per_launch": f"4*S^2*D*H = {attn_ops:.4e} " + ("int8+bf16" if ac is None else "int8") +
                                   f" MFMA ops (S={m}, D={D}, H={HEADS})",
                     "avg_launch_ms": round(t_attn, 3)},
        "wall_s_timed": round(wall, 2),
    }
    if not a.no_side and ac is None and a.model == "c2":
        fp8, vendor = gemm_side_measurements(m, dev)
        out["fp8_gemm_c3"] = fp8
        out["int8_gemm_vs_hipblaslt"] = vendor
        out["h3_shapes"] = h3_side_measurements(dev, a.recipe)
        out["reference_preset"] = preset_side_measurement(m, dev)
    if not a.no_cpu:
        # one traced run of the same block supplies the intermediate tensors the CPU sample starts from
        x_in = x.clone()
        tr = {}
        fused_block(x, w, mod, segments, tab, attn_config=ac, trace=tr, **fq)
        torch.cuda.synchronize()
        out["cpu_baseline"] = cpu_baseline(m, x_in, w, mod, segments, tab, tr)
        del tr
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
