"""rh3_int8_attention_noalloc (the allocation-free attention entry point) against rh3_int8_attention with a
caller workspace on the same inputs: two calls in a row, the second smaller, both bit-identical (the same
kernels run on the same operands; neither size reaches the split last round of the main kernel)."""
import ctypes

import pytest
import torch

from rapid_h3 import _native as nat
from rapid_h3 import attention

pytestmark = pytest.mark.gpu


def _qkv(sq, sk, h, seed, dev):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(sq, h, 128, generator=g).to(torch.bfloat16)
    k = (torch.randn(sk, h, 128, generator=g) + 2.0 * torch.randn(1, h, 128, generator=g)).to(torch.bfloat16)
    v = torch.randn(sk, h, 128, generator=g).to(torch.bfloat16)
    return q.to(dev), k.to(dev), v.to(dev)


def _noalloc(q, k, v, out, scale):
    nat.call("rh3_int8_attention_noalloc", nat.ptr(q), q.stride(0), q.stride(1), nat.ptr(k), k.stride(0),
             k.stride(1), nat.ptr(v), v.stride(0), v.stride(1), q.shape[0], k.shape[0], q.shape[1], float(scale), 1,
             nat.ptr(out), out.stride(0), out.stride(1), nat.stream(q.device))


def test_noalloc_matches_workspace_entry_point(dev):
    for sq, sk, h, seed in ((1200, 1500, 6, 0), (300, 257, 2, 1)):
        print(f"[noalloc] Sq={sq} Sk={sk} H={h} seed={seed}", flush=True)
        q, k, v = _qkv(sq, sk, h, seed, dev)
        ref = attention.attention(q, k, v)                  # rh3_int8_attention, torch workspace
        out = torch.full_like(ref, float("nan"))
        _noalloc(q, k, v, out, 128 ** -0.5)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"Sq={sq} Sk={sk} H={h}"


def test_noalloc_under_graph_capture_allocates_nothing(dev):
    """After one warm-up call on the device (it resolves the scratch array's address), a call leaves the device's free
    memory unchanged, and the call captured in a graph replays bit-identical to the workspace entry point."""
    q, k, v = _qkv(1000, 1100, 4, 3, dev)
    ref = attention.attention(q, k, v)
    out = torch.full_like(ref, float("nan"))
    _noalloc(q, k, v, out, 128 ** -0.5)                     # warm-up, outside capture
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info(dev)[0]
    out.fill_(float("nan"))
    _noalloc(q, k, v, out, 128 ** -0.5)
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info(dev)[0] == free0
    assert torch.equal(out, ref)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _noalloc(q, k, v, out, 128 ** -0.5)
    for i in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {i}"


def test_noalloc_rejects_sizes_beyond_its_scratch(dev):
    q, k, v = _qkv(128, 128, 1, 2, dev)
    out = torch.empty_like(q)
    lib = nat.lib()
    s = 1 << 19                                             # 512k tokens x 1 head: over 16 MiB of operands
    st = lib.rh3_int8_attention_noalloc(nat.ptr(q), 128, 128, nat.ptr(k), 128, 128, nat.ptr(v), 128, 128, s, s, 1,
                                        ctypes.c_float(0.1), 1, nat.ptr(out), 128, 128, nat.stream(dev))
    assert st == 1 and "beyond its" in nat.last_error()
