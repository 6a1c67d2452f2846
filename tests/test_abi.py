"""CPU tests of the C-ABI boundary and the host logic: librh3.so loads without a GPU, exports every
function include/rh3.h declares with the ctypes signatures the host uses, and rejects bad arguments
with a message before touching the device."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    text = open(os.path.join(ROOT, "include", "rh3.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rh3_[a-z0-9_]+)\s*\(", text)))


def test_header_symbols_exported_and_bound():
    from rapid_h3 import _native
    lib = _native.lib()
    names = header_functions()
    assert len(names) >= 16
    for n in names:
        assert hasattr(lib, n), n
        assert n in _native.SIGNATURES, f"{n} declared in rh3.h but not bound in _native"
    assert set(_native.SIGNATURES) == set(names)
    assert lib.rh3_abi_version() == _native.ABI_VERSION == 3


def test_argument_validation_without_gpu():
    from rapid_h3 import _native as nat
    lib = nat.lib()
    fake = ctypes.c_void_p(0x1000)          # never dereferenced: validation fails first
    st = lib.rh3_gemm_i8(fake, 96, fake, fake, 96, fake, None, fake, 16, 4, 16, 96, None, None)
    assert st == 1 and "multiple of 64" in nat.last_error()
    st = lib.rh3_gemm_i8(fake, 64, fake, fake, 64, fake, None, fake, 16, 4, 12, 64, None, None)
    assert st == 1 and "multiple of 8" in nat.last_error()
    st = lib.rh3_quant_rows_i8(fake, 12, 4, 12, fake, 16, fake, None)
    assert st == 1 and "multiple of 8" in nat.last_error()
    st = lib.rh3_quant_norm_mod_i8(fake, 64, 4, 64, None, 1e-6, None, None, None, 2, 64, fake, 64, fake, None)
    assert st == 1 and "idx, shift and scale" in nat.last_error()
    st = lib.rh3_int8_attention(fake, 128, 128, fake, 128, 128, fake, 128, 128, 10, 10, 1, 0.1, 1, fake, 128, 128,
                                fake, 16, None)
    assert st == 1 and "workspace" in nat.last_error()
    st = lib.rh3_attention_forward(10, (1 << 19) + 1, 1, 0.1, fake, 128, 128, fake, 1 << 40, None)
    assert st == 1 and "524288-key limit" in nat.last_error()
    st = lib.rh3_int8_attention_noalloc(fake, 128, 128, fake, 128, 128, fake, 128, 128, 1 << 19, 1 << 19, 1, 0.1, 1,
                                        fake, 128, 128, None)
    assert st == 1 and "beyond its" in nat.last_error()
    st = lib.rh3_int8_attention_rr(fake, 128, 128, fake, 128, 128, fake, 128, 128, 10, 1, fake, 64, fake, fake,
                                   1e-5, 0.1, 1, fake, 128, 128, fake, 1 << 30, None)
    assert st == 1 and "rot_dim" in nat.last_error()
    st = lib.rh3_int8_attention_u8(fake, 128, 128, fake, 128, 128, fake, 128, 128, 10, 10, 1, None, 0, None, None,
                                   1e-5, 0.1, 0, 0.0, 1, 1, 1, fake, 128, 128, fake, 16, None)
    assert st == 1 and "workspace" in nat.last_error()
    st = lib.rh3_int8_attention_u8(fake, 128, 128, fake, 128, 128, fake, 128, 128, 10, 10, 1, None, 0, None, None,
                                   1e-5, 0.1, 11, 0.0, 1, 1, 1, fake, 128, 128, fake, 1 << 30, None)
    assert st == 1 and "nbias" in nat.last_error()
    st = lib.rh3_attention_u8_prepass(fake, 128, 128, fake, 128, 128, fake, 128, 128, 10, 12, 1, fake, 96, fake,
                                      fake, 1e-5, 1, 1, 1, fake, 1 << 30, fake, None)
    assert st == 1 and "self-attention" in nat.last_error()
    st = lib.rh3_rms_rope_qk(fake, 128, 128, fake, 128, 128, 10, 1, fake, 64, fake, fake, 1e-5, None)
    assert st == 1 and "rot_dim" in nat.last_error()
    st = lib.rh3_rms_rope_qk(fake, 100, 128, fake, 128, 128, 10, 1, fake, 128, fake, fake, 1e-5, None)
    assert st == 1 and "multiples of 8" in nat.last_error()
    st = lib.rh3_gemm_fp8_acc(fake, 96, fake, 96, fake, 16, 4, 16, 96, None, None)
    assert st == 1 and "multiple of 64" in nat.last_error()
    with pytest.raises(RuntimeError, match="multiple of 64"):
        nat.call("rh3_gemm_i8", fake, 96, fake, fake, 96, fake, None, fake, 16, 4, 16, 96, None, None)


def test_empty_inputs_are_no_ops():
    from rapid_h3 import _native as nat
    lib = nat.lib()
    assert lib.rh3_quant_rows_i8(None, 0, 0, 64, None, 64, None, None) == 0
    assert lib.rh3_gemm_i8(None, 64, None, None, 64, None, None, None, 8, 0, 8, 64, None, None) == 0
    assert lib.rh3_rms_rope_qk(None, 128, 128, None, 128, 128, 0, 1, None, 128, None, None, 1e-5, None) == 0


def test_workspace_size_matches_layout():
    from rapid_h3 import _native as nat
    lib = nat.lib()
    s, h = 145152, 24
    n = lib.rh3_attention_workspace_bytes(s, s, h)
    sp = (s + 127) // 128 * 128
    nchunk = (s + 255) // 256
    # q8, k8, qs, ks, kmean, the K statistics, V^T, and kn (one key-norm bound per 128-key block)
    expect = (2 * h * sp * 128 + 2 * h * (sp // 128) * 4 + h * 128 * 4 + h * nchunk * 128 * 8 + h * 128 * sp * 2
              + h * (sp // 128) * 4)
    # plus the fp32 partials of the split last round of the main kernel: 2 halves x 128 workgroups x 384
    # queries x 132 floats, reserved when the grid has more than 128 workgroups of 384 queries
    tail = 2 * 128 * 384 * 132 * 4
    assert expect + tail <= n < expect + tail + 9 * 256
    small = lib.rh3_attention_workspace_bytes(384, 384, 128)  # 128 workgroups: no partials
    assert small < lib.rh3_attention_workspace_bytes(385, 385, 128) - tail
    assert lib.rh3_attention_workspace_bytes(0, 5, 1) == 0


def test_host_wrappers_refuse_cpu_tensors():
    import torch
    from rapid_h3 import attention, gemm, quant
    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU"):
        quant.quant_rows_i8(x)
    with pytest.raises(RuntimeError, match="GPU"):
        gemm.int8_gemm(torch.zeros(4, 64, dtype=torch.int8), torch.ones(4, 1), torch.zeros(8, 64, dtype=torch.int8),
                       torch.ones(1, 8))
    q = torch.zeros(8, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU"):
        attention.attention(q, q, q)
    with pytest.raises(RuntimeError, match="128"):
        attention.attention(q[..., :64], q[..., :64], q[..., :64])


def test_dropin_modules_keep_reference_names():
    from rapid_h3 import attn_int8, cutlass_fp8, kernels, triton_fp8
    for mod, names in ((kernels, ["QWeight", "quantize_weight", "quantize_rows", "linear", "gemm_config"]),
                       (cutlass_fp8, ["ext", "fp8_gemm", "int8_gemm", "int8_gemm_qkv_prep", "int8_gemm_gated_residual",
                                      "swiglu_perm", "int8_gemm_swiglu"]),
                       (triton_fp8, ["quant_rows_i8", "quant_rows", "rot_quant_rows_i8", "rot_quant_heads_i8",
                                     "swiglu_rot_quant_rows_i8", "norm_mod_rot_quant_rows_i8", "convrot",
                                     "regular_hadamard", "ROT_GROUP"]),
                       (attn_int8, ["ext", "attention", "attention_bhsd", "attention_rr", "attention_pre",
                                    "attention_rr_bias"])):
        for n in names:
            assert hasattr(mod, n), f"{mod.__name__}.{n}"
    for n in ("int8_attention", "int8_attention_rr", "int8_attention_rr_bias", "int8_prepass", "int8_attention_pre",
              "int8_prepass_pre"):
        assert callable(getattr(attn_int8.ext(), n)), n
    assert attn_int8.CONFIG == int(os.environ.get("RAPIDH3_ATTN_CONFIG", "0"))   # the reference's default 0
    import torch
    p = cutlass_fp8.swiglu_perm(16, "cpu")
    assert p.tolist() == [0, 1, 2, 3, 8, 9, 10, 11, 4, 5, 6, 7, 12, 13, 14, 15]
    with pytest.raises(RuntimeError, match="GPU"):             # no CPU path
        kernels.quantize_rows(torch.zeros(2, 8, dtype=torch.bfloat16), "int8_rowwise")


def test_override_host_logic():
    """RapidH3Int8Attention's host logic (__init__.py:994-1046): segment spans merge, config tags."""
    from rapid_h3 import override
    assert override.merge_spans([(0, 10, "text"), (10, 20, "text"), (20, 50, "video"), (50, 60, "text"),
                                 (60, 60, "text")], {"text"}) == [(0, 20), (50, 60)]
    o = override.make_override(194)
    assert o.rapidh3_rmsrope == 94 and o.rapidh3_rrcheck is False
    assert override.make_override(290).rapidh3_rrcheck is True
    assert not hasattr(override.make_override(194, exact_rows="text"), "rapidh3_rmsrope")
    assert not hasattr(override.make_override(94), "rapidh3_rmsrope")


def test_workspace_layout_offsets():
    """rh3_attention_workspace_layout agrees with the workspace sizes and orders the arrays as declared."""
    from rapid_h3 import _native as nat
    from rapid_h3 import attention
    for numerics, size_fn in ((0, "rh3_attention_workspace_bytes"), (1, "rh3_attention_u8_workspace_bytes")):
        for sq, sk, h in ((300, 300, 2), (1, 129, 3), (145152, 145152, 24)):
            o = attention.workspace_offsets(numerics, sq, sk, h)
            vals = list(o.values())
            assert vals == sorted(vals) and vals[0] == 0 and all(v % 256 == 0 for v in vals)
            assert o["bytes"] == getattr(nat.lib(), size_fn)(sq, sk, h)
    o = attention.workspace_offsets(1, 300, 300, 2)          # Spad 384, 2 statistics chunks
    assert o["qs"] == 2 * 384 * 128 and o["k8"] - o["qs"] == 2 * 384 * 4
    assert o["vt"] - o["side"] == 2 * 3 * 2048 and o["vmin"] - o["vmax"] == 2 * 2 * 128 * 4
