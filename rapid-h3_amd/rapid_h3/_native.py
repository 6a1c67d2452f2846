"""ctypes binding of librh3.so (include/rh3.h). The only route from Python to the HIP kernels.

There is no fallback: if the library is missing or a call fails, a RuntimeError says why. Tensors
cross the boundary as raw device pointers plus element strides; every launch goes on torch's current
HIP stream of the tensor's device.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("RH3_LIB", os.path.join(_HERE, "librh3.so"))

ABI_VERSION = 3  # rh3_abi_version() of the library these signatures describe

_P = ctypes.c_void_p
_I = ctypes.c_int64
_F = ctypes.c_float
_C = ctypes.c_int
_D = ctypes.c_double

# name -> argument types, in header order (include/rh3.h)
SIGNATURES = {
    "rh3_last_error": ([], ctypes.c_char_p),
    "rh3_abi_version": ([], ctypes.c_int),
    "rh3_quant_rows_i8": ([_P, _I, _I, _I, _P, _I, _P, _P], _C),
    "rh3_quant_rows_fp8": ([_P, _I, _I, _I, _P, _I, _P, _P], _C),
    "rh3_quant_norm_mod_i8": ([_P, _I, _I, _I, _P, _F, _P, _P, _P, _C, _I, _P, _I, _P, _P], _C),
    "rh3_quant_heads_i8": ([_P, _I, _I, _I, _I, _P, _I, _P, _P], _C),
    "rh3_quant_swiglu_i8": ([_P, _I, _I, _I, _P, _I, _P, _P], _C),
    "rh3_rot_quant_rows_i8": ([_P, _I, _I, _I, _P, _I, _P, _P], _C),
    "rh3_swiglu_rot_quant_rows_i8": ([_P, _I, _I, _I, _P, _I, _P, _P], _C),
    "rh3_norm_mod_rot_quant_i8": ([_P, _I, _I, _I, _P, _F, _P, _P, _P, _C, _I, _P, _I, _P, _P], _C),
    "rh3_rot_quant_heads_i8": ([_P, _I, _I, _I, _I, _P, _I, _P, _P], _C),
    "rh3_convrot_f32": ([_P, _C, _I, _I, _I, _P, _I, _P], _C),
    "rh3_quant_any": ([_P, _C, _I, _I, _I, _C, _P, _I, _P, _P, _P], _C),
    "rh3_quant_weight_rot_i8": ([_P, _C, _I, _I, _I, _P, _I, _P, _P], _C),
    "rh3_fake_nvfp4": ([_P, _C, _I, _I, _I, _P, _I, _P, _P], _C),
    "rh3_gemm_i8": ([_P, _I, _P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _P, _P], _C),
    "rh3_gemm_i8_swiglu": ([_P, _I, _P, _P, _I, _P, _P, _I, _I, _I, _I, _P, _P], _C),
    "rh3_gemm_i8_gated": ([_P, _I, _P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _P, _P], _C),
    "rh3_gemm_i8_gated_rows": ([_P, _I, _P, _P, _I, _P, _P, _I, _P, _P, _I, _I, _I, _I, _P, _P], _C),
    "rh3_gemm_i8_acc": ([_P, _I, _P, _I, _P, _I, _I, _I, _I, _P, _P], _C),
    "rh3_gemm_i8_qkv": ([_P, _I, _P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _P, _C, _P, _P, _F, _C, _C, _P, _I, _P], _C),
    "rh3_gemm_fp8": ([_P, _I, _P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _P, _P], _C),
    "rh3_gemm_fp8_acc": ([_P, _I, _P, _I, _P, _I, _I, _I, _I, _P, _P], _C),
    "rh3_attention_workspace_bytes": ([_I, _I, _I], ctypes.c_int64),
    "rh3_int8_attention": ([_P, _I, _I, _P, _I, _I, _P, _I, _I, _I, _I, _I, _F, _C, _P, _I, _I, _P, _I, _P], _C),
    "rh3_int8_attention_noalloc": ([_P, _I, _I, _P, _I, _I, _P, _I, _I, _I, _I, _I, _F, _C, _P, _I, _I, _P], _C),
    "rh3_int8_attention_rr": ([_P, _I, _I, _P, _I, _I, _P, _I, _I, _I, _I, _P, _C, _P, _P, _F, _F, _C, _P, _I, _I,
                               _P, _I, _P], _C),
    "rh3_rms_rope_qk": ([_P, _I, _I, _P, _I, _I, _I, _I, _P, _C, _P, _P, _F, _P], _C),
    "rh3_attention_forward": ([_I, _I, _I, _F, _P, _I, _I, _P, _I, _P], _C),
    "rh3_attention_prepass": ([_P, _I, _I, _P, _I, _I, _P, _I, _I, _I, _I, _I, _P, _C, _P, _P, _F, _C, _P, _I,
                               ctypes.POINTER(ctypes.c_void_p), _P], _C),
    "rh3_attention_prepass_qkv": ([_P, _I, _I, _P, _I, _I, _I, _I, _P, _C, _P, _F, _C, _P, _I,
                                   ctypes.POINTER(ctypes.c_void_p), _P], _C),
    "rh3_attention_u8_prepass_qkv": ([_P, _I, _I, _P, _I, _I, _I, _I, _P, _C, _P, _F, _C, _C, _C, _P, _I,
                                      ctypes.POINTER(ctypes.c_void_p), _P], _C),
    "rh3_attention_workspace_layout": ([_C, _I, _I, _I, ctypes.POINTER(ctypes.c_int64)], _C),
    "rh3_attention_u8_workspace_bytes": ([_I, _I, _I], ctypes.c_int64),
    "rh3_int8_attention_u8": ([_P, _I, _I, _P, _I, _I, _P, _I, _I, _I, _I, _I, _P, _C, _P, _P, _F, _F, _C, _D, _C,
                               _C, _C, _P, _I, _I, _P, _I, _P], _C),
    "rh3_attention_u8_prepass": ([_P, _I, _I, _P, _I, _I, _P, _I, _I, _I, _I, _I, _P, _C, _P, _P, _F, _C, _C, _C,
                                  _P, _I, ctypes.POINTER(ctypes.c_void_p), _P], _C),
    "rh3_attention_u8_forward": ([_I, _I, _I, _F, _C, _D, _P, _I, _I, _P, _I, _P], _C),
    "rh3_int8_attention_bk": ([_P, _I, _I, _P, _I, _I, _P, _I, _I, _I, _I, _I, _F, _C, _C, _C, _P, _I, _I, _P, _I,
                               _P], _C),
    "rh3_attention_bk_prepass": ([_P, _I, _I, _P, _I, _I, _P, _I, _I, _I, _I, _I, _C, _C, _C, _P, _I,
                                  ctypes.POINTER(ctypes.c_void_p), _P], _C),
    "rh3_attention_bk_forward": ([_I, _I, _I, _F, _P, _I, _I, _P, _I, _P], _C),
    "rh3_int8_attention_f8": ([_P, _I, _I, _P, _I, _I, _P, _I, _I, _I, _I, _I, _P, _C, _P, _P, _F, _F, _C, _C, _C, _C,
                               _P, _I, _I, _P, _I, _P], _C),
    "rh3_attention_f8_prepass": ([_P, _I, _I, _P, _I, _I, _P, _I, _I, _I, _I, _I, _P, _C, _P, _P, _F, _C, _C, _C,
                                  _P, _I, ctypes.POINTER(ctypes.c_void_p), _P], _C),
    "rh3_attention_f8_forward": ([_I, _I, _I, _F, _C, _P, _I, _I, _P, _I, _P], _C),
}

RH3_DTYPE_BF16 = 1
RH3_DTYPE_F32 = 2
RH3_DTYPE_F16 = 3

_lib = None


def lib():
    """Load librh3.so once; raise if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"librh3.so not found at {LIB_PATH}: build it with `python rapid-h3_amd/build.py` "
                               "(or __graft_entry__.build()); there is no non-HIP fallback")
        lib_ = ctypes.CDLL(LIB_PATH)
        for name, (argt, rest) in SIGNATURES.items():
            f = getattr(lib_, name)
            f.argtypes = argt
            f.restype = rest
        if lib_.rh3_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI version {lib_.rh3_abi_version()}, this binding expects "
                               f"{ABI_VERSION}: rebuild it with `python rapid-h3_amd/build.py`")
        _lib = lib_
    return _lib


def last_error():
    return lib().rh3_last_error().decode()


def call(name, *args):
    """Call an int-status entry point; a nonzero status raises RuntimeError with the library's message."""
    st = getattr(lib(), name)(*args)
    if st != 0:
        raise RuntimeError(f"{name}: {last_error()} (status {st})")


def ptr(t):
    """Device pointer of a tensor, or None for None."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream(device):
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


_GEMM_CTR = {}


def gemm_ctr(device):
    """The GEMM tile counters (8 int32) for a call on torch's current stream of `device`, as a tensor the caller
    holds until the call is enqueued. Eagerly: one buffer per (device, stream), kept for the life of the process, so
    calls on one stream share it in order and calls on different streams never do (the ownership rule of the `ctr`
    argument of the rh3_gemm_* entry points). Under stream capture: a new buffer per call from the caching allocator,
    which then belongs to the graph's private pool. Graphs captured on the same capture stream would otherwise bake
    in one shared buffer and race when replayed on two streams at once."""
    import torch
    st = torch.cuda.current_stream(device)
    if torch.cuda.is_current_stream_capturing():
        return torch.empty(64, dtype=torch.int32, device=st.device)
    key = (st.device.index, st.cuda_stream)
    t = _GEMM_CTR.get(key)
    if t is None:
        t = torch.zeros(64, dtype=torch.int32, device=st.device)
        _GEMM_CTR[key] = t
    return t
