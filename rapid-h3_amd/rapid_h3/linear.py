"""QuantLinear: the reference's _QuantLinear (/root/reference/custom_nodes/rapid_h3/__init__.py:83-167)
without ComfyUI: a replacement forward for one Linear that runs kernels.linear on librh3's kernels.

What it keeps from the reference:
  * the quantized weight is made once and cached; it is remade when the weight changes. The reference keys
    its cache by ComfyUI's patches_uuid (:123-135): a caller that has such an id passes patch_id (a callable
    returning it), and the key is (patch_id(), device); without one the key is the weight tensor's identity,
    storage pointer and version counter, which change when the weight is replaced or updated in place;
  * an already-quantized Comfy int8_convrot weight (int8 [N, K] codes rotated with group 256 plus a
    per-row scale) is adopted as is in int8_rot mode (:107-114), see from_quantized;
  * the bias is added in x.dtype after the GEMM (:158-159);
  * a weight cached in SwiGLU-epilogue row order is returned to natural order (:155-157);
  * measure_every = n > 0 records the relative L2 error against F.linear every n calls into
    stats[name] (:139-165).
  * activations that are not on a GPU or not bf16 / fp16 take torch's F.linear with the weight in x.dtype, as in
    the reference (:147-148): the quantized kernels are for bf16 / fp16 GPU activations only. An adopted
    int8_convrot weight has no bf16 copy; there it is dequantized (codes times scale, rotated back by the
    orthogonal, symmetric blockdiag(H256)), as the reference's QuantizedTensor dequantizes inside F.linear.
What it does not keep: ComfyUI's cast context for off-GPU / LoRA weights (:93-105, needs comfy).
"""
import torch

from . import kernels


class QuantLinear:
    def __init__(self, weight, bias=None, mode="int8_rot", name="linear", measure_every=0, stats=None, patch_id=None):
        if mode not in kernels.MODES or mode == "bf16":
            raise ValueError(f"QuantLinear: mode {mode!r} (one of {kernels.MODES[1:]})")
        self.weight, self.bias, self.mode, self.name = weight, bias, mode, name
        self.patch_id = patch_id
        self.measure_every = int(measure_every)
        self.stats = {} if stats is None else stats
        self.qweight, self.cache_key, self.calls = None, None, 0

    @classmethod
    def from_quantized(cls, qdata, scale, bias=None, group=256, transposed=False, name="linear", **kw):
        """An int8_convrot checkpoint weight taken as is (no bf16 copy); measure_every needs a bf16 weight
        and is off."""
        self = cls(None, bias, "int8_rot", name, 0, kw.get("stats"))
        self.qweight = kernels.adopt_convrot(qdata, scale, group=group, transposed=transposed)
        self.cache_key = "adopted"
        return self

    def _key(self):
        w = self.weight
        if self.patch_id is not None:
            return ("patch", self.patch_id(), str(w.device))
        return (id(w), w.data_ptr(), w._version, str(w.device))

    def qweight_for(self):
        """The cached quantized weight (quantized on first use or after the weight changed)."""
        if self.cache_key == "adopted":
            return self.qweight
        key = self._key()
        if key != self.cache_key:
            self.qweight = kernels.quantize_weight(self.weight.detach(), self.mode)
            self.cache_key = key
        return self.qweight

    def dense_weight(self, device, dtype):
        """The weight for the F.linear route: the module's weight, or the adopted int8_convrot weight dequantized."""
        if self.weight is not None:
            return self.weight.to(device=device, dtype=dtype)
        from .triton_fp8 import ROT_GROUP, regular_hadamard
        q, sc = self.qweight.q, self.qweight.scale
        n, k = q.shape
        w = q.float() * sc.reshape(n, 1).float()
        w = (w.reshape(n, k // ROT_GROUP, ROT_GROUP) @ regular_hadamard(ROT_GROUP, w.device)).reshape(n, k)
        return w.to(device=device, dtype=dtype)

    def __call__(self, x):
        if not x.is_cuda or x.dtype not in (torch.bfloat16, torch.float16):
            b = None if self.bias is None else self.bias.to(device=x.device, dtype=x.dtype)
            return torch.nn.functional.linear(x, self.dense_weight(x.device, x.dtype), b)
        qw = self.qweight_for()
        shape = x.shape
        y = kernels.linear(x.reshape(-1, shape[-1]), qw, self.mode)
        if getattr(qw, "swiglu_perm", False):   # fc1 held in SwiGLU-epilogue order
            from .gemm import swiglu_perm
            y = y[:, torch.argsort(swiglu_perm(y.shape[-1], y.device))]
        if self.bias is not None:
            y = y + self.bias.to(y.dtype)
        y = y.reshape(*shape[:-1], y.shape[-1])
        self.calls += 1
        if self.measure_every and self.calls % self.measure_every == 0 and self.weight is not None:
            ref = torch.nn.functional.linear(x, self.weight.to(x.dtype), None if self.bias is None else
                                             self.bias.to(x.dtype))
            err = ((y.float() - ref.float()).norm() / ref.float().norm().clamp_min(1e-12)).item()
            self.stats.setdefault(self.name, []).append(err)
        return y
