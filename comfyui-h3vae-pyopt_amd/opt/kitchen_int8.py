"""Static row-wise INT8 linears and FFNs of the decoder, on gfx950.

Counterpart of opt/kitchen_int8.py in fishelegs/ComfyUI-H3VAE-PyOpt, which
calls comfy-kitchen 0.2.34: ``quantize_int8_rowwise`` once per weight and
``int8_linear`` (dynamic row quant of the activations + CUTLASS INT8 GEMM) per
call.  Both halves of that contract run on ``libh3vae_hip.so`` here:

* a weight is quantized once, on its own device, by the same row quantizer the
  activations use (``h3v_row_quant``).  That quantizer turns an all-zero row
  into q = -128 with s = 1e-30; such rows are normalised to q = 0, s = 1
  (reference :131-145), any other non-finite or non-positive scale is refused;
* ``h3vae_pyopt::int8_linear`` = ``h3v_row_quant`` of the activation rows, then
  ``h3v_gemm_i8_dequant`` (int32 MFMA sums, fp16(fma(acc * sx, sw, bias))).

``KitchenInt8Linear`` keeps the int8 rows and fp32 scales as buffers (moved by
ComfyUI with the model, counted by its memory estimate) and shares the
source's fp16 bias; the source ``nn.Linear`` is never modified.
"""
from __future__ import annotations

import torch
from torch import nn

from .. import _hip


def _rows(x):
    """[..., K] -> (contiguous [M, K] view, M, K)."""
    k = x.shape[-1]
    m = x.numel() // k if k else 0
    return x.contiguous().view(m, k), m, k


def row_quantize(x):
    """fp16 [..., K] -> (int8 [M, K], fp32 [M, 1]) under the comfy-kitchen row-quant contract."""
    if x.dtype != torch.float16:
        raise ValueError("row quantization requires FP16 input")
    _hip.require_gfx950(x.device, "INT8 row quantization")
    rows, m, k = _rows(x)
    if m == 0 or k == 0:
        raise ValueError("row quantization requires a nonempty input")
    q = torch.empty((m, k), dtype=torch.int8, device=x.device)
    s = torch.empty((m, 1), dtype=torch.float32, device=x.device)
    _hip.call("h3v_row_quant", _hip.ptr(rows), m, k, _hip.ptr(q), _hip.ptr(s), _hip.stream(x.device))
    return q, s


def quantize_int8_rowwise(weight, stochastic_rounding=0):
    """The weight-side quantizer (comfy-kitchen's name): the row quantizer on the fp16 rows."""
    if stochastic_rounding:
        raise ValueError("stochastic rounding is not part of the INT8 contract")
    return row_quantize(weight.detach().to(torch.float16))


def dequant_gemm(q, scale, qweight, weight_scale, bias):
    """int8 [M, K] x int8 [N, K]^T with the dequant epilogue -> fp16 [M, N]."""
    m, k = q.shape
    out = torch.empty((m, qweight.shape[0]), dtype=torch.float16, device=q.device)
    _hip.call("h3v_gemm_i8_dequant", _hip.ptr(q), _hip.ptr(scale), _hip.ptr(qweight), _hip.ptr(weight_scale),
              _hip.ptr(bias), _hip.ptr(out), m, qweight.shape[0], k, _hip.stream(q.device))
    return out


def _check_linear_args(x, qweight, weight_scale, bias):
    n = qweight.shape[0] if qweight.ndim == 2 else -1
    if x.dtype != torch.float16:
        raise ValueError("INT8 linear requires FP16 activations")
    if qweight.dtype != torch.int8 or qweight.ndim != 2 or qweight.shape[1] != x.shape[-1]:
        raise ValueError("INT8 linear requires int8 weight [N, K] matching x")
    if weight_scale.dtype != torch.float32 or weight_scale.numel() != n:
        raise ValueError("INT8 linear requires one FP32 scale per weight row")
    if bias is not None and (bias.dtype != torch.float16 or bias.numel() != n):
        raise ValueError("INT8 linear bias must be FP16 [N]")
    if any(t is not None and (t.device != x.device or not t.is_contiguous()) for t in (qweight, weight_scale, bias)):
        raise ValueError("INT8 linear tensors must be contiguous on one device")


@torch.library.custom_op("h3vae_pyopt::int8_linear", mutates_args=())
def _int8_linear(x: torch.Tensor, qweight: torch.Tensor, weight_scale: torch.Tensor,
                 bias: torch.Tensor | None) -> torch.Tensor:
    """Dynamic row quant of x, then the INT8 GEMM with the dequant epilogue."""
    _check_linear_args(x, qweight, weight_scale, bias)
    q, s = row_quantize(x)
    return dequant_gemm(q, s, qweight, weight_scale, bias).view(*x.shape[:-1], qweight.shape[0])


@_int8_linear.register_fake
def _int8_linear_fake(x, qweight, weight_scale, bias):
    return x.new_empty((*x.shape[:-1], qweight.shape[0]))


def _require_int8_api():
    """What the reference probes in comfy-kitchen: here, the HIP library must load."""
    _hip.lib()


def _validate_source_linear(original, *, require_cuda):
    if not isinstance(original, nn.Linear):
        raise ValueError("kitchen INT8 replacement requires nn.Linear")
    weight, bias = original.weight, original.bias
    if weight.ndim != 2:
        raise ValueError("kitchen INT8 weight must be rank 2")
    if not bool(torch.isfinite(weight.detach()).all()):
        raise ValueError("kitchen INT8 rejects non-finite source weights")
    if bias is not None:
        if bias.ndim != 1 or bias.shape[0] != weight.shape[0]:
            raise ValueError("kitchen INT8 bias shape does not match weight")
        if not bool(torch.isfinite(bias.detach()).all()):
            raise ValueError("kitchen INT8 rejects non-finite source bias")
    if require_cuda:
        if weight.device.type != "cuda" or weight.dtype != torch.float16:
            raise ValueError("kitchen INT8 decoder requires GPU FP16 weights")
        if not _hip.is_gfx950(weight.device):
            raise ValueError("kitchen INT8 decoder requires an AMD MI355X (gfx950) GPU")
        if bias is not None and (bias.device != weight.device or bias.dtype != torch.float16):
            raise ValueError("kitchen INT8 bias must be GPU FP16")
    return original


def quantize_static_weight(original, *, quantize_fn=None, require_cuda=False):
    """-> (int8 [N, K], fp32 [N]) for one nn.Linear, validated; ``quantize_fn`` stands in for CPU tests."""
    _validate_source_linear(original, require_cuda=require_cuda)
    if quantize_fn is None:
        _require_int8_api()
        quantize_fn = quantize_int8_rowwise
    source = original.weight.detach()
    qweight, weight_scale = quantize_fn(source, stochastic_rounding=0)
    if tuple(qweight.shape) != tuple(source.shape) or qweight.dtype != torch.int8:
        raise ValueError(f"INT8 quantizer returned unexpected weight: shape={tuple(qweight.shape)}, "
                         f"dtype={qweight.dtype}, expected shape={tuple(source.shape)}, dtype=torch.int8")
    scale = weight_scale.reshape(-1)
    if scale.numel() != source.shape[0]:
        raise ValueError(f"INT8 weight scale must have one value per output row, got {scale.numel()} "
                         f"for N={source.shape[0]}")
    if scale.dtype != torch.float32:
        raise ValueError(f"INT8 weight scale must be float32, got {scale.dtype}")
    if qweight.device != source.device or scale.device != source.device:
        raise ValueError("INT8 quantized weight changed device")
    empty = (source == 0).all(dim=1)
    bad = ~(torch.isfinite(scale) & (scale > 0))
    if bool((bad & ~empty).any()):
        raise ValueError("INT8 weight scales must be finite and strictly positive")
    qweight, scale = qweight.contiguous(), scale.contiguous()
    if bool(empty.any()):
        qweight = qweight.masked_fill(empty[:, None], 0)
        scale = scale.masked_fill(empty, 1.0)
    return qweight, scale


class KitchenInt8Linear(nn.Module):
    """Inference-only linear with static row-wise INT8 weights (``h3vae_pyopt::int8_linear`` per call)."""

    def __init__(self, original, *, quantize_fn=None, require_cuda=False):
        super().__init__()
        if quantize_fn is None:
            _require_int8_api()
        qweight, weight_scale = quantize_static_weight(original, quantize_fn=quantize_fn, require_cuda=require_cuda)
        self.register_buffer("qweight", qweight)
        self.register_buffer("weight_scale", weight_scale)
        self.bias = original.bias
        self.in_features, self.out_features = original.in_features, original.out_features
        self.source_dtype, self.source_device = original.weight.dtype, original.weight.device
        self.extra_weight_bytes = qweight.numel() + 4 * weight_scale.numel()
        self.train(original.training)

    def _apply(self, fn, recurse=True):
        # a dtype move (ComfyUI offload / reload) must leave the scales in fp32
        scale = self.weight_scale
        out = super()._apply(fn, recurse=recurse)
        self.weight_scale = scale.to(device=self.qweight.device, dtype=torch.float32)
        return out

    def forward(self, x):
        if self.training:
            raise RuntimeError("kitchen INT8 candidate is inference-only; call eval()")
        if torch.is_grad_enabled():
            raise RuntimeError("kitchen INT8 candidate requires torch.no_grad()")
        if x.shape[-1] != self.in_features:
            raise ValueError(f"INT8 input K={x.shape[-1]} does not match K={self.in_features}")
        if x.dtype != self.source_dtype:
            raise ValueError(f"INT8 input dtype must match source dtype {self.source_dtype}, got {x.dtype}")
        if x.device != self.qweight.device:
            raise ValueError("INT8 input and quantized weight must share a device")
        return _int8_linear(x, self.qweight, self.weight_scale, self.bias)


class KitchenInt8FFN(nn.Module):
    """The model's gated SiLU FFN (w1 -> [gate | up] -> SiLU(gate) * up -> w2) with INT8 w1 and/or w2."""

    MODES = {"INT8both": (True, True), "INT8w1": (True, False), "INT8w2": (False, True)}

    def __init__(self, original, mode="INT8both", *, quantize_fn=None, require_cuda=False):
        super().__init__()
        if mode not in self.MODES:
            raise ValueError(f"unsupported INT8 FFN mode: {mode}")
        if not bool(getattr(original, "use_gated", False)):
            raise ValueError("kitchen INT8 experiment requires a gated FFN")
        if not isinstance(getattr(original, "act_fn", None), nn.SiLU):
            raise ValueError("kitchen INT8 experiment requires a SiLU FFN")
        for name in ("w1", "w2"):
            if not isinstance(getattr(original, name, None), nn.Linear):
                raise ValueError(f"kitchen INT8 FFN requires an nn.Linear {name}")
        self.mode, self.use_gated, self.act_fn = mode, True, original.act_fn
        for name, int8 in zip(("w1", "w2"), self.MODES[mode]):
            source = getattr(original, name)
            setattr(self, name, KitchenInt8Linear(source, quantize_fn=quantize_fn, require_cuda=require_cuda)
                    if int8 else source)
        self.train(original.training)

    @property
    def extra_weight_bytes(self):
        return sum(getattr(m, "extra_weight_bytes", 0) for m in (self.w1, self.w2))

    def forward(self, hidden_states):
        gate, up = self.w1(hidden_states).chunk(2, dim=-1)
        return self.w2(self.act_fn(gate) * up)


def install_kitchen_int8_ffn(decoder, mode="INT8both", *, require_cuda=True):
    """Swap every block's FFN for its INT8 form in place; all quantization happens before any swap."""
    if decoder.training:
        raise ValueError("kitchen INT8 candidate requires decoder.eval()")
    blocks = getattr(decoder, "transformer_blocks", None)
    if blocks is None:
        raise ValueError("decoder has no transformer_blocks")
    _require_int8_api()
    built = [KitchenInt8FFN(block.ff, mode, require_cuda=require_cuda) for block in blocks]
    for block, ffn in zip(blocks, built):
        block.ff = ffn
    decoder._h3vae_kitchen_int8_ffn_mode = mode
    return len(built)


__all__ = ["KitchenInt8FFN", "KitchenInt8Linear", "dequant_gemm", "install_kitchen_int8_ffn", "quantize_int8_rowwise",
           "quantize_static_weight", "row_quantize"]
