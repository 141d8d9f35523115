"""INT8 linear / FFN with static row-wise weights on gfx950.

Mirror of opt/kitchen_int8.py in fishelegs/ComfyUI-H3VAE-PyOpt.  The reference
calls comfy-kitchen 0.2.34 (``quantize_int8_rowwise`` for the weights and
``int8_linear`` = dynamic row quant + CUTLASS GEMM for every call).  Here the
same contract runs on ``libh3vae_hip.so``:

* weights: the row quantizer (``h3v_row_quant``) applied to the fp16 weight
  rows once at install time (an all-zero source row is normalised to q=0,
  s=1.0 exactly as the reference does, opt/kitchen_int8.py:131-145);
* ``int8_linear``: ``h3v_row_quant`` on the activation rows, then
  ``h3v_gemm_i8_dequant`` (int32 MFMA accumulation, fp32 scales, fp16 out).

The original fp16 Parameters are not registered as children of the
replacement and are never modified.
"""
from __future__ import annotations

import torch
from torch import nn

from .. import _hip


def _flat_rows(x: torch.Tensor) -> tuple[torch.Tensor, int, int]:
    k = x.shape[-1]
    m = x.numel() // k if k else 0
    return x.reshape(m, k), m, k


def row_quantize(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Row quantization of fp16 [..., K] -> (int8 [M, K], fp32 [M, 1])."""
    if x.dtype != torch.float16:
        raise ValueError("row quantization requires FP16 input")
    _hip.require_gfx950(x.device, "INT8 row quantization")
    x2, m, k = _flat_rows(x.contiguous())
    if m == 0 or k == 0:
        raise ValueError("row quantization requires a nonempty input")
    q = torch.empty((m, k), device=x.device, dtype=torch.int8)
    s = torch.empty((m, 1), device=x.device, dtype=torch.float32)
    _hip.call("h3v_row_quant", _hip.ptr(x2), m, k, _hip.ptr(q), _hip.ptr(s), _hip.stream(x.device))
    return q, s


def quantize_int8_rowwise(weight: torch.Tensor, stochastic_rounding: int = 0):
    """Static weight quantization with the row-quantizer contract (gfx950)."""
    if stochastic_rounding:
        raise ValueError("stochastic rounding is not part of the INT8 contract")
    q, s = row_quantize(weight.detach().to(torch.float16))
    return q, s


def dequant_gemm(q: torch.Tensor, scale: torch.Tensor, qweight: torch.Tensor, weight_scale: torch.Tensor,
                 bias: torch.Tensor | None) -> torch.Tensor:
    m, k = q.shape
    n = qweight.shape[0]
    out = torch.empty((m, n), device=q.device, dtype=torch.float16)
    _hip.call("h3v_gemm_i8_dequant", _hip.ptr(q), _hip.ptr(scale), _hip.ptr(qweight), _hip.ptr(weight_scale),
              _hip.ptr(bias), _hip.ptr(out), m, n, k, _hip.stream(q.device))
    return out


@torch.library.custom_op("h3vae_pyopt::int8_linear", mutates_args=())
def _int8_linear(
    x: torch.Tensor,
    qweight: torch.Tensor,
    weight_scale: torch.Tensor,
    bias: torch.Tensor | None,
) -> torch.Tensor:
    """Dynamic row quant of x + INT8 GEMM with the dequant epilogue."""
    if x.dtype != torch.float16:
        raise ValueError("INT8 linear requires FP16 activations")
    if qweight.dtype != torch.int8 or qweight.ndim != 2 or qweight.shape[1] != x.shape[-1]:
        raise ValueError("INT8 linear requires int8 weight [N, K] matching x")
    if weight_scale.dtype != torch.float32 or weight_scale.numel() != qweight.shape[0]:
        raise ValueError("INT8 linear requires one FP32 scale per weight row")
    if bias is not None and (bias.dtype != torch.float16 or bias.numel() != qweight.shape[0]):
        raise ValueError("INT8 linear bias must be FP16 [N]")
    tensors = (qweight, weight_scale) + (() if bias is None else (bias,))
    if any(t.device != x.device or not t.is_contiguous() for t in tensors):
        raise ValueError("INT8 linear tensors must be contiguous on one device")
    q, s = row_quantize(x)
    out = dequant_gemm(q, s, qweight, weight_scale, bias)
    return out.reshape(*x.shape[:-1], qweight.shape[0])


@_int8_linear.register_fake
def _(x, qweight, weight_scale, bias):
    del weight_scale, bias
    return x.new_empty((*x.shape[:-1], qweight.shape[0]))


def _require_int8_api() -> None:
    """The replacement of the reference's CK API probe: the HIP library must load."""
    _hip.lib()


def _validate_source_linear(original: nn.Module, *, require_cuda: bool) -> nn.Linear:
    if not isinstance(original, nn.Linear):
        raise ValueError("kitchen INT8 replacement requires nn.Linear")
    weight = original.weight
    if weight.ndim != 2:
        raise ValueError("kitchen INT8 weight must be rank 2")
    if not bool(torch.isfinite(weight.detach()).all()):
        raise ValueError("kitchen INT8 rejects non-finite source weights")
    if original.bias is not None:
        bias = original.bias
        if bias.ndim != 1 or bias.shape[0] != weight.shape[0]:
            raise ValueError("kitchen INT8 bias shape does not match weight")
        if not bool(torch.isfinite(bias.detach()).all()):
            raise ValueError("kitchen INT8 rejects non-finite source bias")
    if require_cuda:
        if weight.device.type != "cuda" or weight.dtype != torch.float16:
            raise ValueError("kitchen INT8 decoder requires GPU FP16 weights")
        if not _hip.is_gfx950(weight.device):
            raise ValueError("kitchen INT8 decoder requires an AMD MI355X (gfx950) GPU")
        if original.bias is not None and (
            original.bias.device != weight.device or original.bias.dtype != torch.float16
        ):
            raise ValueError("kitchen INT8 bias must be GPU FP16")
    return original


def quantize_static_weight(
    original: nn.Linear,
    *,
    quantize_fn=None,
    require_cuda: bool = False,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantize one source weight row-wise and validate the static contract.

    ``quantize_fn`` is for CPU tests; the default runs the gfx950 row quantizer.
    """
    _validate_source_linear(original, require_cuda=require_cuda)
    if quantize_fn is None:
        _require_int8_api()
        quantize_fn = quantize_int8_rowwise
    qweight, weight_scale = quantize_fn(original.weight.detach(), stochastic_rounding=0)
    expected_shape = tuple(original.weight.shape)
    if tuple(qweight.shape) != expected_shape or qweight.dtype != torch.int8:
        raise ValueError(
            "INT8 quantizer returned unexpected weight: "
            f"shape={tuple(qweight.shape)}, dtype={qweight.dtype}, "
            f"expected shape={expected_shape}, dtype=torch.int8"
        )
    if qweight.device != original.weight.device:
        raise ValueError("INT8 quantized weight changed device")
    qweight = qweight.contiguous()
    scale = weight_scale.reshape(-1).contiguous()
    if scale.numel() != original.weight.shape[0]:
        raise ValueError(
            "INT8 weight scale must have one value per output row, got "
            f"{scale.numel()} for N={original.weight.shape[0]}"
        )
    if scale.dtype != torch.float32:
        raise ValueError(f"INT8 weight scale must be float32, got {scale.dtype}")
    if scale.device != original.weight.device:
        raise ValueError("INT8 weight scale changed device")
    # The row quantizer maps an all-zero row to q=-128 with s=1e-30; normalise
    # exactly that case to q=0, s=1.  Any other invalid scale is an error.
    zero_rows = torch.all(original.weight.detach() == 0, dim=1)
    invalid_rows = (~torch.isfinite(scale) | (scale <= 0)) & ~zero_rows
    if bool(invalid_rows.any()):
        raise ValueError("INT8 weight scales must be finite and strictly positive")
    if bool(zero_rows.any()):
        qweight = qweight.clone()
        scale = scale.clone()
        qweight[zero_rows] = 0
        scale[zero_rows] = 1.0
    return qweight, scale


class KitchenInt8Linear(nn.Module):
    """Inference-only linear with static row-wise INT8 weights."""

    def __init__(self, original: nn.Linear, *, quantize_fn=None, require_cuda: bool = False):
        super().__init__()
        if quantize_fn is None:
            _require_int8_api()
        source = _validate_source_linear(original, require_cuda=require_cuda)
        qweight, weight_scale = quantize_static_weight(source, quantize_fn=quantize_fn, require_cuda=require_cuda)
        # Both buffers stay in state_dict so ComfyUI's memory accounting sees them.
        self.register_buffer("qweight", qweight)
        self.register_buffer("weight_scale", weight_scale)
        self.bias = source.bias
        self.in_features = source.in_features
        self.out_features = source.out_features
        self.source_dtype = source.weight.dtype
        self.source_device = source.weight.device
        self.extra_weight_bytes = (
            qweight.numel() * qweight.element_size() + weight_scale.numel() * weight_scale.element_size()
        )
        self.train(source.training)

    def _apply(self, fn, recurse=True):
        # A dtype move (ComfyUI offload/reload) must not narrow the FP32 scales.
        original_scale = self.weight_scale
        result = super()._apply(fn, recurse=recurse)
        self.weight_scale = original_scale.to(device=self.qweight.device, dtype=torch.float32)
        return result

    def forward(self, x: torch.Tensor) -> torch.Tensor:
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
    """Source-shaped gated SiLU FFN with selectable INT8 GEMMs."""

    MODES = frozenset(("INT8both", "INT8w1", "INT8w2"))

    def __init__(self, original: nn.Module, mode: str = "INT8both", *, quantize_fn=None, require_cuda: bool = False):
        super().__init__()
        if mode not in self.MODES:
            raise ValueError(f"unsupported INT8 FFN mode: {mode}")
        if not bool(getattr(original, "use_gated", False)):
            raise ValueError("kitchen INT8 experiment requires a gated FFN")
        if not isinstance(getattr(original, "act_fn", None), nn.SiLU):
            raise ValueError("kitchen INT8 experiment requires a SiLU FFN")
        if not isinstance(getattr(original, "w1", None), nn.Linear):
            raise ValueError("kitchen INT8 FFN requires an nn.Linear w1")
        if not isinstance(getattr(original, "w2", None), nn.Linear):
            raise ValueError("kitchen INT8 FFN requires an nn.Linear w2")
        self.mode = mode
        self.use_gated = True
        self.act_fn = original.act_fn
        self.w1 = (KitchenInt8Linear(original.w1, quantize_fn=quantize_fn, require_cuda=require_cuda)
                   if mode in ("INT8both", "INT8w1") else original.w1)
        self.w2 = (KitchenInt8Linear(original.w2, quantize_fn=quantize_fn, require_cuda=require_cuda)
                   if mode in ("INT8both", "INT8w2") else original.w2)
        self.train(original.training)

    @property
    def extra_weight_bytes(self) -> int:
        return sum(getattr(module, "extra_weight_bytes", 0) for module in (self.w1, self.w2))

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        ff_hidden_states = self.w1(hidden_states)
        gate, up = ff_hidden_states.chunk(2, dim=-1)
        ff_hidden_states = self.act_fn(gate) * up
        return self.w2(ff_hidden_states)


def install_kitchen_int8_ffn(decoder: nn.Module, mode: str = "INT8both", *, require_cuda: bool = True) -> int:
    """Replace all decoder FFNs; validation and quantization finish before any assignment."""
    if decoder.training:
        raise ValueError("kitchen INT8 candidate requires decoder.eval()")
    blocks = getattr(decoder, "transformer_blocks", None)
    if blocks is None:
        raise ValueError("decoder has no transformer_blocks")
    _require_int8_api()
    replacements = [KitchenInt8FFN(block.ff, mode, require_cuda=require_cuda) for block in blocks]
    for block, replacement in zip(blocks, replacements):
        block.ff = replacement
    decoder._h3vae_kitchen_int8_ffn_mode = mode
    return len(replacements)


__all__ = [
    "KitchenInt8FFN",
    "KitchenInt8Linear",
    "dequant_gemm",
    "install_kitchen_int8_ffn",
    "quantize_int8_rowwise",
    "quantize_static_weight",
    "row_quantize",
]
