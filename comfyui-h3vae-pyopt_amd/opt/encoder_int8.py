"""INT8 encoder convolution on gfx950.

Mirror of opt/encoder_int8.py in fishelegs/ComfyUI-H3VAE-PyOpt:

* weights are packed once to ``[O, (kd, kh, kw, c)]`` (c fastest) with one
  FP32 scale per output channel (``prepare_int8_weight``, :303-327);
* activations are quantized once per call with one FP32 tensor scale
  (``quantize_activation_tensor``, :384-426 -> ``h3v_tensor_quant_i8``);
* the valid convolution is an implicit GEMM on INT8 MFMA with the
  dequant/bias epilogue fused (``_conv3d_from_quantized``, :509-588 ->
  ``h3v_conv3d_i8``); no im2col tensor is materialised and there is no FP16
  fallback.

Activations and outputs use channels-last-3d (NDHWC) storage.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn

from .. import _hip

# Tile names the reference accepts; the gfx950 kernel picks its own tile from
# the output-channel count, so these only validate the argument.
_TILE_VARIANTS = {
    "64x64x64": (64, 64, 64),
    "128x64x64": (128, 64, 64),
    "128x64x128": (128, 64, 128),
    "128x128x64": (128, 128, 64),
    "128x128x64_pipeline4": (128, 128, 64),
}


@dataclass(frozen=True)
class Int8Conv3DConfig:
    """Static configuration for the supported valid convolution contract."""

    in_channels: int
    out_channels: int
    kernel_size: tuple[int, int, int]
    stride: tuple[int, int, int]
    dilation: tuple[int, int, int] = (1, 1, 1)
    groups: int = 1


def int32_accumulator_bound(config: Int8Conv3DConfig) -> int:
    """Worst-case absolute INT32 dot sum for symmetric int8 operands."""
    reduction = config.in_channels * math.prod(config.kernel_size)
    return reduction * 127 * 127


def validate_int8_weight_buffers(qweight: torch.Tensor, weight_scale: torch.Tensor, config: Int8Conv3DConfig) -> None:
    """Validate static buffers once, outside any timed loop (this synchronises)."""
    expected_qshape = (
        config.out_channels,
        config.kernel_size[0] * config.kernel_size[1] * config.kernel_size[2] * config.in_channels,
    )
    if tuple(qweight.shape) != expected_qshape:
        raise ValueError(f"qweight shape {tuple(qweight.shape)} != packed {expected_qshape}")
    if qweight.dtype != torch.int8 or not qweight.is_contiguous():
        raise ValueError("qweight must be contiguous torch.int8")
    if tuple(weight_scale.shape) != (config.out_channels,):
        raise ValueError("weight_scale must be [out_channels]")
    if weight_scale.dtype != torch.float32 or not weight_scale.is_contiguous():
        raise ValueError("weight_scale must be contiguous FP32")
    if not bool(torch.isfinite(weight_scale).all().item()) or not bool((weight_scale > 0).all().item()):
        raise ValueError("weight_scale must be finite and positive")


def _validate_conv_config(weight, stride, dilation, groups) -> Int8Conv3DConfig:
    if weight.ndim != 5:
        raise ValueError("weight must be [out_channels, in_channels, kd, kh, kw]")
    if groups != 1:
        raise ValueError("INT8 implicit conv currently supports groups=1 only")
    if tuple(dilation) != (1, 1, 1):
        raise ValueError("INT8 implicit conv currently supports dilation=1 only")
    stride = tuple(int(v) for v in stride)
    if any(v not in (1, 2) for v in stride):
        raise ValueError("INT8 implicit conv supports stride values 1 or 2")
    kernel_size = tuple(int(v) for v in weight.shape[-3:])
    if any(v not in (1, 3) for v in kernel_size):
        raise ValueError("INT8 implicit conv supports kernel dimensions 1 or 3")
    return Int8Conv3DConfig(int(weight.shape[1]), int(weight.shape[0]), kernel_size, stride)


_INV127 = torch.tensor(1.0 / 127.0, dtype=torch.float32)


def prepare_int8_weight(weight, *, stride=(1, 1, 1), dilation=(1, 1, 1), groups=1):
    """Pack ``[O, C, kd, kh, kw]`` to ``[O, kd*kh*kw*C]`` INT8 + FP32 ``[O]`` scales.

    scale = amax * fp32(1/127) (the production GPU arithmetic of the reference's
    ``.div(127.0)``), 0 -> 1; q = clamp(round_half_even(w / scale), +-127).
    """
    if weight.numel() == 0 or not weight.is_floating_point():
        raise ValueError("source weight must be a non-empty floating tensor")
    if not bool(torch.isfinite(weight.detach()).all().item()):
        raise ValueError("source weight contains non-finite values")
    config = _validate_conv_config(weight, stride, dilation, groups)
    bound = int32_accumulator_bound(config)
    if bound >= 2**31:
        raise ValueError(f"INT32 accumulator bound {bound} exceeds signed INT32 range")
    source = weight.detach().float().contiguous()
    packed = source.permute(0, 2, 3, 4, 1).reshape(config.out_channels, -1)
    scale = packed.abs().amax(dim=1) * _INV127.to(packed.device)
    scale = torch.where(scale > 0, scale, torch.ones_like(scale))
    qweight = torch.round(packed / scale[:, None]).clamp(-127, 127).to(torch.int8)
    return qweight.contiguous(), scale.float().contiguous(), config


@torch.no_grad()
def quantize_activation_tensor(x: torch.Tensor, *, check_finite: bool = False):
    """Quantize one already-padded FP16 tensor -> (int8 NDHWC, fp32 scalar scale)."""
    if x.ndim != 5:
        raise ValueError("activation must be [B,C,D,H,W]")
    if x.dtype != torch.float16:
        raise ValueError("INT8 implicit conv currently requires FP16 activations")
    if x.device.type != "cuda":
        raise RuntimeError("INT8 activation quantization requires a GPU tensor")
    if check_finite and not bool(torch.isfinite(x).all().item()):
        raise ValueError("INT8 activation quantization rejects non-finite input")
    if x.numel() == 0:
        raise ValueError("INT8 activation quantization requires a nonempty tensor")
    _hip.require_gfx950(x.device, "INT8 activation quantization")
    x = x.contiguous(memory_format=torch.channels_last_3d)
    qx = torch.empty(x.shape, dtype=torch.int8, device=x.device, memory_format=torch.channels_last_3d)
    scale = torch.empty((), dtype=torch.float32, device=x.device)
    scratch = torch.empty((1,), dtype=torch.int32, device=x.device)
    _hip.call("h3v_tensor_quant_i8", _hip.ptr(x), x.numel(), _hip.ptr(qx), _hip.ptr(scale), _hip.ptr(scratch),
              _hip.stream(x.device))
    return qx, scale


def _valid_output_shape(x_shape, config: Int8Conv3DConfig):
    b, _, d, h, w = x_shape
    kd, kh, kw = config.kernel_size
    sd, sh, sw = config.stride
    output = tuple((length - kernel) // step + 1 for length, kernel, step in ((d, kd, sd), (h, kh, sh), (w, kw, sw)))
    if any(v <= 0 for v in output):
        raise ValueError(f"input shape {x_shape} is too small for valid conv")
    return (b, config.out_channels, *output)


@torch.no_grad()
def int8_valid_conv3d(x, qweight, weight_scale, *, config: Int8Conv3DConfig, bias=None, tile_variant="64x64x64"):
    """Quantize x per tensor and run the INT8 valid convolution (no FP16 fallback)."""
    if tile_variant not in _TILE_VARIANTS:
        raise ValueError(f"unknown tile variant {tile_variant!r}")
    if x.ndim != 5 or x.device.type != "cuda":
        raise RuntimeError("INT8 implicit conv requires a GPU 5-D activation")
    if x.dtype != torch.float16:
        raise ValueError("INT8 implicit conv currently requires FP16 activations")
    if qweight.dtype != torch.int8 or qweight.device != x.device:
        raise ValueError("qweight must be GPU torch.int8")
    if not qweight.is_contiguous():
        raise ValueError("qweight must use packed contiguous layout")
    if weight_scale.dtype != torch.float32 or weight_scale.device != x.device:
        raise ValueError("weight_scale must be GPU FP32")
    if tuple(weight_scale.shape) != (config.out_channels,):
        raise ValueError("weight_scale must be [out_channels]")
    if not weight_scale.is_contiguous():
        raise ValueError("weight_scale must be contiguous")
    expected_qshape = (config.out_channels, math.prod(config.kernel_size) * config.in_channels)
    if tuple(qweight.shape) != expected_qshape:
        raise ValueError(f"qweight shape {tuple(qweight.shape)} != packed {expected_qshape}")
    if x.shape[1] != config.in_channels:
        raise ValueError("activation channel count does not match qweight")
    if bias is not None and (bias.device != x.device or bias.dtype != torch.float16 or bias.ndim != 1
                             or bias.numel() != config.out_channels or not bias.is_contiguous()):
        raise ValueError("bias must be contiguous GPU FP16 [out_channels]")
    qx, activation_scale = quantize_activation_tensor(x)
    return _conv3d_from_quantized(qx, activation_scale, qweight, weight_scale, config=config, bias=bias,
                                  tile_variant=tile_variant)


def _conv3d_from_quantized(qx, activation_scale, qweight, weight_scale, *, config: Int8Conv3DConfig, bias,
                           tile_variant: str, causal_prefix_zero: bool = False, residual=None):
    """Launch the implicit-GEMM conv on an int8 NDHWC input.

    Only a producer that guarantees two leading zero temporal planes may set
    causal_prefix_zero; the skipped taps multiply those zeros, so the result is
    identical to the full reduction.  ``residual`` (fp16, the output's shape)
    is added in the epilogue exactly as a following fp16 ``residual + out``.
    """
    if tile_variant not in _TILE_VARIANTS:
        raise ValueError(f"unknown tile variant {tile_variant!r}")
    _hip.require_gfx950(qx.device, "INT8 implicit conv")
    output_shape = _valid_output_shape(tuple(qx.shape), config)
    qx = qx.contiguous(memory_format=torch.channels_last_3d)
    output = torch.empty(output_shape, dtype=torch.float16, device=qx.device, memory_format=torch.channels_last_3d)
    b, c, d, h, w = qx.shape
    kd, kh, kw = config.kernel_size
    sd, sh, sw = config.stride
    if residual is None:
        _hip.call("h3v_conv3d_i8", _hip.ptr(qx), _hip.ptr(activation_scale), _hip.ptr(qweight),
                  _hip.ptr(weight_scale), _hip.ptr(bias), _hip.ptr(output), b, c, d, h, w, config.out_channels, kd, kh,
                  kw, sd, sh, sw, int(bool(causal_prefix_zero)), _hip.stream(qx.device))
        return output
    if residual.shape != output.shape or residual.dtype != torch.float16 or residual.device != output.device:
        raise ValueError("residual must be an fp16 tensor of the convolution output's shape on its device")
    residual = residual.contiguous(memory_format=torch.channels_last_3d)
    _hip.call("h3v_conv3d_i8_residual", _hip.ptr(qx), _hip.ptr(activation_scale), _hip.ptr(qweight),
              _hip.ptr(weight_scale), _hip.ptr(bias), _hip.ptr(residual), _hip.ptr(output), b, c, d, h, w,
              config.out_channels, kd, kh, kw, sd, sh, sw, int(bool(causal_prefix_zero)), _hip.stream(qx.device))
    return output


def _source_pad(x, padding, kernel_size, *, causal: bool, spatial_mode: str, temporal_mode: str):
    """Explicit spatial/temporal padding of the source module (reference :622-652)."""
    pt, ph, pw = padding
    if not (pt or ph or pw):
        return x
    if ph or pw:
        x = F.pad(x, (pw, pw, ph, ph, 0, 0), mode=spatial_mode)
    depth = x.shape[2]
    if depth > 1:
        left = 2 * pt if causal else pt
        right = 0 if causal else pt
        return F.pad(x, (0, 0, 0, 0, left, right), mode=temporal_mode)
    if temporal_mode == "constant":
        if not causal:
            raise ValueError("constant temporal padding requires causal mode")
        zeros = torch.zeros_like(x[:, :, :1]).expand(-1, -1, kernel_size[0] - 1, -1, -1)
        return torch.cat([zeros, x], dim=2)
    return x.expand(-1, -1, x.shape[2] + 2 * pt, -1, -1)


class HipInt8Conv3d(nn.Module):
    """Inference-only INT8 wrapper around one source 3-D convolution."""

    def __init__(self, original: nn.Module, *, assume_padded: bool = False):
        super().__init__()
        if not isinstance(original, nn.Conv3d):
            raise ValueError("expected an nn.Conv3d-compatible source module")
        if not assume_padded and not hasattr(original, "causal"):
            raise ValueError("unpadded wrapper requires a SpatialParallelConv3d-like source; "
                             "use assume_padded=True for ordinary nn.Conv3d")
        config = _validate_conv_config(original.weight, tuple(original.stride), tuple(original.dilation),
                                       int(original.groups))
        qweight, scale, _ = prepare_int8_weight(original.weight, stride=config.stride)
        validate_int8_weight_buffers(qweight, scale, config)
        self.qweight = nn.Parameter(qweight, requires_grad=False)
        self.register_buffer("weight_scale", scale, persistent=True)
        if original.bias is None:
            self.register_buffer("bias", None, persistent=True)
        else:
            if original.bias.ndim != 1 or original.bias.shape[0] != config.out_channels:
                raise ValueError("source bias shape does not match output channels")
            if not bool(torch.isfinite(original.bias.detach()).all().item()):
                raise ValueError("source bias contains non-finite values")
            self.bias = nn.Parameter(original.bias.detach().clone().contiguous(), requires_grad=False)
        self.config = config
        self.padding = tuple(int(v) for v in original.padding)
        self.pad_mode = getattr(original, "pad_mode", "constant")
        self.pad_mode_t = getattr(original, "pad_mode_t", "constant")
        self.causal = bool(getattr(original, "causal", False))
        self.assume_padded = bool(assume_padded)

    @torch.no_grad()
    def forward(self, x):
        if not self.assume_padded:
            x = _source_pad(x, self.padding, self.config.kernel_size, causal=self.causal,
                            spatial_mode=self.pad_mode, temporal_mode=self.pad_mode_t)
        return int8_valid_conv3d(x, self.qweight, self.weight_scale, config=self.config, bias=self.bias)


# Drop-in name of the reference module class.
TritonInt8Conv3d = HipInt8Conv3d

__all__ = [
    "HipInt8Conv3d",
    "Int8Conv3DConfig",
    "TritonInt8Conv3d",
    "int32_accumulator_bound",
    "int8_valid_conv3d",
    "prepare_int8_weight",
    "quantize_activation_tensor",
    "validate_int8_weight_buffers",
]
