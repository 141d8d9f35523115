"""INT8 encoder convolution on gfx950: static weights, per-tensor activations, implicit-GEMM conv.

Counterpart of opt/encoder_int8.py in fishelegs/ComfyUI-H3VAE-PyOpt (E1-E5 of
the hot path):

* ``prepare_int8_weight`` (:303-327) packs ``[O, C, kd, kh, kw]`` to
  ``[O, (kd, kh, kw, c)]`` (c fastest: one 3-D tap is a contiguous channel run)
  with one fp32 scale per output channel;
* ``quantize_activation_tensor`` (:384-426) quantizes an already padded fp16
  tensor with one fp32 scale (``h3v_tensor_quant_i8``, NDHWC int8 out);
* ``_conv3d_from_quantized`` (:509-588) launches the valid conv as an implicit
  GEMM on INT8 MFMA with the dequant / bias (/ residual) epilogue
  (``h3v_conv3d_i8`` / ``h3v_conv3d_i8_residual``); no im2col tensor and no
  FP16 fallback;
* ``int8_valid_conv3d`` / ``HipInt8Conv3d`` (:453-506, :622-717) are the generic
  entry and module wrapper, with the source module's padding done explicitly;
* ``_conv3d_from_quantized_padded`` (no counterpart: the reference pads in a
  separate kernel) writes a stage's last conv straight into its downsample's
  padded input (``h3v_conv3d_i8_residual_padded``).

Activations and outputs are channels-last-3d (NDHWC).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn

from .. import _hip

# Tile names the reference accepts.  The gfx950 kernels choose their own tiles (from the output width
# and channel count), so the name is only validated.
_TILE_VARIANTS = frozenset(("64x64x64", "128x64x64", "128x64x128", "128x128x64", "128x128x64_pipeline4"))
_CL3D = torch.channels_last_3d


@dataclass(frozen=True)
class Int8Conv3DConfig:
    """The convolution contract: channels, kernel, stride (dilation 1, groups 1)."""

    in_channels: int
    out_channels: int
    kernel_size: tuple[int, int, int]
    stride: tuple[int, int, int]
    dilation: tuple[int, int, int] = (1, 1, 1)
    groups: int = 1

    @property
    def taps(self):
        return math.prod(self.kernel_size)

    @property
    def packed_shape(self):
        return (self.out_channels, self.taps * self.in_channels)

    def output_shape(self, x_shape):
        b, _, *extent = x_shape
        out = [(n - k) // s + 1 for n, k, s in zip(extent, self.kernel_size, self.stride)]
        if min(out) <= 0:
            raise ValueError(f"input shape {tuple(x_shape)} is too small for valid conv")
        return (b, self.out_channels, *out)


def int32_accumulator_bound(config: Int8Conv3DConfig) -> int:
    """Largest |sum| of one output for symmetric int8 operands: K * 127^2."""
    return config.in_channels * config.taps * 127 * 127


def validate_int8_weight_buffers(qweight, weight_scale, config: Int8Conv3DConfig) -> None:
    """Static buffers, checked once outside any timed loop (synchronises on the scale check)."""
    if tuple(qweight.shape) != config.packed_shape:
        raise ValueError(f"qweight shape {tuple(qweight.shape)} != packed {config.packed_shape}")
    if qweight.dtype != torch.int8 or not qweight.is_contiguous():
        raise ValueError("qweight must be contiguous torch.int8")
    if tuple(weight_scale.shape) != (config.out_channels,):
        raise ValueError("weight_scale must be [out_channels]")
    if weight_scale.dtype != torch.float32 or not weight_scale.is_contiguous():
        raise ValueError("weight_scale must be contiguous FP32")
    if not bool((torch.isfinite(weight_scale) & (weight_scale > 0)).all()):
        raise ValueError("weight_scale must be finite and positive")


def _config_of(weight, stride, dilation, groups) -> Int8Conv3DConfig:
    if weight.ndim != 5:
        raise ValueError("weight must be [out_channels, in_channels, kd, kh, kw]")
    if groups != 1:
        raise ValueError("INT8 implicit conv currently supports groups=1 only")
    if tuple(dilation) != (1, 1, 1):
        raise ValueError("INT8 implicit conv currently supports dilation=1 only")
    stride = tuple(int(v) for v in stride)
    if not set(stride) <= {1, 2}:
        raise ValueError("INT8 implicit conv supports stride values 1 or 2")
    kernel = tuple(int(v) for v in weight.shape[2:])
    if not set(kernel) <= {1, 3}:
        raise ValueError("INT8 implicit conv supports kernel dimensions 1 or 3")
    return Int8Conv3DConfig(int(weight.shape[1]), int(weight.shape[0]), kernel, stride)


# fp32(1/127): the reference's `.div(127.0)` as its GPU install path computes it (a multiply)
_INV127 = 1.0 / 127.0


def prepare_int8_weight(weight, *, stride=(1, 1, 1), dilation=(1, 1, 1), groups=1):
    """-> (int8 [O, kd*kh*kw*C], fp32 [O], config).

    s = amax * fp32(1/127) per output channel (0 -> 1); q = clamp(round_half_even(w / s), +-127)."""
    if weight.numel() == 0 or not weight.is_floating_point():
        raise ValueError("source weight must be a non-empty floating tensor")
    if not bool(torch.isfinite(weight.detach()).all()):
        raise ValueError("source weight contains non-finite values")
    config = _config_of(weight, stride, dilation, groups)
    bound = int32_accumulator_bound(config)
    if bound >= 2 ** 31:
        raise ValueError(f"INT32 accumulator bound {bound} exceeds signed INT32 range")
    rows = weight.detach().float().permute(0, 2, 3, 4, 1).reshape(config.packed_shape)
    scale = rows.abs().amax(dim=1) * torch.tensor(_INV127, dtype=torch.float32, device=rows.device)
    scale = torch.where(scale > 0, scale, torch.ones_like(scale))
    qweight = torch.round(rows / scale[:, None]).clamp_(-127, 127).to(torch.int8)
    return qweight.contiguous(), scale.contiguous(), config


@torch.no_grad()
def quantize_activation_tensor(x, *, check_finite: bool = False):
    """One already-padded fp16 tensor -> (int8 NDHWC, fp32 scalar scale), per-tensor symmetric."""
    if x.ndim != 5:
        raise ValueError("activation must be [B,C,D,H,W]")
    if x.dtype != torch.float16:
        raise ValueError("INT8 implicit conv currently requires FP16 activations")
    if x.device.type != "cuda":
        raise RuntimeError("INT8 activation quantization requires a GPU tensor")
    if check_finite and not bool(torch.isfinite(x).all()):
        raise ValueError("INT8 activation quantization rejects non-finite input")
    if x.numel() == 0:
        raise ValueError("INT8 activation quantization requires a nonempty tensor")
    _hip.require_gfx950(x.device, "INT8 activation quantization")
    x = x.contiguous(memory_format=_CL3D)
    qx = torch.empty(x.shape, dtype=torch.int8, device=x.device, memory_format=_CL3D)
    scale = torch.empty((), dtype=torch.float32, device=x.device)
    words = int(_hip.lib().h3v_tensor_quant_scratch_words())
    partials = torch.empty((words,), dtype=torch.int32, device=x.device)
    _hip.call("h3v_tensor_quant_i8", _hip.ptr(x), x.numel(), _hip.ptr(qx), _hip.ptr(scale), _hip.ptr(partials), words,
              _hip.stream(x.device))
    return qx, scale


def _check_conv_operands(x, qweight, weight_scale, config, bias):
    dev = x.device
    if qweight.dtype != torch.int8 or qweight.device != dev:
        raise ValueError("qweight must be GPU torch.int8")
    if not qweight.is_contiguous():
        raise ValueError("qweight must use packed contiguous layout")
    if weight_scale.dtype != torch.float32 or weight_scale.device != dev:
        raise ValueError("weight_scale must be GPU FP32")
    if tuple(weight_scale.shape) != (config.out_channels,):
        raise ValueError("weight_scale must be [out_channels]")
    if not weight_scale.is_contiguous():
        raise ValueError("weight_scale must be contiguous")
    if tuple(qweight.shape) != config.packed_shape:
        raise ValueError(f"qweight shape {tuple(qweight.shape)} != packed {config.packed_shape}")
    if x.shape[1] != config.in_channels:
        raise ValueError("activation channel count does not match qweight")
    if bias is not None and (bias.device != dev or bias.dtype != torch.float16 or bias.ndim != 1
                             or bias.numel() != config.out_channels or not bias.is_contiguous()):
        raise ValueError("bias must be contiguous GPU FP16 [out_channels]")


@torch.no_grad()
def int8_valid_conv3d(x, qweight, weight_scale, *, config: Int8Conv3DConfig, bias=None, tile_variant="64x64x64"):
    """Per-tensor quantization of an already padded x, then the INT8 valid conv."""
    if tile_variant not in _TILE_VARIANTS:
        raise ValueError(f"unknown tile variant {tile_variant!r}")
    if x.ndim != 5 or x.device.type != "cuda":
        raise RuntimeError("INT8 implicit conv requires a GPU 5-D activation")
    if x.dtype != torch.float16:
        raise ValueError("INT8 implicit conv currently requires FP16 activations")
    _check_conv_operands(x, qweight, weight_scale, config, bias)
    qx, scale = quantize_activation_tensor(x)
    return _conv3d_from_quantized(qx, scale, qweight, weight_scale, config=config, bias=bias, tile_variant=tile_variant)


def _conv3d_from_quantized(qx, activation_scale, qweight, weight_scale, *, config: Int8Conv3DConfig, bias,
                           tile_variant: str, causal_prefix_zero: bool = False, residual=None, gn_workspace=None,
                           gn_bias=None):
    """The implicit-GEMM conv of an int8 NDHWC input.

    ``causal_prefix_zero`` may be set only by a producer that writes exactly two zero leading frames:
    the taps it skips multiply those zeros, so the result equals the full reduction.  ``residual``
    (fp16, the output's shape) is added in the epilogue as a following fp16 ``residual + out`` would.
    ``gn_workspace`` (fp32, ``gn_workspace_floats`` of the output's D, H, W; geometry of ``gn_stats_fits``):
    the conv also writes the GroupNorm(32) tile statistics of its output (plus ``gn_bias``, fp16 per
    output channel, when given) for ``quantized_temporal_norm_pad(..., partials=gn_workspace)``."""
    if tile_variant not in _TILE_VARIANTS:
        raise ValueError(f"unknown tile variant {tile_variant!r}")
    _hip.require_gfx950(qx.device, "INT8 implicit conv")
    out_shape = config.output_shape(qx.shape)
    qx = qx.contiguous(memory_format=_CL3D)
    out = torch.empty(out_shape, dtype=torch.float16, device=qx.device, memory_format=_CL3D)
    geometry = (*qx.shape, config.out_channels, *config.kernel_size, *config.stride, int(bool(causal_prefix_zero)))
    head = (_hip.ptr(qx), _hip.ptr(activation_scale), _hip.ptr(qweight), _hip.ptr(weight_scale), _hip.ptr(bias))
    if residual is not None:
        if tuple(residual.shape) != out_shape or residual.dtype != torch.float16 or residual.device != out.device:
            raise ValueError("residual must be an fp16 tensor of the convolution output's shape on its device")
        residual = residual.contiguous(memory_format=_CL3D)
    if gn_workspace is not None:
        b, c, d, h, w = qx.shape
        if (config.kernel_size != (3, 3, 3) or config.stride != (1, 1, 1)
                or not gn_stats_fits(c, config.out_channels, *out_shape[2:], batch=b)):
            raise ValueError(f"the statistics epilogue does not take this conv: input {tuple(qx.shape)}, output "
                             f"{out_shape}, kernel {config.kernel_size}, stride {config.stride}")
        need = gn_workspace_floats(*out_shape[2:])
        if (gn_workspace.dtype != torch.float32 or gn_workspace.device != out.device
                or not gn_workspace.is_contiguous() or gn_workspace.numel() < need):
            raise ValueError(f"gn_workspace must be a contiguous fp32 tensor of at least {need} elements on the "
                             "output's device")
        if gn_bias is not None and (gn_bias.shape != (config.out_channels,) or gn_bias.dtype != torch.float16
                                    or gn_bias.device != out.device):
            raise ValueError("gn_bias must be an fp16 vector of the output channels on the output's device")
        _hip.call("h3v_conv3d_i8_gn", *head, _hip.ptr(residual), _hip.ptr(out), c, d, h, w, config.out_channels,
                  int(bool(causal_prefix_zero)), _hip.ptr(None if gn_bias is None else gn_bias.contiguous()),
                  _hip.ptr(gn_workspace), _hip.stream(qx.device))
        return out
    if gn_bias is not None:
        raise ValueError("gn_bias is only taken with gn_workspace")
    if residual is None:
        _hip.call("h3v_conv3d_i8", *head, _hip.ptr(out), *geometry, _hip.stream(qx.device))
        return out
    _hip.call("h3v_conv3d_i8_residual", *head, _hip.ptr(residual), _hip.ptr(out), *geometry, _hip.stream(qx.device))
    return out


def gn_stats_fits(in_channels: int, out_channels: int, out_d: int, out_h: int, out_w: int, *, batch: int = 1) -> bool:
    """Whether ``h3v_conv3d_i8_gn`` takes a stride-1 3x3x3 conv of this geometry and whether it is the
    kernel the plain conv would run anyway: the window conv's strided-pixel form (batch one, Cin % 128 == 0,
    Cout 128 or 256, output width 128 or 256, output height a multiple of 8), at 128 or more 512 x 128
    output tiles (fewer run as the implicit GEMM, which fills the GPU better)."""
    tiles = out_d * (out_h * out_w // 512) * (out_channels // 128)
    return (batch == 1 and in_channels % 128 == 0 and out_channels in (128, 256) and out_w in (128, 256)
            and out_d >= 1 and out_h >= 8 and out_h % 8 == 0 and tiles >= 128)


def gn_workspace_floats(d: int, h: int, w: int) -> int:
    """fp32 elements of the INT8 producer's workspace for an fp16 [1, C, d, h, w] input."""
    n = int(_hip.lib().h3v_gn_norm_pack_workspace_floats(int(d), int(h), int(w)))
    if n <= 0:
        raise ValueError(f"no producer workspace for [D, H, W] = [{d}, {h}, {w}]")
    return n


def padded_output_fits(in_channels: int, out_channels: int, out_h: int, out_w: int) -> bool:
    """Whether ``h3v_conv3d_i8_residual_padded`` takes a stride-1 3x3x3 conv of this geometry (the
    window-in-LDS kernel: Cin % 64 == 0, Cout % 128 == 0, output width 32/64/128/256, output height a
    multiple of 512 / width and at least 2)."""
    return (in_channels % 64 == 0 and out_channels % 128 == 0 and out_w in (32, 64, 128, 256)
            and out_h >= 2 and out_h % (512 // out_w) == 0)


def _conv3d_from_quantized_padded(qx, activation_scale, qweight, weight_scale, *, bias, residual, residual_bias,
                                  front: int, border):
    """The stride-1 3x3x3 conv of a producer's int8 output written into the padded input of a causal
    reflect-padded downsample: [B, Cout, Do + front, Ho + top + bottom, Wo + left + right]
    (channels-last-3d) with the ``front`` leading frames zero and a reflect border ``border`` = (top,
    bottom, left, right) of 0 or 1 per side.  ``residual`` (the output's shape, nullable) is added as
    ``residual + out`` in fp16 would, or, with ``residual_bias``, as one rounding of ``residual + (out +
    residual_bias)`` in fp32."""
    _hip.require_gfx950(qx.device, "INT8 implicit conv")
    config = Int8Conv3DConfig(qx.shape[1], qweight.shape[0], (3, 3, 3), (1, 1, 1))
    b, cout, do, ho, wo = config.output_shape(qx.shape)
    qx = qx.contiguous(memory_format=_CL3D)
    top, bottom, left, right = (int(v) for v in border)
    out = torch.empty((b, cout, do + front, ho + top + bottom, wo + left + right), dtype=torch.float16,
                      device=qx.device, memory_format=_CL3D)
    if front:
        out[:, :, :front].zero_()
    if residual is not None:
        if tuple(residual.shape) != (b, cout, do, ho, wo) or residual.dtype != torch.float16 \
                or residual.device != out.device:
            raise ValueError("residual must be an fp16 tensor of the convolution output's shape on its device")
        residual = residual.contiguous(memory_format=_CL3D)
    if residual_bias is not None and (residual is None or tuple(residual_bias.shape) != (cout,)
                                      or residual_bias.dtype != torch.float16):
        raise ValueError("residual_bias needs a residual and must be an fp16 vector of the output channels")
    _hip.call("h3v_conv3d_i8_residual_padded", _hip.ptr(qx), _hip.ptr(activation_scale), _hip.ptr(qweight),
              _hip.ptr(weight_scale), _hip.ptr(bias), _hip.ptr(residual),
              _hip.ptr(None if residual_bias is None else residual_bias.contiguous()), _hip.ptr(out),
              *qx.shape, cout, 1, int(front), top, bottom, left, right, _hip.stream(qx.device))
    return out


def _source_pad(x, padding, kernel_size, *, causal: bool, spatial_mode: str, temporal_mode: str):
    """The source module's own padding, explicit: spatial border first, then time (reference :622-652).

    Several frames: causal -> 2*pt in front; otherwise pt on both sides.  One frame: zero mode adds
    kd - 1 zero frames in front (causal only); replicate-like modes repeat the frame 2*pt more times."""
    pt, ph, pw = padding
    if not (pt or ph or pw):
        return x
    if ph or pw:
        x = F.pad(x, (pw, pw, ph, ph, 0, 0), mode=spatial_mode)
    if x.shape[2] > 1:
        front, back = (2 * pt, 0) if causal else (pt, pt)
        return F.pad(x, (0, 0, 0, 0, front, back), mode=temporal_mode)
    if temporal_mode != "constant":
        return x.expand(-1, -1, 1 + 2 * pt, -1, -1)
    if not causal:
        raise ValueError("constant temporal padding requires causal mode")
    return torch.cat([x.new_zeros((*x.shape[:2], kernel_size[0] - 1, *x.shape[3:])), x], dim=2)


class HipInt8Conv3d(nn.Module):
    """Inference-only INT8 copy of one source 3-D conv (static weights, per-call activation quant)."""

    def __init__(self, original: nn.Module, *, assume_padded: bool = False):
        super().__init__()
        if not isinstance(original, nn.Conv3d):
            raise ValueError("expected an nn.Conv3d-compatible source module")
        if not assume_padded and not hasattr(original, "causal"):
            raise ValueError("unpadded wrapper requires a SpatialParallelConv3d-like source; "
                             "use assume_padded=True for ordinary nn.Conv3d")
        config = _config_of(original.weight, original.stride, original.dilation, int(original.groups))
        qweight, scale, _ = prepare_int8_weight(original.weight, stride=config.stride)
        validate_int8_weight_buffers(qweight, scale, config)
        self.qweight = nn.Parameter(qweight, requires_grad=False)
        self.register_buffer("weight_scale", scale, persistent=True)
        bias = original.bias
        if bias is None:
            self.register_buffer("bias", None, persistent=True)
        else:
            if bias.ndim != 1 or bias.shape[0] != config.out_channels:
                raise ValueError("source bias shape does not match output channels")
            if not bool(torch.isfinite(bias.detach()).all()):
                raise ValueError("source bias contains non-finite values")
            self.bias = nn.Parameter(bias.detach().clone().contiguous(), requires_grad=False)
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


# the reference module's class name
TritonInt8Conv3d = HipInt8Conv3d

__all__ = ["HipInt8Conv3d", "Int8Conv3DConfig", "TritonInt8Conv3d", "int32_accumulator_bound", "int8_valid_conv3d",
           "prepare_int8_weight", "quantize_activation_tensor", "validate_int8_weight_buffers"]
