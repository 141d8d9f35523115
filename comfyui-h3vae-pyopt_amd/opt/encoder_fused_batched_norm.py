"""Batch-aware per-frame GroupNorm/bias/SiLU/padding for the encoder suffix.

Mirror of opt/encoder_fused_batched_norm.py in fishelegs/ComfyUI-H3VAE-PyOpt
(``batched_temporal_norm_pack`` :15-66, ``BatchedNormPadConv`` :68-72,
``BatchedResidualBlock`` :74-88, ``BatchedSuffix`` :90-108, ``fused_suffix``
:110-111).  The staged encoder batches up to four independent 17-frame clips
for the suffix stages; each clip keeps its own per-frame statistics and its
own causal zero frames.  The producer is one ``h3v_gn_norm_pack_f16`` launch
sequence over batch x depth frames (statistics, merge, fp16 pack).  The
3x3x3 stride-1 convolutions that follow it run as ``h3v_conv3d_f16`` (FP16
operands, fp32 accumulation on the matrix cores, the input window of a tile
in LDS, causal-zero depth taps skipped) when their shape fits the kernel
(Cin % 32 == 0, Cout % 128 == 0, output width 32/64/128/256); other shapes
keep the model's ``F.conv3d``, as in the reference.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F

from .. import _hip
from .encoder_fused_norm_bias import FusedNormPadConv, norm_pack_f16
from .encoder_staged_batch import EncoderSuffix


def pack_conv_weight_f16(weight):
    """fp16 [Cout, Cin, 3, 3, 3] -> [Cout, 27 * Cin] with k = (kd, kh, kw, c), c fastest."""
    if weight.ndim != 5 or tuple(weight.shape[2:]) != (3, 3, 3) or weight.dtype != torch.float16:
        raise ValueError("expected an fp16 [Cout, Cin, 3, 3, 3] weight")
    return weight.permute(0, 2, 3, 4, 1).reshape(weight.shape[0], -1).contiguous()


def conv3d_f16_fits(x_padded, weight, stride):
    """Whether h3v_conv3d_f16 takes this valid 3x3x3 convolution of a padded [B, C, D, H, W] input."""
    b, c, d, h, w = x_padded.shape
    ho, wo = h - 2, w - 2
    return (tuple(stride) == (1, 1, 1) and tuple(weight.shape[2:]) == (3, 3, 3) and weight.shape[1] == c
            and c % 32 == 0 and weight.shape[0] % 128 == 0 and wo in (32, 64, 128, 256) and ho % (512 // wo) == 0
            and d >= 3 and x_padded.dtype == torch.float16)


def _check_conv(x, w_packed, bias):
    if x.ndim != 5 or x.dtype != torch.float16 or w_packed.dtype != torch.float16 or w_packed.ndim != 2:
        raise ValueError("conv3d_f16 requires an fp16 [B, C, D, H, W] input and an fp16 [Cout, 27*C] weight")
    b, c, d, h, w = x.shape
    if w_packed.shape[1] != 27 * c or not w_packed.is_contiguous() or min(d, h, w) < 3:
        raise ValueError("conv3d_f16 requires a packed [Cout, 27*C] weight and an input of at least 3x3x3")
    if bias is not None and (bias.shape != (w_packed.shape[0],) or bias.dtype != torch.float16
                             or not bias.is_contiguous()):
        raise ValueError("conv3d_f16 requires a contiguous fp16 [Cout] bias")
    if b > 1 and not x.is_contiguous(memory_format=torch.channels_last_3d):
        raise ValueError("conv3d_f16 requires a channels-last-3d input")


@torch.library.custom_op("h3vae_encoder::conv3d_f16", mutates_args=(), device_types="cuda")
def conv3d_f16(x: torch.Tensor, w_packed: torch.Tensor, bias: Optional[torch.Tensor], causal_skip: bool) -> torch.Tensor:
    """Valid 3x3x3 stride-1 conv of a padded fp16 [B, C, D, H, W] (channels-last-3d) ->
    fp16 [B, Cout, D-2, H-2, W-2] channels-last-3d; causal_skip assumes two zero leading frames per item."""
    _check_conv(x, w_packed, bias)
    _hip.require_gfx950(x.device, "conv3d_f16")
    if not x.is_contiguous(memory_format=torch.channels_last_3d):
        x = x.contiguous(memory_format=torch.channels_last_3d)
    b, c, d, h, w = x.shape
    cout = w_packed.shape[0]
    out = torch.empty((b, cout, d - 2, h - 2, w - 2), device=x.device, dtype=x.dtype,
                      memory_format=torch.channels_last_3d)
    _hip.call("h3v_conv3d_f16", _hip.ptr(x), _hip.ptr(w_packed), _hip.ptr(bias), _hip.ptr(out), b, c, d, h, w, cout,
              int(bool(causal_skip)), _hip.stream(x.device))
    return out


@conv3d_f16.register_fake
def _fake_conv(x, w_packed, bias, causal_skip):
    _check_conv(x, w_packed, bias)
    b, c, d, h, w = x.shape
    return torch.empty((b, w_packed.shape[0], d - 2, h - 2, w - 2), device=x.device, dtype=x.dtype,
                       memory_format=torch.channels_last_3d)


class _PackedWeights:
    """Packed fp16 copies of conv weights, made once per weight tensor (weights are read-only)."""

    def __init__(self):
        self._cache = {}

    def get(self, weight):
        key = (weight.data_ptr(), tuple(weight.shape), weight.device)
        packed = self._cache.get(key)
        if packed is None:
            packed = self._cache[key] = pack_conv_weight_f16(weight.detach())
        return packed


_PACKED = _PackedWeights()


def suffix_conv3d(y, weight, bias, stride):
    """The FP16 conv after a producer (two zero leading frames per item): h3v_conv3d_f16 when it fits."""
    if conv3d_f16_fits(y, weight, stride) and _hip.is_gfx950(y.device):
        return conv3d_f16(y, _PACKED.get(weight), bias, True)
    return F.conv3d(y, weight, bias, stride=stride)


def _validate(x, pre_bias, weight, bias):
    b, c, d, h, w = x.shape
    if b not in (1, 3, 4) or c not in (256, 512, 1024) or min(h, w) < 2 or x.dtype != torch.float16:
        raise ValueError("Supported: FP16 B=1/3/4 C=256/512/1024 H/W>=2")
    if b > 1 and x.stride(0) != d * x.stride(2):
        raise ValueError("Batch and time must be contiguous adjacent frame spans")
    if (b * c * (d + 2) * (h + 2) * (w + 2) >= 2 ** 31
            or sum((size - 1) * stride for size, stride in zip(x.shape, x.stride())) >= 2 ** 31):
        raise ValueError("Tensor exceeds validated int32 indexing range")
    for v in (weight, bias, pre_bias):
        if v is not None and (v.shape != (c,) or v.dtype != x.dtype or v.device != x.device or not v.is_contiguous()):
            raise ValueError("Expected FP16 contiguous channel vectors on input device")


@torch.library.custom_op("h3vae_encoder::batched_temporal_norm_pack", mutates_args=(), device_types="cuda")
def batched_temporal_norm_pack(x: torch.Tensor, pre_bias: Optional[torch.Tensor], weight: torch.Tensor,
                               bias: torch.Tensor, eps: float) -> torch.Tensor:
    """x fp16 [B, C, D, H, W] -> fp16 [B, C, D+2, H+2, W+2] channels-last-3d (per-item causal/reflect pad)."""
    _validate(x, pre_bias, weight, bias)
    return norm_pack_f16(x, weight, bias, eps, pre_bias)


@batched_temporal_norm_pack.register_fake
def _fake(x, pre_bias, weight, bias, eps):
    _validate(x, pre_bias, weight, bias)
    b, c, d, h, w = x.shape
    return torch.empty((b, c, d + 2, h + 2, w + 2), device=x.device, dtype=x.dtype,
                       memory_format=torch.channels_last_3d)


class BatchedNormPadConv(FusedNormPadConv):
    def forward(self, x):
        y = batched_temporal_norm_pack(x, None, self.norm_weight, self.norm_bias, self.eps)
        return suffix_conv3d(y, self.weight, self.bias, self.stride) if self.with_conv else y


class BatchedResidualBlock(torch.nn.Module):
    """norm1/conv1 -> norm2 (+ conv1 bias folded in as pre-bias)/conv2 -> + shortcut, clip-batched."""

    def __init__(self, block):
        super().__init__()
        if block.use_fused_norm or block.conv1.bias is None:
            raise ValueError("Expected original encoder block")
        self.first = BatchedNormPadConv(block.norm1, block.conv1, with_conv=False)
        self.second = BatchedNormPadConv(block.norm2, block.conv2, with_conv=False)
        self.shortcut = getattr(block, "nin_shortcut", None)

    def forward(self, x, zq=None):
        if zq is not None:
            raise ValueError("Unconditional inference only")
        h = suffix_conv3d(self.first(x), self.first.weight, None, self.first.stride)
        h = batched_temporal_norm_pack(h, self.first.bias, self.second.norm_weight, self.second.norm_bias,
                                       self.second.eps)
        h = suffix_conv3d(h, self.second.weight, self.second.bias, self.second.stride)
        return (self.shortcut(x) if self.shortcut is not None else x) + h


class BatchedSuffix(EncoderSuffix):
    def __init__(self, encoder, quant_conv, all_stages=False):
        super().__init__(encoder, quant_conv, 2)
        for i in range(len(self.stages) if all_stages else 1):
            original = encoder.down[i + 2]
            stage = torch.nn.Module()
            stage.block = torch.nn.ModuleList([BatchedResidualBlock(block) for block in original.block])
            if hasattr(original, "downsample"):
                stage.downsample = original.downsample
            self.stages[i] = stage
        self.final = BatchedNormPadConv(encoder.norm_out, encoder.conv_out) if all_stages else None

    def forward(self, h):
        for stage in self.stages:
            for block in stage.block:
                h = block(h)
            if hasattr(stage, "downsample"):
                h = stage.downsample(h)
        h = self.final(h) if self.final is not None else self.conv_out(F.silu(self.norm_out(h)))
        return self.quant_conv(h)


def fused_suffix(encoder, quant_conv, all_stages=False):
    return BatchedSuffix(encoder, quant_conv, all_stages)
