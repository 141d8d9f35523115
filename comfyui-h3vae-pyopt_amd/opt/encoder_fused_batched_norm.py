"""Batch-aware per-frame GroupNorm/bias/SiLU/padding for the encoder suffix.

Mirror of opt/encoder_fused_batched_norm.py in fishelegs/ComfyUI-H3VAE-PyOpt
(``batched_temporal_norm_pack`` :15-66, ``BatchedNormPadConv`` :68-72,
``BatchedResidualBlock`` :74-88, ``BatchedSuffix`` :90-108, ``fused_suffix``
:110-111).  The staged encoder batches up to four independent 17-frame clips
for the suffix stages; each clip keeps its own per-frame statistics and its
own causal zero frames.  The producer is one ``h3v_gn_norm_pack_f16`` launch
sequence over batch x depth frames (statistics, merge, fp16 pack).  The
3x3x3 convolutions that follow it, the ``nin_shortcut`` projections and the
stages' downsample convs run as ``h3v_conv3d_f16`` (FP16 operands, fp32
accumulation on the matrix cores, causal-zero depth taps skipped); the
48-channel ``quant_conv`` is one channels-last GEMM.  With ``all_stages`` every
suffix layer is native; a shape outside the kernels' gates raises.
"""
from __future__ import annotations

from typing import Optional

import torch

from .encoder_fp16_conv import PointwiseConv
from .encoder_fused_norm_bias import FusedNormPadConv, norm_pack_f16
from .encoder_internal_padding import ImplicitTemporalPadConv3d
from .encoder_staged_batch import EncoderSuffix


def _validate(x, pre_bias, weight, bias):
    b, c, d, h, w = x.shape
    # B = 2 is accepted here: the reference's check (B in 1/3/4) rejects the batch of two clips that
    # encode_staged forms for 2 mod 4 clips at staged batch 4 (and for every batch at staged batch 2).
    if b not in (1, 2, 3, 4) or c not in (256, 512, 1024) or min(h, w) < 2 or x.dtype != torch.float16:
        raise ValueError("Supported: FP16 B=1..4 C=256/512/1024 H/W>=2")
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
        return self.conv(y, causal_skip=True) if self.with_conv else y


class BatchedResidualBlock(torch.nn.Module):
    """norm1/conv1 -> norm2 (+ conv1 bias folded in as pre-bias)/conv2 -> + shortcut, clip-batched."""

    def __init__(self, block):
        super().__init__()
        if block.use_fused_norm or block.conv1.bias is None:
            raise ValueError("Expected original encoder block")
        self.first = BatchedNormPadConv(block.norm1, block.conv1, with_conv=False)
        self.second = BatchedNormPadConv(block.norm2, block.conv2, with_conv=False)
        self.shortcut = getattr(block, "nin_shortcut", None)
        self.shortcut_conv = PointwiseConv(self.shortcut) if self.shortcut is not None else None

    def forward(self, x, zq=None):
        if zq is not None:
            raise ValueError("Unconditional inference only")
        residual = self.shortcut_conv(x) if self.shortcut_conv is not None else x
        h = self.first.conv(self.first(x), with_bias=False, causal_skip=True)
        h = batched_temporal_norm_pack(h, self.first.bias, self.second.norm_weight, self.second.norm_bias,
                                       self.second.eps)
        # the closing residual add runs in the second conv's epilogue (fp16(residual + fp16 conv))
        return self.second.conv(h, causal_skip=True, residual=residual)


class SuffixDownsample(torch.nn.Module):
    """A suffix stage's downsample conv, its causal / reflect padding written by the pack kernel."""

    def __init__(self, downsample):
        super().__init__()
        self.conv = ImplicitTemporalPadConv3d(downsample.conv)

    def forward(self, x):
        return self.conv(x)


class BatchedSuffix(EncoderSuffix):
    def __init__(self, encoder, quant_conv, all_stages=False):
        super().__init__(encoder, quant_conv, 2)
        for i in range(len(self.stages) if all_stages else 1):
            original = encoder.down[i + 2]
            stage = torch.nn.Module()
            stage.block = torch.nn.ModuleList([BatchedResidualBlock(block) for block in original.block])
            if hasattr(original, "downsample"):
                stage.downsample = SuffixDownsample(original.downsample)
            self.stages[i] = stage
        self.final = BatchedNormPadConv(encoder.norm_out, encoder.conv_out) if all_stages else None
        self.quant = PointwiseConv(quant_conv) if all_stages else None

    def head(self, h):
        if self.final is None:
            return super().head(h)
        return self.quant(self.final(h))


def fused_suffix(encoder, quant_conv, all_stages=False):
    return BatchedSuffix(encoder, quant_conv, all_stages)
