"""Last stage-1 block: residual + bias + right/bottom reflect + causal zero pack, then the downsample conv.

Mirror of opt/encoder_fused_residual_pack.py in fishelegs/ComfyUI-H3VAE-PyOpt.
``residual_downsample_pack`` (:36-55) becomes ``h3v_residual_downsample_pack``:
y = fp16(residual + (x + bias)) with fp32 adds and one rounding, written into
the padded NDHWC input of the stride-(2,2,2) downsample convolution.
``ResidualDownsampleBlock`` (:63-85) runs the INT8 residual body, the pack
and the FP16 stride-(2,2,2) downsample convolution (``h3v_conv3d_f16``).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .. import _hip
from .encoder_fp16_conv import NativeConv
from .encoder_fused_norm_bias import BiasFusedResidualBlock


def _validate_pack(x, residual, bias):
    if x.ndim != 5:
        raise ValueError("Validated scope: batch-one FP16 rank-5 input")
    b, c, d, h, w = x.shape
    if b != 1 or c <= 0 or c % 8 or d < 1 or min(h, w) < 2 or x.dtype != torch.float16:
        raise ValueError("Validated scope: batch-one FP16, C a multiple of 8, H/W>=2")
    if residual.shape != x.shape or residual.dtype != x.dtype or residual.device != x.device:
        raise ValueError("Residual must match input")
    if bias.shape != (c,) or bias.dtype != x.dtype or bias.device != x.device or not bias.is_contiguous():
        raise ValueError("Expected contiguous FP16 channel bias")
    if c * (d + 2) * (h + 1) * (w + 1) >= 2**31:
        raise ValueError("Output exceeds validated int32 index range")


@torch.library.custom_op("h3vae_encoder::residual_downsample_pack", mutates_args=(), device_types="cuda")
def residual_downsample_pack(x: torch.Tensor, residual: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    """-> fp16 [1, C, D+2, H+1, W+1] channels-last-3d."""
    _validate_pack(x, residual, bias)
    _hip.require_gfx950(x.device, "residual downsample pack")
    b, c, d, h, w = x.shape
    x = x.contiguous(memory_format=torch.channels_last_3d)
    residual = residual.contiguous(memory_format=torch.channels_last_3d)
    y = torch.empty((b, c, d + 2, h + 1, w + 1), device=x.device, dtype=x.dtype,
                    memory_format=torch.channels_last_3d)
    _hip.call("h3v_residual_downsample_pack", _hip.ptr(x), _hip.ptr(residual), _hip.ptr(bias), _hip.ptr(y), c, d, h,
              w, _hip.stream(x.device))
    return y


@residual_downsample_pack.register_fake
def _fake(x, residual, bias):
    b, c, d, h, w = x.shape
    return torch.empty((b, c, d + 2, h + 1, w + 1), device=x.device, dtype=x.dtype,
                       memory_format=torch.channels_last_3d)


class ResidualDownsampleBlock(BiasFusedResidualBlock):
    """Stage-1 final identity-shortcut block fused with its causal reflect downsample (reference :63-85)."""

    def __init__(self, block, downsample):
        super().__init__(block)
        conv = downsample.conv
        if (self.shortcut is not None or conv.padding != (1, 0, 0) or conv.stride != (2, 2, 2)
                or conv.pad_mode != "reflect" or conv.pad_mode_t != "constant" or not conv.causal
                or conv.spatial_parallel):
            raise ValueError("Expected stage1 final identity-shortcut block and causal reflect downsample")
        self.down_weight = conv.weight
        self.down_bias = conv.bias
        self.down = NativeConv(conv.weight, conv.bias, (2, 2, 2))

    def forward(self, x, zq=None):
        if zq is not None:
            raise ValueError("Unconditional inference only")
        return self.forward_partials(x)[0]

    def forward_partials(self, x, x_partials=None):
        """``(forward(x), None)``; ``x_partials`` as in ``BiasFusedResidualBlock.forward_partials`` (read by the
        first norm in INT8 mode).  The first conv hands its tile statistics to the second norm."""
        if self.int8_first is not None and self.int8_first.fuse_norm and self.int8_second.fuse_norm:
            from .encoder_int8 import padded_output_fits
            h, w = x.shape[3:]
            if padded_output_fits(self.int8_second.config.in_channels, self.int8_second.config.out_channels, h, w):
                # The second conv writes the pack's output itself: fp16(x + (conv + second.bias)) into the
                # downsample's padded input (two zero frames, bottom / right reflect); bit-identical to the
                # conv followed by residual_downsample_pack, without re-reading the conv output.
                h1, hp = self.int8_first.forward_norm(x, self.first.norm_weight, self.first.norm_bias,
                                                      self.first.eps, x_partials=x_partials, emit_partials=True,
                                                      partials_bias=self.first.bias)
                padded = self.int8_second.forward_norm(h1, self.second.norm_weight, self.second.norm_bias,
                                                       self.second.eps, pre_bias=self.first.bias, residual=x,
                                                       residual_bias=self.second.bias, pad_front=2,
                                                       pad_border=(0, 1, 0, 1), x_partials=hp)
                return self.down(padded), None
        # second.bias is added by the pack, not by the second convolution
        h = self._residual_body(x, None)
        h = residual_downsample_pack(h, x, self.second.bias)
        return self.down(h), None
