"""Encoder residual block whose norm/SiLU/pad producers carry the conv bias.

Mirror of opt/encoder_fused_norm_bias.py (``BiasFusedResidualBlock``,
:121-140) and of the norm-pack holder ``FusedNormPadConv``
(opt/encoder_fused_temporal_norm.py:101-118; opaque op
opt/encoder_fused_norm_opaque.py:10-21) in fishelegs/ComfyUI-H3VAE-PyOpt.

With INT8 wrappers installed and norm fusion on (the gfx950 default), a block
is two ``h3vae_encoder::int8_norm_conv3d`` calls.  The first conv's bias is
not applied in its epilogue; it is folded into the second producer as
``pre_bias`` (v = fp16(v + bias) before the statistics).  The block input
(or its ``nin_shortcut`` projection) is added last.

Without INT8 wrappers (the FP16 encoder mode) the same producers emit fp16
through ``h3v_gn_norm_pack_f16`` (one fused statistics + pack launch
sequence) and the convolutions run in FP16 through ``h3v_conv3d_f16``
(``NativeConv``; the ``nin_shortcut`` through ``PointwiseConv``);
nothing in this file ever falls back from the INT8 path to them.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .. import _hip
from .encoder_fp16_conv import NativeConv, PointwiseConv


def _check_channel_vectors(x, *vectors):
    c = x.shape[1]
    for parameter in vectors:
        if (parameter.shape != (c,) or parameter.dtype != x.dtype or parameter.device != x.device
                or not parameter.is_contiguous()):
            raise ValueError("Expected contiguous FP16 channel vectors on input device")


def norm_pack_f16(x, weight, bias, eps, pre_bias=None):
    """Per-frame GroupNorm(32) + SiLU + 2 causal zero frames + reflect pad 1, fp16 out (``h3v_gn_norm_pack_f16``).

    x: fp16 [B, C, D, H, W] whose batch and time are adjacent frame spans (B == 1, or
    x.stride(0) == D * x.stride(2)); it is made channels-last-3d if it is not.  Statistics are
    per (batch item, frame).  -> fp16 [B, C, D+2, H+2, W+2] channels-last-3d.
    """
    b, c, d, h, w = x.shape
    _hip.require_gfx950(x.device, "norm_pack_f16")
    if not x.is_contiguous(memory_format=torch.channels_last_3d):
        x = x.contiguous(memory_format=torch.channels_last_3d)
    y = torch.empty((b, c, d + 2, h + 2, w + 2), device=x.device, dtype=x.dtype, memory_format=torch.channels_last_3d)
    stats = torch.empty((b * d, 32, 2), device=x.device, dtype=torch.float32)
    ws = torch.empty(int(_hip.lib().h3v_gn_norm_pack_f16_workspace_floats(b, c, d, h, w)), device=x.device,
                     dtype=torch.float32)
    _hip.call("h3v_gn_norm_pack_f16", _hip.ptr(x), _hip.ptr(pre_bias), _hip.ptr(weight), _hip.ptr(bias), float(eps),
              b, c, d, h, w, _hip.ptr(y), _hip.ptr(stats), _hip.ptr(ws), _hip.stream(x.device))
    return y


def fused_temporal_norm_pad(x, weight, bias, eps, pre_bias=None):
    """FP16 encoder mode producer (reference opt/encoder_fused_temporal_norm.py:83-99 and
    opt/encoder_fused_norm_bias.py:14-39): batch one, C divisible by 32 (kernel: 128 ... 1024).

    -> fp16 [1, C, D+2, H+2, W+2] channels-last-3d, one ``h3v_gn_norm_pack_f16`` call.
    """
    b, c, d, h, w = x.shape
    if b != 1 or x.dtype != torch.float16 or c % 32 or min(h, w) < 2:
        raise ValueError("Validated scope: batch-one FP16, C divisible by 32, spatial >=2")
    if c not in (128, 256, 512, 1024):
        raise ValueError("Validated scope: C in 128, 256, 512, 1024")
    _check_channel_vectors(x, weight, bias, *(() if pre_bias is None else (pre_bias,)))
    return norm_pack_f16(x, weight, bias, eps, pre_bias)


@torch.library.custom_op("h3vae_encoder::temporal_norm_pack", mutates_args=(), device_types="cuda")
def temporal_norm_pack(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, eps: float) -> torch.Tensor:
    return fused_temporal_norm_pad(x, weight, bias, eps)


@temporal_norm_pack.register_fake
def _fake_norm_pack(x, weight, bias, eps):
    b, c, d, h, w = x.shape
    return torch.empty((b, c, d + 2, h + 2, w + 2), device=x.device, dtype=x.dtype,
                       memory_format=torch.channels_last_3d)


@torch.library.custom_op("h3vae_encoder::bias_temporal_norm_pack", mutates_args=(), device_types="cuda")
def bias_temporal_norm_pack(x: torch.Tensor, pre_bias: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor,
                            eps: float) -> torch.Tensor:
    return fused_temporal_norm_pad(x, weight, bias, eps, pre_bias=pre_bias)


@bias_temporal_norm_pack.register_fake
def _fake_bias_norm_pack(x, pre_bias, weight, bias, eps):
    b, c, d, h, w = x.shape
    return torch.empty((b, c, d + 2, h + 2, w + 2), device=x.device, dtype=x.dtype,
                       memory_format=torch.channels_last_3d)


class FusedNormPadConv(torch.nn.Module):
    """GroupNorm(32) + SiLU + causal/reflect pad feeding a 3x3x3 conv (reference :101-118)."""

    def __init__(self, norm, conv, config=(128, 32, 4), with_conv=True):
        super().__init__()
        if type(norm).__name__ != "TemporalIsolatedSpatialParallelGroupNorm" or norm.num_groups != 32:
            raise ValueError("Expected temporal-isolated GroupNorm with 32 groups")
        if (conv.padding != (1, 1, 1) or conv.kernel_size != (3, 3, 3) or not conv.causal
                or conv.pad_mode != "reflect" or conv.pad_mode_t != "constant" or conv.spatial_parallel):
            raise ValueError("Expected single-GPU causal 3x3x3 reflect-padded conv")
        self.norm_weight = norm.weight
        self.norm_bias = norm.bias
        self.eps = norm.eps
        self.weight = conv.weight
        self.bias = conv.bias
        self.stride = conv.stride
        self.config = config
        self.with_conv = with_conv
        # the FP16 conv after the producer (FP16 encoder mode); packs its weight on first use only
        self.conv = NativeConv(conv.weight, conv.bias, conv.stride)

    def forward(self, x):
        y = temporal_norm_pack(x, self.norm_weight, self.norm_bias, self.eps)
        return self.conv(y, causal_skip=True) if self.with_conv else y


# The reference's opaque-op subclass has the same behaviour here (every producer is an opaque op).
OpaqueFusedNormPadConv = FusedNormPadConv


class BiasFusedResidualBlock(torch.nn.Module):
    """Residual block: norm1/conv1 -> norm2(+conv1 bias)/conv2 -> + shortcut (reference :121-140)."""

    def __init__(self, block):
        super().__init__()
        if block.use_fused_norm or block.conv1.bias is None:
            raise ValueError("Expected original residual block with conv1 bias")
        self.first = OpaqueFusedNormPadConv(block.norm1, block.conv1, with_conv=False)
        self.second = OpaqueFusedNormPadConv(block.norm2, block.conv2, with_conv=False)
        self.shortcut = getattr(block, "nin_shortcut", None)
        self.shortcut_conv = PointwiseConv(self.shortcut) if self.shortcut is not None else None
        # INT8 wrappers are installed by encoder_int8_integration.install_int8_encoder_prefix;
        # None keeps the FP16 encoder mode.
        self.int8_first = None
        self.int8_second = None
        # The padded conv that reads this block's output (the stage's downsample), when the block is the
        # last of its stage: the INT8 second conv then writes that conv's padded input directly.
        self.padded_consumer = None

    def _residual_body(self, x, second_bias):
        if self.int8_first is not None and self.int8_first.fuse_norm:
            h = self.int8_first.forward_norm(x, self.first.norm_weight, self.first.norm_bias, self.first.eps)
            return self.int8_second.forward_norm(h, self.second.norm_weight, self.second.norm_bias,
                                                 self.second.eps, pre_bias=self.first.bias)
        first_input = self.first(x)
        h = (self.int8_first(first_input) if self.int8_first is not None
             else self.first.conv(first_input, with_bias=False, causal_skip=True))
        second_input = bias_temporal_norm_pack(h, self.first.bias, self.second.norm_weight,
                                               self.second.norm_bias, self.second.eps)
        return (self.int8_second(second_input) if self.int8_second is not None
                else self.second.conv(second_input, with_bias=second_bias is not None, causal_skip=True))

    def _padded_form(self, out_like):
        """(front, border) when the INT8 second conv can write the padded input of ``padded_consumer``
        for an output shaped like ``out_like``, else None."""
        consumer = self.padded_consumer
        if consumer is None or self.int8_second is None or not self.int8_second.fuse_norm:
            return None
        from .encoder_int8 import padded_output_fits
        _, c, _, h, w = out_like.shape
        if not padded_output_fits(self.int8_second.config.in_channels, c, h, w):
            return None
        return consumer.padded_input_form(out_like)

    def forward(self, x, zq=None):
        """(shortcut(x) or x) + body(x), the add fused into the second conv's epilogue where that conv is a
        kernel of this package (bit-identical to the separate fp16 add of the reference, :141)."""
        if zq is not None:
            raise ValueError("Unconditional inference only")
        return self.forward_partials(x)[0]

    def forward_partials(self, x, x_partials=None):
        """``(forward(x), partials)``.  In INT8 mode the first conv writes the GroupNorm tile statistics of
        its output (plus the first bias, the second norm's pre-bias) for the second norm, and the second
        conv those of the block's output for the norm that reads it next (the next block's first norm),
        returned as ``partials``; None where the convs' geometry has no statistics epilogue or the block
        writes the padded form.  ``x_partials``: the statistics of ``x`` that the previous block's second
        conv wrote (no bias), read by the first norm instead of its own statistics pass."""
        residual = self.shortcut_conv(x) if self.shortcut_conv is not None else x
        if self.int8_first is not None and self.int8_first.fuse_norm:
            h, hp = self.int8_first.forward_norm(x, self.first.norm_weight, self.first.norm_bias, self.first.eps,
                                                 x_partials=x_partials, emit_partials=True,
                                                 partials_bias=self.first.bias)
            form = self._padded_form(residual)
            if form is not None:
                from .encoder_fp16_conv import tag_padded_input
                padded = self.int8_second.forward_norm(h, self.second.norm_weight, self.second.norm_bias,
                                                       self.second.eps, pre_bias=self.first.bias, residual=residual,
                                                       pad_front=form[0], pad_border=form[1], x_partials=hp)
                return tag_padded_input(padded, *form), None
            return self.int8_second.forward_norm(h, self.second.norm_weight, self.second.norm_bias, self.second.eps,
                                                 pre_bias=self.first.bias, residual=residual, x_partials=hp,
                                                 emit_partials=True)
        if self.int8_first is None:
            h = self.first.conv(self.first(x), with_bias=False, causal_skip=True)
            second_input = bias_temporal_norm_pack(h, self.first.bias, self.second.norm_weight,
                                                   self.second.norm_bias, self.second.eps)
            return self.second.conv(second_input, causal_skip=True, residual=residual), None
        return residual + self._residual_body(x, self.second.bias), None
