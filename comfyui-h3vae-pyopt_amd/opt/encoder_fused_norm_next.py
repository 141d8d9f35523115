"""Encoder prefix with bias-fused residual blocks (stages 0 and 1).

Mirror of ``next_fused_prefix`` (opt/encoder_fused_norm_next.py:7-28) in
fishelegs/ComfyUI-H3VAE-PyOpt for its bias-fused variants.  The returned
prefix shares every weight with ``encoder``; the original modules are not
modified.  ``extend_bias_pack`` (the production choice) also fuses the last
stage-1 block with the downsample through the residual pack.
"""
from __future__ import annotations

import torch

from .encoder_fused_norm_bias import BiasFusedResidualBlock
from .encoder_fused_residual_pack import ResidualDownsampleBlock
from .encoder_internal_padding import ImplicitTemporalPadConv3d
from .encoder_staged_batch import EncoderPrefix

VARIANTS = ("bias", "extend_bias", "extend_bias_pack")


def next_fused_prefix(encoder, variant="extend_bias_pack"):
    if variant not in VARIANTS:
        raise ValueError(f"unsupported prefix variant {variant!r}; expected one of {VARIANTS}")
    prefix = EncoderPrefix(encoder, 2)
    stages = (0, 1) if variant.startswith("extend") else (0,)
    for idx in stages:
        stage = torch.nn.Module()
        stage.block = torch.nn.ModuleList([BiasFusedResidualBlock(b) for b in encoder.down[idx].block])
        if hasattr(encoder.down[idx], "downsample"):
            stage.downsample = encoder.down[idx].downsample
        prefix.stages[idx] = stage
    if variant == "extend_bias_pack":
        prefix.stages[1].block[-1] = ResidualDownsampleBlock(encoder.down[1].block[-1], encoder.down[1].downsample)
        del prefix.stages[1].downsample
        # A stage-0 downsample conv run as pack + native conv lets the stage's last block write that
        # conv's padded input directly (INT8 mode).
        down0 = getattr(prefix.stages[0], "downsample", None)
        conv0 = getattr(down0, "conv", None)
        if isinstance(conv0, ImplicitTemporalPadConv3d):
            prefix.stages[0].block[-1].padded_consumer = conv0
    return prefix
