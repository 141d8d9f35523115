"""Causal temporal zero padding folded into the convolution call (FP16 encoder layers).

Mirror of opt/encoder_internal_padding.py in fishelegs/ComfyUI-H3VAE-PyOpt.
The spatial reflect pad stays explicit; the left-only causal zero frames are
requested from the convolution as symmetric temporal padding and the extra
tail outputs are dropped.  Used for ``down.0.downsample.conv`` (and, in this
build's runtime, ``conv_in``), FP16 layers outside the INT8 path.  On gfx950
the zero frames and the reflect border are written by one pack kernel
(``h3v_causal_reflect_pack``; for conv_in's 3 channels ``h3v_tap_fold_pack``,
which also folds the 3x3 spatial taps into 32 channels) and the convolution
runs as ``h3v_conv3d_f16`` over exactly the kept outputs.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .encoder_fp16_conv import native_device, padded_causal_conv3d


class ImplicitTemporalPadConv3d(torch.nn.Module):
    def __init__(self, original):
        super().__init__()
        if not (getattr(original, "causal", False) and getattr(original, "pad_mode_t", None) == "constant"
                and not getattr(original, "spatial_parallel", False) and original.groups == 1
                and original.dilation == (1, 1, 1) and original.padding[0] > 0):
            raise ValueError("Only single-GPU causal zero-temporal-padding convolutions are supported")
        self.weight = original.weight
        self.bias = original.bias
        self.padding = original.padding
        self.stride = original.stride
        self.kernel_size = original.kernel_size
        self.pad_mode = original.pad_mode

    def forward(self, x):
        depth = x.shape[2]
        left = 2 * self.padding[0] if depth > 1 else self.kernel_size[0] - 1
        output_depth = (depth + left - self.kernel_size[0]) // self.stride[0] + 1
        ph, pw = self.padding[1:]
        if self.pad_mode == "reflect" and native_device(x):
            return padded_causal_conv3d(x, self.weight, self.bias, self.stride, left, ph, ph, pw, pw)
        if ph or pw:
            x = F.pad(x, (pw, pw, ph, ph, 0, 0), mode=self.pad_mode)
        y = F.conv3d(x, self.weight, self.bias, stride=self.stride, padding=(left, 0, 0))
        return y[:, :, :output_depth]


def replace_selected(encoder, names):
    replacements = []
    for name in names:
        parent_path, _, leaf = name.rpartition(".")
        parent = encoder.get_submodule(parent_path) if parent_path else encoder
        original = getattr(parent, leaf)
        setattr(parent, leaf, ImplicitTemporalPadConv3d(original))
        replacements.append((parent, leaf, original))
    return replacements


def restore_selected(replacements):
    for parent, leaf, original in replacements:
        setattr(parent, leaf, original)
