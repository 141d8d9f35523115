"""The model's causal padded convolutions, with their padding written by a pack kernel.

Counterpart of opt/encoder_internal_padding.py in fishelegs/ComfyUI-H3VAE-PyOpt
(``ImplicitTemporalPadConv3d`` :14-35, ``replace_selected`` / ``restore_selected``
:38-56), which moves the causal zero frames of ``down.0.downsample.conv`` into
the cuDNN call.  Here a wrapped conv never materialises ``F.pad`` output: one
HIP pack (``h3v_causal_reflect_pack``) writes the zero frames and the reflect
border into a channels-last-3d buffer and ``h3v_conv3d_f16`` convolves it over
exactly the output frames the model keeps (3-channel ``conv_in`` folds its
spatial taps in the pack instead, see ``encoder_fp16_conv.PaddedCausalConv``).

The model pads a causal conv with ``2 * pt`` zero frames in front (``kd - 1``
for a one-frame input) and a reflect border of ``ph`` / ``pw`` on every side,
or of one row and one column at the far edges when ``right_bottom_only`` is
set (the stride-2 downsample convs).  This build wraps ``conv_in``, every
downsample conv of the prefix and of the suffix stages the same way.
"""
from __future__ import annotations

import contextlib
from dataclasses import dataclass

import torch

from .encoder_fp16_conv import PaddedCausalConv


@dataclass
class _PartialsSlot:
    partials: object = None


def _reflect_border(conv):
    """(top, bottom, left, right) reflect rows / columns the model pads around a frame."""
    _, ph, pw = conv.padding
    if getattr(conv, "right_bottom_only", False):
        return (0, 1, 0, 1)
    return (ph, ph, pw, pw)


class ImplicitTemporalPadConv3d(torch.nn.Module):
    """A causal zero-time / reflect-space padded conv of the model, run as pack + native conv."""

    def __init__(self, original):
        super().__init__()
        supported = (getattr(original, "causal", False) and getattr(original, "pad_mode_t", None) == "constant"
                     and getattr(original, "pad_mode", None) == "reflect"
                     and not getattr(original, "spatial_parallel", False) and original.groups == 1
                     and tuple(original.dilation) == (1, 1, 1) and original.padding[0] > 0)
        if not supported:
            raise ValueError("Only single-GPU causal zero-temporal-padding convolutions are supported")
        self.weight, self.bias = original.weight, original.bias
        self.kernel_size, self.stride, self.padding = tuple(original.kernel_size), tuple(original.stride), \
            tuple(original.padding)
        self.pad_mode = original.pad_mode
        # zero frames in front of a clip / of a single image
        self.front_video, self.front_image = 2 * self.padding[0], self.kernel_size[0] - 1
        self.native = PaddedCausalConv(self.weight, self.bias, self.stride, _reflect_border(original))
        self._partials_slot = None

    def forward(self, x):
        front = self.front_video if x.shape[2] > 1 else self.front_image
        slot = self._partials_slot
        if slot is not None:
            out, slot.partials = self.native.forward_partials(x, front)
            return out
        return self.native(x, front)

    def forward_partials(self, x):
        """``(forward(x), partials)``: the conv also writes the GroupNorm statistics of its output for the INT8
        norm that reads it next (``GnPartials``), or None where its geometry has no statistics epilogue."""
        return self.native.forward_partials(x, self.front_video if x.shape[2] > 1 else self.front_image)

    @contextlib.contextmanager
    def partials_requested(self):
        """Inside the block, a call of this conv by the module that owns it (the model's downsample module
        calls it as ``self.conv(x)``) also forms the statistics of ``forward_partials`` and leaves them in the
        yielded slot's ``partials``."""
        slot = _PartialsSlot()
        self._partials_slot = slot
        try:
            yield slot
        finally:
            self._partials_slot = None

    def padded_input_form(self, x):
        """(front, border) of the padded input this conv builds for ``x`` when its reflect border is 0 or 1
        per side, the form ``h3v_conv3d_i8_residual_padded`` writes, else None."""
        native = self.native
        if native.folded or any(b not in (0, 1) for b in native.border) or min(x.shape[3:]) < 2:
            return None
        return (self.front_video if x.shape[2] > 1 else self.front_image), native.border


@dataclass
class _Swap:
    owner: torch.nn.Module
    name: str
    original: torch.nn.Module

    def undo(self):
        self.owner._modules[self.name] = self.original


def replace_selected(encoder, names):
    """Wrap the named convs of ``encoder`` in place; -> handles for ``restore_selected``.

    Every named conv is checked and wrapped before any is swapped in, so a conv the wrapper refuses (for
    instance a ``conv_in`` whose spatial padding is not reflect) raises ``ValueError`` naming it and leaves
    the encoder untouched."""
    planned = []
    for path in names:
        *owner_path, leaf = path.split(".")
        owner = encoder.get_submodule(".".join(owner_path))
        original = owner._modules[leaf]
        try:
            wrapper = ImplicitTemporalPadConv3d(original)
        except ValueError as exc:
            raise ValueError(f"{path}: {exc} (causal={getattr(original, 'causal', None)!r}, "
                             f"pad_mode={getattr(original, 'pad_mode', None)!r}, "
                             f"pad_mode_t={getattr(original, 'pad_mode_t', None)!r}); no conv was replaced") from exc
        planned.append((_Swap(owner, leaf, original), wrapper))
    for swap, wrapper in planned:
        swap.owner._modules[swap.name] = wrapper
    return [swap for swap, _ in planned]


def restore_selected(replacements):
    for swap in reversed(replacements):
        swap.undo()
