"""FP16 encoder convolutions on the matrix cores (``h3v_conv3d_f16``).

The reference runs every FP16 convolution of the encoder outside the INT8
path as ``F.conv3d`` (cuDNN): the 3x3x3 convs after the fp16 producers
(opt/encoder_fused_batched_norm.py:83,94,96; opt/encoder_fused_norm_bias.py
:135,139; opt/encoder_fused_temporal_norm.py:118), the stride-2 downsample
after the residual pack (opt/encoder_fused_residual_pack.py:85), the stage-0
downsample with its temporal padding folded into the call
(opt/encoder_internal_padding.py:34), and the 1x1x1 ``nin_shortcut``
projections.  Here they run as one HIP entry: fp16 operands, fp32
accumulation on ``v_mfma_f32_32x32x16_f16``, ``fp16(acc + bias)`` once.
Stride-1 3x3x3 convs whose output rows tile into 512-voxel blocks keep the
input window of a tile in LDS; every other geometry is an implicit GEMM.

Inputs are channels-last-3d and already padded; weights are packed once per
weight tensor to [Cout, kd*kh*kw*Cin] (c fastest).  ``conv3d_f16_fits`` is the
shape gate (Cin a multiple of 32).  ``conv_in`` (3 input channels, a model
layer the reference leaves alone) runs through ``padded_causal_conv3d`` too:
its 3x3 spatial taps and channels are folded into 32 channels by one pack
kernel (``h3v_tap_fold_pack``), leaving a 3x1x1 conv with K = 96.
"""
from __future__ import annotations

from typing import List, Optional, Tuple

import torch
import torch.nn.functional as F
from torch import nn

from .. import _hip


def pack_conv_weight_f16(weight):
    """fp16 [Cout, Cin, kd, kh, kw] -> [Cout, kd*kh*kw*Cin] with k = (kd, kh, kw, c), c fastest."""
    if weight.ndim != 5 or weight.dtype != torch.float16:
        raise ValueError("expected an fp16 [Cout, Cin, kd, kh, kw] weight")
    return weight.permute(0, 2, 3, 4, 1).reshape(weight.shape[0], -1).contiguous()


def fold_conv_weight_f16(weight, cf=32):
    """fp16 [Cout, C, 3, 3, 3] (9C <= cf) -> [Cout, 3 * cf]: k = (kd, (kh*3 + kw)*C + c), zero beyond 9C."""
    if weight.ndim != 5 or weight.dtype != torch.float16 or tuple(weight.shape[2:]) != (3, 3, 3) or 9 * weight.shape[1] > cf:
        raise ValueError("expected an fp16 [Cout, C, 3, 3, 3] weight with 9 * C <= folded channels")
    o, c = weight.shape[:2]
    folded = weight.new_zeros((o, 3, cf))
    folded[:, :, :9 * c] = weight.permute(0, 2, 3, 4, 1).reshape(o, 3, 9 * c)
    return folded.reshape(o, 3 * cf).contiguous()


def conv3d_f16_fits(x, weight, stride):
    """Whether h3v_conv3d_f16 takes the valid convolution of x [B, C, D, H, W] with weight at stride."""
    if x.ndim != 5 or weight.ndim != 5 or x.dtype != torch.float16 or weight.dtype != torch.float16:
        return False
    b, c, d, h, w = x.shape
    kd, kh, kw = weight.shape[2:]
    sd, sh, sw = tuple(stride)
    if weight.shape[1] != c or c % 32 or min(d - kd, h - kh, w - kw) < 0 or min(sd, sh, sw) < 1:
        return False
    m = b * ((d - kd) // sd + 1) * ((h - kh) // sh + 1) * ((w - kw) // sw + 1)
    return x.numel() * 2 < 2 ** 32 and weight.numel() * 2 < 2 ** 31 and m < 2 ** 31


def _check_conv(x, w_packed, bias, kernel_size, stride, residual=None):
    if x.ndim != 5 or x.dtype != torch.float16 or w_packed.dtype != torch.float16 or w_packed.ndim != 2:
        raise ValueError("conv3d_f16 requires an fp16 [B, C, D, H, W] input and an fp16 [Cout, K] packed weight")
    if len(kernel_size) != 3 or len(stride) != 3 or min(kernel_size) < 1 or min(stride) < 1:
        raise ValueError("conv3d_f16 requires three positive kernel sizes and strides")
    b, c, d, h, w = x.shape
    kd, kh, kw = kernel_size
    if w_packed.shape[1] != kd * kh * kw * c or not w_packed.is_contiguous():
        raise ValueError("conv3d_f16 requires a packed [Cout, kd*kh*kw*C] weight")
    if d < kd or h < kh or w < kw:
        raise ValueError("conv3d_f16 requires an input at least as large as the kernel")
    if bias is not None and (bias.shape != (w_packed.shape[0],) or bias.dtype != torch.float16
                             or not bias.is_contiguous()):
        raise ValueError("conv3d_f16 requires a contiguous fp16 [Cout] bias")
    if b > 1 and not x.is_contiguous(memory_format=torch.channels_last_3d):
        raise ValueError("conv3d_f16 requires a channels-last-3d input")
    if residual is not None and (residual.dtype != torch.float16
                                 or tuple(residual.shape) != _out_shape(x, w_packed, kernel_size, stride)):
        raise ValueError("conv3d_f16 requires an fp16 residual of the output's shape")


def _out_shape(x, w_packed, kernel_size, stride):
    b, _, d, h, w = x.shape
    return (b, w_packed.shape[0], (d - kernel_size[0]) // stride[0] + 1, (h - kernel_size[1]) // stride[1] + 1,
            (w - kernel_size[2]) // stride[2] + 1)


@torch.library.custom_op("h3vae_encoder::conv3d_f16", mutates_args=(), device_types="cuda")
def conv3d_f16(x: torch.Tensor, w_packed: torch.Tensor, bias: Optional[torch.Tensor], kernel_size: List[int],
               stride: List[int], causal_skip: bool, residual: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Valid conv of a padded fp16 [B, C, D, H, W] (channels-last-3d) -> fp16 [B, Cout, Do, Ho, Wo] channels-last-3d.

    causal_skip (3-deep kernels at depth stride 1) assumes two zero leading frames per item; residual (the
    output's shape) is added as a separate fp16 add would: fp16(residual + fp16 output)."""
    _check_conv(x, w_packed, bias, kernel_size, stride, residual)
    _hip.require_gfx950(x.device, "conv3d_f16")
    if not x.is_contiguous(memory_format=torch.channels_last_3d):
        x = x.contiguous(memory_format=torch.channels_last_3d)
    if residual is not None and not residual.is_contiguous(memory_format=torch.channels_last_3d):
        residual = residual.contiguous(memory_format=torch.channels_last_3d)
    b, c, d, h, w = x.shape
    out = torch.empty(_out_shape(x, w_packed, kernel_size, stride), device=x.device, dtype=x.dtype,
                      memory_format=torch.channels_last_3d)
    cout = w_packed.shape[0]
    # convs too small to fill the chip split their reduction over a workspace of fp32 partial sums
    floats = int(_hip.lib().h3v_conv3d_f16_workspace_floats(b, c, d, h, w, cout, *kernel_size, *stride))
    if floats < 0:
        raise ValueError(_hip.lib().h3v_last_error().decode(errors="replace"))
    ws = torch.empty(floats, device=x.device, dtype=torch.float32) if floats else None
    _hip.call("h3v_conv3d_f16_ws", _hip.ptr(x), _hip.ptr(w_packed), _hip.ptr(bias), _hip.ptr(residual), _hip.ptr(out),
              b, c, d, h, w, cout, *kernel_size, *stride, int(bool(causal_skip)), _hip.ptr(ws), floats,
              _hip.stream(x.device))
    return out


@conv3d_f16.register_fake
def _fake_conv(x, w_packed, bias, kernel_size, stride, causal_skip, residual=None):
    _check_conv(x, w_packed, bias, kernel_size, stride, residual)
    return torch.empty(_out_shape(x, w_packed, kernel_size, stride), device=x.device, dtype=x.dtype,
                       memory_format=torch.channels_last_3d)


def conv3d_f16_gn_fits(x, w_packed, kernel_size, stride):
    """Whether ``conv3d_f16_gn`` takes this conv: one clip, 128 output channels, output frames of a multiple
    of 256 pixels, Cin % 32 == 0."""
    if x.ndim != 5 or w_packed.ndim != 2:
        return False
    b, c, _, _, _ = x.shape
    _, _, do, ho, wo = _out_shape(x, w_packed, kernel_size, stride)
    return b == 1 and c % 32 == 0 and w_packed.shape[0] == 128 and do >= 1 and (ho * wo) % 256 == 0


@torch.library.custom_op("h3vae_encoder::conv3d_f16_gn", mutates_args=(), device_types="cuda")
def conv3d_f16_gn(x: torch.Tensor, w_packed: torch.Tensor, bias: Optional[torch.Tensor], kernel_size: List[int],
                  stride: List[int], causal_skip: bool) -> Tuple[torch.Tensor, torch.Tensor]:
    """``conv3d_f16`` (no residual) that also writes the GroupNorm(32) partial statistics of its output for the
    INT8 producer that normalises it next (``h3v_conv3d_f16_gn``): -> (out, workspace), the workspace in that
    producer's layout over 256-pixel chunks, in the order of its own statistics pass, so the producer's
    results are bit-identical to those of its own pass.  ``conv3d_f16_gn_fits`` geometry only."""
    _check_conv(x, w_packed, bias, kernel_size, stride)
    if not conv3d_f16_gn_fits(x, w_packed, kernel_size, stride):
        raise ValueError(f"conv3d_f16_gn: input {tuple(x.shape)}, Cout {w_packed.shape[0]} is outside its gate "
                         "(one clip, Cout 128, output frames of a multiple of 256 pixels)")
    _hip.require_gfx950(x.device, "conv3d_f16_gn")
    if not x.is_contiguous(memory_format=torch.channels_last_3d):
        x = x.contiguous(memory_format=torch.channels_last_3d)
    _, c, d, h, w = x.shape
    shape = _out_shape(x, w_packed, kernel_size, stride)
    out = torch.empty(shape, device=x.device, dtype=x.dtype, memory_format=torch.channels_last_3d)
    floats = int(_hip.lib().h3v_gn_norm_pack_workspace_floats(*shape[2:]))
    ws = torch.empty(floats, device=x.device, dtype=torch.float32)
    _hip.call("h3v_conv3d_f16_gn", _hip.ptr(x), _hip.ptr(w_packed), _hip.ptr(bias), _hip.ptr(out), c, d, h, w,
              w_packed.shape[0], *kernel_size, *stride, int(bool(causal_skip)), _hip.ptr(ws), _hip.stream(x.device))
    return out, ws


@conv3d_f16_gn.register_fake
def _fake_conv_gn(x, w_packed, bias, kernel_size, stride, causal_skip):
    _check_conv(x, w_packed, bias, kernel_size, stride)
    shape = _out_shape(x, w_packed, kernel_size, stride)
    return (torch.empty(shape, device=x.device, dtype=x.dtype, memory_format=torch.channels_last_3d),
            x.new_empty((0,), dtype=torch.float32))


def _check_pack(x, front, pads):
    if x.ndim != 5 or x.dtype != torch.float16 or x.shape[1] % 8 or x.numel() == 0:
        raise ValueError("causal_reflect_pack requires a nonempty fp16 [B, C, D, H, W] input with C % 8 == 0")
    top, bottom, left, right = pads
    h, w = x.shape[3:]
    if front < 0 or min(pads) < 0 or max(top, bottom) >= h or max(left, right) >= w:
        raise ValueError("causal_reflect_pack: reflect padding must be smaller than the padded dimension")


@torch.library.custom_op("h3vae_encoder::causal_reflect_pack", mutates_args=(), device_types="cuda")
def causal_reflect_pack(x: torch.Tensor, front: int, top: int, bottom: int, left: int, right: int) -> torch.Tensor:
    """fp16 [B, C, D, H, W] -> [B, C, D+front, H+top+bottom, W+left+right] channels-last-3d:
    ``front`` zero frames per item, then x with its spatial border reflected."""
    _check_pack(x, front, (top, bottom, left, right))
    _hip.require_gfx950(x.device, "causal_reflect_pack")
    x = x.contiguous(memory_format=torch.channels_last_3d)
    b, c, d, h, w = x.shape
    out = torch.empty((b, c, d + front, h + top + bottom, w + left + right), device=x.device, dtype=x.dtype,
                      memory_format=torch.channels_last_3d)
    _hip.call("h3v_causal_reflect_pack", _hip.ptr(x), _hip.ptr(out), b, c, d, h, w, front, top, bottom, left, right,
              _hip.stream(x.device))
    return out


@causal_reflect_pack.register_fake
def _fake_pack(x, front, top, bottom, left, right):
    _check_pack(x, front, (top, bottom, left, right))
    b, c, d, h, w = x.shape
    return torch.empty((b, c, d + front, h + top + bottom, w + left + right), device=x.device, dtype=x.dtype,
                       memory_format=torch.channels_last_3d)


def _check_fold(x, front):
    if x.ndim != 5 or x.dtype != torch.float16 or not 1 <= x.shape[1] <= 3 or x.numel() == 0:
        raise ValueError("tap_fold_pack requires a nonempty fp16 [B, C, D, H, W] input with C in 1..3")
    if min(x.shape[3:]) < 2 or front < 0:
        raise ValueError("tap_fold_pack requires H, W >= 2 and front >= 0")


@torch.library.custom_op("h3vae_encoder::tap_fold_pack", mutates_args=(), device_types="cuda")
def tap_fold_pack(x: torch.Tensor, front: int) -> torch.Tensor:
    """fp16 [B, C<=3, D, H, W] -> [B, 32, D+front, H, W] channels-last-3d: channel (kh*3 + kw)*C + c holds the
    (kh, kw) tap of the reflect-padded input (a 3x3x3 conv over x = a 3x1x1 conv over this)."""
    _check_fold(x, front)
    _hip.require_gfx950(x.device, "tap_fold_pack")
    x = x.contiguous(memory_format=torch.channels_last_3d)
    b, c, d, h, w = x.shape
    out = torch.empty((b, 32, d + front, h, w), device=x.device, dtype=x.dtype, memory_format=torch.channels_last_3d)
    _hip.call("h3v_tap_fold_pack", _hip.ptr(x), _hip.ptr(out), b, c, d, h, w, front, 32, _hip.stream(x.device))
    return out


@tap_fold_pack.register_fake
def _fake_fold(x, front):
    _check_fold(x, front)
    b, _, d, h, w = x.shape
    return torch.empty((b, 32, d + front, h, w), device=x.device, dtype=x.dtype, memory_format=torch.channels_last_3d)


def _weight_stamp(weight):
    """What identifies the contents of a weight: storage, device, dtype, shape and in-place version
    (inference tensors carry no version counter; their in-place updates are not seen)."""
    return (weight.data_ptr(), weight.device, weight.dtype, tuple(weight.shape),
            -1 if weight.is_inference() else weight._version)


class PackedConvWeight(nn.Module):
    """The packed fp16 copy of one conv weight, owned by the module that runs the conv.

    The copy is made on first use and kept as a non-persistent buffer, so it moves and is freed
    with its owner (``.to()``, an offload of the runtime): no packed copy outlives the module or
    stays behind on a GPU, and a conv that never runs never holds one.  Each use compares the
    source weight with the stamp taken at packing and repacks when it changed (an in-place
    state-dict load, a move of the model's weights).

    The runtime runs encoder tiles on several streams at once, and the copy is shared by all of
    them, so on a GPU (re)packing waits for the device twice: before, because another stream may
    still read the old copy, and after, because the packing kernel runs on the current stream and
    the next tile's convs on another stream must not read the copy before it is written."""

    def __init__(self, weight, fold=False):
        super().__init__()
        self.fold = bool(fold)
        self.register_buffer("packed", None, persistent=False)
        self._stamp = None

    def forward(self, weight):
        stamp = _weight_stamp(weight)
        if self.packed is None or stamp != self._stamp:
            source = weight.detach()
            if source.is_cuda:
                torch.cuda.synchronize(source.device)
            self.packed = fold_conv_weight_f16(source) if self.fold else pack_conv_weight_f16(source)
            self._stamp = stamp
            if source.is_cuda:
                torch.cuda.synchronize(source.device)
        return self.packed


def native_device(x):
    """x lives on a gfx950 GPU, where these kernels run."""
    return x.is_cuda and _hip.is_gfx950(x.device)


def _require_native(x, what):
    if not native_device(x):
        raise RuntimeError(f"{what} runs on an AMD MI355X (gfx950) GPU only; got a tensor on {x.device}")


class NativeConv(nn.Module):
    """One FP16 convolution of the model run as ``h3v_conv3d_f16`` on an already padded input.

    Shares the model's weight and bias; owns their packed copy.  Shapes outside the kernel's gate
    (``conv3d_f16_fits``) raise: there is no second implementation to fall back to."""

    def __init__(self, weight, bias, stride):
        super().__init__()
        if weight.ndim != 5:
            raise ValueError("NativeConv expects a [Cout, Cin, kd, kh, kw] weight")
        self.weight, self.bias = weight, bias
        self.stride = tuple(int(s) for s in stride)
        self.packed_weight = PackedConvWeight(weight)

    def forward(self, x, *, with_bias=True, causal_skip=False, residual=None):
        _require_native(x, "FP16 encoder convolution")
        if not conv3d_f16_fits(x, self.weight, self.stride):
            raise ValueError(f"FP16 encoder convolution: input {tuple(x.shape)} / weight {tuple(self.weight.shape)} "
                             f"at stride {self.stride} is outside h3v_conv3d_f16's gate (Cin % 32 == 0, fp16)")
        kernel = list(self.weight.shape[2:])
        skip = bool(causal_skip) and kernel[0] == 3 and self.stride[0] == 1
        return conv3d_f16(x, self.packed_weight(self.weight), self.bias if with_bias else None, kernel,
                          list(self.stride), skip, residual)

    def forward_partials(self, x, *, causal_skip=False):
        """``(forward(x), partials)``: where ``conv3d_f16_gn`` takes the geometry, the conv also writes the
        GroupNorm statistics of its output (``GnPartials`` over 256-pixel chunks) for the INT8 norm that reads
        it next; otherwise ``(forward(x), None)``."""
        _require_native(x, "FP16 encoder convolution")
        kernel = list(self.weight.shape[2:])
        packed = self.packed_weight(self.weight)
        if not conv3d_f16_fits(x, self.weight, self.stride) or not conv3d_f16_gn_fits(x, packed, kernel,
                                                                                      self.stride):
            return self.forward(x, causal_skip=causal_skip), None
        from .encoder_int8_norm import PIXEL_CHUNK, GnPartials
        skip = bool(causal_skip) and kernel[0] == 3 and self.stride[0] == 1
        out, ws = conv3d_f16_gn(x, packed, self.bias, kernel, list(self.stride), skip)
        return out, GnPartials(ws, PIXEL_CHUNK)


class PointwiseConv(nn.Module):
    """A 1x1x1 ``nn.Conv3d`` over channels-last-3d activations.

    Cin % 32 == 0 (``nin_shortcut``) runs as ``h3v_conv3d_f16``; other widths (the 48-channel
    ``quant_conv``) are a plain [rows, Cin] x [Cin, Cout] GEMM through torch's BLAS (hipBLASLt) over
    the channels-last rows, with the bias added in the same call."""

    def __init__(self, conv):
        super().__init__()
        if (tuple(conv.kernel_size) != (1, 1, 1) or tuple(conv.padding) != (0, 0, 0) or tuple(conv.stride) != (1, 1, 1)
                or tuple(conv.dilation) != (1, 1, 1) or conv.groups != 1):
            raise ValueError("PointwiseConv expects a 1x1x1, stride-1, unpadded, ungrouped Conv3d")
        self.weight, self.bias = conv.weight, conv.bias
        self.conv = NativeConv(conv.weight, conv.bias, (1, 1, 1)) if conv.weight.shape[1] % 32 == 0 else None

    def forward(self, x):
        _require_native(x, "pointwise convolution")
        if self.conv is not None:
            return self.conv(x.contiguous(memory_format=torch.channels_last_3d))
        b, c, d, h, w = x.shape
        rows = x.permute(0, 2, 3, 4, 1).reshape(-1, c)
        y = F.linear(rows, self.weight.view(self.weight.shape[0], c), self.bias)
        return y.view(b, d, h, w, -1).permute(0, 4, 1, 2, 3)


_PADDED_INPUT = "_h3v_padded_input"


def tag_padded_input(padded, front, border):
    """The interior ``padded[:, :, front:, top:top + H, left:left + W]`` of a padded conv input that a
    producer wrote directly, tagged so that ``PaddedCausalConv`` with the same front and border uses
    ``padded`` as it is instead of packing the interior again.  The view holds the unpadded tensor's
    values, so any other consumer sees the ordinary output."""
    top, bottom, left, right = border
    h = padded.shape[3] - top - bottom
    w = padded.shape[4] - left - right
    view = padded[:, :, front:, top:top + h, left:left + w]
    setattr(view, _PADDED_INPUT, (padded, int(front), tuple(border)))
    return view


def padded_input_of(x, front, border):
    """The tagged padded buffer behind ``x`` when it was written for this front and border, else None.
    (Views made under inference mode do not record their base, so the check compares the view's data
    pointer and strides with the interior of the tagged buffer.)"""
    tag = getattr(x, _PADDED_INPUT, None)
    if tag is None:
        return None
    padded, tfront, tborder = tag
    if tfront != front or tborder != tuple(border):
        return None
    top, _, left, _ = tborder
    inner = padded[:, :, front:, top:top + x.shape[3], left:left + x.shape[4]]
    if x.shape != inner.shape or x.stride() != inner.stride() or x.data_ptr() != inner.data_ptr():
        return None
    return padded


class PaddedCausalConv(nn.Module):
    """Zero frames in front + reflect border + valid conv (conv_in, the downsample convs).

    The padding is written by one pack kernel and the conv runs over exactly the kept outputs.
    A 3-channel stride-1 3x3x3 conv with a border of 1 (conv_in) folds its 3x3 spatial taps into 32
    channels in the pack (``h3v_tap_fold_pack``) and becomes a 3x1x1 conv with K = 96."""

    def __init__(self, weight, bias, stride, border):
        super().__init__()
        self.weight, self.bias = weight, bias
        self.stride, self.border = tuple(int(s) for s in stride), tuple(int(b) for b in border)
        self.folded = (weight.shape[1] <= 3 and tuple(weight.shape[2:]) == (3, 3, 3) and self.stride == (1, 1, 1)
                       and self.border == (1, 1, 1, 1))
        if self.folded:
            self.packed_weight = PackedConvWeight(weight, fold=True)
        else:
            self.conv = NativeConv(weight, bias, stride)

    def forward(self, x, front):
        return self.forward_partials(x, front, want=False)[0]

    def forward_partials(self, x, front, want=True):
        """``(forward(x, front), partials)``: with ``want`` and where ``conv3d_f16_gn`` takes the conv, it also
        writes the GroupNorm statistics of its output (``GnPartials``, 256-pixel chunks) for the INT8 norm that
        reads it next; otherwise partials is None."""
        _require_native(x, "padded causal convolution")
        if self.folded:
            if min(x.shape[3:]) < 2:
                raise ValueError("conv_in requires H, W >= 2")
            folded, packed = tap_fold_pack(x, front), self.packed_weight(self.weight)
            if want and conv3d_f16_gn_fits(folded, packed, [3, 1, 1], [1, 1, 1]):
                from .encoder_int8_norm import PIXEL_CHUNK, GnPartials
                out, ws = conv3d_f16_gn(folded, packed, self.bias, [3, 1, 1], [1, 1, 1], front == 2)
                return out, GnPartials(ws, PIXEL_CHUNK)
            return conv3d_f16(folded, packed, self.bias, [3, 1, 1], [1, 1, 1], front == 2), None
        top, bottom, left, right = self.border
        written = padded_input_of(x, front, self.border)
        if written is None:
            if x.shape[1] % 8 or max(top, bottom) >= x.shape[3] or max(left, right) >= x.shape[4]:
                raise ValueError(f"padded causal convolution: input {tuple(x.shape)} needs C % 8 == 0 and a "
                                 f"reflect border {self.border} smaller than H, W")
            written = causal_reflect_pack(x, front, top, bottom, left, right)
        # (else the producing conv already wrote this conv's padded input)
        if want:
            return self.conv.forward_partials(written, causal_skip=front == 2)
        return self.conv(written, causal_skip=front == 2), None
