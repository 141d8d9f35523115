"""INT8 wiring for the H3 encoder prefix: custom ops, module state, install policy.

Mirror of opt/encoder_int8_integration.py in fishelegs/ComfyUI-H3VAE-PyOpt.
Only the two residual blocks of encoder prefix stages 0 and 1 are replaced
(eight 3x3x3 convolutions).  With the fused producer the GroupNorm / SiLU /
padding / quantization and the causal-zero-skipping convolution run as one
custom op (``h3vae_encoder::int8_norm_conv3d``).
"""
from __future__ import annotations

from typing import Any

import torch
from torch import nn

from .. import _hip
from .encoder_int8 import Int8Conv3DConfig, _conv3d_from_quantized, int8_valid_conv3d, prepare_int8_weight

INT8_ENCODER_POLICY = {
    "stages": (0, 1),
    "blocks_per_stage": 2,
    "convolutions_per_block": ("first", "second"),
    "quantized_conv_count": 8,
    "kernel": (3, 3, 3),
    "tile_variants_by_input_channels": {128: "128x128x64", 256: "128x128x64"},
    "gfx950_auto_tile_variant": "128x128x64_pipeline4",
    "gfx950_auto_norm_absmax_fusion": True,
    "excluded": ("conv_in", "conv_out", "downsample", "nin_shortcut", "encoder suffix", "quant_conv"),
}


def _resolve_tile_variant(input_channels: int, requested: str | None, gfx950: bool = False) -> str:
    """Tile name of an installed module (the fused path is selected on gfx950)."""
    if requested not in (None, "auto"):
        return str(requested)
    if gfx950 and input_channels in (128, 256):
        return INT8_ENCODER_POLICY["gfx950_auto_tile_variant"]
    try:
        return INT8_ENCODER_POLICY["tile_variants_by_input_channels"][int(input_channels)]
    except KeyError as exc:
        raise ValueError("INT8 encoder stage-aware tile policy only supports input channels "
                         f"128 or 256, got {input_channels}") from exc


def _output_shape(x, qweight, kernel, stride):
    if x.ndim != 5:
        raise ValueError("INT8 encoder activation must be rank 5")
    if qweight.ndim != 2:
        raise ValueError("INT8 encoder qweight must be rank 2")
    output_dims = tuple((length - k) // s + 1 for length, k, s in zip(x.shape[-3:], kernel, stride))
    if any(value <= 0 for value in output_dims):
        raise ValueError(f"activation shape {tuple(x.shape)} is too small for valid conv")
    return (x.shape[0], qweight.shape[0], *output_dims)


@torch.library.custom_op("h3vae_encoder::int8_valid_conv3d_integration", mutates_args=(), device_types="cuda")
def int8_valid_conv3d_integration(x: torch.Tensor, qweight: torch.Tensor, weight_scale: torch.Tensor,
                                  bias: torch.Tensor, kernel_d: int, kernel_h: int, kernel_w: int, stride_d: int,
                                  stride_h: int, stride_w: int, apply_bias: bool, tile_variant: str) -> torch.Tensor:
    """Opaque graph boundary around the INT8 valid convolution."""
    taps = int(kernel_d) * int(kernel_h) * int(kernel_w)
    config = Int8Conv3DConfig(int(qweight.shape[1]) // taps, int(qweight.shape[0]),
                              (int(kernel_d), int(kernel_h), int(kernel_w)),
                              (int(stride_d), int(stride_h), int(stride_w)))
    return int8_valid_conv3d(x, qweight, weight_scale, config=config, bias=bias if apply_bias else None,
                             tile_variant=tile_variant)


@int8_valid_conv3d_integration.register_fake
def _int8_valid_conv3d_integration_fake(x, qweight, weight_scale, bias, kernel_d, kernel_h, kernel_w, stride_d,
                                        stride_h, stride_w, apply_bias, tile_variant):
    del weight_scale, bias, apply_bias, tile_variant
    shape = _output_shape(x, qweight, (int(kernel_d), int(kernel_h), int(kernel_w)),
                          (int(stride_d), int(stride_h), int(stride_w)))
    return torch.empty(shape, device=x.device, dtype=x.dtype, memory_format=torch.channels_last_3d)


@torch.library.custom_op("h3vae_encoder::int8_norm_conv3d", mutates_args=(), device_types="cuda")
def int8_norm_conv3d(x: torch.Tensor, norm_weight: torch.Tensor, norm_bias: torch.Tensor,
                     pre_bias: torch.Tensor | None, eps: float, qweight: torch.Tensor, weight_scale: torch.Tensor,
                     bias: torch.Tensor | None) -> torch.Tensor:
    """GroupNorm/SiLU/padding/quantization then the causal-skipping INT8 conv."""
    from .encoder_int8_norm import quantized_temporal_norm_pad

    qx, scale = quantized_temporal_norm_pad(x, norm_weight, norm_bias, eps, pre_bias=pre_bias)
    return _conv3d_from_quantized(qx, scale, qweight, weight_scale,
                                  config=Int8Conv3DConfig(x.shape[1], qweight.shape[0], (3, 3, 3), (1, 1, 1)),
                                  bias=bias, tile_variant="128x128x64_pipeline4",
                                  # the producer writes exactly two causal zero planes
                                  causal_prefix_zero=True)


@int8_norm_conv3d.register_fake
def _int8_norm_conv3d_fake(x, norm_weight, norm_bias, pre_bias, eps, qweight, weight_scale, bias):
    return torch.empty((x.shape[0], qweight.shape[0], *x.shape[2:]), device=x.device, dtype=x.dtype,
                       memory_format=torch.channels_last_3d)


@torch.library.custom_op("h3vae_encoder::int8_norm_conv3d_residual", mutates_args=(), device_types="cuda")
def int8_norm_conv3d_residual(x: torch.Tensor, norm_weight: torch.Tensor, norm_bias: torch.Tensor,
                              pre_bias: torch.Tensor | None, eps: float, qweight: torch.Tensor,
                              weight_scale: torch.Tensor, bias: torch.Tensor | None,
                              residual: torch.Tensor) -> torch.Tensor:
    """``residual + int8_norm_conv3d(...)`` in one conv launch: the residual block's closing add
    (opt/encoder_fused_norm_bias.py:141) fused into the conv epilogue, bit-identical to the add."""
    from .encoder_int8_norm import quantized_temporal_norm_pad

    qx, scale = quantized_temporal_norm_pad(x, norm_weight, norm_bias, eps, pre_bias=pre_bias)
    return _conv3d_from_quantized(qx, scale, qweight, weight_scale,
                                  config=Int8Conv3DConfig(x.shape[1], qweight.shape[0], (3, 3, 3), (1, 1, 1)),
                                  bias=bias, tile_variant="128x128x64_pipeline4", causal_prefix_zero=True,
                                  residual=residual)


@int8_norm_conv3d_residual.register_fake
def _int8_norm_conv3d_residual_fake(x, norm_weight, norm_bias, pre_bias, eps, qweight, weight_scale, bias, residual):
    return torch.empty((x.shape[0], qweight.shape[0], *x.shape[2:]), device=x.device, dtype=x.dtype,
                       memory_format=torch.channels_last_3d)


@torch.library.custom_op("h3vae_encoder::int8_norm_conv3d_residual_padded", mutates_args=("x_partials",),
                  device_types="cuda")
def int8_norm_conv3d_residual_padded(x: torch.Tensor, norm_weight: torch.Tensor, norm_bias: torch.Tensor,
                                     pre_bias: torch.Tensor | None, eps: float, qweight: torch.Tensor,
                                     weight_scale: torch.Tensor, bias: torch.Tensor | None,
                                     residual: torch.Tensor | None, residual_bias: torch.Tensor | None,
                                     front: int, border: list[int],
                                     x_partials: torch.Tensor | None, x_chunk: int) -> torch.Tensor:
    """The last conv of an encoder stage written as the padded input of the stage's causal stride-2
    downsample: ``[B, Cout, D + front, H + top + bottom, W + left + right]``, zero leading frames, a reflect
    border (top, bottom, left, right) of 0 or 1 per side.  The
    residual add is that of ``int8_norm_conv3d_residual``, or with ``residual_bias`` the stage-1 residual
    pack's ``residual + (out + bias)`` (opt/encoder_fused_residual_pack.py:12-33); the pack kernel that
    would re-read the conv output (there, or ``causal_reflect_pack`` before the stage-0 downsample) is
    not run.  ``x_partials``, ``x_chunk``: GroupNorm statistics of ``x`` as in ``int8_norm_conv3d_tiles``."""
    from .encoder_int8 import _conv3d_from_quantized_padded
    from .encoder_int8_norm import GnPartials, quantized_temporal_norm_pad

    partials = None if x_partials is None else GnPartials(x_partials, int(x_chunk))
    qx, scale = quantized_temporal_norm_pad(x, norm_weight, norm_bias, eps, pre_bias=pre_bias, partials=partials)
    return _conv3d_from_quantized_padded(qx, scale, qweight, weight_scale, bias=bias, residual=residual,
                                         residual_bias=residual_bias, front=int(front), border=border)


@int8_norm_conv3d_residual_padded.register_fake
def _int8_norm_conv3d_residual_padded_fake(x, norm_weight, norm_bias, pre_bias, eps, qweight, weight_scale, bias,
                                           residual, residual_bias, front, border, x_partials, x_chunk):
    b, _, d, h, w = x.shape
    top, bottom, left, right = border
    return torch.empty((b, qweight.shape[0], d + int(front), h + top + bottom, w + left + right), device=x.device,
                       dtype=x.dtype, memory_format=torch.channels_last_3d)


@torch.library.custom_op("h3vae_encoder::int8_norm_conv3d_tiles", mutates_args=("x_partials",), device_types="cuda")
def int8_norm_conv3d_tiles(x: torch.Tensor, norm_weight: torch.Tensor, norm_bias: torch.Tensor,
                           pre_bias: torch.Tensor | None, eps: float, qweight: torch.Tensor,
                           weight_scale: torch.Tensor, bias: torch.Tensor | None, residual: torch.Tensor | None,
                           x_partials: torch.Tensor | None, x_chunk: int, emit: bool,
                           partials_bias: torch.Tensor | None) -> tuple[torch.Tensor, torch.Tensor]:
    """``int8_norm_conv3d`` (or ``_residual``) with GroupNorm statistics on either side: the producer reads
    those of ``x`` from ``x_partials`` (written by the conv that produced ``x`` over ``x_chunk``-pixel chunks,
    with ``pre_bias`` as its statistics bias; the workspace is reused by the producer) instead of its own
    statistics pass, and with ``emit`` the conv writes those of its output's 512-pixel tiles plus
    ``partials_bias`` into the returned workspace (``gn_stats_fits`` geometry; without ``emit`` the second
    output is empty)."""
    from .encoder_int8 import gn_workspace_floats
    from .encoder_int8_norm import GnPartials, quantized_temporal_norm_pad

    partials = None if x_partials is None else GnPartials(x_partials, int(x_chunk))
    qx, scale = quantized_temporal_norm_pad(x, norm_weight, norm_bias, eps, pre_bias=pre_bias, partials=partials)
    ws = None
    if emit:
        ws = torch.empty((gn_workspace_floats(*x.shape[2:]),), device=x.device, dtype=torch.float32)
    out = _conv3d_from_quantized(qx, scale, qweight, weight_scale,
                                 config=Int8Conv3DConfig(x.shape[1], qweight.shape[0], (3, 3, 3), (1, 1, 1)),
                                 bias=bias, tile_variant="128x128x64_pipeline4", causal_prefix_zero=True,
                                 residual=residual, gn_workspace=ws, gn_bias=partials_bias if emit else None)
    return out, (ws if ws is not None else x.new_empty((0,), dtype=torch.float32))


@int8_norm_conv3d_tiles.register_fake
def _int8_norm_conv3d_tiles_fake(x, norm_weight, norm_bias, pre_bias, eps, qweight, weight_scale, bias, residual,
                                 x_partials, x_chunk, emit, partials_bias):
    out = torch.empty((x.shape[0], qweight.shape[0], *x.shape[2:]), device=x.device, dtype=x.dtype,
                      memory_format=torch.channels_last_3d)
    return out, x.new_empty((0,), dtype=torch.float32)


class Int8FusedValidConv3d(nn.Module):
    """Static-weight INT8 wrapper for an already-padded fused Conv3d call."""

    def __init__(self, source: nn.Module, *, apply_bias: bool, tile_variant: str = "128x64x64") -> None:
        super().__init__()
        source_weight = getattr(source, "weight", None)
        source_bias = getattr(source, "bias", None)
        if not isinstance(source_weight, torch.Tensor) or source_weight.ndim != 5:
            raise ValueError("INT8 encoder source must expose a rank-5 weight")
        if source_bias is None or not isinstance(source_bias, torch.Tensor):
            raise ValueError("INT8 encoder integration requires a source bias")
        if source_bias.ndim != 1 or source_bias.shape[0] != source_weight.shape[0]:
            raise ValueError("source bias must match the convolution output channels")
        if source_bias.device != source_weight.device:
            raise ValueError("source weight and bias must share a device")
        if source_weight.dtype != torch.float16:
            raise ValueError("INT8 encoder integration requires FP16 source weights")
        if source_bias.dtype != torch.float16:
            raise ValueError("INT8 encoder integration requires an FP16 source bias")
        if not bool(torch.isfinite(source_bias.detach()).all().item()):
            raise ValueError("source bias contains non-finite values")
        stride = tuple(int(value) for value in getattr(source, "stride", (1, 1, 1)))
        if tuple(source_weight.shape[-3:]) != (3, 3, 3):
            raise ValueError("the initial INT8 encoder policy only supports 3x3x3")
        qweight, weight_scale, config = prepare_int8_weight(source_weight, stride=stride)
        # A non-trainable Parameter so ComfyUI's ModelPatcher moves it on offload/reload.
        self.qweight = nn.Parameter(qweight.contiguous(), requires_grad=False)
        self.register_buffer("weight_scale", weight_scale.float().contiguous(), persistent=True)
        self.bias = nn.Parameter(source_bias.detach().clone().contiguous(), requires_grad=False)
        self.config = config
        self.apply_bias = bool(apply_bias)
        self.tile_variant = str(tile_variant)
        self.fuse_norm = False

    def _apply(self, fn, recurse=True):
        # module.to(device, dtype) must keep INT8 weights, FP32 scales and the FP16 bias bit for bit.
        # The reference (opt/encoder_int8_integration.py:268-282) keeps a copy of the scale only; its
        # bias goes through the requested dtype and back, which rounds it on a bf16 move.
        original_scale = self.weight_scale.detach().clone()
        original_bias = self.bias.detach().clone()
        result = super()._apply(fn, recurse=recurse)
        self.qweight.data = self.qweight.data.to(device=self.qweight.device, dtype=torch.int8)
        self.weight_scale.data = original_scale.to(device=self.weight_scale.device, dtype=torch.float32)
        self.bias.data = original_bias.to(device=self.bias.device, dtype=torch.float16)
        return result

    def forward_norm(self, x, norm_weight, norm_bias, eps, pre_bias=None, residual=None, residual_bias=None,
                     pad_front=None, pad_border=None, x_partials=None, emit_partials=False, partials_bias=None):
        """Fused producer + conv; ``residual`` adds the block's closing residual in the conv epilogue.
        ``pad_front`` and ``pad_border`` (with ``residual_bias`` optional) return the padded input of the
        stage's downsample instead (``int8_norm_conv3d_residual_padded``).

        GroupNorm statistics (``int8_norm_conv3d_tiles``): ``x_partials`` (``GnPartials``) holds those of ``x``,
        written by the conv that produced ``x`` with ``pre_bias`` as its statistics bias; with
        ``emit_partials`` the call returns ``(out, partials)``, ``partials`` the tile statistics of ``out``
        plus ``partials_bias`` for the norm that reads ``out``, or None where the conv's geometry has no
        statistics epilogue (``gn_stats_fits``)."""
        if not self.fuse_norm:
            raise RuntimeError("INT8 norm fusion is not enabled for this convolution")
        if x.dtype != torch.float16:
            raise RuntimeError("INT8 encoder convolution requires FP16 activations")
        if x.device != self.qweight.device:
            raise RuntimeError("INT8 encoder activation and qweight must be on the same device")
        bias = self.bias if self.apply_bias else None
        from .encoder_int8_norm import TILE_CHUNK, GnPartials
        x_ws, x_chunk = (None, TILE_CHUNK) if x_partials is None else x_partials
        if pad_front is not None:
            if emit_partials:
                raise ValueError("the padded form writes no tile statistics")
            return int8_norm_conv3d_residual_padded(x, norm_weight, norm_bias, pre_bias, eps, self.qweight,
                                                    self.weight_scale, bias, residual, residual_bias, int(pad_front),
                                                    [int(v) for v in pad_border], x_ws, int(x_chunk))
        if residual_bias is not None:
            raise ValueError("residual_bias is only taken with pad_front")
        if x_partials is not None or emit_partials:
            from .encoder_int8 import gn_stats_fits
            b, _, d, h, w = x.shape
            emit = bool(emit_partials) and gn_stats_fits(self.config.in_channels, self.config.out_channels, d, h, w,
                                                         batch=b)
            out, partials = int8_norm_conv3d_tiles(x, norm_weight, norm_bias, pre_bias, eps, self.qweight,
                                                   self.weight_scale, bias, residual, x_ws, int(x_chunk), emit,
                                                   partials_bias if emit else None)
            if not emit_partials:
                return out
            return out, (GnPartials(partials, TILE_CHUNK) if emit else None)
        if partials_bias is not None:
            raise ValueError("partials_bias is only taken with emit_partials")
        if residual is not None:
            return int8_norm_conv3d_residual(x, norm_weight, norm_bias, pre_bias, eps, self.qweight,
                                             self.weight_scale, bias, residual)
        return int8_norm_conv3d(x, norm_weight, norm_bias, pre_bias, eps, self.qweight, self.weight_scale, bias)

    def forward(self, x):
        if x.dtype != torch.float16:
            raise RuntimeError("INT8 encoder convolution requires FP16 activations")
        if x.device != self.qweight.device:
            raise RuntimeError("INT8 encoder activation and qweight must be on the same device")
        k, s = self.config.kernel_size, self.config.stride
        return int8_valid_conv3d_integration(x, self.qweight, self.weight_scale, self.bias, k[0], k[1], k[2], s[0],
                                             s[1], s[2], self.apply_bias, self.tile_variant)


def _check_encoder_platform(prefix: nn.Module) -> None:
    devices = {parameter.device for parameter in prefix.parameters()}
    if not devices:
        raise RuntimeError("int8_encode requires encoder prefix parameters")
    if any(device.type != "cuda" for device in devices):
        raise RuntimeError("int8_encode requires all encoder prefix parameters on the GPU; got "
                           + ", ".join(sorted(str(d) for d in devices)))
    if len(devices) != 1:
        raise RuntimeError("int8_encode requires all encoder prefix parameters on one GPU; got "
                           + ", ".join(sorted(str(d) for d in devices)))
    _hip.require_gfx950(next(iter(devices)), "int8_encode")


def install_int8_encoder_prefix(prefix: nn.Module, *, require_cuda: bool = True,
                                tile_variant: str | None = "auto") -> dict[str, Any]:
    """Install exactly the eight approved prefix residual convolutions (atomically)."""
    if require_cuda:
        _check_encoder_platform(prefix)
    stages = getattr(prefix, "stages", None)
    if not isinstance(stages, nn.ModuleList) or len(stages) < 2:
        raise ValueError("INT8 encoder prefix must expose at least two stages")
    pending, installed = [], []
    for stage_index in INT8_ENCODER_POLICY["stages"]:
        blocks = getattr(stages[stage_index], "block", None)
        if not isinstance(blocks, nn.ModuleList) or len(blocks) != 2:
            raise ValueError(f"INT8 encoder policy expected two blocks at stage {stage_index}")
        for block_index, block in enumerate(blocks):
            block_type = type(block).__name__
            if block_type not in {"BiasFusedResidualBlock", "ResidualDownsampleBlock"}:
                raise ValueError(f"stage {stage_index} block {block_index} has unsupported type {block_type}")
            is_residual_downsample = block_type == "ResidualDownsampleBlock"
            if stage_index == 1 and block_index == 1:
                if not is_residual_downsample or not hasattr(block, "down_weight"):
                    raise ValueError("stage 1 final block must be ResidualDownsampleBlock")
            elif is_residual_downsample:
                raise ValueError(f"unexpected ResidualDownsampleBlock at stage {stage_index} block {block_index}")
            for field in ("first", "second"):
                source = getattr(block, field, None)
                if source is None:
                    raise ValueError(f"stage {stage_index} block {block_index} lacks {field}")
                if getattr(block, f"int8_{field}", None) is not None:
                    raise ValueError(f"stage {stage_index} block {block_index} {field} already has an INT8 wrapper")
                # The last stage-1 block adds second.bias in its residual pack.
                apply_bias = not (field == "first" or (stage_index == 1 and block_index == 1 and field == "second"))
                device = source.weight.device
                selected = _resolve_tile_variant(int(source.weight.shape[1]), tile_variant,
                                                 _hip.is_gfx950(device) if device.type == "cuda" else False)
                wrapper = Int8FusedValidConv3d(source, apply_bias=apply_bias, tile_variant=selected)
                wrapper.fuse_norm = (tile_variant in (None, "auto") and selected == "128x128x64_pipeline4"
                                     and wrapper.config.stride == (1, 1, 1))
                pending.append((block, field, wrapper))
                installed.append({"path": f"stages.{stage_index}.block.{block_index}.{field}",
                                  "weight_shape": list(source.weight.shape),
                                  "input_channels": int(source.weight.shape[1]),
                                  "stride": list(wrapper.config.stride), "apply_bias": apply_bias,
                                  "tile_variant": selected, "fuse_norm": wrapper.fuse_norm})
    expected = int(INT8_ENCODER_POLICY["quantized_conv_count"])
    if len(installed) != expected:
        raise RuntimeError(f"INT8 encoder policy installed {len(installed)} convolutions, expected {expected}")
    for block, field, wrapper in pending:
        setattr(block, f"int8_{field}", wrapper)
    return {"enabled": True, "count": len(installed), "policy": dict(INT8_ENCODER_POLICY),
            "tile_variant": "stage-aware-input-channels",
            "tile_variants": sorted({item["tile_variant"] for item in installed}), "convolutions": installed}


__all__ = ["INT8_ENCODER_POLICY", "Int8FusedValidConv3d", "install_int8_encoder_prefix",
           "int8_norm_conv3d", "int8_valid_conv3d_integration"]
