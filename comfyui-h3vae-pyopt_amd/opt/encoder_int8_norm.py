"""INT8 producer for the batch-one H3 encoder prefix.

Mirror of opt/encoder_int8_norm.py in fishelegs/ComfyUI-H3VAE-PyOpt
(``quantized_temporal_norm_pad``, :77-110).  One call of
``h3v_gn_norm_pack_i8`` runs per-frame GroupNorm(32) statistics, then two
recompute passes of norm / FP16 round / SiLU / FP16 round / causal + reflect
padding: the first finds the absmax, the second writes padded INT8 directly.
No full-sized FP16 intermediate is allocated.
"""
from __future__ import annotations

from typing import NamedTuple

import torch

from .. import _hip

# chunk sizes of the partial statistics a conv can hand to the producer (h3v_gn_norm_pack_i8_partials)
TILE_CHUNK = 512    # the INT8 window conv's 8-row x 64-column output tiles (h3v_conv3d_i8_gn)
PIXEL_CHUNK = 256   # 256-pixel runs of a frame in the producer's own order (h3v_conv3d_f16_gn)


class GnPartials(NamedTuple):
    """GroupNorm(32) partial statistics of a conv output, written by that conv into the producer workspace
    of the INT8 norm that reads the output next, and the chunk size they were formed over."""
    workspace: torch.Tensor
    chunk: int


def _validate(x, weight, bias, pre_bias):
    if x.ndim != 5 or x.device.type != "cuda":
        raise ValueError("INT8 norm producer requires a CUDA rank-5 input")
    b, c, d, h, w = x.shape
    if b != 1 or x.dtype != torch.float16 or c not in (128, 256) or d < 1 or min(h, w) < 2:
        raise ValueError("INT8 norm producer requires batch-one FP16 C=128/256, D>=1, H/W>=2")
    if c * (d + 2) * (h + 2) * (w + 2) >= 2**31:
        raise ValueError("Padded output exceeds int32 index range")
    for parameter in (weight, bias) + (() if pre_bias is None else (pre_bias,)):
        if (parameter is None or parameter.shape != (c,) or parameter.dtype != x.dtype
                or parameter.device != x.device or not parameter.is_contiguous()):
            raise ValueError("Expected contiguous FP16 channel vectors on input device")


def quantized_temporal_norm_pad(x, weight, bias, eps, *, pre_bias=None, return_stats=False, partials=None):
    """-> (q int8 [1, C, D+2, H+2, W+2] channels-last-3d, scale fp32 scalar).

    ``partials`` (``GnPartials``): the producer workspace that the conv which wrote ``x`` filled with the
    GroupNorm statistics of ``x`` (plus ``pre_bias``, which must be the bias that conv was given as its
    statistics bias), over 512-pixel window-conv tiles or 256-pixel runs; the statistics pass is then
    skipped (``h3v_gn_norm_pack_i8_partials``).  The workspace is reused for the rest of the call."""
    _validate(x, weight, bias, pre_bias)
    _hip.require_gfx950(x.device, "INT8 norm producer")
    _, c, d, h, w = x.shape
    x = x.contiguous(memory_format=torch.channels_last_3d)
    qy = torch.empty((1, c, d + 2, h + 2, w + 2), device=x.device, dtype=torch.int8,
                     memory_format=torch.channels_last_3d)
    scale = torch.empty((), device=x.device, dtype=torch.float32)
    stats = torch.empty((d, 32, 2), device=x.device, dtype=torch.float32)
    nws = int(_hip.lib().h3v_gn_norm_pack_workspace_floats(d, h, w))
    scratch = torch.empty((1,), device=x.device, dtype=torch.int32)
    tail = (_hip.ptr(qy), _hip.ptr(scale), _hip.ptr(stats))
    if partials is None:
        workspace = torch.empty((nws,), device=x.device, dtype=torch.float32)
        _hip.call("h3v_gn_norm_pack_i8", _hip.ptr(x), _hip.ptr(pre_bias), _hip.ptr(weight), _hip.ptr(bias),
                  float(eps), c, d, h, w, *tail, _hip.ptr(workspace), _hip.ptr(scratch), _hip.stream(x.device))
    else:
        workspace, chunk = partials
        if (workspace.dtype != torch.float32 or workspace.device != x.device or not workspace.is_contiguous()
                or workspace.numel() < nws):
            raise ValueError(f"partials must be a contiguous fp32 workspace of at least {nws} elements on x's device")
        if chunk == TILE_CHUNK and (h % 8 or w % 64):
            raise ValueError(f"tile statistics need H % 8 == 0 and W % 64 == 0 (got {h} x {w})")
        if chunk == PIXEL_CHUNK and (h * w) % PIXEL_CHUNK:
            raise ValueError(f"256-pixel statistics need H * W % 256 == 0 (got {h} x {w})")
        if chunk not in (TILE_CHUNK, PIXEL_CHUNK):
            raise ValueError(f"partials chunk must be {TILE_CHUNK} or {PIXEL_CHUNK} (got {chunk})")
        _hip.call("h3v_gn_norm_pack_i8_partials", _hip.ptr(x), _hip.ptr(pre_bias), _hip.ptr(weight), _hip.ptr(bias),
                  float(eps), c, d, h, w, int(chunk), *tail, _hip.ptr(workspace), _hip.ptr(scratch),
                  _hip.stream(x.device))
    if return_stats:
        return qy, scale, stats
    return qy, scale
