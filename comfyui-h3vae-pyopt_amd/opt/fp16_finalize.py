"""Exact-order FP32 pixel finalisation of the decoder output.

Mirror of opt/fp16_finalize.py in fishelegs/ComfyUI-H3VAE-PyOpt
(``validate`` :6-16, ``finalize_pixels`` :45-54): decoded ImageNet-normalised
pixels [B, 3, T, H, W] (fp16 or fp32, any strides) become contiguous fp32
pixels clamp(x * std[c] + mean[c], 0, 1), the multiply and the add rounded
separately (no FMA), NaN and an in-range -0 kept.  One HIP kernel
(``h3v_finalize_pixels``); the optional ``out`` is written in place.
"""
from __future__ import annotations

import ctypes

import torch

from .. import _hip


def validate(x, std, mean, out=None):
    if x.ndim != 5 or x.shape[1] != 3 or x.numel() == 0:
        raise ValueError("nonempty B,3,T,H,W tensor required")
    if x.dtype not in (torch.float16, torch.float32):
        raise ValueError("FP16 or FP32 decoded pixels required")
    for v in (std, mean):
        if v.numel() != 3 or v.dtype != torch.float32 or not v.is_contiguous() or v.device != x.device:
            raise ValueError("three contiguous FP32 channel constants on same device required")
    if out is not None and (out.shape != x.shape or out.dtype != torch.float32 or out.device != x.device
                            or not out.is_contiguous()):
        raise ValueError("contiguous FP32 output with matching shape/device required")


def finalize_pixels(x, std, mean, out=None):
    validate(x, std, mean, out)
    if not _hip.is_gfx950(x.device):
        raise ValueError("AMD MI355X (gfx950) GPU required")
    if torch.is_grad_enabled():
        raise RuntimeError("inference only")
    if out is None:
        out = torch.empty(x.shape, device=x.device, dtype=torch.float32)
    b, _, t, h, w = x.shape
    strides = (ctypes.c_int64 * 5)(*x.stride())
    _hip.call("h3v_finalize_pixels", _hip.ptr(x), int(x.dtype == torch.float16), b, t, h, w,
              ctypes.cast(strides, ctypes.c_void_p), _hip.ptr(std), _hip.ptr(mean), _hip.ptr(out),
              _hip.stream(x.device))
    return out
