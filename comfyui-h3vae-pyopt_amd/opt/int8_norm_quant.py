"""The norm2 producer: residual + fp32 RMS statistics + INT8 row quantization, and its linear op.

Counterpart of opt/int8_norm_quant.py in fishelegs/ComfyUI-H3VAE-PyOpt.  Its
Triton ``kernel`` / ``residual_quant`` (:16-69) is ``h3v_residual_rms_quant``:
raw = fma(a, g, x); h = fp16(raw); inv = 1/sqrt(sum(raw^2)/K + eps) over a fixed
reduction tree; act = fp16(h * inv * w); the comfy-kitchen row quantizer on
act.  ``h3vae_norm_exp::residual_rms_linear`` feeds those rows to the INT8
GEMM.  Row widths 1024, 2048 and 4096 (H3 uses 2048, the synthetic benchmark
shapes 1024).  ``clone_norm_quant_decoder`` (reference :87-136) builds
``decoder_int8.Int8Block`` blocks.
"""
from __future__ import annotations

import os

import torch

from .. import _hip
from ._checks import ROW_WIDTHS
from .decoder_int8 import norm_ffn_decoder
from .int8_swiglu_fused import prequantized_linear


def validate(x, a, g, w, eps, warps):
    if x.ndim < 2 or x.shape[-1] not in ROW_WIDTHS or x.numel() == 0:
        raise ValueError(f"nonempty residual rows of width {ROW_WIDTHS} required")
    k = x.shape[-1]
    if a.shape != x.shape or tuple(g.shape) != (k,) or tuple(w.shape) != (k,):
        raise ValueError("residual/scale/RMS weight shape mismatch")
    if not all(t.dtype == torch.float16 and t.is_contiguous() and t.device == x.device for t in (x, a, g, w)):
        raise ValueError("contiguous FP16 tensors on the same device required")
    if not 0 < eps < 1 or warps not in (4, 8, 16):
        raise ValueError("invalid epsilon or warp count")


def residual_quant(x, a, g, w, eps, warps=8, round_stats=False):
    """-> (h fp16 like x, q int8 [M, K], s fp32 [M, 1]); ``warps`` is validated and otherwise unused."""
    validate(x, a, g, w, eps, warps)
    if round_stats:
        raise ValueError("round_stats=True is not part of the production norm2 contract")
    _hip.require_gfx950(x.device, "residual RMS quantization")
    k = x.shape[-1]
    m = x.numel() // k
    h = torch.empty_like(x)
    q = torch.empty((m, k), dtype=torch.int8, device=x.device)
    s = torch.empty((m, 1), dtype=torch.float32, device=x.device)
    _hip.call("h3v_residual_rms_quant", _hip.ptr(x), _hip.ptr(a), _hip.ptr(g), _hip.ptr(w), float(eps), m, k,
              _hip.ptr(h), _hip.ptr(q), _hip.ptr(s), _hip.stream(x.device))
    return h, q, s


@torch.library.custom_op("h3vae_norm_exp::residual_rms_linear", mutates_args=())
def residual_rms_linear(x: torch.Tensor, a: torch.Tensor, g: torch.Tensor, w: torch.Tensor, qw: torch.Tensor,
                        ws: torch.Tensor, bias: torch.Tensor | None, eps: float, warps: int
                        ) -> tuple[torch.Tensor, torch.Tensor]:
    h, q, s = residual_quant(x, a, g, w, eps, warps)
    return h, prequantized_linear(q, s, qw, ws, bias).view(*x.shape[:-1], qw.shape[0])


@residual_rms_linear.register_fake
def _fake(x, a, g, w, qw, ws, bias, eps, warps):
    return torch.empty_like(x), x.new_empty((*x.shape[:-1], qw.shape[0]))


def clone_norm_quant_decoder(raw, warps=8):
    """Copy of an INT8-FFN decoder with the fused norm2 / FFN chain in every block."""
    if os.environ.get("MINIMAX_H3_VAE_DECODER_VIT_FP32_NORM", "1").lower() not in ("1", "true", "yes", "on"):
        raise ValueError("experimental fusion requires FP32 norm enabled")
    if warps not in (4, 8, 16):
        raise ValueError("unsupported warp count")
    return norm_ffn_decoder(raw, warps)
