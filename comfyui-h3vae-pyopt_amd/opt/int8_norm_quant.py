"""Residual + FP32 RMS statistics + INT8 row quantization (the norm2 producer).

Mirror of opt/int8_norm_quant.py in fishelegs/ComfyUI-H3VAE-PyOpt.  The
Triton ``kernel`` (:22-43) becomes ``h3v_residual_rms_quant``:
raw = fma(a, g, x); h = fp16(raw); inv = 1/sqrt(sum(raw*raw)/K + eps) with a
fixed reduction tree; act = fp16(h * inv * w); row quantization of act.
Row width K in {1024, 2048, 4096} (the H3 decoder uses 2048, the synthetic
configuration 1024).
"""
from __future__ import annotations

import os

import torch
from torch import nn

from .. import _hip
from ._checks import ROW_WIDTHS
from .int8_ffn_up_fused import fused_residual_ffn, supports_fused_ffn_up
from .int8_swiglu_fused import clone_fused_decoder, prequantized_linear, swiglu_int8_linear


def validate(x, a, g, w, eps, warps):
    if x.ndim < 2 or x.shape[-1] not in ROW_WIDTHS or x.numel() == 0:
        raise ValueError(f"nonempty residual rows of width {ROW_WIDTHS} required")
    k = x.shape[-1]
    if a.shape != x.shape or g.shape != (k,) or w.shape != (k,):
        raise ValueError("residual/scale/RMS weight shape mismatch")
    if any(t.dtype != torch.float16 or not t.is_contiguous() or t.device != x.device for t in (x, a, g, w)):
        raise ValueError("contiguous FP16 tensors on the same device required")
    if not 0 < eps < 1 or warps not in (4, 8, 16):
        raise ValueError("invalid epsilon or warp count")


def residual_quant(x, a, g, w, eps, warps=8, round_stats=False):
    """-> (h fp16 like x, q int8 [M, K], s fp32 [M, 1]).  warps is accepted for API parity."""
    validate(x, a, g, w, eps, warps)
    if round_stats:
        raise ValueError("round_stats=True is not part of the production norm2 contract")
    _hip.require_gfx950(x.device, "residual RMS quantization")
    k = x.shape[-1]
    m = x.numel() // k
    h = torch.empty_like(x)
    q = torch.empty((m, k), device=x.device, dtype=torch.int8)
    s = torch.empty((m, 1), device=x.device, dtype=torch.float32)
    _hip.call("h3v_residual_rms_quant", _hip.ptr(x), _hip.ptr(a), _hip.ptr(g), _hip.ptr(w), float(eps), m, k,
              _hip.ptr(h), _hip.ptr(q), _hip.ptr(s), _hip.stream(x.device))
    return h, q, s


@torch.library.custom_op("h3vae_norm_exp::residual_rms_linear", mutates_args=())
def residual_rms_linear(x: torch.Tensor, a: torch.Tensor, g: torch.Tensor, w: torch.Tensor, qw: torch.Tensor,
                        ws: torch.Tensor, bias: torch.Tensor | None, eps: float, warps: int
                        ) -> tuple[torch.Tensor, torch.Tensor]:
    h, q, s = residual_quant(x, a, g, w, eps, warps)
    out = prequantized_linear(q, s, qw, ws, bias)
    return h, out.reshape(*x.shape[:-1], qw.shape[0])


@residual_rms_linear.register_fake
def _fake(x, a, g, w, qw, ws, bias, eps, warps):
    return torch.empty_like(x), x.new_empty((*x.shape[:-1], qw.shape[0]))


class NormQuantBlock(nn.Module):
    def __init__(self, block, warps=8):
        super().__init__()
        if not isinstance(block.norm2, nn.RMSNorm) or not block.use_scale:
            raise ValueError("scaled residual block with RMSNorm required")
        width = block.norm2.normalized_shape
        if len(width) != 1 or width[0] not in ROW_WIDTHS or block.norm2.weight is None:
            raise ValueError(f"affine RMSNorm of width {ROW_WIDTHS} required")
        self.norm1, self.norm2 = block.norm1, block.norm2
        self.attn, self.ff = block.attn, block.ff
        self.scale1, self.scale2 = block.scale1, block.scale2
        self.warps = warps
        self.fuse_ffn_up = supports_fused_ffn_up(self.scale1.device)
        self.train(block.training)

    def _apply(self, fn, recurse=True):
        result = super()._apply(fn, recurse=recurse)
        self.fuse_ffn_up = supports_fused_ffn_up(self.scale1.device)
        return result

    def forward(self, hidden_states, rotary_pos_emb=None, pack_info=None):
        if self.training or torch.is_grad_enabled():
            raise RuntimeError("eval + inference/no_grad required")
        if pack_info is None:
            pack_info = {}
        normed = self.norm1(hidden_states.float()).to(hidden_states.dtype)
        attn = self.attn(normed, rotary_pos_emb, pack_info)
        w1, w2 = self.ff.w1, self.ff.w2
        if self.fuse_ffn_up:
            h, out = fused_residual_ffn(hidden_states, attn, self.scale1, self.norm2.weight, w1.qweight,
                                        w1.weight_scale, w1.bias, w2.qweight, w2.weight_scale, w2.bias,
                                        self.norm2.eps, self.warps)
            return h + out * self.scale2
        h, hidden = residual_rms_linear(hidden_states, attn, self.scale1, self.norm2.weight, w1.qweight,
                                        w1.weight_scale, w1.bias, self.norm2.eps, self.warps)
        out = swiglu_int8_linear(hidden, w2.qweight, w2.weight_scale, w2.bias, 16)
        return h + out * self.scale2


def clone_norm_quant_decoder(raw, warps=8):
    if os.environ.get("MINIMAX_H3_VAE_DECODER_VIT_FP32_NORM", "1").lower() not in ("1", "true", "yes", "on"):
        raise ValueError("experimental fusion requires FP32 norm enabled")
    if warps not in (4, 8, 16):
        raise ValueError("unsupported warp count")
    result = clone_fused_decoder(raw, 16)
    result.transformer_blocks = nn.ModuleList([NormQuantBlock(block, warps).eval() for block in result.transformer_blocks])
    return result
