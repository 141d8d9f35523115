"""Fused QK RMSNorm + partial rotate-half RoPE.

Mirror of opt/decoder_fused_qk_rope.py in fishelegs/ComfyUI-H3VAE-PyOpt.
``_qk_rope`` (:12-35) becomes ``h3v_qk_rope``: per (token, head) the q and k
rows (64 dims) are RMS-normalised in FP32 without affine and rounded to FP16,
then the first 48 dims get rotate-half RoPE with FP16-rounded products summed
in FP32; dims 48..63 pass through.
"""
from __future__ import annotations

import copy
import os

import torch

from .. import _hip


@torch.library.custom_op("h3vae_decoder::qk_rope", mutates_args=(), device_types="cuda")
def qk_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, heads: int, eps: float,
            rows: int) -> tuple[torch.Tensor, torch.Tensor]:
    """x [B, N, heads*3*64] -> q, k [B, N, heads, 64].  rows is accepted for API parity."""
    if rows not in (4, 8, 16, 32):
        raise ValueError("rows must be one of the tested configurations: 4, 8, 16, 32")
    b, n, _ = x.shape
    d = x.shape[-1] // (3 * heads)
    if not (x.is_contiguous() and cos.is_contiguous() and sin.is_contiguous()):
        raise ValueError("qk_rope requires contiguous inputs")
    if not (x.dtype == torch.float16 and cos.dtype == torch.float16 and sin.dtype == torch.float16):
        raise ValueError("qk_rope requires FP16 inputs")
    if d != 64 or x.shape[-1] != heads * 3 * d or cos.shape != (b, n, 1, 48) or sin.shape != cos.shape:
        raise ValueError("qk_rope requires head_dim 64 and cos/sin [B, N, 1, 48]")
    _hip.require_gfx950(x.device, "qk_rope")
    q = torch.empty((b, n, heads, d), device=x.device, dtype=x.dtype)
    k = torch.empty_like(q)
    _hip.call("h3v_qk_rope", _hip.ptr(x), _hip.ptr(cos), _hip.ptr(sin), b * n, heads, d, 48, float(eps),
              _hip.ptr(q), _hip.ptr(k), _hip.stream(x.device))
    return q, k


@qk_rope.register_fake
def _fake(x, cos, sin, heads, eps, rows):
    shape = (*x.shape[:2], heads, x.shape[-1] // (3 * heads))
    return x.new_empty(shape), x.new_empty(shape)


class FusedQKAttention(torch.nn.Module):
    """Attention wrapper: to_qkv -> fused QK norm/RoPE -> attention -> to_out."""

    def __init__(self, original, rows=8):
        super().__init__()
        if (getattr(original, "spatial_parallel", False) or not isinstance(original.norm_q, torch.nn.RMSNorm)
                or not isinstance(original.norm_k, torch.nn.RMSNorm)):
            raise ValueError("single-device RMSNorm attention required")
        if (original.norm_q.weight is not None or original.norm_k.weight is not None or original.dim_head != 64
                or original.norm_q.eps != original.norm_k.eps):
            raise ValueError("expected head=64 and unaffined equal-eps QK norms")
        self.original = original
        self.rows = rows

    def forward(self, x, rotary_pos_emb=None, pack_info=None):
        if rotary_pos_emb is None:
            return self.original(x, rotary_pos_emb, pack_info or {})
        b, n, _ = x.shape
        a = self.original
        qkv = a.to_qkv(x)
        q, k = qk_rope(qkv, *rotary_pos_emb, a.heads, a.norm_q.eps, self.rows)
        v = qkv.view(b, n, a.heads, 3 * a.dim_head)[..., 2 * a.dim_head:]
        y = a.perform_attention(q, k, v, pack_info or {})
        return a.to_out(y.reshape(b, n, -1))


def clone_with_qk_fusion(raw, rows=8):
    """Copy the decoder's module containers with every attention wrapped in FusedQKAttention.

    Weights are shared read-only and the original decoder is left intact
    (reference opt/decoder_fused_qk_rope.py:76-89).
    """
    if raw.training or os.environ.get("MINIMAX_H3_VAE_DECODER_VIT_FP32_NORM", "1").lower() in ("0", "false", "no",
                                                                                               "off"):
        raise ValueError("QK fusion requires eval inference with FP32 norm enabled")
    decoder = copy.copy(raw)
    decoder._modules = raw._modules.copy()
    blocks = []
    for block in raw.transformer_blocks:
        new = copy.copy(block)
        new._modules = block._modules.copy()
        new.attn = FusedQKAttention(block.attn, rows).eval()
        blocks.append(new)
    decoder.transformer_blocks = torch.nn.ModuleList(blocks)
    return decoder
