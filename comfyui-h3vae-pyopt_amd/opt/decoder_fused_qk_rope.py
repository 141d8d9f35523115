"""Fused QK RMSNorm + partial rotate-half RoPE.

Mirror of opt/decoder_fused_qk_rope.py in fishelegs/ComfyUI-H3VAE-PyOpt.
``_qk_rope`` (:12-35) becomes ``h3v_qk_rope``: per (token, head) the q and k
rows (64 dims) are RMS-normalised in FP32 without affine and rounded to FP16,
then the first 48 dims get rotate-half RoPE with FP16-rounded products summed
in FP32; dims 48..63 pass through.

The attention between the fused QK-RoPE and the output projection, which the
reference hands to the model's ``perform_attention`` (:66-74), runs as
``h3v_attention_d64`` (``attention_d64`` below): q and k straight from the
QK-RoPE outputs and v as the strided slice of the QKV projection, no copies.
The kernel computes unmasked attention over each (batch, head).  A call that
carries a non-empty ``pack_info`` (the model code's packed-sequence metadata,
whose layout the reference leaves to the external model) or no rotary table
raises ``ValueError`` rather than running a different path; a wrapper built
with ``native_attention=False`` keeps the model's ``perform_attention`` for
every call, as the reference does.
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


def _check_attention(q, k, v):
    if not (q.ndim == 4 and q.shape == k.shape == v.shape and q.shape[-1] == 64):
        raise ValueError("attention_d64 requires q, k, v of one shape [B, N, H, 64]")
    if not (q.dtype == k.dtype == v.dtype == torch.float16) or not (q.device == k.device == v.device):
        raise ValueError("attention_d64 requires FP16 q, k, v on one device")
    b, n, h, _ = q.shape
    if b == 0 or n == 0 or h == 0:
        raise ValueError("attention_d64 requires a nonempty input")
    for t in (q, k, v):
        st = t.stride()
        if st[3] != 1 or st[1] % 8 or st[2] % 8 or st[1] <= 0 or st[2] <= 0 or (b > 1 and st[0] != n * st[1]):
            raise ValueError("attention_d64 requires contiguous head dims, token/head strides that are multiples of 8 "
                             "and the batch stride tokens * token stride")
        if t.data_ptr() % 16:
            raise ValueError("attention_d64 requires 16-byte aligned q, k, v")


@torch.library.custom_op("h3vae_decoder::attention_d64", mutates_args=(), device_types="cuda")
def attention_d64(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float) -> torch.Tensor:
    """softmax(scale * q k^T) v per (batch, head): q, k, v [B, N, H, 64] fp16 (strided) -> [B, N, H, 64]."""
    _check_attention(q, k, v)
    if not (0.0 < scale < 1e30):
        raise ValueError("attention_d64 requires a positive finite scale")
    _hip.require_gfx950(q.device, "attention_d64")
    b, n, h, d = q.shape
    o = torch.empty((b, n, h, d), device=q.device, dtype=q.dtype)
    _hip.call("h3v_attention_d64", _hip.ptr(q), q.stride(1), q.stride(2), _hip.ptr(k), k.stride(1), k.stride(2),
              _hip.ptr(v), v.stride(1), v.stride(2), _hip.ptr(o), o.stride(1), o.stride(2), b, n, h, float(scale),
              _hip.stream(q.device))
    return o


@attention_d64.register_fake
def _fake_attention(q, k, v, scale):
    _check_attention(q, k, v)
    return q.new_empty(q.shape)


class FusedQKAttention(torch.nn.Module):
    """Attention wrapper: to_qkv -> fused QK norm/RoPE -> attention -> to_out."""

    def __init__(self, original, rows=8, native_attention=True):
        super().__init__()
        if (getattr(original, "spatial_parallel", False) or not isinstance(original.norm_q, torch.nn.RMSNorm)
                or not isinstance(original.norm_k, torch.nn.RMSNorm)):
            raise ValueError("single-device RMSNorm attention required")
        if (original.norm_q.weight is not None or original.norm_k.weight is not None or original.dim_head != 64
                or original.norm_q.eps != original.norm_k.eps):
            raise ValueError("expected head=64 and unaffined equal-eps QK norms")
        self.original = original
        self.rows = rows
        self.native_attention = bool(native_attention)

    def forward(self, x, rotary_pos_emb=None, pack_info=None):
        if rotary_pos_emb is None:
            if self.native_attention:
                raise ValueError("FusedQKAttention with native attention needs the rotary table (cos, sin); "
                                 "build it with native_attention=False to run the model's own attention")
            return self.original(x, rotary_pos_emb, pack_info or {})
        b, n, _ = x.shape
        a = self.original
        qkv = a.to_qkv(x)
        q, k = qk_rope(qkv, *rotary_pos_emb, a.heads, a.norm_q.eps, self.rows)
        v = qkv.view(b, n, a.heads, 3 * a.dim_head)[..., 2 * a.dim_head:]
        return a.to_out(run_attention(self, q, k, v, pack_info).reshape(b, n, -1))


def run_attention(wrapper, q, k, v, pack_info):
    """The attention of a FusedQKAttention ``wrapper`` on q, k, v [B, N, H, 64]: ``attention_d64`` (unmasked)
    when the wrapper is native, else the model's ``perform_attention``.  A native wrapper refuses a non-empty
    ``pack_info``: the kernel has no packed-sequence masking, and the call must not silently change path."""
    a = wrapper.original
    if not getattr(wrapper, "native_attention", False):
        return a.perform_attention(q, k, v, pack_info or {})
    if pack_info:
        raise ValueError("attention_d64 computes unmasked attention and cannot apply pack_info "
                         f"(keys {sorted(map(str, pack_info))}); build the decoder with "
                         "clone_with_qk_fusion(..., native_attention=False) to use the model's perform_attention")
    return attention_d64(q, k, v, a.dim_head ** -0.5)


def clone_with_qk_fusion(raw, rows=8, native_attention=True):
    """Copy the decoder's module containers with every attention wrapped in FusedQKAttention.

    Weights are shared read-only and the original decoder is left intact
    (reference opt/decoder_fused_qk_rope.py:76-89).  ``native_attention=False``
    keeps the model's ``perform_attention`` for every call (the reference's
    behaviour); the default runs ``attention_d64`` and refuses calls with a
    non-empty ``pack_info`` or without a rotary table.
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
        new.attn = FusedQKAttention(block.attn, rows, native_attention).eval()
        blocks.append(new)
    decoder.transformer_blocks = torch.nn.ModuleList(blocks)
    return decoder
