"""Residual / norm1 / INT8-QKV fusion and the decoder block carry protocol.

Mirror of opt/int8_norm1_quant.py in fishelegs/ComfyUI-H3VAE-PyOpt.

* ``residual_qkv`` (:126-162) runs ``h3v_residual_norm1_quant`` in place on
  ``h`` (raw = fma(o, g, h); h <- fp16(raw); the published W16 reduction tree
  for sum(raw^2); n = fp16((h * inv) * w); row quantization) followed by the
  INT8 QKV GEMM ``h3v_gemm_i8_dequant``.
* ``_Norm1QuantBlock`` (:185-269) passes the residual between blocks as a
  carry ``(h, out, scale2)`` instead of materialising ``h + out * scale2``:
  block 0 normalises with ``rms_fp16_x2_w16``; blocks 1.. fold the previous
  block's residual into their norm1 producer; the last block hands the carry
  to the final LayerNorm (``_FinalNormAdapter`` -> ``residual_ln_w8``).

The reference gates the fused path to its validated SM120 B4 shape
``[4, 1797, 2048]`` and a 36-block stack.  Here the kernels take any row
count and widths 1024/2048/4096, so the gate is: contiguous FP16
``[B, N, D]`` rows with D the decoder width, on an MI355X (gfx950) device.
"""
from __future__ import annotations

import torch
from torch import nn

from .. import _hip
from . import decoder_block0_norm as _BLOCK0_HELPER
from . import decoder_final_norm as _FINAL_HELPER
from ._checks import ROW_WIDTHS
from .int8_swiglu_fused import prequantized_linear

_EPS = 1.0e-5
_FFN_WARPS = 8

block0_rms_fp16 = _BLOCK0_HELPER.rms_fp16_x2_w16


def supports_norm1_quant(device):
    """The fused producer runs on MI355X (gfx950) only."""
    return _hip.is_gfx950(device)


def produce_norm1(h, o, g, w, eps=_EPS):
    """In-place h producer -> (q int8 [M, K], s fp32 [M, 1])."""
    k = h.shape[-1]
    m = h.numel() // k
    q = torch.empty((m, k), device=h.device, dtype=torch.int8)
    scale = torch.empty((m, 1), device=h.device, dtype=torch.float32)
    _hip.call("h3v_residual_norm1_quant", _hip.ptr(h), _hip.ptr(o), _hip.ptr(g), _hip.ptr(w), float(eps), m, k,
              _hip.ptr(h), _hip.ptr(q), _hip.ptr(scale), _hip.stream(h.device))
    return q, scale


def residual_qkv_impl(h, o, g, w, qw, ws, bias):
    """In-place H producer followed by the INT8 QKV GEMM."""
    k = h.shape[-1] if h.ndim else 0
    tensors = (h, o, g, w, qw, ws) + (() if bias is None else (bias,))
    if (h.ndim < 2 or k not in ROW_WIDTHS or h.numel() == 0 or o.shape != h.shape or g.shape != (k,)
            or w.shape != (k,) or qw.ndim != 2 or qw.shape[1] != k or ws.shape != (qw.shape[0],)
            or h.dtype != torch.float16 or o.dtype != torch.float16 or g.dtype != torch.float16
            or w.dtype != torch.float16 or qw.dtype != torch.int8 or ws.dtype != torch.float32
            or any(t.device != h.device or not t.is_contiguous() for t in tensors)
            or (bias is not None and (bias.shape != (qw.shape[0],) or bias.dtype != torch.float16))):
        raise ValueError(f"expected contiguous [..., K] FP16 inputs (K in {ROW_WIDTHS}) and INT8 QKV [N, K]")
    if torch.is_grad_enabled():
        raise RuntimeError("norm1 fusion requires inference/no_grad")
    _hip.require_gfx950(h.device, "norm1 fusion")
    if h.data_ptr() == o.data_ptr():
        raise ValueError("residual H and FFN output must have distinct storage")
    q, scale = produce_norm1(h, o, g, w)
    return prequantized_linear(q, scale, qw, ws, bias).reshape(*h.shape[:-1], qw.shape[0])


@torch.library.custom_op("h3vae_norm1::residual_qkv", mutates_args=("h",))
def residual_qkv(h: torch.Tensor, o: torch.Tensor, g: torch.Tensor, w: torch.Tensor, qw: torch.Tensor,
                 ws: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
    return residual_qkv_impl(h, o, g, w, qw, ws, bias)


@residual_qkv.register_fake
def _fake_residual_qkv(h, o, g, w, qw, ws, bias):
    del o, g, w, ws, bias
    return h.new_empty((*h.shape[:-1], qw.shape[0]))


class _FinalNormAdapter(nn.Module):
    """Final LayerNorm that also accepts the last block's carry (reference :31-46)."""

    def __init__(self, original):
        super().__init__()
        self.weight, self.bias = original.weight, original.bias
        self.normalized_shape, self.eps = original.normalized_shape, original.eps
        self.train(original.training)

    def forward(self, states):
        if isinstance(states, tuple):
            if self.training or torch.is_grad_enabled():
                raise RuntimeError("eval + inference/no_grad required")
            h, out, gate = states
            return _FINAL_HELPER.final_residual_ln_w8(h, out, gate, self.weight, self.bias)
        return torch.nn.functional.layer_norm(states, self.normalized_shape, self.weight, self.bias, self.eps)


def _carry_safe_unpad(original_unpad):
    """A carry tuple only passes a zero-length unpad, unchanged (reference :49-60)."""
    def unpad(states, pad_len):
        if isinstance(states, tuple):
            if pad_len != 0:
                raise RuntimeError("final residual carry requires zero sequence padding")
            unpadded = original_unpad(states, pad_len)
            if unpadded is not states:
                raise RuntimeError("zero unpadding must preserve final residual carry")
            return unpadded
        return original_unpad(states, pad_len)
    return unpad


def _qk_rope_for(attn):
    """The fused QK-norm/RoPE op of a FusedQKAttention module (reference :165-174)."""
    from . import decoder_fused_qk_rope as fused
    if type(attn) is not fused.FusedQKAttention:
        raise ValueError("expected the runtime FusedQKAttention class")
    return fused.qk_rope


def _attention_from_qkv(attn, qkv, rotary, pack_info, qk_rope):
    a = attn.original
    b, n, _ = qkv.shape
    q, k = qk_rope(qkv, *rotary, a.heads, a.norm_q.eps, attn.rows)
    v = qkv.view(b, n, a.heads, 3 * a.dim_head)[..., 2 * a.dim_head:]
    y = a.perform_attention(q, k, v, pack_info)
    return a.to_out(y.reshape(b, n, -1))


class _Norm1QuantBlock(nn.Module):
    """Decoder block speaking the (h, out, scale2) carry protocol (reference :185-269)."""

    def __init__(self, src, first, last, norm1_enabled):
        super().__init__()
        self.norm1, self.norm2, self.attn, self.ff = src.norm1, src.norm2, src.attn, src.ff
        self.scale1, self.scale2 = src.scale1, src.scale2
        self.warps, self.fuse_ffn_up = src.warps, src.fuse_ffn_up
        self.norm1_enabled = bool(norm1_enabled)
        self.fuse_norm1 = self.norm1_enabled and supports_norm1_quant(self.scale1.device)
        self.qk_rope = _qk_rope_for(self.attn)
        self.first, self.last = first, last
        self.train(src.training)

    def _apply(self, fn, recurse=True):
        from .int8_ffn_up_fused import supports_fused_ffn_up
        out = super()._apply(fn, recurse=recurse)
        self.fuse_ffn_up = supports_fused_ffn_up(self.scale1.device)
        self.fuse_norm1 = self.norm1_enabled and supports_norm1_quant(self.scale1.device)
        return out

    def _ffn_pair(self, h, attn):
        from .int8_ffn_up_fused import fused_residual_ffn
        from .int8_norm_quant import residual_rms_linear
        from .int8_swiglu_fused import swiglu_int8_linear
        w1, w2 = self.ff.w1, self.ff.w2
        if self.fuse_ffn_up:
            return fused_residual_ffn(h, attn, self.scale1, self.norm2.weight, w1.qweight, w1.weight_scale, w1.bias,
                                      w2.qweight, w2.weight_scale, w2.bias, self.norm2.eps, self.warps)
        h, hidden = residual_rms_linear(h, attn, self.scale1, self.norm2.weight, w1.qweight, w1.weight_scale,
                                        w1.bias, self.norm2.eps, self.warps)
        out = swiglu_int8_linear(hidden, w2.qweight, w2.weight_scale, w2.bias, 16)
        return h, out

    def _target_shape(self, h):
        return (self.fuse_norm1 and h.ndim == 3 and h.shape[-1] == self.scale1.shape[0] and h.numel() > 0
                and h.dtype == torch.float16 and h.is_cuda and h.is_contiguous())

    def forward(self, states, rotary_pos_emb=None, pack_info=None):
        if self.training or torch.is_grad_enabled():
            raise RuntimeError("eval + inference/no_grad required")
        pack_info = {} if pack_info is None else pack_info
        chain = False
        if isinstance(states, tuple):
            h, prev_out, prev_scale2 = states
            can_fuse = (not self.first and self._target_shape(h) and prev_out.shape == h.shape
                        and prev_out.dtype == torch.float16 and prev_out.is_contiguous()
                        and rotary_pos_emb is not None)
            if can_fuse:
                linear = self.attn.original.to_qkv
                qkv = residual_qkv(h, prev_out, prev_scale2, self.norm1.weight, linear.qweight, linear.weight_scale,
                                   linear.bias)
                attn = _attention_from_qkv(self.attn, qkv, rotary_pos_emb, pack_info, self.qk_rope)
                states, chain = h, True
            else:
                states = h + prev_out * prev_scale2
                normed = self.norm1(states.float()).to(states.dtype)
                attn = self.attn(normed, rotary_pos_emb, pack_info)
        else:
            if self.first and self._target_shape(states):
                normed = block0_rms_fp16(states, self.norm1.weight)
            else:
                normed = self.norm1(states.float()).to(states.dtype)
            attn = self.attn(normed, rotary_pos_emb, pack_info)
            chain = self._target_shape(states) and rotary_pos_emb is not None

        h, out = self._ffn_pair(states, attn)
        if self.last:
            if self._target_shape(h):
                return h, out, self.scale2
            return h + out * self.scale2
        return (h, out, self.scale2) if chain else h + out * self.scale2


def _validate_blocks(blocks):
    """Every block must already be the INT8 norm2/FFN block with INT8 QKV/out (reference :272-299)."""
    from .kitchen_int8 import KitchenInt8Linear
    if not blocks:
        raise ValueError("norm1 fusion expects at least one decoder block")
    width = blocks[0].scale1.shape[0] if blocks[0].scale1.ndim == 1 else -1
    if width not in ROW_WIDTHS:
        raise ValueError(f"norm1 fusion requires decoder width in {ROW_WIDTHS}")
    for block in blocks:
        if (block.training or block.warps != _FFN_WARPS or not isinstance(block.norm1, nn.RMSNorm)
                or not isinstance(block.norm2, nn.RMSNorm) or block.norm1.normalized_shape != (width,)
                or block.norm2.normalized_shape != (width,) or block.norm1.weight is None
                or block.norm2.weight is None or block.norm1.eps != _EPS or block.norm2.eps != _EPS
                or block.scale1.shape != (width,) or block.scale2.shape != (width,)
                or block.scale1.dtype != torch.float16 or block.scale2.dtype != torch.float16
                or block.norm1.weight.dtype != torch.float16 or block.norm2.weight.dtype != torch.float16):
            raise ValueError("norm1 fusion requires the validated FP16 block contract of one decoder width")
        _qk_rope_for(block.attn)
        a = block.attn.original
        if (not isinstance(a.to_qkv, KitchenInt8Linear) or not isinstance(a.to_out, KitchenInt8Linear)
                or not isinstance(block.ff.w1, KitchenInt8Linear) or not isinstance(block.ff.w2, KitchenInt8Linear)
                or a.to_qkv.qweight.shape != (3 * width, width) or a.to_qkv.weight_scale.shape != (3 * width,)):
            raise ValueError("expected an already-quantized INT8 decoder; refusing requantization")
    return width


def clone_norm1_quant_decoder(raw, *, enabled=False):
    """Clone an already-INT8 decoder with the carry protocol (reference :302-343)."""
    from .int8_attention_out import clone_containers
    if raw.training:
        raise ValueError("eval decoder required")
    blocks = getattr(raw, "transformer_blocks", None)
    if blocks is None or len(blocks) == 0:
        raise ValueError("expected a decoder with transformer_blocks")
    result = clone_containers(raw)
    try:
        device = next(raw.parameters()).device
    except StopIteration as exc:
        raise ValueError("decoder has no parameters") from exc
    if not enabled:
        result._h3vae_norm1_quant_enabled = False
        return result.eval()
    if not supports_norm1_quant(device):
        raise RuntimeError("norm1 fusion requires an AMD MI355X (gfx950) GPU")
    _hip.lib()

    # A carry tuple cannot pass a sequence-parallel gather or a nonzero unpad.
    if getattr(raw, "spatial_parallel", True):
        raise RuntimeError("authored final LayerNorm requires spatial_parallel=false")
    width = _validate_blocks(list(result.transformer_blocks))
    norm = getattr(raw, "norm_out", None)
    if (type(norm) is not nn.LayerNorm or getattr(norm.forward, "__func__", None) is not nn.LayerNorm.forward
            or norm.normalized_shape != (width,) or norm.eps != _EPS or norm.weight is None or norm.bias is None
            or norm.weight.dtype != torch.float16 or norm.bias.dtype != torch.float16):
        raise ValueError("final LayerNorm requires affine FP16 decoder-width/eps-1e-5")

    blocks = list(result.transformer_blocks)
    result.transformer_blocks = nn.ModuleList([
        _Norm1QuantBlock(block, i == 0, i == len(blocks) - 1, norm1_enabled=True).eval()
        for i, block in enumerate(blocks)
    ])
    result.norm_out = _FinalNormAdapter(result.norm_out).eval()
    result._unpad_for_sp = _carry_safe_unpad(result._unpad_for_sp)
    result._h3vae_norm1_quant_enabled = True
    return result.eval()
