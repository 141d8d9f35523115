"""The INT8 decoder of the H3 VAE: one block type for every fused wiring the runtime offers.

The reference builds its fused INT8 decoder in layers, each cloning the previous
one: ``clone_norm_quant_decoder`` (opt/int8_norm_quant.py:87-136: the norm2
producer fused with the INT8 FFN), ``clone_qkv_int8_decoder`` /
``clone_attention_out_decoder`` (opt/int8_qkv.py:33-41,
opt/int8_attention_out.py:40-52: INT8 QKV and attention-out linears) and
``clone_norm1_quant_decoder`` (opt/int8_norm1_quant.py:185-343: the residual
carry between blocks).  Here one module, ``Int8Block``, covers all of them; the
wiring functions in those files build it.

``Int8Block`` runs, per call:

* norm1 + attention.  ``carry`` off: the model's fp32 RMSNorm, then the
  attention (fused QK-RMSNorm/RoPE, INT8 or model QKV / out linears).  ``carry``
  on and the previous block handed over ``(h, out, scale2)``: one
  ``h3vae_norm1::residual_qkv`` call folds ``h + out * scale2`` into the norm1
  producer (in place on ``h``) and runs the QKV GEMM; block 0 normalises with
  ``h3vae_norm1_block0::rms_fp16_x2_w16``.
* norm2 + FFN.  ``h3vae_int8_ffn::residual_ffn`` (residual + RMSNorm + row
  quant, FFN-up + SwiGLU + requant, FFN-down) on gfx950; elsewhere
  ``residual_rms_linear`` then ``swiglu_int8_linear``.
* the hand-over.  ``carry`` off: ``h + out * scale2``.  ``carry`` on: the
  tuple ``(h, out, scale2)``; the last block hands it to ``CarryLayerNorm``
  (``h3vae_final_ln::residual_ln_w8``) through the decoder's unpad hook, which
  lets a carry through only with zero padding.

A ``carry`` block runs only the fused kernels.  Rows the carry kernels cannot
take (not contiguous fp16 ``[B, N, width]`` on a gfx950 GPU, or no rotary
table), a plain tensor reaching a block after the first, or a carry reaching
block 0 raise ``ValueError``.  The reference drops to eager torch for those
calls (opt/int8_norm1_quant.py:218-252, non-B4 shapes); here the decode-fusion
mode never changes path silently.
"""
from __future__ import annotations

import torch
from torch import nn

from .. import _hip
from ._checks import ROW_WIDTHS
from ._modules import require_inference, share_containers
from .kitchen_int8 import KitchenInt8Linear

EPS = 1.0e-5
FFN_WARPS = 8


def attention_of(block):
    """The model attention inside a block (under its FusedQKAttention wrapper, if any)."""
    return getattr(block.attn, "original", block.attn)


def chosen_blocks(count, indices=None):
    """Block indices to convert: all by default; otherwise a nonempty list of distinct in-range ints."""
    picked = list(range(count)) if indices is None else list(indices)
    if not picked or len(set(picked)) != len(picked):
        raise ValueError("nonempty unique block indices required")
    for i in picked:
        if type(i) is not int or not 0 <= i < count:
            raise ValueError("block index out of range or not an integer")
    return picked


def source_linear(block, name, *, square):
    """The block attention's ``name`` projection, checked: nn.Linear, width in ROW_WIDTHS, eval mode,
    N = K (``square``) or N = 3K."""
    attention = attention_of(block)
    linear = getattr(attention, name, None)
    label = "output" if square else "QKV"
    if not isinstance(linear, nn.Linear):
        raise ValueError(f"expected original nn.Linear {label} projection")
    wanted = linear.in_features if square else 3 * linear.in_features
    if linear.in_features not in ROW_WIDTHS or linear.out_features != wanted:
        raise ValueError(f"{label} projection requires K in {ROW_WIDTHS} and N = {'K' if square else '3K'}")
    if linear.training:
        raise ValueError(f"{label} projection inference requires eval()")
    return attention, linear


def quantize_attention_linears(decoder, name, indices, *, square):
    """Replace ``name`` of the chosen blocks' attention in ``decoder`` by INT8 linears (in place)."""
    blocks = decoder.transformer_blocks
    picked = chosen_blocks(len(blocks), indices)
    sources = [source_linear(blocks[i], name, square=square) for i in picked]
    built = [KitchenInt8Linear(linear, require_cuda=True).eval() for _, linear in sources]
    for (attention, _), linear in zip(sources, built):
        setattr(attention, name, linear)
    return decoder


class Int8Block(nn.Module):
    """A decoder block with the fused INT8 norm2 / FFN chain, optionally speaking the residual carry."""

    def __init__(self, block, *, warps=FFN_WARPS, carry=False, first=False, last=False):
        super().__init__()
        self.norm1, self.norm2, self.attn, self.ff = block.norm1, block.norm2, block.attn, block.ff
        self.scale1, self.scale2 = block.scale1, block.scale2
        self.warps = warps
        self.carry, self.first, self.last = bool(carry), bool(first), bool(last)
        self._rope = None
        if self.carry:
            from .decoder_fused_qk_rope import FusedQKAttention, qk_rope
            if type(self.attn) is not FusedQKAttention:
                raise ValueError("expected the runtime FusedQKAttention class")
            self._rope = qk_rope
        self._platform()
        self.train(block.training)

    def _platform(self):
        native = _hip.is_gfx950(self.scale1.device)
        self.fuse_ffn_up = native
        self.fuse_norm1 = self.carry and native

    def _apply(self, fn, recurse=True):
        out = super()._apply(fn, recurse=recurse)
        self._platform()
        return out

    def _eligible(self, h):
        """Rows the fused carry kernels take."""
        return (self.fuse_norm1 and h.ndim == 3 and h.numel() > 0 and h.shape[-1] == self.scale1.shape[0]
                and h.dtype == torch.float16 and h.is_cuda and h.is_contiguous())

    def _model_norm1(self, h):
        return self.norm1(h.float()).to(h.dtype)

    def _attention_from_qkv(self, qkv, rotary, pack_info):
        from .decoder_fused_qk_rope import run_attention
        wrapper, a = self.attn, self.attn.original
        b, n, _ = qkv.shape
        q, k = self._rope(qkv, *rotary, a.heads, a.norm_q.eps, wrapper.rows)
        v = qkv.view(b, n, a.heads, 3 * a.dim_head)[..., 2 * a.dim_head:]
        return a.to_out(run_attention(wrapper, q, k, v, pack_info).reshape(b, n, -1))

    def _require_rows(self, h, rotary):
        """Refuse rows the carry kernels cannot take (no eager fallback in the decode-fusion mode)."""
        if not self._eligible(h):
            got = (f"{tuple(h.shape)} {h.dtype} on {h.device}, contiguous={h.is_contiguous()}"
                   if isinstance(h, torch.Tensor) else type(h).__name__)
            platform = "" if self.fuse_norm1 else " (the block's parameters are not on a gfx950 GPU)"
            raise ValueError(f"fused INT8 decoder block: the carry kernels take contiguous fp16 [B, N, "
                             f"{self.scale1.shape[0]}] rows on a gfx950 GPU{platform}; got {got}")
        if rotary is None:
            raise ValueError("fused INT8 decoder block: the carry path needs the rotary table (cos, sin)")

    def _enter(self, states, rotary, pack_info):
        """-> (residual stream, attention output)."""
        if isinstance(states, tuple):
            if not self.carry or self.first:
                raise ValueError("a residual carry (h, out, scale2) reached a block that does not take one "
                                 f"(carry={self.carry}, first={self.first})")
            h, prev_out, prev_scale2 = states
            self._require_rows(h, rotary)
            if not (isinstance(prev_out, torch.Tensor) and prev_out.shape == h.shape
                    and prev_out.dtype == torch.float16 and prev_out.is_contiguous()):
                raise ValueError("the carried block output must be contiguous fp16 of the residual's shape")
            from .int8_norm1_quant import residual_qkv
            lin = self.attn.original.to_qkv
            qkv = residual_qkv(h, prev_out, prev_scale2, self.norm1.weight, lin.qweight, lin.weight_scale, lin.bias)
            return h, self._attention_from_qkv(qkv, rotary, pack_info)
        if self.carry:
            if not self.first:
                raise ValueError("a fused INT8 decoder block after the first needs the previous block's residual "
                                 "carry (h, out, scale2), got a plain tensor")
            self._require_rows(states, rotary)
            from .decoder_block0_norm import rms_fp16_x2_w16
            return states, self.attn(rms_fp16_x2_w16(states, self.norm1.weight), rotary, pack_info)
        return states, self.attn(self._model_norm1(states), rotary, pack_info)

    def _ffn(self, h, attn):
        w1, w2 = self.ff.w1, self.ff.w2
        if self.fuse_ffn_up:
            from .int8_ffn_up_fused import fused_residual_ffn
            return fused_residual_ffn(h, attn, self.scale1, self.norm2.weight, w1.qweight, w1.weight_scale, w1.bias,
                                      w2.qweight, w2.weight_scale, w2.bias, self.norm2.eps, self.warps)
        from .int8_norm_quant import residual_rms_linear
        from .int8_swiglu_fused import swiglu_int8_linear
        h, hidden = residual_rms_linear(h, attn, self.scale1, self.norm2.weight, w1.qweight, w1.weight_scale,
                                        w1.bias, self.norm2.eps, self.warps)
        return h, swiglu_int8_linear(hidden, w2.qweight, w2.weight_scale, w2.bias, 16)

    def forward(self, states, rotary_pos_emb=None, pack_info=None):
        require_inference(self)
        pack_info = {} if pack_info is None else pack_info
        h, attn = self._enter(states, rotary_pos_emb, pack_info)
        h, out = self._ffn(h, attn)
        if self.carry:
            return h, out, self.scale2
        return h + out * self.scale2


class CarryLayerNorm(nn.Module):
    """The decoder's final LayerNorm, also taking the last block's carry (reference opt/int8_norm1_quant.py:31-46).

    In a carry decoder the last ``Int8Block`` always hands over the tuple (or has raised), so the tensor branch
    is the standalone adapter's contract only: the model's own LayerNorm of a plain tensor, as in the reference."""

    def __init__(self, original):
        super().__init__()
        self.weight, self.bias = original.weight, original.bias
        self.normalized_shape, self.eps = original.normalized_shape, original.eps
        self.train(original.training)

    def forward(self, states):
        if not isinstance(states, tuple):
            return nn.functional.layer_norm(states, self.normalized_shape, self.weight, self.bias, self.eps)
        require_inference(self)
        from .decoder_final_norm import final_residual_ln_w8
        h, out, gate = states
        return final_residual_ln_w8(h, out, gate, self.weight, self.bias)


def carry_unpad(unpad):
    """The decoder's sequence-parallel unpad hook, letting a carry tuple through only unchanged."""
    def hook(states, pad_len):
        if not isinstance(states, tuple):
            return unpad(states, pad_len)
        if pad_len != 0:
            raise RuntimeError("final residual carry requires zero sequence padding")
        if unpad(states, pad_len) is not states:
            raise RuntimeError("zero unpadding must preserve final residual carry")
        return states
    return hook


def norm_ffn_decoder(raw, warps=FFN_WARPS):
    """Copy of a decoder with INT8 FFNs whose blocks run the fused norm2 / FFN chain (no carry)."""
    from .int8_swiglu_fused import require_backend
    require_backend()
    if raw.training:
        raise ValueError("decoder.eval() required")
    result = share_containers(raw)
    blocks = []
    for block in result.transformer_blocks:
        if getattr(block.ff, "mode", None) != "INT8both":
            raise ValueError("requires an existing INT8both FFN")
        if not isinstance(block.norm2, nn.RMSNorm) or not getattr(block, "use_scale", False):
            raise ValueError("scaled residual block with RMSNorm required")
        width = block.norm2.normalized_shape
        if len(width) != 1 or width[0] not in ROW_WIDTHS or block.norm2.weight is None:
            raise ValueError(f"affine RMSNorm of width {ROW_WIDTHS} required")
        blocks.append(Int8Block(block, warps=warps).eval())
    result.transformer_blocks = nn.ModuleList(blocks)
    return result


def _check_carry_blocks(blocks):
    """Every block: an INT8 norm2 / FFN block of one width with INT8 QKV / out linears and fp16 norms."""
    width = blocks[0].scale1.shape[0] if blocks[0].scale1.ndim == 1 else -1
    if width not in ROW_WIDTHS:
        raise ValueError(f"norm1 fusion requires decoder width in {ROW_WIDTHS}")
    for block in blocks:
        norms_ok = all(isinstance(n, nn.RMSNorm) and n.normalized_shape == (width,) and n.weight is not None
                       and n.eps == EPS and n.weight.dtype == torch.float16 for n in (block.norm1, block.norm2))
        gates_ok = all(s.shape == (width,) and s.dtype == torch.float16 for s in (block.scale1, block.scale2))
        if block.training or getattr(block, "warps", None) != FFN_WARPS or not norms_ok or not gates_ok:
            raise ValueError("norm1 fusion requires the validated FP16 block contract of one decoder width")
        from .decoder_fused_qk_rope import FusedQKAttention
        if type(block.attn) is not FusedQKAttention:
            raise ValueError("expected the runtime FusedQKAttention class")
        a = block.attn.original
        linears = (a.to_qkv, a.to_out, block.ff.w1, block.ff.w2)
        if not all(isinstance(lin, KitchenInt8Linear) for lin in linears) \
                or tuple(a.to_qkv.qweight.shape) != (3 * width, width) or tuple(a.to_qkv.weight_scale.shape) != (3 * width,):
            raise ValueError("expected an already-quantized INT8 decoder; refusing requantization")
    return width


def carry_decoder(raw):
    """Copy of an INT8 decoder (INT8 QKV / out / FFN, fused norm2 blocks) with the residual carry."""
    if getattr(raw, "spatial_parallel", True):
        raise RuntimeError("authored final LayerNorm requires spatial_parallel=false")
    result = share_containers(raw)
    blocks = list(result.transformer_blocks)
    width = _check_carry_blocks(blocks)
    norm = getattr(raw, "norm_out", None)
    if (type(norm) is not nn.LayerNorm or getattr(norm.forward, "__func__", None) is not nn.LayerNorm.forward
            or norm.normalized_shape != (width,) or norm.eps != EPS or norm.weight is None or norm.bias is None
            or norm.weight.dtype != torch.float16 or norm.bias.dtype != torch.float16):
        raise ValueError("final LayerNorm requires affine FP16 decoder-width/eps-1e-5")
    last = len(blocks) - 1
    result.transformer_blocks = nn.ModuleList(
        [Int8Block(b, warps=b.warps, carry=True, first=i == 0, last=i == last).eval() for i, b in enumerate(blocks)])
    result.norm_out = CarryLayerNorm(result.norm_out).eval()
    result._unpad_for_sp = carry_unpad(result._unpad_for_sp)
    result._h3vae_norm1_quant_enabled = True
    return result.eval()
