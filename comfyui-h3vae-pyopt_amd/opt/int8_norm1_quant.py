"""Residual / norm1 / INT8-QKV fusion and the decoder block carry protocol.

Counterpart of opt/int8_norm1_quant.py in fishelegs/ComfyUI-H3VAE-PyOpt.

* ``residual_qkv`` (:126-162) runs ``h3v_residual_norm1_quant`` in place on
  ``h`` (raw = fma(o, g, h); h <- fp16(raw); the published W16 reduction tree
  for sum(raw^2); n = fp16((h * inv) * w); row quantization) followed by the
  INT8 QKV GEMM ``h3v_gemm_i8_dequant``.
* ``clone_norm1_quant_decoder`` (:302-343) makes the blocks pass the
  residual between them as a carry ``(h, out, scale2)`` instead of
  materialising ``h + out * scale2`` (``decoder_int8.Int8Block`` with
  ``carry``): block 0 normalises with ``rms_fp16_x2_w16``; blocks 1.. fold
  the previous block's residual into their norm1 producer; the last block
  hands the carry to the final LayerNorm (``residual_ln_w8``).

The reference gates the fused path to its validated SM120 B4 shape
``[4, 1797, 2048]`` and a 36-block stack.  Here the kernels take any row
count and widths 1024/2048/4096, so the gate is: contiguous FP16
``[B, N, D]`` rows with D the decoder width, on an MI355X (gfx950) device.
"""
from __future__ import annotations

import torch
from torch import nn

from .. import _hip
from ._checks import ROW_WIDTHS
from ._modules import share_containers
from .decoder_int8 import carry_decoder
from .int8_swiglu_fused import prequantized_linear

_EPS = 1.0e-5


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


def clone_norm1_quant_decoder(raw, *, enabled=False):
    """Copy of an already-INT8 decoder whose blocks pass the residual carry (reference :302-343).

    ``enabled=False`` returns a plain copy; enabling it off an MI355X raises."""
    if raw.training:
        raise ValueError("eval decoder required")
    blocks = getattr(raw, "transformer_blocks", None)
    if blocks is None or len(blocks) == 0:
        raise ValueError("expected a decoder with transformer_blocks")
    try:
        device = next(raw.parameters()).device
    except StopIteration as exc:
        raise ValueError("decoder has no parameters") from exc
    if not enabled:
        result = share_containers(raw)
        result._h3vae_norm1_quant_enabled = False
        return result.eval()
    if not supports_norm1_quant(device):
        raise RuntimeError("norm1 fusion requires an AMD MI355X (gfx950) GPU")
    _hip.lib()
    return carry_decoder(raw)
