"""No-rotation SwiGLU + row-wise INT8 quantization and the prequantized GEMM.

Mirror of opt/int8_swiglu_fused.py in fishelegs/ComfyUI-H3VAE-PyOpt.  The
reference's Triton quantizer (``quant``, :22-38) becomes
``h3v_swiglu_row_quant`` and its CK CUTLASS GEMM (``prequantized_linear``,
:78-107) becomes ``h3v_gemm_i8_dequant``.  Unsupported inputs fail; there is
no fallback and no re-quantization.
"""
from __future__ import annotations

import copy
from functools import lru_cache

import torch
from torch import nn

from .. import _hip


def validate_input(x):
    if x.dtype != torch.float16 or x.ndim < 2 or not x.is_contiguous():
        raise ValueError("contiguous FP16 input with at least two dimensions required")
    if x.shape[-1] <= 0 or x.shape[-1] % 2 or x.numel() == 0:
        raise ValueError("nonempty [gate | up] rows of even width required")
    if x.shape[-1] // 2 > 16384:
        raise ValueError("experimental quantizer K exceeds 16384")


def quantize_swiglu(x, *, num_warps=8):
    """fp16 [..., 2K] -> (int8 [M, K], fp32 [M, 1]); num_warps is accepted for API parity."""
    validate_input(x)
    if num_warps not in (4, 8, 16):
        raise ValueError("unsupported warp count")
    _hip.require_gfx950(x.device, "SwiGLU INT8 quantization")
    k = x.shape[-1] // 2
    rows = x.numel() // (2 * k)
    q = torch.empty((rows, k), device=x.device, dtype=torch.int8)
    scale = torch.empty((rows, 1), device=x.device, dtype=torch.float32)
    _hip.call("h3v_swiglu_row_quant", _hip.ptr(x), rows, k, _hip.ptr(q), _hip.ptr(scale), _hip.stream(x.device))
    return q, scale


@lru_cache(maxsize=1)
def require_backend():
    """The reference pins comfy-kitchen 0.2.34 here; the backend is the HIP library."""
    return _hip.lib()


def prequantized_linear(q, scale, weight, weight_scale, bias=None):
    """INT8 GEMM with the dequant epilogue, consuming already-quantized rows once."""
    require_backend()
    m, k = q.shape
    n = weight.shape[0]
    if q.dtype != torch.int8 or weight.dtype != torch.int8 or weight.shape[1] != k:
        raise ValueError("INT8 matrix dimensions/types do not match")
    if scale.dtype != torch.float32 or weight_scale.dtype != torch.float32:
        raise ValueError("FP32 scales required")
    if scale.numel() != m or weight_scale.numel() != n:
        raise ValueError("one scale per activation/weight row required")
    tensors = (q, scale, weight, weight_scale) + (() if bias is None else (bias,))
    if any(t.device != q.device or not t.is_contiguous() for t in tensors):
        raise ValueError("contiguous tensors on the same GPU device required")
    _hip.require_gfx950(q.device, "INT8 GEMM")
    if bias is not None and (bias.dtype != torch.float16 or bias.numel() != n):
        raise ValueError("FP16 bias matching output channels required")
    out = torch.empty((m, n), device=q.device, dtype=torch.float16)
    _hip.call("h3v_gemm_i8_dequant", _hip.ptr(q), _hip.ptr(scale), _hip.ptr(weight), _hip.ptr(weight_scale),
              _hip.ptr(bias), _hip.ptr(out), m, n, k, _hip.stream(q.device))
    return out


@torch.library.custom_op("h3vae_exp::swiglu_int8_linear", mutates_args=())
def swiglu_int8_linear(x: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor,
                       bias: torch.Tensor | None, warps: int) -> torch.Tensor:
    q, scale = quantize_swiglu(x, num_warps=warps)
    out = prequantized_linear(q, scale, weight, weight_scale, bias)
    return out.reshape(*x.shape[:-1], weight.shape[0])


@swiglu_int8_linear.register_fake
def _fake(x, weight, weight_scale, bias, warps):
    return x.new_empty((*x.shape[:-1], weight.shape[0]))


class FusedFFN(nn.Module):
    def __init__(self, original, warps=8):
        super().__init__()
        if getattr(original, "mode", None) != "INT8both":
            raise ValueError("requires an existing INT8both FFN")
        self.w1, self.w2 = original.w1, original.w2
        self.warps = warps
        self.train(original.training)

    def forward(self, x):
        if self.training or torch.is_grad_enabled():
            raise RuntimeError("eval + no_grad/inference_mode required")
        hidden = self.w1(x)
        return swiglu_int8_linear(hidden, self.w2.qweight, self.w2.weight_scale, self.w2.bias, self.warps)


def clone_fused_decoder(raw, warps=8):
    require_backend()
    if raw.training:
        raise ValueError("decoder.eval() required")

    def clone(module):
        new = copy.copy(module)
        new._parameters = module._parameters.copy()
        new._buffers = module._buffers.copy()
        new._modules = {key: None if child is None else clone(child) for key, child in module._modules.items()}
        return new

    result = clone(raw)
    for block in result.transformer_blocks:
        block.ff = FusedFFN(block.ff, warps).eval()
    return result
