"""SwiGLU + INT8 row quantization of the FFN activation, and the GEMM on prequantized rows.

Counterpart of opt/int8_swiglu_fused.py in fishelegs/ComfyUI-H3VAE-PyOpt: its
Triton quantizer (``quant`` :22-38, ``quantize_swiglu`` :52-65) is
``h3v_swiglu_row_quant`` and its comfy-kitchen CUTLASS call
(``prequantized_linear`` :78-107) is ``h3v_gemm_i8_dequant``.  The op
``h3vae_exp::swiglu_int8_linear`` chains the two: fp16 [gate | up] rows ->
int8 SiLU(gate) * up rows + fp32 row scales -> the down projection.  The
non-fused FFN (``FusedFFN``: INT8 w1 GEMM, then this op) is the arithmetic the
fused FFN-up path must reproduce bit for bit.
"""
from __future__ import annotations

from functools import lru_cache

import torch
from torch import nn

from .. import _hip
from ._modules import require_inference, share_containers


def validate_input(x):
    if x.dtype != torch.float16 or x.ndim < 2 or not x.is_contiguous():
        raise ValueError("contiguous FP16 input with at least two dimensions required")
    width = x.shape[-1]
    if width <= 0 or width % 2 or x.numel() == 0:
        raise ValueError("nonempty [gate | up] rows of even width required")
    if width // 2 > 16384:
        raise ValueError("experimental quantizer K exceeds 16384")


def quantize_swiglu(x, *, num_warps=8):
    """fp16 [..., 2N] -> (int8 [M, N], fp32 [M, 1]); ``num_warps`` is validated and otherwise unused."""
    validate_input(x)
    if num_warps not in (4, 8, 16):
        raise ValueError("unsupported warp count")
    _hip.require_gfx950(x.device, "SwiGLU INT8 quantization")
    n = x.shape[-1] // 2
    m = x.numel() // (2 * n)
    q = torch.empty((m, n), dtype=torch.int8, device=x.device)
    s = torch.empty((m, 1), dtype=torch.float32, device=x.device)
    _hip.call("h3v_swiglu_row_quant", _hip.ptr(x), m, n, _hip.ptr(q), _hip.ptr(s), _hip.stream(x.device))
    return q, s


@lru_cache(maxsize=1)
def require_backend():
    """Where the reference pins comfy-kitchen 0.2.34: the backend is the HIP library."""
    return _hip.lib()


def prequantized_linear(q, scale, weight, weight_scale, bias=None):
    """INT8 GEMM of already-quantized rows with the dequant epilogue -> fp16 [M, N]."""
    require_backend()
    if q.dtype != torch.int8 or weight.dtype != torch.int8 or q.ndim != 2 or weight.ndim != 2 \
            or weight.shape[1] != q.shape[1]:
        raise ValueError("INT8 matrix dimensions/types do not match")
    m, n = q.shape[0], weight.shape[0]
    if scale.dtype != torch.float32 or weight_scale.dtype != torch.float32:
        raise ValueError("FP32 scales required")
    if scale.numel() != m or weight_scale.numel() != n:
        raise ValueError("one scale per activation/weight row required")
    if any(t is not None and (t.device != q.device or not t.is_contiguous())
           for t in (scale, weight, weight_scale, bias)) or not q.is_contiguous():
        raise ValueError("contiguous tensors on the same GPU device required")
    _hip.require_gfx950(q.device, "INT8 GEMM")
    if bias is not None and (bias.dtype != torch.float16 or bias.numel() != n):
        raise ValueError("FP16 bias matching output channels required")
    out = torch.empty((m, n), dtype=torch.float16, device=q.device)
    _hip.call("h3v_gemm_i8_dequant", _hip.ptr(q), _hip.ptr(scale), _hip.ptr(weight), _hip.ptr(weight_scale),
              _hip.ptr(bias), _hip.ptr(out), m, n, q.shape[1], _hip.stream(q.device))
    return out


@torch.library.custom_op("h3vae_exp::swiglu_int8_linear", mutates_args=())
def swiglu_int8_linear(x: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor,
                       bias: torch.Tensor | None, warps: int) -> torch.Tensor:
    q, s = quantize_swiglu(x, num_warps=warps)
    return prequantized_linear(q, s, weight, weight_scale, bias).view(*x.shape[:-1], weight.shape[0])


@swiglu_int8_linear.register_fake
def _fake(x, weight, weight_scale, bias, warps):
    return x.new_empty((*x.shape[:-1], weight.shape[0]))


class FusedFFN(nn.Module):
    """An INT8 FFN whose activation requant runs in the SwiGLU quantizer (reference :124-141)."""

    def __init__(self, original, warps=8):
        super().__init__()
        if getattr(original, "mode", None) != "INT8both":
            raise ValueError("requires an existing INT8both FFN")
        self.w1, self.w2, self.warps = original.w1, original.w2, warps
        self.train(original.training)

    def forward(self, x):
        require_inference(self)
        w2 = self.w2
        return swiglu_int8_linear(self.w1(x), w2.qweight, w2.weight_scale, w2.bias, self.warps)


def clone_fused_decoder(raw, warps=8):
    """A copy of an INT8-FFN decoder whose FFNs are ``FusedFFN``; the source keeps its modules."""
    require_backend()
    if raw.training:
        raise ValueError("decoder.eval() required")
    result = share_containers(raw)
    for block in result.transformer_blocks:
        block.ff = FusedFFN(block.ff, warps).eval()
    return result
