"""INT8 FFN-up GEMM with the paired SwiGLU epilogue, activation requant and down GEMM.

Mirror of opt/int8_ffn_up_fused.py in fishelegs/ComfyUI-H3VAE-PyOpt.
``up_swiglu`` (:50-89) becomes ``h3v_gemm_i8_swiglu`` (one MFMA GEMM whose N
tiles hold matching gate and up weight rows, so the SiLU(gate)*up epilogue is
register-local), ``quantize_act`` (:91-104) becomes ``h3v_row_quant`` over the
fp16 activation, and the down projection is ``h3v_gemm_i8_dequant``.  The
residual FFN op chains the same arithmetic as dequant GEMM + SwiGLU row
quantizer (see ``quantize_ffn_up``), which is bit-identical and faster.
INT32 accumulation, FP32 scales with an FMA bias, FP16 rounding of the linear
output and of the activation, and the row-quantizer contract are unchanged.
"""
from __future__ import annotations

import torch

from .. import _hip

# Workgroup tile of the gfx950 kernel: (BM, BN weight rows, BK, waves, LDS stages).
CONFIG = (256, 256, 64, 4, 2)


def supports_fused_ffn_up(device):
    """The fused kernels run on MI355X (gfx950) only."""
    return _hip.is_gfx950(device)


def validate_prequantized(q, scale, weight, weight_scale, bias):
    if q.ndim != 2 or q.shape[0] == 0 or q.shape[1] == 0:
        raise ValueError("nonempty INT8 activation matrix required")
    if weight.ndim != 2 or weight.shape[0] % 2 or weight.shape[1] != q.shape[1]:
        raise ValueError("INT8 FFN-up weight must be [2N, K] with K matching the activation")
    n = weight.shape[0] // 2
    # The activation output is indexed as row * N; keep M * N inside 2^31.
    if q.shape[0] > (1 << 31) // n:
        raise ValueError("INT8 FFN-up M exceeds 32-bit output indexing bound")
    if q.dtype != torch.int8 or weight.dtype != torch.int8:
        raise ValueError("INT8 activations and weights required")
    if scale.dtype != torch.float32 or weight_scale.dtype != torch.float32:
        raise ValueError("FP32 activation and weight scales required")
    if scale.shape != (q.shape[0], 1) or weight_scale.shape != (2 * n,):
        raise ValueError("one activation/weight scale per row required")
    if bias is not None and (bias.shape != (2 * n,) or bias.dtype != torch.float16):
        raise ValueError("FP16 bias with one element per weight row required")
    values = (q, scale, weight, weight_scale) + (() if bias is None else (bias,))
    if any(not value.is_contiguous() or value.device != q.device for value in values):
        raise ValueError("contiguous tensors on the same device required")


def up_swiglu(q, scale, weight, weight_scale, bias=None):
    """fp16 act [M, N] = SwiGLU of the dequantized FFN-up GEMM."""
    validate_prequantized(q, scale, weight, weight_scale, bias)
    _hip.require_gfx950(q.device, "fused INT8 FFN-up")
    m, k = q.shape
    n = weight.shape[0] // 2
    act = torch.empty((m, n), device=q.device, dtype=torch.float16)
    _hip.call("h3v_gemm_i8_swiglu", _hip.ptr(q), _hip.ptr(scale), _hip.ptr(weight), _hip.ptr(weight_scale),
              _hip.ptr(bias), _hip.ptr(act), m, n, k, _hip.stream(q.device))
    return act


def quantize_ffn_up(q, scale, weight, weight_scale, bias=None):
    """Consume prequantized norm output and return the INT8 SwiGLU rows and scales.

    Runs as the dequant GEMM over all 2N weight rows (fp16 [gate | up] rows)
    followed by the SwiGLU row quantizer.  This is bit-identical to
    ``up_swiglu`` + row quantization (the G1 epilogue and the SiLU/product
    rounding are the same operations) and faster on MI355X: the SiLU work
    overlaps the quantizer's memory stream instead of following the MFMA
    main loop (measured 400 us vs 437 us at M=7188, N=8192, K=2048).
    """
    validate_prequantized(q, scale, weight, weight_scale, bias)
    if not supports_fused_ffn_up(q.device):
        raise ValueError("fused INT8 FFN-up requires an AMD MI355X (gfx950) GPU")
    if torch.is_grad_enabled():
        raise RuntimeError("fused INT8 FFN-up requires inference/no_grad")
    m, k = q.shape
    n = weight.shape[0] // 2
    gate_up = torch.empty((m, 2 * n), device=q.device, dtype=torch.float16)
    stream = _hip.stream(q.device)
    _hip.call("h3v_gemm_i8_dequant", _hip.ptr(q), _hip.ptr(scale), _hip.ptr(weight), _hip.ptr(weight_scale),
              _hip.ptr(bias), _hip.ptr(gate_up), m, 2 * n, k, stream)
    qout = torch.empty((m, n), device=q.device, dtype=torch.int8)
    sout = torch.empty((m, 1), device=q.device, dtype=torch.float32)
    _hip.call("h3v_swiglu_row_quant", _hip.ptr(gate_up), m, n, _hip.ptr(qout), _hip.ptr(sout), stream)
    return qout, sout


def _residual_ffn_impl(x, a, g, norm_weight, up_weight, up_scale, up_bias, down_weight, down_scale, down_bias,
                       eps, warps):
    from .int8_norm_quant import residual_quant
    from .int8_swiglu_fused import prequantized_linear, require_backend

    require_backend()
    if down_weight.ndim != 2 or down_weight.shape != (x.shape[-1], up_weight.shape[0] // 2):
        raise ValueError("INT8 FFN-down weight must be [K, N] for an FFN-up weight [2N, K]")
    h, q, scale = residual_quant(x, a, g, norm_weight, eps, warps)
    qout, sout = quantize_ffn_up(q, scale, up_weight, up_scale, up_bias)
    del q, scale
    out = prequantized_linear(qout, sout, down_weight, down_scale, down_bias)
    return h, out.reshape(*x.shape[:-1], down_weight.shape[0])


@torch.library.custom_op("h3vae_int8_ffn::residual_ffn", mutates_args=())
def fused_residual_ffn(x: torch.Tensor, a: torch.Tensor, g: torch.Tensor, norm_weight: torch.Tensor,
                       up_weight: torch.Tensor, up_scale: torch.Tensor, up_bias: torch.Tensor | None,
                       down_weight: torch.Tensor, down_scale: torch.Tensor, down_bias: torch.Tensor | None,
                       eps: float, warps: int) -> tuple[torch.Tensor, torch.Tensor]:
    return _residual_ffn_impl(x, a, g, norm_weight, up_weight, up_scale, up_bias, down_weight, down_scale,
                              down_bias, eps, warps)


@fused_residual_ffn.register_fake
def _fake(x, a, g, norm_weight, up_weight, up_scale, up_bias, down_weight, down_scale, down_bias, eps, warps):
    return torch.empty_like(x), x.new_empty((*x.shape[:-1], down_weight.shape[0]))
