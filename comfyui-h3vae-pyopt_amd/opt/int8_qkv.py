"""INT8 QKV projections on the fused-FFN decoder.

Mirror of opt/int8_qkv.py in fishelegs/ComfyUI-H3VAE-PyOpt.  Each selected
block's ``to_qkv`` (``nn.Linear`` D -> 3D) becomes a ``KitchenInt8Linear``:
static row-wise INT8 weights, then per call the activation row quantizer and
the INT8 MFMA GEMM with the dequant epilogue.  The source decoder and its
weights are left intact; the clone shares read-only tensors.
"""
from __future__ import annotations

import torch
from torch import nn

from ._checks import ROW_WIDTHS
from .int8_norm_quant import clone_norm_quant_decoder
from .kitchen_int8 import KitchenInt8Linear


def qkv_linear(block):
    """-> (attention module, source nn.Linear) after checking the QKV contract (reference :12-21)."""
    attention = getattr(block.attn, "original", block.attn)
    source = getattr(attention, "to_qkv", None)
    if not isinstance(source, nn.Linear):
        raise ValueError("expected original nn.Linear QKV projection")
    if source.in_features not in ROW_WIDTHS or source.out_features != 3 * source.in_features:
        raise ValueError(f"QKV projection requires K in {ROW_WIDTHS} and N = 3K")
    if source.training:
        raise ValueError("QKV inference requires eval()")
    return attention, source


def selected_indices(count, indices=None):
    """Validated block indices (reference :24-30)."""
    result = tuple(range(count)) if indices is None else tuple(indices)
    if not result or len(set(result)) != len(result):
        raise ValueError("nonempty unique block indices required")
    if any(type(i) is not int or i < 0 or i >= count for i in result):
        raise ValueError("block index out of range or not an integer")
    return result


def clone_qkv_int8_decoder(raw, *, indices=None, warps=8):
    """Clone via the norm2/FFN fusion and install INT8 QKV on the chosen blocks (reference :33-41)."""
    chosen = selected_indices(len(raw.transformer_blocks), indices)
    for i in chosen:
        qkv_linear(raw.transformer_blocks[i])
    result = clone_norm_quant_decoder(raw, warps)
    for i in chosen:
        attention, source = qkv_linear(result.transformer_blocks[i])
        attention.to_qkv = KitchenInt8Linear(source, require_cuda=True).eval()
    return result


def qkv_inventory(decoder):
    rows = []
    for i, block in enumerate(decoder.transformer_blocks):
        attention = getattr(block.attn, "original", block.attn)
        linear = attention.to_qkv
        if isinstance(linear, KitchenInt8Linear):
            if linear.qweight.dtype != torch.int8 or linear.weight_scale.dtype != torch.float32:
                raise RuntimeError("QKV quantized state has invalid dtype")
            rows.append({"block": i, "shape": list(linear.qweight.shape), "qweight_dtype": str(linear.qweight.dtype),
                         "scale_dtype": str(linear.weight_scale.dtype), "device": str(linear.qweight.device)})
    return rows
