"""INT8 QKV projections of the decoder (on the fused norm2 / FFN decoder).

Counterpart of opt/int8_qkv.py in fishelegs/ComfyUI-H3VAE-PyOpt
(``clone_qkv_int8_decoder`` :33-41): the chosen blocks' ``to_qkv``
(``nn.Linear`` D -> 3D) become ``KitchenInt8Linear`` (static row-wise INT8
weights; per call the activation row quantizer and the INT8 MFMA GEMM with the
dequant epilogue).  Built on a container copy; the source decoder is untouched.
"""
from __future__ import annotations

from .decoder_int8 import attention_of, chosen_blocks, quantize_attention_linears, source_linear
from .int8_norm_quant import clone_norm_quant_decoder


def qkv_linear(block):
    """-> (attention module, its D -> 3D nn.Linear) after checking the QKV contract."""
    return source_linear(block, "to_qkv", square=False)


def clone_qkv_int8_decoder(raw, *, indices=None, warps=8):
    """Fused norm2 / FFN copy of ``raw`` with INT8 QKV linears in the chosen blocks (all by default)."""
    for i in chosen_blocks(len(raw.transformer_blocks), indices):
        qkv_linear(raw.transformer_blocks[i])
    return quantize_attention_linears(clone_norm_quant_decoder(raw, warps), "to_qkv", indices, square=False)


def qkv_inventory(decoder):
    """Per block with an INT8 QKV projection: its shape, dtypes and device."""
    from .kitchen_int8 import KitchenInt8Linear
    rows = []
    for i, block in enumerate(decoder.transformer_blocks):
        linear = attention_of(block).to_qkv
        if isinstance(linear, KitchenInt8Linear):
            rows.append({"block": i, "shape": list(linear.qweight.shape), "qweight_dtype": str(linear.qweight.dtype),
                         "scale_dtype": str(linear.weight_scale.dtype), "device": str(linear.qweight.device)})
    return rows
