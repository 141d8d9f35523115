"""INT8 attention output projections of the decoder (after INT8 QKV).

Counterpart of opt/int8_attention_out.py in fishelegs/ComfyUI-H3VAE-PyOpt
(``clone_attention_out_decoder`` :40-48, ``from_raw_decoder`` :51-52): the
chosen blocks' ``to_out`` (``nn.Linear`` D -> D, bias) become
``KitchenInt8Linear``.  ``from_raw_decoder`` is the runtime's full INT8
decoder: fused norm2 / FFN chain + INT8 QKV + INT8 attention-out.
"""
from __future__ import annotations

from ._modules import share_containers
from .decoder_int8 import chosen_blocks, quantize_attention_linears, source_linear
from .int8_qkv import clone_qkv_int8_decoder

# the reference's name for the container copy (opt/int8_attention_out.py:13-25)
clone_containers = share_containers


def out_linear(block):
    """-> (attention module, its D -> D nn.Linear) after checking the output-projection contract."""
    return source_linear(block, "to_out", square=True)


def clone_attention_out_decoder(baseline, *, indices=None):
    """Copy of ``baseline`` with INT8 attention-out linears in the chosen blocks (all by default)."""
    for i in chosen_blocks(len(baseline.transformer_blocks), indices):
        out_linear(baseline.transformer_blocks[i])
    return quantize_attention_linears(share_containers(baseline), "to_out", indices, square=True)


def from_raw_decoder(raw, *, warps=8):
    """INT8 QKV + fused norm2 / FFN + INT8 attention-out on a decoder whose FFNs are INT8."""
    return clone_attention_out_decoder(clone_qkv_int8_decoder(raw, warps=warps))


def out_inventory(decoder):
    """Per block with an INT8 output projection: its shape, dtypes and device."""
    from .decoder_int8 import attention_of
    from .kitchen_int8 import KitchenInt8Linear
    rows = []
    for i, block in enumerate(decoder.transformer_blocks):
        linear = attention_of(block).to_out
        if isinstance(linear, KitchenInt8Linear):
            rows.append({"block": i, "shape": list(linear.qweight.shape), "qweight_dtype": str(linear.qweight.dtype),
                         "scale_dtype": str(linear.weight_scale.dtype), "device": str(linear.qweight.device)})
    return rows
