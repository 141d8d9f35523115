"""Final residual + LayerNorm for the last decoder block's carry.

Mirror of opt/decoder_final_norm.py in fishelegs/ComfyUI-H3VAE-PyOpt
(``final_residual_ln_w8``, :35-86): raw = fma(o, gate, h); mean and variance
over the row (a fixed two-pass reduction order replaces the reference's
compiler-owned Welford order); y = fp16(fma((raw - mean) * inv, gamma, beta)).
"""
from __future__ import annotations

import torch

from .. import _hip
from ._checks import ROW_WIDTHS

EPS = 9.999999747378752e-06


def validate_metadata(h, o, gate, gamma, beta, *, require_cuda):
    tensors = (h, o, gate, gamma, beta)
    k = h.shape[-1] if h.ndim else 0
    if (h.ndim < 2 or k not in ROW_WIDTHS or tuple(o.shape) != tuple(h.shape)
            or any(tuple(v.shape) != (k,) for v in tensors[2:])
            or any(v.dtype != torch.float16 or not v.is_contiguous() for v in tensors)
            or any(v.device != h.device for v in tensors)):
        raise ValueError(f"expected contiguous FP16 [..., K] H/O (K in {ROW_WIDTHS}) and width-K vectors on one device")
    if require_cuda:
        _hip.require_gfx950(h.device, "final LayerNorm")


def final_residual_ln_w8_impl(h, o, gate, gamma, beta):
    validate_metadata(h, o, gate, gamma, beta, require_cuda=True)
    if torch.is_grad_enabled():
        raise RuntimeError("final LayerNorm requires inference/no_grad")
    y = torch.empty_like(h, memory_format=torch.contiguous_format)
    k = h.shape[-1]
    _hip.call("h3v_residual_layernorm", _hip.ptr(h), _hip.ptr(o), _hip.ptr(gate), _hip.ptr(gamma), _hip.ptr(beta),
              EPS, h.numel() // k, k, _hip.ptr(y), _hip.stream(h.device))
    return y


@torch.library.custom_op("h3vae_final_ln::residual_ln_w8", mutates_args=())
def final_residual_ln_w8(h: torch.Tensor, o: torch.Tensor, gate: torch.Tensor, gamma: torch.Tensor,
                         beta: torch.Tensor) -> torch.Tensor:
    return final_residual_ln_w8_impl(h, o, gate, gamma, beta)


@final_residual_ln_w8.register_fake
def _fake(h, o, gate, gamma, beta):
    validate_metadata(h, o, gate, gamma, beta, require_cuda=False)
    return torch.empty_like(h, memory_format=torch.contiguous_format)
