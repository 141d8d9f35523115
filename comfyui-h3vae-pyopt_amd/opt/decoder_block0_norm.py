"""Block-0 FP16 RMSNorm (no residual carry).

Mirror of opt/decoder_block0_norm.py in fishelegs/ComfyUI-H3VAE-PyOpt
(``rms_fp16_x2_w16``, :39-95): out = fp16((x * inv) * gamma) with
inv = 1/sqrt(sum(x^2)/K + EPS_F32), summed with the published W16 tree.
"""
from __future__ import annotations

import torch

from .. import _hip
from ._checks import ROW_WIDTHS

_EPS_F32 = 9.999999747378752e-06


def _validate_metadata(x, gamma, *, require_cuda):
    k = x.shape[-1] if x.ndim else 0
    if (x.ndim < 2 or k not in ROW_WIDTHS or tuple(gamma.shape) != (k,) or x.dtype != torch.float16
            or gamma.dtype != torch.float16 or not x.is_contiguous() or not gamma.is_contiguous()
            or x.device != gamma.device):
        raise ValueError(f"expected contiguous [..., K] (K in {ROW_WIDTHS}) and gamma [K], both FP16 on one device")
    if require_cuda:
        _hip.require_gfx950(x.device, "block0 RMS")


def rms_fp16_x2_w16_impl(x: torch.Tensor, gamma: torch.Tensor) -> torch.Tensor:
    _validate_metadata(x, gamma, require_cuda=True)
    if torch.is_grad_enabled():
        raise RuntimeError("block0 RMS requires inference/no_grad")
    output = torch.empty_like(x, memory_format=torch.contiguous_format)
    k = x.shape[-1]
    _hip.call("h3v_rms_fp16", _hip.ptr(x), _hip.ptr(gamma), _EPS_F32, x.numel() // k, k, _hip.ptr(output),
              _hip.stream(x.device))
    return output


@torch.library.custom_op("h3vae_norm1_block0::rms_fp16_x2_w16", mutates_args=())
def rms_fp16_x2_w16(x: torch.Tensor, gamma: torch.Tensor) -> torch.Tensor:
    return rms_fp16_x2_w16_impl(x, gamma)


@rms_fp16_x2_w16.register_fake
def _fake_rms_fp16_x2_w16(x, gamma):
    _validate_metadata(x, gamma, require_cuda=False)
    return torch.empty_like(x, memory_format=torch.contiguous_format)
