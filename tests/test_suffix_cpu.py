"""CPU checks of the encoder suffix's FP16 conv routing: the packed weight layout the kernel reads, the
shape gate that picks h3v_conv3d_f16 over the model's F.conv3d, and the op's host-side guards."""
from __future__ import annotations

import importlib

import pytest
import torch


@pytest.fixture(scope="module")
def bn(pkg):
    return importlib.import_module(f"{pkg.__name__}.opt.encoder_fused_batched_norm")


def test_packed_weight_layout(bn):
    gen = torch.Generator().manual_seed(2)
    w = torch.randn(5, 7, 3, 3, 3, generator=gen).half()
    p = bn.pack_conv_weight_f16(w)
    assert p.shape == (5, 27 * 7) and p.is_contiguous()
    for o, c, kd, kh, kw in [(0, 0, 0, 0, 0), (4, 6, 2, 2, 2), (2, 3, 1, 0, 2), (3, 5, 0, 2, 1)]:
        assert p[o, ((kd * 3 + kh) * 3 + kw) * 7 + c] == w[o, c, kd, kh, kw]
    with pytest.raises(ValueError):
        bn.pack_conv_weight_f16(w.float())
    with pytest.raises(ValueError):
        bn.pack_conv_weight_f16(w[:, :, :1])


@pytest.mark.parametrize("shape,cout,stride,fits", [
    ((4, 256, 19, 66, 66), 256, (1, 1, 1), True),      # suffix stage at tile 256: 64 x 64
    ((4, 512, 11, 34, 34), 512, (1, 1, 1), True),      # 32 x 32
    ((4, 1024, 7, 18, 18), 1024, (1, 1, 1), False),    # 16 x 16: model conv
    ((4, 256, 19, 66, 66), 48, (1, 1, 1), False),      # conv_out to the latent moments
    ((4, 256, 19, 66, 66), 256, (1, 2, 2), False),
    ((1, 16, 5, 66, 66), 128, (1, 1, 1), False),       # Cin % 32
    ((1, 32, 5, 14, 66), 128, (1, 1, 1), False),       # Ho = 12 not a multiple of 8 at Wo 64
])
def test_fits_gate(bn, shape, cout, stride, fits):
    x = torch.empty(shape, dtype=torch.float16, device="meta")
    w = torch.empty((cout, shape[1], 3, 3, 3), dtype=torch.float16, device="meta")
    assert bn.conv3d_f16_fits(x, w, stride) is fits


def test_conv_op_guards_on_meta(bn):
    x = torch.empty((2, 64, 5, 6, 66), dtype=torch.float16, device="meta").contiguous(
        memory_format=torch.channels_last_3d)
    w = torch.empty((128, 27 * 64), dtype=torch.float16, device="meta")
    y = bn.conv3d_f16(x, w, None, True)
    assert y.shape == (2, 128, 3, 4, 64) and y.is_contiguous(memory_format=torch.channels_last_3d)
    with pytest.raises(ValueError, match="packed"):
        bn.conv3d_f16(x, w[:, :100], None, True)
    with pytest.raises(ValueError, match="channels-last"):
        bn.conv3d_f16(x.contiguous(), w, None, True)
    with pytest.raises(ValueError, match="bias"):
        bn.conv3d_f16(x, w, torch.empty(64, dtype=torch.float16, device="meta"), True)
    with pytest.raises(ValueError, match="fp16"):
        bn.conv3d_f16(x.float(), w, None, True)
