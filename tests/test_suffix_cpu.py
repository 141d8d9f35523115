"""CPU checks of the FP16 encoder convs: the packed weight layout the kernel reads, the shape gate of
h3v_conv3d_f16, the packed copies' ownership, and the ops' host-side guards (meta tensors)."""
from __future__ import annotations

import importlib

import pytest
import torch


@pytest.fixture(scope="module")
def fc(pkg):
    return importlib.import_module(f"{pkg.__name__}.opt.encoder_fp16_conv")


def test_packed_weight_layout(fc):
    gen = torch.Generator().manual_seed(2)
    w = torch.randn(5, 7, 3, 3, 3, generator=gen).half()
    p = fc.pack_conv_weight_f16(w)
    assert p.shape == (5, 27 * 7) and p.is_contiguous()
    for o, c, kd, kh, kw in [(0, 0, 0, 0, 0), (4, 6, 2, 2, 2), (2, 3, 1, 0, 2), (3, 5, 0, 2, 1)]:
        assert p[o, ((kd * 3 + kh) * 3 + kw) * 7 + c] == w[o, c, kd, kh, kw]
    w1 = torch.randn(4, 6, 1, 1, 1, generator=gen).half()
    assert torch.equal(fc.pack_conv_weight_f16(w1), w1.reshape(4, 6))
    with pytest.raises(ValueError):
        fc.pack_conv_weight_f16(w.float())
    with pytest.raises(ValueError):
        fc.pack_conv_weight_f16(w[0])


@pytest.mark.parametrize("shape,cout,kernel,stride,fits", [
    ((4, 256, 19, 66, 66), 256, 3, (1, 1, 1), True),      # suffix stage at tile 256: 64 x 64
    ((4, 1024, 7, 18, 18), 1024, 3, (1, 1, 1), True),     # 16 x 16 stage (implicit GEMM)
    ((4, 256, 19, 66, 66), 48, 3, (1, 1, 1), True),       # conv_out to the latent moments
    ((1, 128, 19, 258, 258), 128, 3, (1, 2, 2), True),    # stage-0 downsample
    ((1, 256, 19, 129, 129), 256, 3, (2, 2, 2), True),    # stage-1 downsample
    ((1, 128, 17, 128, 128), 256, 1, (1, 1, 1), True),    # nin_shortcut
    ((1, 3, 19, 258, 258), 128, 3, (1, 1, 1), False),     # conv_in: 3 channels
    ((1, 16, 5, 66, 66), 128, 3, (1, 1, 1), False),       # Cin % 32
    ((1, 32, 2, 66, 66), 128, 3, (1, 1, 1), False),       # shallower than the kernel
])
def test_fits_gate(fc, shape, cout, kernel, stride, fits):
    x = torch.empty(shape, dtype=torch.float16, device="meta")
    w = torch.empty((cout, shape[1], kernel, kernel, kernel), dtype=torch.float16, device="meta")
    assert fc.conv3d_f16_fits(x, w, stride) is fits
    assert fc.conv3d_f16_fits(x.float(), w, stride) is False


def test_conv_op_guards_on_meta(fc):
    x = torch.empty((2, 64, 5, 6, 66), dtype=torch.float16, device="meta").contiguous(
        memory_format=torch.channels_last_3d)
    w = torch.empty((128, 27 * 64), dtype=torch.float16, device="meta")
    y = fc.conv3d_f16(x, w, None, [3, 3, 3], [1, 1, 1], True)
    assert y.shape == (2, 128, 3, 4, 64) and y.is_contiguous(memory_format=torch.channels_last_3d)
    assert fc.conv3d_f16(x, w, None, [3, 3, 3], [1, 2, 2], False).shape == (2, 128, 3, 2, 32)
    with pytest.raises(ValueError, match="packed"):
        fc.conv3d_f16(x, w[:, :100], None, [3, 3, 3], [1, 1, 1], True)
    with pytest.raises(ValueError, match="channels-last"):
        fc.conv3d_f16(x.contiguous(), w, None, [3, 3, 3], [1, 1, 1], True)
    with pytest.raises(ValueError, match="bias"):
        fc.conv3d_f16(x, w, torch.empty(64, dtype=torch.float16, device="meta"), [3, 3, 3], [1, 1, 1], True)
    with pytest.raises(ValueError, match="fp16"):
        fc.conv3d_f16(x.float(), w, None, [3, 3, 3], [1, 1, 1], True)
    with pytest.raises(ValueError, match="strides"):
        fc.conv3d_f16(x, w, None, [3, 3, 3], [1, 0, 1], True)


def test_pack_op_guards_on_meta(fc):
    x = torch.empty((1, 128, 5, 16, 16), dtype=torch.float16, device="meta")
    y = fc.causal_reflect_pack(x, 2, 1, 1, 1, 1)
    assert y.shape == (1, 128, 7, 18, 18) and y.is_contiguous(memory_format=torch.channels_last_3d)
    with pytest.raises(ValueError, match="smaller"):
        fc.causal_reflect_pack(x, 2, 16, 0, 0, 0)
    with pytest.raises(ValueError, match="C % 8"):
        fc.causal_reflect_pack(x[:, :12], 2, 1, 1, 1, 1)


def test_cpu_tensors_raise_no_fallback(fc):
    """Off the GPU the native conv modules refuse to run: there is no second implementation."""
    gen = torch.Generator().manual_seed(1)
    w = torch.nn.Parameter(torch.randn(64, 32, 3, 3, 3, generator=gen).half(), requires_grad=False)
    conv = fc.NativeConv(w, None, (1, 2, 2))
    with pytest.raises(RuntimeError, match="gfx950"):
        conv(torch.randn(1, 32, 5, 6, 6, generator=gen).half())
    padded = fc.PaddedCausalConv(w, None, (1, 2, 2), (1, 1, 1, 1))
    with pytest.raises(RuntimeError, match="gfx950"):
        padded(torch.randn(1, 32, 5, 6, 6, generator=gen).half(), 2)
    point = fc.PointwiseConv(torch.nn.Conv3d(48, 48, 1).half())
    with pytest.raises(RuntimeError, match="gfx950"):
        point(torch.randn(1, 48, 2, 3, 3, generator=gen).half())
    with pytest.raises(ValueError, match="1x1x1"):
        fc.PointwiseConv(torch.nn.Conv3d(48, 48, 3))


def test_packed_weight_tracks_its_source_and_moves_with_its_owner(fc):
    gen = torch.Generator().manual_seed(3)
    w = torch.nn.Parameter(torch.randn(4, 32, 3, 3, 3, generator=gen).half(), requires_grad=False)
    owner = torch.nn.Module()
    owner.packed = fc.PackedConvWeight(w)
    assert owner.packed.packed is None                         # nothing is packed before the first use
    p1 = owner.packed(w)
    assert owner.packed(w) is p1                               # reused while unchanged
    assert torch.equal(p1, fc.pack_conv_weight_f16(w.detach()))
    with torch.no_grad():
        w.mul_(2)                                              # in-place update (a state-dict load) repacks
    p2 = owner.packed(w)
    assert p2 is not p1 and torch.equal(p2, fc.pack_conv_weight_f16(w.detach()))
    assert "packed.packed" not in owner.state_dict()          # derived data: not saved
    owner.to("meta")                                           # the copy moves (and is freed) with its owner
    assert owner.packed.packed.device.type == "meta"
    with torch.inference_mode():                               # weights created under inference mode
        wi = torch.randn(4, 32, 3, 3, 3, generator=gen).half()
        folded = fc.PackedConvWeight(wi[:, :3], fold=True)
        assert torch.equal(folded(wi[:, :3]), fc.fold_conv_weight_f16(wi[:, :3]))


def test_folded_conv_in_weight_layout(fc):
    gen = torch.Generator().manual_seed(4)
    w = torch.randn(6, 3, 3, 3, 3, generator=gen).half()
    f = fc.fold_conv_weight_f16(w)
    assert f.shape == (6, 96) and f.is_contiguous()
    for o, c, kd, kh, kw in [(0, 0, 0, 0, 0), (5, 2, 2, 2, 2), (3, 1, 1, 0, 2)]:
        assert f[o, kd * 32 + (kh * 3 + kw) * 3 + c] == w[o, c, kd, kh, kw]
    assert not f.view(6, 3, 32)[:, :, 27:].any()
    with pytest.raises(ValueError):
        fc.fold_conv_weight_f16(torch.zeros(6, 4, 3, 3, 3, dtype=torch.float16))
    x = torch.empty((1, 3, 5, 16, 16), dtype=torch.float16, device="meta")
    y = fc.tap_fold_pack(x, 2)
    assert y.shape == (1, 32, 7, 16, 16) and y.is_contiguous(memory_format=torch.channels_last_3d)
    with pytest.raises(ValueError, match="C in 1..3"):
        fc.tap_fold_pack(torch.empty((1, 4, 5, 16, 16), dtype=torch.float16, device="meta"), 2)
