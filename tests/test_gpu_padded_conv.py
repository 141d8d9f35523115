"""GPU parity: the padded-output INT8 conv (h3v_conv3d_i8_residual_padded) and the encoder stage ends that use it.

The last conv of a prefix stage writes its result straight into the padded input of the stage's causal
stride-2 downsample: `front` leading frames (zeroed by the op, not written by the kernel) and a reflect
border of 0 or 1 per side (row -1 = row 1, row H = row H - 2, likewise columns: stage 0's downsample reflects
all four sides, stage 1's only the bottom and right).  Every case is compared bit for bit with the separate path:
h3v_conv3d_i8 / h3v_conv3d_i8_residual (bitwise against the oracle in test_gpu_conv.py), then the padding
built on the CPU, and for the stage-1 form (residual + pack bias) the oracle's residual_downsample_pack.
"""
from __future__ import annotations

import importlib

import numpy as np
import pytest
import torch

import h3_arch
from _util import assert_bitwise, ndhwc, np_

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
SENTINEL = 0x7E01   # a NaN pattern no conv output takes


def _pad_np(v, front, border):
    """fp16 NDHWC [B, D, H, W, C] -> [B, D + front, H + top + bottom, W + left + right, C]: zero frames and
    a reflect border (top, bottom, left, right) of 0 or 1 per side (numpy's reflect mode)."""
    top, bottom, left, right = border
    out = np.pad(v, ((0, 0), (0, 0), (top, bottom), (left, right), (0, 0)), mode="reflect")
    return np.concatenate([np.zeros((v.shape[0], front, *out.shape[2:]), np.float16), out], axis=1)


# (batch, cin, cout, output frames, output height, output width, front, border, residual form)
CASES = [(1, 128, 128, 3, 8, 64, 2, (1, 1, 1, 1), "residual"),        # stage-0 form: residual, conv bias
         (1, 256, 256, 3, 4, 128, 2, (0, 1, 0, 1), "residual_bias"),  # stage-1 form: residual + pack bias
         (2, 64, 128, 2, 16, 32, 1, (1, 0, 0, 1), "none"),
         (1, 128, 128, 2, 2, 256, 0, (1, 1, 1, 1), "residual"),       # two rows: rows 0 and 1 both borders
         (1, 128, 128, 2, 8, 256, 2, (1, 1, 1, 1), "residual"),       # 8-row tiles of 64-column blocks
         (1, 256, 256, 2, 8, 128, 2, (0, 1, 0, 1), "residual_bias"),  # the same at the stage-1 form
         (1, 128, 256, 3, 8, 64, 2, (0, 1, 0, 1), "residual_bias"),
         (1, 128, 128, 3, 8, 64, 2, (0, 0, 0, 0), "residual")]


@pytest.mark.parametrize("case", CASES)
def test_padded_conv_matches_conv_then_pack(ops, oracle, case):
    b, cin, cout, d, h, w, front, border, form = case
    top, bottom, left, right = border
    print(f"h3v_conv3d_i8_residual_padded {case}", flush=True)
    hip = ops.hip
    gen = torch.Generator().manual_seed(cin + 7 * cout + 31 * w + front)
    qx = torch.randint(-127, 128, (b, d + 2, h + 2, w + 2, cin), generator=gen, dtype=torch.int8)
    qx[:, :2] = 0                                                     # the producer's causal zero frames
    qw = torch.randint(-127, 128, (cout, 27 * cin), generator=gen, dtype=torch.int8)
    xs = torch.tensor([0.0123])
    ws = torch.rand(cout, generator=gen) * 1e-3 + 1e-4
    bias = (torch.randn(cout, generator=gen) * 0.5).half() if form != "residual_bias" else None
    res = (torch.randn(b, d, h, w, cout, generator=gen) * 2).half() if form != "none" else None
    rb = (torch.randn(cout, generator=gen) * 0.5).half() if form == "residual_bias" else None
    dq, dw, dxs, dws = qx.to(DEV), qw.to(DEV), xs.to(DEV), ws.to(DEV)
    dbias = bias.to(DEV) if bias is not None else None
    dres = res.to(DEV) if res is not None else None
    drb = rb.to(DEV) if rb is not None else None
    p, st = hip.ptr, hip.stream(DEV)
    geo = (b, cin, d + 2, h + 2, w + 2, cout)
    out = torch.full((b, d + front, h + top + bottom, w + left + right, cout), 0, dtype=torch.int16, device=DEV)
    out.fill_(SENTINEL - 65536 if SENTINEL > 32767 else SENTINEL)
    out = out.view(torch.float16)
    hip.call("h3v_conv3d_i8_residual_padded", p(dq), p(dxs), p(dw), p(dws), p(dbias), p(dres), p(drb), p(out),
             *geo, 1, front, *border, st)
    y = torch.empty((b, d, h, w, cout), dtype=torch.float16, device=DEV)
    if form == "residual":
        hip.call("h3v_conv3d_i8_residual", p(dq), p(dxs), p(dw), p(dws), p(dbias), p(dres), p(y), *geo,
                 3, 3, 3, 1, 1, 1, 1, st)
    else:
        hip.call("h3v_conv3d_i8", p(dq), p(dxs), p(dw), p(dws), p(dbias), p(y), *geo, 3, 3, 3, 1, 1, 1, 1, st)
    torch.cuda.synchronize()
    yv = np_(y)
    if form == "residual_bias":
        v = (np_(res).astype(np.float32) + (yv.astype(np.float32) + np_(rb).astype(np.float32))).astype(np.float16)
        if b == 1 and front == 2:   # the oracle's stage-1 pack of the unpadded conv output
            if border == (0, 1, 0, 1):
                assert_bitwise(_pad_np(v[None, 0], 2, border)[0],
                               oracle.residual_downsample_pack(yv[0], np_(res)[0], np_(rb)), "pack restatement")
    else:
        v = yv
    got = np_(out)
    assert_bitwise(got[:, front:], _pad_np(v, front, border)[:, front:], f"padded output {case}")
    if front:
        assert (got[:, :front].view(np.uint16) == SENTINEL).all(), "frames below front must not be written"


@pytest.fixture(scope="module")
def padded_prefix(pkg):
    """The INT8 prefix as the runtime wires it: downsample convs run as pack + native conv, stage 1's last
    block fused with its downsample, stage 0's last block linked to its downsample conv."""
    mod = lambda n: importlib.import_module(f"{pkg.__name__}.opt.{n}")
    torch.manual_seed(3)
    enc = h3_arch.H3Encoder().half().to(DEV).eval().to(memory_format=torch.channels_last_3d)
    mod("encoder_internal_padding").replace_selected(enc, ["down.0.downsample.conv"])
    prefix = mod("encoder_fused_norm_next").next_fused_prefix(enc, "extend_bias_pack")
    meta = mod("encoder_int8_integration").install_int8_encoder_prefix(prefix, require_cuda=True)
    assert meta["count"] == 8 and all(c["fuse_norm"] for c in meta["convolutions"])
    return prefix, mod


def _cl(t):
    return t.contiguous(memory_format=torch.channels_last_3d)


def test_stage0_end_writes_the_downsample_input(padded_prefix):
    """Stage 0's last block returns a view of the downsample's padded input; the block output and the
    downsample output equal those of the block + causal_reflect_pack path bit for bit."""
    print("stage 0 end: block -> padded downsample input", flush=True)
    prefix, mod = padded_prefix
    block, down = prefix.stages[0].block[-1], prefix.stages[0].downsample
    assert block.padded_consumer is down.conv
    gen = torch.Generator().manual_seed(41)
    x = _cl(torch.randn(1, 128, 5, 64, 64, generator=gen).half().to(DEV))
    with torch.inference_mode():
        y = block(x)
        border = down.conv.native.border
        assert mod("encoder_fp16_conv").padded_input_of(y, 2, border) is not None
        z = down(y)
        consumer, block.padded_consumer = block.padded_consumer, None
        try:
            y_ref = block(x)
            z_ref = down(y_ref)
        finally:
            block.padded_consumer = consumer
        torch.cuda.synchronize()
    assert mod("encoder_fp16_conv").padded_input_of(y_ref, 2, border) is None
    assert_bitwise(ndhwc(y), ndhwc(y_ref), "stage-0 block output")
    assert z.shape == z_ref.shape == (1, 128, 5, 32, 32)
    assert_bitwise(ndhwc(z), ndhwc(z_ref), "stage-0 downsample output")


def test_stage1_end_fused_equals_conv_then_pack(padded_prefix):
    """Stage 1's ResidualDownsampleBlock at a shape the padded conv takes (output width 32) equals its
    body, then residual_downsample_pack, then the downsample conv, bit for bit."""
    print("stage 1 end: ResidualDownsampleBlock at 32 x 32", flush=True)
    prefix, mod = padded_prefix
    block = prefix.stages[1].block[-1]
    gen = torch.Generator().manual_seed(43)
    x = _cl(torch.randn(1, 256, 5, 32, 32, generator=gen).half().to(DEV))
    with torch.inference_mode():
        y = block(x)
        body = block._residual_body(x, None)
        pk = mod("encoder_fused_residual_pack").residual_downsample_pack(body, x, block.second.bias)
        ref = block.down(pk)
        torch.cuda.synchronize()
    assert y.shape == ref.shape == (1, 256, 3, 16, 16)
    assert_bitwise(ndhwc(y), ndhwc(ref), "stage-1 downsample block")
