"""GPU: GroupNorm statistics written by the FP16 implicit-GEMM conv's epilogue (h3v_conv3d_f16_gn) for the
INT8 producer that normalises the conv's output next (conv_in -> stage 0's first norm, the stage-0
downsample -> stage 1's first norm), bit for bit.

* the conv's output equals h3v_conv3d_f16's (same kernel, the statistics only add to the epilogue);
* the workspace's averages, M2 and channel extremes equal those the producer's own statistics pass
  (gn_partial, 256-pixel chunks) writes, and the producer reading them (h3v_gn_norm_pack_i8_partials,
  chunk 256) gives the same stats, scale and int8 codes as the producer with its own pass; the stats
  equal the oracle's gn_stats;
* the INT8 encoder prefix with conv_in and the downsample handing their statistics along gives the same
  output as the prefix whose first norms run their own statistics pass.
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
CL = torch.channels_last_3d


def _producer_pair(hip, out, ws_conv, gamma, beta):
    """(own-pass results, partials results, own workspace): h3v_gn_norm_pack_i8 into a fresh workspace and
    h3v_gn_norm_pack_i8_partials (chunk 256) on the conv's workspace, each -> (q, scale, stats)."""
    _, c, d, h, w = out.shape
    nws = int(hip.lib().h3v_gn_norm_pack_workspace_floats(d, h, w))
    ws_own = torch.empty(nws, device=DEV)
    results = []
    for entry, ws in (("h3v_gn_norm_pack_i8", ws_own), ("h3v_gn_norm_pack_i8_partials", ws_conv)):
        q = torch.empty((1, c, d + 2, h + 2, w + 2), dtype=torch.int8, device=DEV, memory_format=CL)
        scale = torch.empty((), device=DEV)
        stats = torch.empty((d, 32, 2), device=DEV)
        scratch = torch.empty(1, dtype=torch.int32, device=DEV)
        head = (hip.ptr(out), None, hip.ptr(gamma), hip.ptr(beta), 1e-6, c, d, h, w)
        chunk = () if entry == "h3v_gn_norm_pack_i8" else (256,)
        hip.call(entry, *head, *chunk, hip.ptr(q), hip.ptr(scale), hip.ptr(stats), hip.ptr(ws), hip.ptr(scratch),
                 hip.stream(DEV))
        results.append((q, scale, stats))
    torch.cuda.synchronize()
    return results[0], results[1], ws_own


def _statistics_words(ws, d, h, w, c=128):
    """The averages, M2 and channel-extreme words of a producer workspace in the 256-pixel layout."""
    n = h * w // 256
    return ws[:2 * d * 32 * n + d * n * c].detach().cpu().numpy().view(np.uint32)


def _check(ops, oracle, out_plain, out, ws, seed):
    assert_bitwise(out, np_(out_plain), "conv output")
    _, c, d, h, w = out.shape
    gen = torch.Generator().manual_seed(seed)
    gamma = (1 + 0.3 * torch.randn(c, generator=gen)).half().to(DEV)
    beta = (0.3 * torch.randn(c, generator=gen)).half().to(DEV)
    (q0, s0, st0), (q1, s1, st1), ws_own = _producer_pair(ops.hip, out, ws, gamma, beta)
    assert np.array_equal(_statistics_words(ws, d, h, w), _statistics_words(ws_own, d, h, w)), "partial statistics"
    assert_bitwise(np_(st1).view(np.uint32), np_(st0).view(np.uint32), "stats")
    assert np_(s1).view(np.uint32) == np_(s0).view(np.uint32)
    assert torch.equal(q1, q0), "int8 codes"
    rstats = oracle.gn_stats(ndhwc(out)[0], 1e-6)
    assert_bitwise(np_(st1).view(np.uint32), rstats.view(np.uint32), "stats against the oracle")


@pytest.mark.parametrize("d, h, w, front", [(5, 64, 64, 2), (3, 32, 48, 2), (1, 16, 16, 2), (4, 64, 32, 0)])
def test_conv_in_statistics(ops, oracle, pkg, d, h, w, front):
    """conv_in's form: tap-folded 3 -> 32 channels, 3x1x1 conv with K = 96 (64-byte K steps)."""
    print(f"conv3d_f16_gn conv_in x [1, 3, {d}, {h}, {w}] front={front}", flush=True)
    f16 = importlib.import_module(f"{pkg.__name__}.opt.encoder_fp16_conv")
    gen = torch.Generator().manual_seed(d * 1000 + h + w)
    x = (torch.rand(1, 3, d, h, w, generator=gen) * 2 - 1).half().to(DEV).contiguous(memory_format=CL)
    weight = (torch.randn(128, 3, 3, 3, 3, generator=gen) * 0.2).half().to(DEV)
    bias = (torch.randn(128, generator=gen) * 0.1).half().to(DEV)
    with torch.inference_mode():
        folded = f16.tap_fold_pack(x, front)
        packed = f16.fold_conv_weight_f16(weight)
        plain = f16.conv3d_f16(folded, packed, bias, [3, 1, 1], [1, 1, 1], front == 2)
        out, ws = f16.conv3d_f16_gn(folded, packed, bias, [3, 1, 1], [1, 1, 1], front == 2)
    _check(ops, oracle, plain, out, ws, d + h)


@pytest.mark.parametrize("d, h, w", [(5, 65, 129), (2, 33, 65), (3, 33, 33)])
def test_downsample_statistics(ops, oracle, pkg, d, h, w):
    """The stage-0 downsample's form: Cin 128, stride (1, 2, 2) over a padded input (128-byte K steps); the
    output frames are (h - 1) / 2 x (w - 1) / 2 pixels."""
    print(f"conv3d_f16_gn stride (1, 2, 2) x [1, 128, {d + 2}, {h}, {w}]", flush=True)
    f16 = importlib.import_module(f"{pkg.__name__}.opt.encoder_fp16_conv")
    gen = torch.Generator().manual_seed(d * 100 + h + w)
    x = torch.randn(1, 128, d + 2, h, w, generator=gen).half().to(DEV).contiguous(memory_format=CL)
    x[:, :, :2] = 0
    weight = (torch.randn(128, 128, 3, 3, 3, generator=gen) * (128 * 27) ** -0.5).half().to(DEV)
    bias = (torch.randn(128, generator=gen) * 0.1).half().to(DEV)
    packed = f16.pack_conv_weight_f16(weight)
    assert f16.conv3d_f16_gn_fits(x, packed, [3, 3, 3], [1, 2, 2])
    with torch.inference_mode():
        out, ws = f16.conv3d_f16_gn(x, packed, bias, [3, 3, 3], [1, 2, 2], True)
        # h3v_conv3d_f16 itself (the op may split the reduction of so small a conv over a workspace; the
        # stage-0 downsample of config 5, 1088 tiles, does not)
        plain = torch.empty_like(out)
        hip = ops.hip
        hip.call("h3v_conv3d_f16", hip.ptr(x), hip.ptr(packed), hip.ptr(bias), None, hip.ptr(plain), 1, 128, d + 2,
                 h, w, 128, 3, 3, 3, 1, 2, 2, 1, hip.stream(DEV))
    _check(ops, oracle, plain, out, ws, d + w)


def test_conv3d_f16_gn_rejects_other_geometries(ops):
    hip = ops.hip
    z = torch.zeros(64, device=DEV)
    with pytest.raises(ValueError, match="128 output channels"):   # Cout 64
        hip.call("h3v_conv3d_f16_gn", hip.ptr(z), hip.ptr(z), None, hip.ptr(z), 32, 3, 16, 16, 64, 3, 1, 1, 1, 1, 1,
                 1, hip.ptr(z), hip.stream(DEV))
    with pytest.raises(ValueError, match="multiple of 256 pixels"):   # 10 x 16 output frame
        hip.call("h3v_conv3d_f16_gn", hip.ptr(z), hip.ptr(z), None, hip.ptr(z), 32, 3, 10, 16, 128, 3, 1, 1, 1, 1,
                 1, 1, hip.ptr(z), hip.stream(DEV))


@pytest.fixture(scope="module")
def int8_prefix_wrapped(pkg):
    """The INT8 encoder prefix as the runtime builds it: conv_in and the stage-0 downsample conv wrapped."""
    pad = importlib.import_module(f"{pkg.__name__}.opt.encoder_internal_padding")
    nn_ = importlib.import_module(f"{pkg.__name__}.opt.encoder_fused_norm_next")
    integ = importlib.import_module(f"{pkg.__name__}.opt.encoder_int8_integration")
    torch.manual_seed(11)
    enc = h3_arch.H3Encoder().half().to(DEV).eval()
    pad.replace_selected(enc, ["down.0.downsample.conv", "conv_in"])
    prefix = nn_.next_fused_prefix(enc, "extend_bias_pack")
    meta = integ.install_int8_encoder_prefix(prefix, require_cuda=True)
    assert meta["count"] == 8
    return prefix


def test_prefix_hands_conv_statistics_along(int8_prefix_wrapped, pkg, monkeypatch):
    """x [1, 3, 5, 128, 256]: stage 0 at 5 x 128 x 256, stage 1 at 5 x 64 x 128, as at config 5 but five
    frames.  With and without conv_in's and the downsample's statistics the prefix output is bit-identical."""
    staged = importlib.import_module(f"{pkg.__name__}.opt.encoder_staged_batch")
    prefix = int8_prefix_wrapped
    print("INT8 prefix x [1, 3, 5, 128, 256] with and without the conv statistics", flush=True)
    gen = torch.Generator().manual_seed(5)
    x = (torch.rand(1, 3, 5, 128, 256, generator=gen) * 2 - 1).half().to(DEV).contiguous(memory_format=CL)
    with torch.inference_mode():
        assert staged._reads_partials(prefix.stages[0]) and staged._reads_partials(prefix.stages[1])
        _, p_in = prefix.conv_in.forward_partials(x)
        assert p_in is not None and p_in.chunk == 256
        with_stats = prefix(x)
        torch.cuda.synchronize()
        monkeypatch.setattr(staged, "_reads_partials", lambda stage: False)
        own_pass = prefix(x)
        torch.cuda.synchronize()
    assert_bitwise(with_stats, np_(own_pass), "prefix output")
