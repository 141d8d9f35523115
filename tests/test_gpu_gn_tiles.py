"""GPU: GroupNorm statistics written by the INT8 window conv's epilogue (h3v_conv3d_i8_gn) and read by
the INT8 producer (h3v_gn_norm_pack_i8_partials), against the CPU oracle, bit for bit.

* the conv's output is that of h3v_conv3d_i8 / h3v_conv3d_i8_residual (the statistics path shares the
  kernel and only adds to the epilogue);
* the workspace holds exactly oracle.gn_partials_tiled of that output (plus gn_bias): the per-tile
  averages, M2 and channel extremes in the producer's workspace layout;
* the producer on an oracle-filled workspace gives the oracle's stats, scale and int8 codes
  (gn_stats_tiled, then norm_pack);
* the encoder's INT8 residual blocks hand the statistics along (first conv -> second norm, a block's
  second conv -> the next block's first norm) and match the oracle chain that sums each norm's statistics
  in the order the GPU used.
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


def _split_workspace(ws, d, h, w, c):
    """(avg [d,32,n], m2 [d,32,n], ext [d,n,c] uint32) of a producer workspace in the 512-pixel tile layout."""
    n = (h // 8) * (w // 64)
    a = ws.detach().cpu().numpy()
    k = d * 32 * n
    avg = a[:k].reshape(d, 32, n)
    m2 = a[k:2 * k].reshape(d, 32, n)
    ext = a[2 * k:2 * k + d * n * c].view(np.uint32).reshape(d, n, c)
    return avg, m2, ext


def _fill_workspace(ws, avg, m2, ext):
    d, _, n = avg.shape
    k = d * 32 * n
    host = np.zeros(ws.numel(), np.float32)
    host[:k] = avg.reshape(-1)
    host[k:2 * k] = m2.reshape(-1)
    host[2 * k:2 * k + ext.size] = ext.reshape(-1).view(np.float32)
    ws.copy_(torch.from_numpy(host))


# cin, cout, output d, h, w, residual, gn_bias, causal_skip
CASES = [(128, 128, 2, 16, 128, False, False, 0), (128, 128, 3, 8, 256, True, False, 1),
         (256, 256, 2, 8, 128, False, True, 0), (128, 256, 2, 16, 128, True, True, 1),
         (256, 128, 1, 24, 256, False, True, 0)]


@pytest.mark.parametrize("case", CASES)
def test_conv_gn_output_and_partials(ops, oracle, case):
    cin, cout, do, ho, wo, with_res, with_bias, causal = case
    print(f"conv3d_i8_gn cin={cin} cout={cout} out={do}x{ho}x{wo} residual={with_res} gn_bias={with_bias} "
          f"causal_skip={causal}", flush=True)
    hip = ops.hip
    gen = torch.Generator().manual_seed(cin + cout + do * 7 + ho + wo)
    q = torch.randint(-127, 128, (1, do + 2, ho + 2, wo + 2, cin), generator=gen, dtype=torch.int8)
    if causal:
        q[:, :2] = 0                                   # the producer's two zero leading frames
    qw = torch.randint(-127, 128, (cout, 27 * cin), generator=gen, dtype=torch.int8)
    xs = torch.tensor([0.004], dtype=torch.float32)
    wsc = (torch.rand(cout, generator=gen) * 2e-3 + 1e-4).float()
    bias = (torch.randn(cout, generator=gen) * 0.2).half()
    res = (torch.randn(1, do, ho, wo, cout, generator=gen)).half() if with_res else None
    gb = (torch.randn(cout, generator=gen) * 0.5).half() if with_bias else None
    qd, qwd, xsd, wsd, bd = (t.to(DEV) for t in (q, qw, xs, wsc, bias))
    rd = res.to(DEV) if res is not None else None
    gbd = gb.to(DEV) if gb is not None else None
    plain = torch.empty((1, do, ho, wo, cout), dtype=torch.float16, device=DEV)
    fused = torch.full_like(plain, float("nan"))
    nws = int(hip.lib().h3v_gn_norm_pack_workspace_floats(do, ho, wo))
    ws = torch.full((nws,), float("nan"), device=DEV)
    geo = (1, cin, do + 2, ho + 2, wo + 2, cout, 3, 3, 3, 1, 1, 1, causal)
    head = (hip.ptr(qd), hip.ptr(xsd), hip.ptr(qwd), hip.ptr(wsd), hip.ptr(bd))
    if rd is None:
        hip.call("h3v_conv3d_i8", *head, hip.ptr(plain), *geo, hip.stream(DEV))
    else:
        hip.call("h3v_conv3d_i8_residual", *head, hip.ptr(rd), hip.ptr(plain), *geo, hip.stream(DEV))
    hip.call("h3v_conv3d_i8_gn", *head, hip.ptr(rd), hip.ptr(fused), cin, do + 2, ho + 2, wo + 2, cout, causal,
             hip.ptr(gbd), hip.ptr(ws), hip.stream(DEV))
    torch.cuda.synchronize()
    assert_bitwise(fused.cpu(), plain.cpu().numpy(), "conv output")
    avg, m2, ext = _split_workspace(ws, do, ho, wo, cout)
    want_avg, want_m2, want_ext = oracle.gn_partials_tiled(plain.cpu().numpy()[0], None if gb is None else gb.numpy())
    assert np.array_equal(avg.view(np.uint32), want_avg.view(np.uint32)), "tile averages"
    assert np.array_equal(m2.view(np.uint32), want_m2.view(np.uint32)), "tile M2"
    assert np.array_equal(ext, want_ext), "tile channel extremes"


def test_conv_gn_rejects_other_geometry(ops):
    hip = ops.hip
    z = torch.zeros(16, device=DEV)
    with pytest.raises(ValueError, match="output width 128 or 256"):
        hip.call("h3v_conv3d_i8_gn", hip.ptr(z), hip.ptr(z), hip.ptr(z), hip.ptr(z), None, None, hip.ptr(z),
                 128, 4, 10, 66, 128, 0, None, hip.ptr(z), hip.stream(DEV))
    with pytest.raises(ValueError, match="Cout 128 or 256"):
        hip.call("h3v_conv3d_i8_gn", hip.ptr(z), hip.ptr(z), hip.ptr(z), hip.ptr(z), None, None, hip.ptr(z),
                 128, 4, 10, 130, 384, 0, None, hip.ptr(z), hip.stream(DEV))


@pytest.mark.parametrize("c,d,h,w,pre", [(128, 3, 16, 128, False), (256, 2, 8, 256, True), (128, 2, 24, 64, True)])
def test_norm_pack_partials_matches_oracle(ops, oracle, c, d, h, w, pre):
    print(f"gn_norm_pack_i8_partials C={c} D={d} {h}x{w} pre_bias={pre}", flush=True)
    hip = ops.hip
    gen = torch.Generator().manual_seed(c + d + h + w)
    x = (torch.randn(d, h, w, c, generator=gen) * 1.5 + 0.2).half()
    gamma = (1 + 0.3 * torch.randn(c, generator=gen)).half()
    beta = (0.3 * torch.randn(c, generator=gen)).half()
    pb = (0.5 * torch.randn(c, generator=gen)).half() if pre else None
    xn, pbn = x.numpy(), (None if pb is None else pb.numpy())
    avg, m2, ext = oracle.gn_partials_tiled(xn, pbn)
    nws = int(hip.lib().h3v_gn_norm_pack_workspace_floats(d, h, w))
    ws = torch.empty(nws, device=DEV)
    _fill_workspace(ws, avg, m2, ext)
    # device copies bound to names: a temporary's memory could be handed to the next one before the launch
    xd, gd, bd = x.to(DEV), gamma.to(DEV), beta.to(DEV)
    pbd = None if pb is None else pb.to(DEV)
    q = torch.empty((d + 2, h + 2, w + 2, c), dtype=torch.int8, device=DEV)
    scale = torch.empty(1, device=DEV)
    stats = torch.empty((d, 32, 2), device=DEV)
    scratch = torch.empty(1, dtype=torch.int32, device=DEV)
    hip.call("h3v_gn_norm_pack_i8_partials", hip.ptr(xd), hip.ptr(pbd), hip.ptr(gd), hip.ptr(bd), 1e-6, c, d, h, w,
             512, hip.ptr(q), hip.ptr(scale), hip.ptr(stats), hip.ptr(ws), hip.ptr(scratch), hip.stream(DEV))
    torch.cuda.synchronize()
    rstats = oracle.gn_stats_tiled(xn, 1e-6, pbn)
    assert np.array_equal(np_(stats).view(np.uint32), rstats.view(np.uint32)), "stats"
    _, _, amax = oracle.norm_pack(xn, gamma.numpy(), beta.numpy(), rstats, pbn, want_fp16=False)
    rs = oracle.scale_from_amax(amax)
    assert np_(scale)[0] == rs
    _, rq, _ = oracle.norm_pack(xn, gamma.numpy(), beta.numpy(), rstats, pbn, scale=rs, want_fp16=False)
    assert np.array_equal(np_(q), rq), "int8 codes"


def test_norm_pack_partials_rejects_untiled_frames(ops):
    hip = ops.hip
    z = torch.zeros(16, device=DEV)
    with pytest.raises(ValueError, match="multiple of 512"):
        hip.call("h3v_gn_norm_pack_i8_partials", hip.ptr(z), None, hip.ptr(z), hip.ptr(z), 1e-6, 128, 1, 8, 40,
                 512, hip.ptr(z), hip.ptr(z), hip.ptr(z), hip.ptr(z), hip.ptr(z), hip.stream(DEV))
    with pytest.raises(ValueError, match="multiple of 256"):
        hip.call("h3v_gn_norm_pack_i8_partials", hip.ptr(z), None, hip.ptr(z), hip.ptr(z), 1e-6, 128, 1, 8, 40,
                 256, hip.ptr(z), hip.ptr(z), hip.ptr(z), hip.ptr(z), hip.ptr(z), hip.stream(DEV))
    with pytest.raises(ValueError, match="chunk must be"):
        hip.call("h3v_gn_norm_pack_i8_partials", hip.ptr(z), None, hip.ptr(z), hip.ptr(z), 1e-6, 128, 1, 8, 64,
                 128, hip.ptr(z), hip.ptr(z), hip.ptr(z), hip.ptr(z), hip.ptr(z), hip.stream(DEV))


# -- the encoder blocks ----------------------------------------------------------------------------------

@pytest.fixture(scope="module")
def int8_prefix(pkg):
    nn_ = importlib.import_module(f"{pkg.__name__}.opt.encoder_fused_norm_next")
    integ = importlib.import_module(f"{pkg.__name__}.opt.encoder_int8_integration")
    torch.manual_seed(7)
    enc = h3_arch.H3Encoder().half().to(DEV).eval()
    prefix = nn_.next_fused_prefix(enc, "extend_bias_pack")
    meta = integ.install_int8_encoder_prefix(prefix, require_cuda=True)
    assert meta["count"] == 8 and all(c["fuse_norm"] for c in meta["convolutions"])
    return prefix


def _oracle_block(oracle, block, x_nd, tiled_first, tiled_second):
    f, s = block.first, block.second
    i1, i2 = block.int8_first, block.int8_second
    h1, _, _ = oracle.norm_conv3d(x_nd, np_(f.norm_weight), np_(f.norm_bias), f.eps, np_(i1.qweight),
                                  np_(i1.weight_scale), None, None, tiled=tiled_first)
    h2, _, _ = oracle.norm_conv3d(h1, np_(s.norm_weight), np_(s.norm_bias), s.eps, np_(i2.qweight),
                                  np_(i2.weight_scale), np_(i2.bias) if i2.apply_bias else None, np_(f.bias),
                                  tiled=tiled_second)
    return h2


def test_stage0_blocks_hand_statistics_along(int8_prefix, pkg, oracle):
    """Stage 0 at 4 x 64 x 256 (128 tiles per conv): block 0's first norm runs its own statistics pass, its
    second norm and block 1's two norms read the tile statistics of the conv before them."""
    ei = importlib.import_module(f"{pkg.__name__}.opt.encoder_int8")
    assert ei.gn_stats_fits(128, 128, 4, 64, 256)
    print("stage-0 blocks 0 and 1 with tile statistics, x [1, 128, 4, 64, 256]", flush=True)
    b0, b1 = int8_prefix.stages[0].block
    gen = torch.Generator().manual_seed(31)
    x = torch.randn(1, 128, 4, 64, 256, generator=gen).half().to(DEV).contiguous(memory_format=CL)
    with torch.inference_mode():
        y0, p0 = b0.forward_partials(x)
        assert p0 is not None
        y1, _ = b1.forward_partials(y0, p0)
        torch.cuda.synchronize()
    xn = ndhwc(x)[0]
    h2 = _oracle_block(oracle, b0, xn, tiled_first=False, tiled_second=True)
    want0 = (xn.astype(np.float32) + h2.astype(np.float32)).astype(np.float16)
    assert_bitwise(ndhwc(y0)[0], want0, "block 0")
    g2 = _oracle_block(oracle, b1, want0, tiled_first=True, tiled_second=True)
    want1 = (want0.astype(np.float32) + g2.astype(np.float32)).astype(np.float16)
    assert_bitwise(ndhwc(y1)[0], want1, "block 1")


def test_stage1_blocks_hand_statistics_along(int8_prefix, pkg, oracle):
    """Stage 1 at 4 x 64 x 128 (Cout 256: 128 tiles per conv), block 0 with its 128 -> 256 shortcut; block
    1 (the residual downsample block) reads block 0's output statistics in its first norm, and its first
    conv's in its second norm, whose conv writes the downsample's padded input."""
    print("stage-1 blocks 0 and 1 with tile statistics, x [1, 128, 4, 64, 128]", flush=True)
    b0, b1 = int8_prefix.stages[1].block
    gen = torch.Generator().manual_seed(37)
    x = torch.randn(1, 128, 4, 64, 128, generator=gen).half().to(DEV).contiguous(memory_format=CL)
    with torch.inference_mode():
        y0, p0 = b0.forward_partials(x)
        shortcut = b0.shortcut_conv(x)
        assert p0 is not None
        y1, p1 = b1.forward_partials(y0, p0)
        # block 1's INT8 steps as forward_partials runs them (the producer leaves p0's statistics in place)
        h1, hp = b1.int8_first.forward_norm(y0, b1.first.norm_weight, b1.first.norm_bias, b1.first.eps,
                                            x_partials=p0, emit_partials=True, partials_bias=b1.first.bias)
        assert hp is not None
        padded = b1.int8_second.forward_norm(h1, b1.second.norm_weight, b1.second.norm_bias, b1.second.eps,
                                             pre_bias=b1.first.bias, residual=y0, residual_bias=b1.second.bias,
                                             pad_front=2, pad_border=(0, 1, 0, 1), x_partials=hp)
        down = b1.down(padded)
        torch.cuda.synchronize()
    assert p1 is None
    assert_bitwise(y1, np_(down), "block 1 = its steps")
    xn = ndhwc(x)[0]
    h2 = _oracle_block(oracle, b0, xn, tiled_first=False, tiled_second=True)
    want0 = (ndhwc(shortcut)[0].astype(np.float32) + h2.astype(np.float32)).astype(np.float16)
    assert_bitwise(ndhwc(y0)[0], want0, "stage-1 block 0")
    g2 = _oracle_block(oracle, b1, want0, tiled_first=True, tiled_second=True)
    packed = oracle.residual_downsample_pack(g2, want0, np_(b1.second.bias))
    assert_bitwise(ndhwc(padded)[0], packed, "stage-1 block 1 padded output")
