"""GPU: h3v_gn_norm_pack_i8_noalloc (static scratch, no allocation) == h3v_gn_norm_pack_i8.

Both entry points are called through the C ABI on the same inputs; q, the scale
and the per-frame statistics must agree bit for bit.  Two calls run back to
back on the no-allocation entry point, the second on a smaller input (and with
a pre-bias), so whatever the first call left in the shared scratch must not
leak into the second.  A size beyond the scratch is rejected on the host.
"""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _inputs(gen, c, d, h, w, pre_bias):
    x = torch.randn(d, h, w, c, generator=gen).half()
    gamma = (1 + 0.1 * torch.randn(c, generator=gen)).half()
    beta = (0.1 * torch.randn(c, generator=gen)).half()
    pb = (0.1 * torch.randn(c, generator=gen)).half() if pre_bias else None
    return [None if t is None else t.to(DEV) for t in (x, gamma, beta, pb)]


def _outputs(c, d, h, w):
    q = torch.full((d + 2, h + 2, w + 2, c), 77, device=DEV, dtype=torch.int8)
    return q, torch.full((), -1.0, device=DEV), torch.full((d, 32, 2), -1.0, device=DEV)


def _with_workspace(hip, x, gamma, beta, pb, c, d, h, w):
    q, scale, stats = _outputs(c, d, h, w)
    ws = torch.empty(int(hip.lib().h3v_gn_norm_pack_workspace_floats(d, h, w)), device=DEV)
    amax = torch.empty(1, device=DEV, dtype=torch.int32)
    hip.call("h3v_gn_norm_pack_i8", hip.ptr(x), hip.ptr(pb), hip.ptr(gamma), hip.ptr(beta), 1e-6, c, d, h, w,
             hip.ptr(q), hip.ptr(scale), hip.ptr(stats), hip.ptr(ws), hip.ptr(amax), hip.stream(DEV))
    return q, scale, stats


def _no_alloc(hip, x, gamma, beta, pb, c, d, h, w):
    q, scale, stats = _outputs(c, d, h, w)
    hip.call("h3v_gn_norm_pack_i8_noalloc", hip.ptr(x), hip.ptr(pb), hip.ptr(gamma), hip.ptr(beta), 1e-6, c, d, h,
             w, hip.ptr(q), hip.ptr(scale), hip.ptr(stats), hip.stream(DEV))
    return q, scale, stats


def test_no_alloc_matches_workspace_entry(ops):
    hip = ops.hip
    gen = torch.Generator().manual_seed(20261002)
    # the larger call first, then a smaller one with a pre-bias and the other channel count
    cases = [(256, 5, 64, 96, False), (128, 2, 16, 24, True)]
    for c, d, h, w, pre in cases:
        print(f"no-alloc norm pack C={c} D={d} H={h} W={w} pre_bias={pre}", flush=True)
        args = _inputs(gen, c, d, h, w, pre)
        got = _no_alloc(hip, *args, c, d, h, w)
        torch.cuda.synchronize()
        want = _with_workspace(hip, *args, c, d, h, w)
        torch.cuda.synchronize()
        for g, r, name in zip(got, want, ("q", "scale", "stats")):
            assert torch.equal(g.view(torch.int8) if name == "q" else g.view(torch.int32),
                               r.view(torch.int8) if name == "q" else r.view(torch.int32)), (name, c, d, h, w)
        assert float(got[1]) > 0


def test_no_alloc_rejects_beyond_scratch(ops):
    hip = ops.hip
    c, d, h, w = 128, 63, 256, 256     # 63 frames of 256 x 256 need more than the 2^21-float scratch
    need = int(hip.lib().h3v_gn_norm_pack_workspace_floats(d, h, w))
    assert need > 1 << 21
    tiny = torch.zeros(16, device=DEV, dtype=torch.float16)
    with pytest.raises(ValueError, match="static scratch"):
        hip.call("h3v_gn_norm_pack_i8_noalloc", hip.ptr(tiny), None, hip.ptr(tiny), hip.ptr(tiny), 1e-6, c, d, h, w,
                 hip.ptr(tiny), hip.ptr(tiny), hip.ptr(tiny), hip.stream(DEV))
