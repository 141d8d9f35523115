"""GPU parity: decoder attention (h3v_attention_d64) against the float64 oracle.

Tolerance: the kernel rounds the softmax weights to fp16 for the P.V product and
the output to fp16; against float64 it stays within |err| <= 2e-3 + 4e-3 |ref|
for N(0, 1) values (half an fp16 ulp of the output is 2.4e-4 |ref|).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
ATOL, RTOL = 2e-3, 4e-3


def _qkv(b, n, h, seed, qk_scale=1.0):
    """q, k [B, N, H, 64] contiguous and v as the strided slice of a [B, N, H*192] projection."""
    gen = torch.Generator().manual_seed(seed)
    qkv = torch.randn(b, n, h * 192, generator=gen).half()
    q = (torch.randn(b, n, h, 64, generator=gen) * qk_scale).half()
    k = (torch.randn(b, n, h, 64, generator=gen) * qk_scale).half()
    qkv_d = qkv.to(DEV)
    v_d = qkv_d.view(b, n, h, 192)[..., 128:]
    v = qkv.view(b, n, h, 192)[..., 128:]
    return q, k, v, q.to(DEV), k.to(DEV), v_d


def _check(ops, oracle, q, k, v, out, queries=None):
    ref = oracle.attention(q.numpy(), k.numpy(), v.numpy(), 0.125, queries)
    got = out.cpu().numpy().astype(np.float64)
    if queries is not None:
        got = got[:, queries]
    err = np.abs(got - ref)
    bound = ATOL + RTOL * np.abs(ref)
    worst = float((err / bound).max())
    assert worst <= 1.0, f"max err {err.max():.3e} ({worst:.2f} of the bound)"


@pytest.mark.parametrize("b,n,h", [(1, 1, 1), (1, 2, 2), (2, 63, 1), (1, 64, 2), (3, 65, 1), (1, 129, 2),
                                   (2, 200, 3), (1, 513, 1), (2, 1025, 1), (1, 1100, 2), (1, 1537, 1)])
def test_attention_small_shapes_match_oracle(ops, oracle, b, n, h):
    """Key-block (64) and wave (64 queries) edges, and the workgroup edges: a workgroup holds 8 waves of 64
    queries (512), so 513, 1025, 1100 and 1537 tokens put ragged workgroups after full ones; one token, odd
    batches and heads.  Every query is checked."""
    q, k, v, qd, kd, vd = _qkv(b, n, h, seed=b * 1000 + n * 10 + h)
    with torch.inference_mode():
        out = ops.decoder_fused_qk_rope.attention_d64(qd, kd, vd, 0.125)
    torch.cuda.synchronize()
    assert out.shape == (b, n, h, 64) and out.is_contiguous()
    _check(ops, oracle, q, k, v, out)


def test_attention_h3_shape_sampled(ops, oracle):
    """H3 decoder call: B4 x 1797 tokens x 32 heads; the last query and key blocks are ragged."""
    print("attention H3 [4, 1797, 32, 64]", flush=True)
    b, n, h = 4, 1797, 32
    q, k, v, qd, kd, vd = _qkv(b, n, h, seed=1797)
    with torch.inference_mode():
        out = ops.decoder_fused_qk_rope.attention_d64(qd, kd, vd, 0.125)
    torch.cuda.synchronize()
    rng = np.random.default_rng(5)
    # workgroup (512-query) and wave (64-query) edges, the ragged tail, random others
    edges = [0, 1, 63, 64, 127, 128, 511, 512, 1023, 1024, 1535, 1536, 1791, 1792, 1795, 1796]
    queries = np.unique(np.concatenate([edges, rng.integers(0, n, 40)]))
    _check(ops, oracle, q, k, v, out, queries)


def test_attention_large_scores_online_max(ops, oracle):
    """Scores ~ N(0, 64): the running maximum changes across key blocks and exp would overflow without it."""
    q, k, v, qd, kd, vd = _qkv(2, 300, 2, seed=77, qk_scale=2.83)
    with torch.inference_mode():
        out = ops.decoder_fused_qk_rope.attention_d64(qd, kd, vd, 0.125)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    _check(ops, oracle, q, k, v, out)


@pytest.mark.parametrize("direction", [1, -1])
def test_attention_score_ramp_moves_the_lazy_maximum(ops, oracle, direction):
    """The kernel's reference maximum moves only when a score exceeds it by more than 8 / (scale * log2 e)
    (a weight above 2^8).  Key norms growing with the key index make the maximum jump past that margin in
    many blocks (the O and l rescale runs repeatedly); the reverse ramp sets it in the first block and
    leaves later weights tiny (no rescale after block 0, deep exponents)."""
    b, n, h = 1, 700, 2
    q, k, v, qd, kd, vd = _qkv(b, n, h, seed=91 + direction)
    ramp = torch.linspace(0.2, 6.0, n) if direction > 0 else torch.linspace(6.0, 0.2, n)
    k = (k.float() * ramp.view(1, n, 1, 1)).half()
    kd = k.to(DEV)
    with torch.inference_mode():
        out = ops.decoder_fused_qk_rope.attention_d64(qd, kd, vd, 0.125)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    _check(ops, oracle, q, k, v, out)


def test_attention_cfg4_sampled_and_against_torch_sdpa(ops, oracle):
    """one 256x256 tile, 16384 tokens x 16 heads; also compared with torch's SDPA."""
    print("attention cfg4 [1, 16384, 16, 64]", flush=True)
    b, n, h = 1, 16384, 16
    q, k, v, qd, kd, vd = _qkv(b, n, h, seed=4)
    with torch.inference_mode():
        out = ops.decoder_fused_qk_rope.attention_d64(qd, kd, vd, 0.125)
        sdpa = torch.nn.functional.scaled_dot_product_attention(
            qd.transpose(1, 2), kd.transpose(1, 2), vd.transpose(1, 2).contiguous(), scale=0.125).transpose(1, 2)
    torch.cuda.synchronize()
    rng = np.random.default_rng(6)
    edges = [0, 511, 512, 8191, 8192, 16383]
    queries = np.unique(np.concatenate([edges, rng.integers(0, n, 24)]))
    _check(ops, oracle, q, k, v, out, queries)
    assert float((out.float() - sdpa.float()).abs().max()) < 4e-3


def test_attention_rejects_bad_layouts(ops):
    qd = torch.zeros(1, 8, 2, 64, dtype=torch.float16, device=DEV)
    att = ops.decoder_fused_qk_rope.attention_d64
    with pytest.raises(ValueError, match="one shape"):
        att(qd, qd[:, :4], qd, 0.125)
    with pytest.raises(ValueError, match="FP16"):
        att(qd.float(), qd.float(), qd.float(), 0.125)
    odd = torch.zeros(1, 8, 2, 68, dtype=torch.float16, device=DEV)[..., :64]    # head stride 68
    with pytest.raises(ValueError, match="strides"):
        att(odd, odd, odd, 0.125)
    with pytest.raises(ValueError, match="scale"):
        att(qd, qd, qd, 0.0)
