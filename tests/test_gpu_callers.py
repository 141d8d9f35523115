"""GPU parity of the hot path's callers against the CPU oracle (bit for bit).

* E9: the encoder prefix blocks with INT8 wrappers (BiasFusedResidualBlock,
  ResidualDownsampleBlock) and the residual downsample pack kernel;
* N5/N6/O1/F7/R2: the decoder carry protocol on a reconstructed H3 decoder
  with INT8 QKV / attention-out / FFN installs, block 0 RMS, fused
  residual+norm1+QKV for blocks 1.., and the final residual LayerNorm.

The FP16 layers outside the INT8 path (nin_shortcut, downsample convs, and
attention itself) are evaluated by the same call (h3v_conv3d_f16 through
opt/encoder_fp16_conv.py; their own parity is in test_gpu_conv_f16.py) on
identical inputs on both sides.  The decoder chain test uses the elementwise attention
stand-in of tests/h3_arch.py so every value stays checkable bit for bit.
"""
from __future__ import annotations

import importlib

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import h3_arch
from _util import assert_bitwise, ndhwc, np_

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


@pytest.fixture(scope="module")
def mods(pkg):
    names = ["int8_qkv", "int8_attention_out", "int8_norm1_quant", "decoder_fused_qk_rope", "kitchen_int8",
             "encoder_fused_norm_bias", "encoder_fused_residual_pack", "encoder_fused_norm_next",
             "encoder_int8_integration", "decoder_block0_norm", "decoder_final_norm", "encoder_fp16_conv"]
    return {n: importlib.import_module(f"{pkg.__name__}.opt.{n}") for n in names}


def _cl(t):
    return t.contiguous(memory_format=torch.channels_last_3d)


@pytest.mark.parametrize("shape", [(256, 3, 8, 8), (128, 2, 5, 7), (64, 1, 2, 2), (256, 17, 128, 128)])
def test_residual_downsample_pack_matches_oracle(mods, oracle, shape):
    c, d, h, w = shape
    print(f"residual_downsample_pack C={c} D={d} H={h} W={w}", flush=True)
    gen = torch.Generator().manual_seed(20261002 + c + d)
    x = torch.randn(1, c, d, h, w, generator=gen).half()
    r = torch.randn(1, c, d, h, w, generator=gen).half()
    b = (0.5 * torch.randn(c, generator=gen)).half()
    with torch.inference_mode():
        y = mods["encoder_fused_residual_pack"].residual_downsample_pack(_cl(x.to(DEV)), r.to(DEV), b.to(DEV))
        torch.cuda.synchronize()
    assert y.shape == (1, c, d + 2, h + 1, w + 1) and y.is_contiguous(memory_format=torch.channels_last_3d)
    want = oracle.residual_downsample_pack(ndhwc(x)[0], ndhwc(r)[0], np_(b))
    assert_bitwise(ndhwc(y)[0], want, f"pack {shape}")


@pytest.fixture(scope="module")
def int8_prefix(mods):
    torch.manual_seed(7)
    enc = h3_arch.H3Encoder().half().to(DEV).eval()
    prefix = mods["encoder_fused_norm_next"].next_fused_prefix(enc, "extend_bias_pack")
    meta = mods["encoder_int8_integration"].install_int8_encoder_prefix(prefix, require_cuda=True)
    assert meta["count"] == 8 and all(c["fuse_norm"] for c in meta["convolutions"])
    return enc, prefix


def _oracle_body(oracle, block, x_nd):
    """Two fused norm+conv layers of a block on the oracle -> fp16 NDHWC [D, H, W, Cout]."""
    f, s = block.first, block.second
    i1, i2 = block.int8_first, block.int8_second
    h1, _, _ = oracle.norm_conv3d(x_nd, np_(f.norm_weight), np_(f.norm_bias), f.eps, np_(i1.qweight),
                                  np_(i1.weight_scale), None, None)
    h2, _, _ = oracle.norm_conv3d(h1, np_(s.norm_weight), np_(s.norm_bias), s.eps, np_(i2.qweight),
                                  np_(i2.weight_scale), np_(i2.bias) if i2.apply_bias else None, np_(f.bias))
    return h2


@pytest.mark.parametrize("where", [(0, 0, 128, 16), (0, 1, 128, 16), (1, 0, 128, 8)])
def test_bias_fused_block_matches_oracle(int8_prefix, mods, oracle, where):
    stage, index, cin, hw = where
    print(f"BiasFusedResidualBlock stage={stage} block={index}", flush=True)
    _, prefix = int8_prefix
    block = prefix.stages[stage].block[index]
    gen = torch.Generator().manual_seed(11 + stage * 10 + index)
    x = _cl(torch.randn(1, cin, 5, hw, hw, generator=gen).half().to(DEV))
    with torch.inference_mode():
        y = block(x)
        shortcut = block.shortcut_conv(x) if block.shortcut_conv is not None else x
        torch.cuda.synchronize()
    h2 = _oracle_body(oracle, block, ndhwc(x)[0])
    want = (ndhwc(shortcut)[0].astype(np.float32) + h2.astype(np.float32)).astype(np.float16)
    assert_bitwise(ndhwc(y)[0], want, f"block {stage}.{index}")


def test_residual_downsample_block_matches_oracle(int8_prefix, mods, oracle):
    print("ResidualDownsampleBlock stage=1 block=1", flush=True)
    _, prefix = int8_prefix
    block = prefix.stages[1].block[1]
    gen = torch.Generator().manual_seed(23)
    x = _cl(torch.randn(1, 256, 5, 8, 8, generator=gen).half().to(DEV))
    with torch.inference_mode():
        y = block(x)
        body = block._residual_body(x, None)
        pk = mods["encoder_fused_residual_pack"].residual_downsample_pack(body, x, block.second.bias)
        # the FP16 downsample conv on the very same tensor
        conv = block.down(pk)
        torch.cuda.synchronize()
    h2 = _oracle_body(oracle, block, ndhwc(x)[0])
    assert_bitwise(ndhwc(body)[0], h2, "residual body")
    packed = oracle.residual_downsample_pack(h2, ndhwc(x)[0], np_(block.second.bias))
    assert_bitwise(ndhwc(pk)[0], packed, "residual pack")
    assert y.shape == (1, 256, 3, 4, 4)
    assert_bitwise(ndhwc(y), ndhwc(conv), "downsample block")


def test_prefix_runs_all_int8_blocks(int8_prefix):
    enc, prefix = int8_prefix
    gen = torch.Generator().manual_seed(5)
    x = _cl(torch.rand(1, 3, 17, 32, 32, generator=gen).half().to(DEV) * 2 - 1)
    with torch.inference_mode():
        y = prefix(x)
        ref = enc.down[1].downsample(enc.down[1].block[1](enc.down[1].block[0](
            enc.down[0].downsample(enc.down[0].block[1](enc.down[0].block[0](enc.conv_in(x)))))))
        torch.cuda.synchronize()
    assert y.shape == ref.shape == (1, 256, 9, 8, 8)
    assert torch.isfinite(y).all()
    # INT8 quantisation error against the FP16 modules stays small
    rel = (y.float() - ref.float()).norm() / ref.float().norm()
    assert rel < 0.1, float(rel)


# -- decoder ---------------------------------------------------------------------------------------------

def _int8_decoder(mods, raw, native_attention=False):
    # by default the model's perform_attention (the architecture's "sum" stand-in) keeps the chain bit-exact
    dec = mods["decoder_fused_qk_rope"].clone_with_qk_fusion(raw, 8, native_attention=native_attention)
    mods["kitchen_int8"].install_kitchen_int8_ffn(dec, mode="INT8both", require_cuda=True)
    dec = mods["int8_attention_out"].from_raw_decoder(dec, warps=8)
    return mods["int8_norm1_quant"].clone_norm1_quant_decoder(dec, enabled=True)


def _oracle_decoder(oracle, dec, x, cos, sin):
    """The carry protocol restated with oracle functions -> fp16 [B, N, D]."""
    b, n, d = x.shape
    m = b * n
    blocks = dec.transformer_blocks
    eps_rms = 9.999999747378752e-06   # fp32(1e-5), the block-0 RMS and final LayerNorm epsilon
    states = np_(x).reshape(m, d)
    carry = None
    for i, blk in enumerate(blocks):
        a = blk.attn.original
        qkv_l, out_l, w1, w2 = a.to_qkv, a.to_out, blk.ff.w1, blk.ff.w2
        if i == 0:
            normed = oracle.rms_fp16(states, np_(blk.norm1.weight), eps_rms)
            qkv = oracle.int8_linear(normed, np_(qkv_l.qweight), np_(qkv_l.weight_scale), np_(qkv_l.bias))
        else:
            h, out, gate = carry
            states, q1, s1 = oracle.residual_rms_quant(h, out, gate, np_(blk.norm1.weight), 1e-5, recipe=0)
            qkv = oracle.gemm_dequant(oracle.gemm_acc(q1, np_(qkv_l.qweight)), s1, np_(qkv_l.weight_scale),
                                      np_(qkv_l.bias))
        q, k = oracle.qk_rope(qkv.reshape(b, n, 3 * d), np_(cos), np_(sin), a.heads, a.norm_q.eps)
        v = qkv.reshape(b, n, a.heads, 3 * a.dim_head)[..., 2 * a.dim_head:]
        y = (q + k) + v
        attn = oracle.int8_linear(y.reshape(m, d), np_(out_l.qweight), np_(out_l.weight_scale), np_(out_l.bias))
        h, q2, s2 = oracle.residual_rms_quant(states, attn, np_(blk.scale1), np_(blk.norm2.weight), blk.norm2.eps,
                                              recipe=1)
        act = oracle.gemm_swiglu(oracle.gemm_acc(q2, np_(w1.qweight)), s2, np_(w1.weight_scale), np_(w1.bias))
        aq, asc = oracle.row_quant(act)
        out = oracle.gemm_dequant(oracle.gemm_acc(aq, np_(w2.qweight)), asc, np_(w2.weight_scale), np_(w2.bias))
        carry = (h, out, np_(blk.scale2))
    h, out, gate = carry
    y = oracle.residual_layernorm(h, out, gate, np_(dec.norm_out.weight), np_(dec.norm_out.bias), eps_rms)
    return y.reshape(b, n, d)


@pytest.mark.parametrize("dim,hidden,depth,batch,tokens", [(1024, 1024, 3, 2, 96), (2048, 2048, 2, 1, 130)])
def test_decoder_carry_chain_matches_oracle(mods, oracle, dim, hidden, depth, batch, tokens):
    print(f"decoder carry chain D={dim} F={hidden} blocks={depth} B={batch} N={tokens}", flush=True)
    torch.manual_seed(dim + depth)
    raw = h3_arch.H3Decoder(dim=dim, hidden=hidden, depth=depth).half().to(DEV).eval()
    raw.set_mix("sum")
    with torch.inference_mode():
        dec = _int8_decoder(mods, raw)
        blocks = dec.transformer_blocks
        assert [(b.first, b.last) for b in blocks] == [(i == 0, i == depth - 1) for i in range(depth)]
        assert all(b.fuse_norm1 and b.fuse_ffn_up for b in blocks)
        gen = torch.Generator().manual_seed(31)
        x = torch.randn(batch, tokens, dim, generator=gen).half().to(DEV)
        cos, sin = (t.to(DEV) for t in h3_arch.rope_tables(batch, tokens))
        y = dec(x, (cos, sin), {})
        torch.cuda.synchronize()
    # static weights: the row quantizer applied to each fp16 weight
    lin = blocks[0].attn.original.to_qkv
    wq, ws = oracle.row_quant(np_(raw.transformer_blocks[0].attn.to_qkv.weight))
    assert np.array_equal(np_(lin.qweight), wq) and np.array_equal(np_(lin.weight_scale), ws)
    want = _oracle_decoder(oracle, dec, x, cos, sin)
    assert_bitwise(y, want, "decoder carry chain")


@pytest.mark.parametrize("native_attention", [False, True])
def test_decoder_int8_close_to_fp16_model(mods, native_attention):
    """The INT8 decoder (with the model's SDPA, or with h3v_attention_d64) against the fp16 model."""
    torch.manual_seed(3)
    raw = h3_arch.H3Decoder(dim=1024, hidden=2048, depth=3).half().to(DEV).eval()
    gen = torch.Generator().manual_seed(9)
    x = torch.randn(2, 200, 1024, generator=gen).half().to(DEV)
    cos, sin = (t.to(DEV) for t in h3_arch.rope_tables(2, 200))
    with torch.inference_mode():
        ref = raw(x, (cos, sin), {})
        y = _int8_decoder(mods, raw, native_attention)(x, (cos, sin), {})
        torch.cuda.synchronize()
    assert torch.isfinite(y).all()
    rel = (y.float() - ref.float()).norm() / ref.float().norm()
    assert rel < 0.05, float(rel)
