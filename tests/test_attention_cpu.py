"""CPU contracts of the decoder attention op: metadata guards and fake shapes (no launches)."""
from __future__ import annotations

import importlib

import pytest
import torch


@pytest.fixture(scope="module")
def qk(pkg):
    return importlib.import_module(f"{pkg.__name__}.opt.decoder_fused_qk_rope")


def test_attention_guards_before_any_launch(qk):
    """The metadata guards (shared by the op and its fake) raise ValueError; CPU tensors never reach a kernel."""
    q = torch.zeros(2, 8, 2, 64, dtype=torch.float16, device="meta")
    att = torch.ops.h3vae_decoder.attention_d64
    with pytest.raises(ValueError, match="one shape"):
        att(q, q[:, :4], q, 0.125)
    with pytest.raises(ValueError, match="64"):
        att(q[..., :32], q[..., :32], q[..., :32], 0.125)
    with pytest.raises(ValueError, match="strides"):
        att(q.transpose(1, 2), q.transpose(1, 2), q.transpose(1, 2), 0.125)
    with pytest.raises(ValueError, match="nonempty"):
        att(q[:, :0], q[:, :0], q[:, :0], 0.125)
    cpu = torch.zeros(2, 8, 2, 64, dtype=torch.float16)
    with pytest.raises((NotImplementedError, RuntimeError)):
        att(cpu, cpu, cpu, 0.125)                 # no CPU implementation, no fallback


def test_attention_fake_shape_and_strided_v(qk):
    qkv = torch.empty(2, 9, 3 * 192, dtype=torch.float16, device="meta")
    v = qkv.view(2, 9, 3, 192)[..., 128:]
    q = torch.empty(2, 9, 3, 64, dtype=torch.float16, device="meta")
    out = torch.ops.h3vae_decoder.attention_d64(q, q, v, 0.125)
    assert out.shape == (2, 9, 3, 64) and out.is_contiguous()


def test_batched_norm_pack_guards_on_meta(pkg):
    """Reference opt/encoder_fused_batched_norm.py:37-49 scope checks, raised by the op's fake as well."""
    bn = importlib.import_module(f"{pkg.__name__}.opt.encoder_fused_batched_norm")
    op = torch.ops.h3vae_encoder.batched_temporal_norm_pack
    c = 256
    x = torch.empty(4, c, 3, 8, 8, dtype=torch.float16, device="meta").contiguous(memory_format=torch.channels_last_3d)
    v = torch.empty(c, dtype=torch.float16, device="meta")
    y = op(x, None, v, v, 1e-6)
    assert y.shape == (4, c, 5, 10, 10) and y.is_contiguous(memory_format=torch.channels_last_3d)
    assert op(x[:2], None, v, v, 1e-6).shape == (2, c, 5, 10, 10)     # two clips: accepted (the reference raises)
    x5 = torch.empty(5, c, 3, 8, 8, dtype=torch.float16, device="meta").contiguous(memory_format=torch.channels_last_3d)
    with pytest.raises(ValueError, match="B=1..4"):
        op(x5, None, v, v, 1e-6)
    with pytest.raises(ValueError, match="adjacent"):
        op(x.contiguous(), None, v, v, 1e-6)
    with pytest.raises(ValueError, match="channel vectors"):
        op(x, v[:8], v, v, 1e-6)
    assert bn.fused_suffix is not None
