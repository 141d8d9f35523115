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
