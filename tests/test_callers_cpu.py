"""CPU contracts of the hot path's callers: decoder install/carry wiring, encoder prefix wiring.

Mirrors the reference's CPU tests of these modules (tests/test_int8_qkv.py,
tests/test_int8_attention_out.py, tests/test_int8_norm1_quant.py) on this
build's modules and a reconstructed H3 model (tests/h3_arch.py).
"""
from __future__ import annotations

import copy
import importlib
from unittest.mock import Mock, patch

import pytest
import torch

import h3_arch


@pytest.fixture(scope="module")
def mods(pkg):
    names = ["int8_qkv", "int8_attention_out", "int8_norm1_quant", "decoder_int8", "_modules", "decoder_fused_qk_rope",
             "encoder_fused_norm_bias",
             "encoder_fused_residual_pack", "encoder_fused_norm_next", "encoder_staged_batch",
             "encoder_internal_padding", "encoder_int8_integration"]
    return {n: importlib.import_module(f"{pkg.__name__}.opt.{n}") for n in names}


def _block(width=2048):
    block = torch.nn.Module()
    block.attn = torch.nn.Module()
    block.attn.original = torch.nn.Module()
    block.attn.original.to_qkv = torch.nn.Linear(width, width * 3, device="meta")
    block.attn.original.to_out = torch.nn.Linear(width, width, device="meta")
    block.eval()
    return block


# -- N6 / O1 install helpers (reference tests/test_int8_qkv.py, tests/test_int8_attention_out.py) ----------

def test_chosen_blocks(mods):
    sel = mods["decoder_int8"].chosen_blocks
    assert sel(36) == list(range(36))
    assert sel(36, [3, 7]) == [3, 7]
    for bad in ([], [1, 1], [-1], [36], [True], [1.0]):
        with pytest.raises(ValueError):
            sel(36, bad)


def test_qkv_and_out_linear_validation(mods):
    qkv_linear, out_linear = mods["int8_qkv"].qkv_linear, mods["int8_attention_out"].out_linear
    for width in (1024, 2048, 4096):
        block = _block(width)
        assert qkv_linear(block)[1] is block.attn.original.to_qkv
        assert out_linear(block)[1] is block.attn.original.to_out
    block = _block()
    block.train()
    for fn in (qkv_linear, out_linear):
        with pytest.raises(ValueError):
            fn(block)
        with pytest.raises(ValueError):
            fn(_block(128))
    block = _block()
    block.attn.original.to_out = torch.nn.Identity()
    with pytest.raises(ValueError):
        out_linear(block)


def test_share_containers_alias_and_sharing(mods):
    clone_containers = mods["_modules"].share_containers
    assert mods["int8_attention_out"].clone_containers is clone_containers
    raw = _block()
    raw.alias = raw.attn
    raw.register_buffer("probe", torch.ones(2))
    clone = clone_containers(raw)
    assert clone.attn is not raw.attn
    assert clone.alias is clone.attn
    assert clone.probe is raw.probe
    assert clone.attn.original.to_out.weight is raw.attn.original.to_out.weight
    clone.probe = torch.zeros(2)
    assert torch.equal(raw.probe, torch.ones(2))


def test_qkv_replacement_scope_original_untouched(mods):
    m = mods["int8_qkv"]
    raw = torch.nn.Module()
    raw.transformer_blocks = torch.nn.ModuleList([_block(), _block()])
    raw.eval()
    clone = copy.deepcopy(raw)
    replacement = torch.nn.Identity()
    with patch.object(m, "clone_norm_quant_decoder", return_value=clone), \
            patch.object(mods["decoder_int8"], "KitchenInt8Linear", return_value=replacement) as factory:
        result = m.clone_qkv_int8_decoder(raw, indices=[1])
    assert isinstance(raw.transformer_blocks[1].attn.original.to_qkv, torch.nn.Linear)
    assert isinstance(result.transformer_blocks[0].attn.original.to_qkv, torch.nn.Linear)
    assert result.transformer_blocks[1].attn.original.to_qkv is replacement
    assert factory.call_count == 1 and factory.call_args.kwargs["require_cuda"]


def test_out_replacement_scope_original_untouched(mods):
    m = mods["int8_attention_out"]
    raw = torch.nn.Module()
    raw.transformer_blocks = torch.nn.ModuleList([_block(), _block()])
    raw.eval()
    replacement = torch.nn.Identity()
    with patch.object(mods["decoder_int8"], "KitchenInt8Linear", return_value=replacement) as factory:
        result = m.clone_attention_out_decoder(raw, indices=[1])
    for i in range(2):
        assert isinstance(raw.transformer_blocks[i].attn.original.to_out, torch.nn.Linear)
        assert (result.transformer_blocks[i].attn.original.to_qkv.weight
                is raw.transformer_blocks[i].attn.original.to_qkv.weight)
    assert isinstance(result.transformer_blocks[0].attn.original.to_out, torch.nn.Linear)
    assert result.transformer_blocks[1].attn.original.to_out is replacement
    assert factory.call_count == 1 and factory.call_args.kwargs["require_cuda"]


# -- N5 carry protocol (reference tests/test_int8_norm1_quant.py) -------------------------------------------

def test_final_adapter_shares_parameters_and_keeps_tensor_path(mods):
    source = torch.nn.LayerNorm(2048, eps=1e-5, dtype=torch.float16).eval()
    adapter = mods["decoder_int8"].CarryLayerNorm(source).eval()
    assert set(adapter.state_dict()) == set(source.state_dict())
    assert adapter.weight is source.weight and adapter.bias is source.bias
    with torch.inference_mode():
        x = torch.randn(2, 7, 2048, dtype=torch.float16)
        assert torch.equal(adapter(x), source(x))
        adapter.to(dtype=torch.float32)
        assert adapter.weight is source.weight
        assert torch.equal(adapter(x.float()), source(x.float()))


def test_carry_unpad_rules(mods):
    carry_unpad = mods["decoder_int8"].carry_unpad
    original = Mock(side_effect=lambda states, pad: states)
    unpad = carry_unpad(original)
    carry = (object(), object(), object())
    assert unpad(carry, 0) is carry
    original.reset_mock()
    with pytest.raises(RuntimeError, match="zero sequence padding"):
        unpad(carry, 1)
    original.assert_not_called()
    tensor = torch.empty(2, 5, 3)
    assert unpad(tensor, 1) is tensor
    original.assert_called_once_with(tensor, 1)
    with pytest.raises(RuntimeError, match="preserve final residual carry"):
        carry_unpad(lambda s, p: tuple(list(s)))((object(), object(), object()), 0)


def test_norm1_platform_gate_and_disabled_clone(mods):
    n1 = mods["int8_norm1_quant"]
    assert not n1.supports_norm1_quant("cpu")
    dec = h3_arch.H3Decoder(dim=1024, hidden=512, depth=2).eval()
    clone = n1.clone_norm1_quant_decoder(dec, enabled=False)
    assert clone is not dec and clone._h3vae_norm1_quant_enabled is False
    assert clone.transformer_blocks[0].ff.w1.weight is dec.transformer_blocks[0].ff.w1.weight
    with pytest.raises(RuntimeError, match="gfx950"):
        n1.clone_norm1_quant_decoder(dec, enabled=True)
    with pytest.raises(ValueError, match="eval"):
        n1.clone_norm1_quant_decoder(dec.train())


def test_qk_fusion_clone_wraps_every_attention(mods):
    qk = mods["decoder_fused_qk_rope"]
    dec = h3_arch.H3Decoder(dim=1024, hidden=512, depth=3).eval()
    fused = qk.clone_with_qk_fusion(dec, rows=8)
    assert all(type(b.attn) is qk.FusedQKAttention for b in fused.transformer_blocks)
    assert all(type(b.attn) is h3_arch.H3Attention for b in dec.transformer_blocks)
    assert fused.transformer_blocks[1].attn.original is dec.transformer_blocks[1].attn
    int8_block = mods["decoder_int8"].Int8Block
    assert int8_block(fused.transformer_blocks[0], carry=True)._rope is qk.qk_rope
    with pytest.raises(ValueError, match="FusedQKAttention"):
        int8_block(dec.transformer_blocks[0], carry=True)


# -- no silent eager fallback in the decode-fusion mode ----------------------------------------------------

def test_native_attention_refuses_pack_info_and_missing_rotary(mods):
    qk = mods["decoder_fused_qk_rope"]
    dec = h3_arch.H3Decoder(dim=1024, hidden=512, depth=1).eval()
    native = qk.clone_with_qk_fusion(dec, rows=8).transformer_blocks[0].attn
    q = k = v = torch.zeros(1, 4, 16, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="cannot apply pack_info"):
        qk.run_attention(native, q, k, v, {"cu_seqlens": torch.tensor([0, 4])})
    with torch.inference_mode(), pytest.raises(ValueError, match="rotary table"):
        native(torch.zeros(1, 4, 1024), None, {})
    # the model's attention only on explicit request (the reference's behaviour), pack_info passed through
    model = qk.clone_with_qk_fusion(dec, rows=8, native_attention=False).transformer_blocks[0].attn
    with patch.object(model.original, "perform_attention", return_value="model") as perform:
        assert qk.run_attention(model, q, k, v, {"cu_seqlens": 1}) == "model"
    perform.assert_called_once_with(q, k, v, {"cu_seqlens": 1})


def test_carry_blocks_raise_instead_of_eager_fallback(mods):
    qk, d8 = mods["decoder_fused_qk_rope"], mods["decoder_int8"]
    fused = qk.clone_with_qk_fusion(h3_arch.H3Decoder(dim=1024, hidden=512, depth=2).eval(), rows=8)
    first = d8.Int8Block(fused.transformer_blocks[0], carry=True, first=True).eval()
    second = d8.Int8Block(fused.transformer_blocks[1], carry=True, last=True).eval()
    plain = d8.Int8Block(fused.transformer_blocks[1]).eval()
    h = torch.zeros(1, 4, 1024, dtype=torch.float16)
    rotary = (torch.zeros(1, 4, 1, 48, dtype=torch.float16),) * 2
    with torch.inference_mode():
        # rows the carry kernels cannot take (here: CPU tensors; the block is not on a gfx950 GPU)
        with pytest.raises(ValueError, match="carry kernels take contiguous fp16"):
            first(h, rotary, {})
        with pytest.raises(ValueError, match="carry kernels take contiguous fp16"):
            second((h, h, h[0, 0]), rotary, {})
        # a plain tensor after block 0, a carry into block 0 or into a block built without carry
        with pytest.raises(ValueError, match="previous block's residual carry"):
            second(h, rotary, {})
        with pytest.raises(ValueError, match="does not take one"):
            first((h, h, h[0, 0]), rotary, {})
        with pytest.raises(ValueError, match="does not take one"):
            plain((h, h, h[0, 0]), rotary, {})
    # rows the kernels take, but no rotary table
    with patch.object(second, "_eligible", return_value=True), pytest.raises(ValueError, match="rotary table"):
        second._require_rows(h, None)


# -- E9 / C1 encoder wiring ---------------------------------------------------------------------------------

def test_prefix_structure_and_int8_policy(mods):
    enc = h3_arch.H3Encoder().half().eval()
    prefix = mods["encoder_fused_norm_next"].next_fused_prefix(enc, "extend_bias_pack")
    nb = mods["encoder_fused_norm_bias"]
    rp = mods["encoder_fused_residual_pack"]
    assert [type(b) for b in prefix.stages[0].block] == [nb.BiasFusedResidualBlock] * 2
    assert type(prefix.stages[1].block[0]) is nb.BiasFusedResidualBlock
    assert type(prefix.stages[1].block[1]) is rp.ResidualDownsampleBlock
    assert hasattr(prefix.stages[0], "downsample") and not hasattr(prefix.stages[1], "downsample")
    assert prefix.stages[1].block[0].shortcut is enc.down[1].block[0].nin_shortcut
    assert prefix.stages[1].block[1].down_weight is enc.down[1].downsample.conv.weight
    assert type(enc.down[1].block[1]) is h3_arch.ResnetBlock3D
    meta = mods["encoder_int8_integration"].install_int8_encoder_prefix(prefix, require_cuda=False)
    assert meta["count"] == 8
    applied = [c["apply_bias"] for c in meta["convolutions"]]
    # first convs never add their bias (it becomes the next producer's pre_bias); the last block's
    # second bias is added by the residual pack (reference opt/encoder_int8_integration.py:403-409)
    assert applied == [False, True, False, True, False, True, False, False]
    with pytest.raises(ValueError, match="already has an INT8 wrapper"):
        mods["encoder_int8_integration"].install_int8_encoder_prefix(prefix, require_cuda=False)
    with pytest.raises(ValueError):
        mods["encoder_fused_norm_next"].next_fused_prefix(enc, "extend")


def test_implicit_temporal_pad_geometry_and_no_cpu_fallback(mods):
    """The wrapper reads the model's padding (2*pt zero frames in front, kd-1 for one frame; a reflect
    border of ph/pw, or right/bottom only) and runs only on the GPU: a CPU input raises."""
    ip = mods["encoder_internal_padding"]
    torch.manual_seed(3)
    conv = h3_arch.CausalConv3d(8, 8, 3, stride=(1, 2, 2), padding=(1, 1, 1)).double()
    implicit = ip.ImplicitTemporalPadConv3d(conv)
    assert (implicit.front_video, implicit.front_image) == (2, 2)
    assert implicit.native.border == (1, 1, 1, 1) and implicit.native.stride == (1, 2, 2)
    down = h3_arch.Downsample(8, (2, 2, 2), (1, 0, 0), right_bottom=True)
    assert ip.ImplicitTemporalPadConv3d(down.conv).native.border == (0, 1, 0, 1)
    conv_in = h3_arch.CausalConv3d(3, 16)
    assert ip.ImplicitTemporalPadConv3d(conv_in).native.folded
    with pytest.raises(RuntimeError, match="gfx950"):
        implicit(torch.randn(1, 8, 5, 10, 12, dtype=torch.float64))
    flat = h3_arch.CausalConv3d(8, 8, 3, padding=(0, 1, 1))
    with pytest.raises(ValueError, match="causal zero-temporal-padding"):
        ip.ImplicitTemporalPadConv3d(flat)
    parent = torch.nn.Module()
    parent.child = torch.nn.Module()
    parent.child.conv = conv
    rep = ip.replace_selected(parent, ["child.conv"])
    assert type(parent.child.conv).__name__ == "ImplicitTemporalPadConv3d"
    ip.restore_selected(rep)
    assert parent.child.conv is conv


def test_non_reflect_conv_in_is_refused_before_any_swap(mods):
    ip = mods["encoder_internal_padding"]
    enc = h3_arch.H3Encoder()
    down, conv_in = enc.down[0].downsample.conv, enc.conv_in
    conv_in.pad_mode = "replicate"
    with pytest.raises(ValueError, match="conv_in: .*pad_mode='replicate'.*no conv was replaced"):
        ip.replace_selected(enc, ["down.0.downsample.conv", "conv_in"])
    assert enc.down[0].downsample.conv is down and enc.conv_in is conv_in


def test_encode_staged_clips_batches_and_token_drop(mods):
    staged = mods["encoder_staged_batch"].encode_staged
    calls = []

    def prefix(x):
        assert x.shape[2] == 17
        return x[:, :, ::4][:, :, :5] * 1.0   # 17 frames -> 5 latent frames

    def suffix(batch):
        calls.append(batch.shape[0])
        return batch * 2.0

    video = torch.arange(40, dtype=torch.float32).view(1, 1, 40, 1, 1).expand(1, 2, 40, 2, 2).contiguous()
    out = staged(video, prefix, suffix, clip_length=17, token_drop=3, batch_size=2, cut=2)
    # 40 frames -> 3 clips (last frame repeated 11 times) -> 15 latent frames - 3 dropped
    assert out.shape == (1, 2, 12, 2, 2)
    assert calls == [2, 1]
    frames = [0, 4, 8, 12, 16, 17, 21, 25, 29, 33, 34, 38]
    expected = torch.tensor([2.0 * min(f, 39) for f in frames])
    assert torch.equal(out[0, 0, :, 0, 0], expected)
    with pytest.raises(ValueError):
        staged(video, prefix, suffix, clip_length=17, token_drop=3, batch_size=4, cut=1)
    with pytest.raises(ValueError):
        staged(video[0], prefix, suffix, clip_length=17, token_drop=3, batch_size=2, cut=2)


def test_residual_pack_validation(mods):
    validate = mods["encoder_fused_residual_pack"]._validate_pack
    x = torch.empty((1, 256, 3, 4, 4), dtype=torch.float16, device="meta")
    b = torch.empty((256,), dtype=torch.float16, device="meta")
    validate(x, x, b)
    for bad in (x[:, :250], x.float(), torch.empty((2, 256, 3, 4, 4), dtype=torch.float16, device="meta"),
                x[..., :1]):
        with pytest.raises(ValueError):
            validate(bad, bad, b[: bad.shape[1]] if bad.ndim == 5 else b)
    with pytest.raises(ValueError):
        validate(x, x, b[:128])
