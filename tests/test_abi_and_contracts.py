"""CPU: the C-ABI library and host-side contracts (no kernel launches).

* libh3vae_hip.so loads and exports every entry point declared in
  include/h3vae_hip.h, and the ctypes table covers them all;
* bench.py refuses --gpus above 1 with a message;
* the reference's CPU contract tests, adapted: shape/dtype/layout guards on
  meta tensors, fake (meta) op outputs, weight-quantizer validation with an
  injected quantize function, explicit failure on CPU tensors (no fallback).
"""
from __future__ import annotations

import re
import sys
from pathlib import Path

import pytest
import torch
from torch import nn

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "h3vae_hip.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(h3v_[a-z0-9_]+)\s*\(", text)))


def test_library_loads_and_exports_every_declared_symbol(ops):
    lib = ops.hip.lib()
    names = _declared()
    assert len(names) >= 15
    for name in names:
        assert hasattr(lib, name), name
    table = set(ops.hip.SIGNATURES) | set(ops.hip.SPECIAL)
    assert set(names) == table
    assert lib.h3v_abi_version() == ops.hip.ABI_VERSION
    # per-chunk (avg, M2) partials, per-chunk packed fp16 channel extremes (sized for 256 channels), the 64 KB
    # quantize table, 64 floats of counters, one absmax candidate word per (frame, group)
    assert lib.h3v_gn_norm_pack_workspace_floats(17, 256, 256) == \
        2 * 17 * 256 * 32 + 17 * 256 * 256 + 65536 // 4 + 64 + 17 * 32
    assert lib.h3v_gn_norm_pack_workspace_floats(0, 1, 1) == -1
    # K splits of the FP16 conv: conv_out (1024 -> 48 on 4 x 5 x 16 x 16, 20 row tiles of 256) 12 ways,
    # the 16^2 1024-channel conv (80 tiles of 256 x 256) 3 ways; full-chip convs and window-kernel convs none
    ws = lib.h3v_conv3d_f16_workspace_floats
    assert ws(4, 1024, 7, 18, 18, 48, 3, 3, 3, 1, 1, 1) == 12 * 5120 * 48
    assert ws(4, 1024, 7, 18, 18, 1024, 3, 3, 3, 1, 1, 1) == 3 * 5120 * 1024
    assert ws(1, 128, 19, 258, 258, 128, 3, 3, 3, 1, 2, 2) == 0
    assert ws(4, 256, 11, 66, 66, 256, 3, 3, 3, 1, 1, 1) == 0
    assert ws(1, 128, 2, 18, 18, 128, 3, 3, 3, 1, 1, 1) == -1


def test_entry_points_reject_bad_arguments_before_any_launch(ops):
    """Host-side checks return H3V_EINVAL with a message; nothing touches a device."""
    with pytest.raises(ValueError, match="null pointer"):
        ops.hip.call("h3v_gemm_i8_dequant", None, None, None, None, None, None, 4, 4, 64, None)
    with pytest.raises(ValueError, match="positive"):
        ops.hip.call("h3v_gemm_i8_i32", 1, 1, 1, 0, 4, 64, None)
    with pytest.raises(ValueError, match="accumulator"):
        ops.hip.call("h3v_gemm_i8_i32", 1, 1, 1, 4, 4, 1 << 20, None)
    with pytest.raises(ValueError, match="row width"):
        ops.hip.call("h3v_rms_fp16", 16, 16, 1e-5, 4, 1000, 16, None)
    with pytest.raises(ValueError, match="head_dim 64"):
        ops.hip.call("h3v_qk_rope", 16, 16, 16, 4, 2, 32, 48, 1e-6, 16, 16, None)
    with pytest.raises(ValueError, match="C must be 128 or 256"):
        ops.hip.call("h3v_gn_norm_pack_i8", 16, None, 16, 16, 1e-6, 64, 1, 4, 4, 16, 16, 16, 16, 16, None)
    with pytest.raises(ValueError, match="too small"):
        ops.hip.call("h3v_conv3d_i8", 16, 16, 16, 16, None, 16, 1, 8, 2, 4, 4, 8, 3, 3, 3, 1, 1, 1, 0, None)
    with pytest.raises(ValueError, match="nonempty"):
        ops.hip.call("h3v_tensor_quant_i8", 16, 0, 16, 16, 16, 1024, None)
    with pytest.raises(ValueError, match="scratch holds 1 words"):   # the one-word amax buffer of an older contract
        ops.hip.call("h3v_tensor_quant_i8", 16, 64, 16, 16, 16, 1, None)
    with pytest.raises(ValueError, match="blocks in"):
        ops.hip.call("h3v_probe_mfma_rate", 16, 16, 16, 16, 0, 1, 16, 16, None)
    pad = ("h3v_conv3d_i8_residual_padded", 16, 32, 48, 64, None)
    with pytest.raises(ValueError, match="output width"):   # output width 30 is not a window-kernel width
        ops.hip.call(*pad, 80, None, 96, 1, 128, 4, 10, 32, 128, 1, 2, 1, 1, 1, 1, None)
    with pytest.raises(ValueError, match="needs a residual"):
        ops.hip.call(*pad, None, 80, 96, 1, 128, 4, 18, 34, 128, 1, 2, 0, 1, 0, 1, None)
    with pytest.raises(ValueError, match="alias"):
        ops.hip.call(*pad, 96, None, 96, 1, 128, 4, 18, 34, 128, 1, 2, 0, 1, 0, 1, None)
    with pytest.raises(ValueError, match="front"):
        ops.hip.call(*pad, 80, None, 96, 1, 128, 4, 18, 34, 128, 1, -1, 0, 1, 0, 1, None)
    with pytest.raises(ValueError, match="reflect border"):
        ops.hip.call(*pad, 80, None, 96, 1, 128, 4, 18, 34, 128, 1, 2, 0, 2, 0, 1, None)
    with pytest.raises(ValueError, match="16-byte"):
        ops.hip.call(*pad, 80, None, 98, 1, 128, 4, 18, 34, 128, 1, 2, 1, 1, 1, 1, None)
    # 4 operand sets x 8 MFMAs x 8 waves x 32^3 MACs x 2 ops per iteration
    assert ops.hip.lib().h3v_probe_mfma_ops_per_block(1) == 4 * 8 * 8 * 32 ** 3 * 2


# ---------------------------------------------------------------------------
# reference CPU contracts, adapted (tests/test_int8_ffn_up_fused.py)
# ---------------------------------------------------------------------------

def _ffn_inputs(rows=3, k=2048, n=8192):
    return (torch.empty(rows, k, dtype=torch.int8, device="meta"),
            torch.empty(rows, 1, dtype=torch.float32, device="meta"),
            torch.empty(2 * n, k, dtype=torch.int8, device="meta"),
            torch.empty(2 * n, dtype=torch.float32, device="meta"),
            torch.empty(2 * n, dtype=torch.float16, device="meta"))


def test_ffn_up_shape_dtype_layout_scale_guards(ops):
    validate = ops.int8_ffn_up_fused.validate_prequantized
    values = _ffn_inputs()
    validate(*values)
    validate(*values[:-1], None)
    validate(*_ffn_inputs(k=1024, n=4096))           # the synthetic D=1024 configuration
    cases = [(0, torch.empty(3, 2048, dtype=torch.float16, device="meta")),
             (0, torch.empty(3, 2047, dtype=torch.int8, device="meta")),
             (0, torch.empty(0, 2048, dtype=torch.int8, device="meta")),
             (1, torch.empty(3, 1, dtype=torch.float16, device="meta")),
             (1, torch.empty(3, dtype=torch.float32, device="meta")),
             (2, torch.empty(16383, 2048, dtype=torch.int8, device="meta")),
             (3, torch.empty(16384, dtype=torch.float16, device="meta")),
             (4, torch.empty(16384, dtype=torch.float32, device="meta")),
             (0, torch.empty(2048, 3, dtype=torch.int8, device="meta").t())]
    for index, bad in cases:
        changed = list(values)
        changed[index] = bad
        with pytest.raises(ValueError):
            validate(*changed)


def test_ffn_up_output_indexing_boundary_without_storage(ops):
    validate = ops.int8_ffn_up_fused.validate_prequantized
    validate(*_ffn_inputs(rows=262144))
    with pytest.raises(ValueError, match="32-bit output indexing"):
        validate(*_ffn_inputs(rows=262145))


def test_fake_outputs_have_honest_shapes_and_no_alias(ops):
    x = torch.empty(2, 3, 2048, dtype=torch.float16, device="meta")
    g = torch.empty(2048, dtype=torch.float16, device="meta")
    _, _, w, ws, b = _ffn_inputs()
    down = torch.empty(2048, 8192, dtype=torch.int8, device="meta")
    ds = torch.empty(2048, dtype=torch.float32, device="meta")
    h, out = ops.int8_ffn_up_fused.fused_residual_ffn(x, torch.empty_like(x), g, g, w, ws, b, down, ds, g, 1e-5, 8)
    assert h.shape == x.shape and out.shape == x.shape
    assert h.dtype == torch.float16 and out.dtype == torch.float16
    assert h is not x and out is not x and h is not out
    qw = torch.empty(6144, 2048, dtype=torch.int8, device="meta")
    qkv = ops.int8_norm1_quant.residual_qkv(x, torch.empty_like(x), g, g, qw,
                                            torch.empty(6144, dtype=torch.float32, device="meta"), None)
    assert qkv.shape == (2, 3, 6144)
    xq = torch.empty(2, 5, 32 * 192, dtype=torch.float16, device="meta")
    cs = torch.empty(2, 5, 1, 48, dtype=torch.float16, device="meta")
    q, k = ops.decoder_fused_qk_rope.qk_rope(xq, cs, cs, 32, 1e-6, 8)
    assert q.shape == (2, 5, 32, 64) and k.shape == (2, 5, 32, 64)
    y = ops.decoder_block0_norm.rms_fp16_x2_w16(x, g)
    assert y.shape == x.shape and y.dtype == torch.float16
    y = ops.decoder_final_norm.final_residual_ln_w8(x, x, g, g, g)
    assert y.shape == x.shape


def test_encoder_fake_shapes(ops):
    integ = ops.encoder_int8_integration
    x = torch.empty(2, 6, 5, 8, 10, dtype=torch.float16, device="meta")
    qw = torch.empty(7, 6 * 27, dtype=torch.int8, device="meta")
    y = integ.int8_valid_conv3d_integration(x, qw, torch.empty(7, device="meta"), torch.empty(7, device="meta"),
                                            3, 3, 3, 1, 1, 1, True, "128x128x64")
    assert tuple(y.shape) == (2, 7, 3, 6, 8)         # reference tests/test_encoder_int8_integration.py:233-243
    x = torch.empty(1, 128, 5, 8, 10, dtype=torch.float16, device="meta")
    qw = torch.empty(256, 128 * 27, dtype=torch.int8, device="meta")
    y = integ.int8_norm_conv3d(x, torch.empty(128, dtype=torch.float16, device="meta"),
                               torch.empty(128, dtype=torch.float16, device="meta"), None, 1e-6, qw,
                               torch.empty(256, device="meta"), None)
    assert tuple(y.shape) == (1, 256, 5, 8, 10)
    assert y.is_contiguous(memory_format=torch.channels_last_3d)
    y = integ.int8_norm_conv3d_residual_padded(x, torch.empty(128, dtype=torch.float16, device="meta"),
                                               torch.empty(128, dtype=torch.float16, device="meta"), None, 1e-6, qw,
                                               torch.empty(256, device="meta"), None, None, None, 2, [0, 1, 0, 1],
                                               None, 512)
    assert tuple(y.shape) == (1, 256, 7, 9, 11)      # two leading frames, one reflected row and column
    assert y.is_contiguous(memory_format=torch.channels_last_3d)


def test_ops_fail_loudly_on_cpu_tensors(ops):
    """No silent fallback: CPU inputs raise before any computation."""
    x = torch.randn(2, 2048).half()
    with pytest.raises(RuntimeError, match="gfx950"):
        ops.kitchen_int8.row_quantize(x)
    with pytest.raises(ValueError, match="CUDA rank-5"):
        ops.encoder_int8_norm.quantized_temporal_norm_pad(torch.empty((1, 128, 1, 2, 2), dtype=torch.float16),
                                                          torch.ones(128), torch.zeros(128), 1e-6)
    with pytest.raises(RuntimeError):
        ops.int8_norm_quant.residual_quant(x, x, x[0], x[0], 1e-5)
    q = torch.zeros(3, 2048, dtype=torch.int8)
    with pytest.raises(RuntimeError):
        ops.int8_swiglu_fused.prequantized_linear(q, torch.ones(3, 1), q, torch.ones(3))


# ---------------------------------------------------------------------------
# static weight quantization contract (tests/test_kitchen_int8.py, adapted)
# ---------------------------------------------------------------------------

def _fake_rowwise(weight, stochastic_rounding=0):
    del stochastic_rounding
    scale = weight.detach().abs().amax(dim=-1, keepdim=True).float()
    scale = (scale / 127.0).clamp(min=1e-30)
    q = torch.where(scale > 1e-30, (weight.detach().float() / scale).round(), torch.full_like(scale, -128.0))
    return q.clamp(-128, 127).to(torch.int8), scale


def test_zero_row_normalised_and_scales_fp32(ops):
    source = nn.Linear(5, 3).eval()
    with torch.no_grad():
        source.weight[1].zero_()
    original = source.weight.detach().clone()
    cand = ops.kitchen_int8.KitchenInt8Linear(source, quantize_fn=_fake_rowwise).eval()
    assert tuple(cand.qweight.shape) == (3, 5) and tuple(cand.weight_scale.shape) == (3,)
    assert cand.weight_scale.dtype == torch.float32
    assert torch.equal(cand.qweight[1], torch.zeros(5, dtype=torch.int8))
    assert float(cand.weight_scale[1]) == 1.0
    assert torch.equal(source.weight, original)
    cand.to(dtype=torch.float16)
    assert cand.weight_scale.dtype == torch.float32 and cand.qweight.dtype == torch.int8


def test_nonfinite_and_bad_scales_rejected(ops):
    source = nn.Linear(5, 3).eval()
    with torch.no_grad():
        source.weight[0, 0] = float("nan")
    with pytest.raises(ValueError, match="non-finite source weights"):
        ops.kitchen_int8.KitchenInt8Linear(source, quantize_fn=_fake_rowwise)
    source = nn.Linear(5, 3).eval()

    def bad(weight, stochastic_rounding=0):
        return torch.zeros_like(weight, dtype=torch.int8), torch.zeros(weight.shape[0], 1)

    with pytest.raises(ValueError, match="strictly positive"):
        ops.kitchen_int8.KitchenInt8Linear(source, quantize_fn=bad)


def test_forward_rejects_training_and_grad(ops):
    cand = ops.kitchen_int8.KitchenInt8Linear(nn.Linear(5, 3).eval(), quantize_fn=_fake_rowwise)
    cand.train()
    with pytest.raises(RuntimeError, match="inference-only"):
        cand(torch.randn(2, 5))
    cand.eval()
    with torch.enable_grad(), pytest.raises(RuntimeError, match="no_grad"):
        cand(torch.randn(2, 5, requires_grad=True))


# ---------------------------------------------------------------------------
# encoder weight preparation and install policy
# ---------------------------------------------------------------------------

def test_prepare_int8_weight_matches_oracle_on_cpu(ops, oracle):
    import numpy as np
    w = torch.randn(5, 3, 3, 1, 3)
    q, s, cfg = ops.encoder_int8.prepare_int8_weight(w, stride=(2, 1, 2))
    assert tuple(q.shape) == (5, 27) and cfg.stride == (2, 1, 2)
    ops.encoder_int8.validate_int8_weight_buffers(q, s, cfg)
    assert ops.encoder_int8.int32_accumulator_bound(cfg) < 2 ** 31
    rq, rs = oracle.prepare_conv_weight(w.numpy())
    assert np.array_equal(q.numpy(), rq) and np.array_equal(s.numpy(), rs)


def test_int8_module_keeps_int8_and_has_no_cpu_fallback(ops):
    source = nn.Conv3d(2, 3, 1, bias=True).eval()
    cand = ops.encoder_int8.TritonInt8Conv3d(source, assume_padded=True).eval()
    assert isinstance(cand.qweight, nn.Parameter) and not cand.qweight.requires_grad
    cand.to(dtype=torch.float16)
    assert cand.qweight.dtype == torch.int8
    with pytest.raises(RuntimeError, match="GPU"):
        cand(torch.randn(1, 2, 2, 3, 4))


def test_tile_policy(ops):
    resolve = ops.encoder_int8_integration._resolve_tile_variant
    assert resolve(128, "auto", gfx950=True) == "128x128x64_pipeline4"
    assert resolve(256, None, gfx950=False) == "128x128x64"
    assert resolve(64, "128x64x64") == "128x64x64"
    with pytest.raises(ValueError):
        resolve(64, "auto")


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus 2 exits with status 2 and says so, before torch is imported."""
    import subprocess
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2", "--steps", "1", "--warmup", "0"],
                          capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert proc.returncode == 2
    assert "measures one MI355X" in proc.stderr and "--gpus 1" in proc.stderr
    assert proc.stdout == ""
