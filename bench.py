"""Benchmark: the H3 VAE INT8 hot path of one full-clip encode + decode on one MI355X.

One step = the INT8 hot path of encoding and decoding a synthetic
1x3x124x768x1344 clip at tile 256 (tile batch 4), with random-init H3-shaped
weights resident in HBM:

* encode: 28 spatial tiles x 8 clips of 17 frames = 224 prefix calls, each
  running the 8 INT8 residual convolutions of encoder stages 0-1 as fused
  GroupNorm/SiLU/pad/quant producer + causal-skipping INT8 conv
  (stage 0: 4 x C128 @ 17x256x256; stage 1: 128->256 and 3 x 256->256 @ 17x128x128);
* decode: 49 decoder calls of 4 tiles (M = 4 x 1797 = 7188 tokens, width
  2048), 36 blocks each: norm1 producer + QKV GEMM (block 0: RMSNorm + row
  quant + GEMM), QK-RMSNorm-RoPE, attention-out row quant + GEMM, norm2
  producer, FFN-up GEMM + SwiGLU requant, FFN-down GEMM; final residual LayerNorm.

The FP16 layers outside the INT8 path (conv_in, downsample and suffix convs,
scaled-dot-product attention, output projection, blending) are not part of
the step.  Kernels are called through the C ABI on preallocated buffers.

Prints one JSON line (rank 0, N=1).  `--gpus N` with N > 1 exits: this build
measures one GPU.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

INT8_PEAK_TOPS = 5033.2  # 256 CU x 8192 int8 ops/clk x 2.4 GHz (dense)
HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2516.6  # 256 CU x 4096 fp16 flops/clk x 2.4 GHz (dense MFMA)

# H3 shapes
ENC_CALLS = 224            # 28 tiles x 8 clips
DEC_CALLS = 49             # 7 temporal chunks x 28 tiles / batch 4
DEC_BLOCKS = 36
DEC_M = 4 * 1797
DEC_D = 2048
DEC_HEADS = 32


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=3)
    p.add_argument("--warmup", type=int, default=1)
    p.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU baseline sample")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-configs", action="store_true", help="skip the per-config (BASELINE configs 1-4) kernel timings")
    p.add_argument("--vs-torch", action="store_true",
                   help="also time the model's F.conv3d (MIOpen) on the FP16 conv configs; its first call per shape "
                        "runs MIOpen's solver search, which takes minutes")
    p.add_argument("--configs-only", action="store_true",
                   help="run only the per-config kernel timings and print them as JSON (for rocprofv3 kernel traces)")
    p.add_argument("--traffic-sample", action="store_true",
                   help="run only a 1 GiB elementwise copy and three stage-0 fused layers (for rocprofv3 --pmc)")
    p.add_argument("--enc-calls", type=int, default=ENC_CALLS, help=argparse.SUPPRESS)
    p.add_argument("--dec-calls", type=int, default=DEC_CALLS, help=argparse.SUPPRESS)
    return p.parse_args()


class Workload:
    """Preallocated synthetic inputs, weights and scratch for the hot path."""

    def __init__(self, torch, hip, kitchen, enc, seed=20261002):
        self.torch, self.hip = torch, hip
        dev = self.dev = torch.device("cuda:0")
        g = torch.Generator(device=dev).manual_seed(seed)
        f16, i8, f32 = torch.float16, torch.int8, torch.float32

        def randn(*shape, scale=1.0):
            return (torch.randn(*shape, generator=g, device=dev, dtype=torch.float32) * scale).to(f16)

        def linear(n, k):
            """Random-init nn.Linear weight N(0, 0.02) quantized per row by the INT8 weight quantizer."""
            q, s = kitchen.quantize_int8_rowwise(randn(n, k, scale=0.02))
            return q, s.reshape(-1).contiguous(), randn(n, scale=0.02)

        def conv(cout, cin):
            """Kaiming-normal 3x3x3 conv weight packed + quantized per output channel (E1)."""
            w = randn(cout, cin, 3, 3, 3, scale=(2.0 / (27 * cin)) ** 0.5)
            qw, ws, _ = enc.prepare_int8_weight(w)
            return qw, ws

        # ---------------- encoder (stage 0 @256^2 C128, stage 1 @128^2) ----------------
        t = 17
        self.enc_layers = []   # (cin, cout, h, w)
        self.enc_layers += [(128, 128, 256, 256)] * 4
        self.enc_layers += [(128, 256, 128, 128)] + [(256, 256, 128, 128)] * 3
        self.enc_w = []
        for cin, cout, h, w in self.enc_layers:
            qw, ws = conv(cout, cin)
            bias = randn(cout, scale=0.02)
            gamma = torch.ones(cin, device=dev, dtype=f16)        # unit GroupNorm affine at init
            beta = torch.zeros(cin, device=dev, dtype=f16)
            self.enc_w.append((qw, ws, bias, gamma, beta))
        self.x0 = randn(t, 256, 256, 128)                         # NDHWC stage-0 input
        self.x1 = randn(t, 128, 128, 128)                         # stage-1 input (after the FP16 downsample)
        self.a0 = torch.empty((t, 256, 256, 128), device=dev, dtype=f16)
        self.a1 = torch.empty((t, 256, 256, 128), device=dev, dtype=f16)
        self.b0 = torch.empty((t, 128, 128, 256), device=dev, dtype=f16)
        self.b1 = torch.empty((t, 128, 128, 256), device=dev, dtype=f16)
        self.q = torch.empty((t + 2) * 258 * 258 * 128, device=dev, dtype=i8)
        self.qscale = torch.empty(1, device=dev, dtype=f32)
        self.stats = torch.empty((t, 32, 2), device=dev, dtype=f32)
        nws = int(hip.lib().h3v_gn_norm_pack_workspace_floats(t, 256, 256))
        self.gn_ws = torch.empty(nws, device=dev, dtype=f32)
        self.amax = torch.empty(1, device=dev, dtype=torch.int32)
        self.t = t

        # ---------------- decoder (36 blocks, width 2048) ----------------
        m, d = DEC_M, DEC_D
        self.blocks = []
        for _ in range(DEC_BLOCKS):
            blk = {
                "g1": torch.ones(d, device=dev, dtype=f16), "g2": torch.ones(d, device=dev, dtype=f16),
                "scale1": randn(d, scale=0.1), "scale2": randn(d, scale=0.1),
            }
            blk["qkv"], blk["qkv_s"], blk["qkv_b"] = linear(6144, d)
            blk["out"], blk["out_s"], blk["out_b"] = linear(d, d)
            blk["up"], blk["up_s"], blk["up_b"] = linear(16384, d)
            blk["down"], blk["down_s"], blk["down_b"] = linear(d, 8192)
            self.blocks.append(blk)
        self.ln_g = torch.ones(d, device=dev, dtype=f16)
        self.ln_b = torch.zeros(d, device=dev, dtype=f16)
        self.tokens0 = randn(m, d)
        self.attn_y = randn(m, d)                     # stand-in for the SDPA output
        cos_sin = torch.rand(m, 48, generator=g, device=dev) * 6.283
        self.cos, self.sin = cos_sin.cos().to(f16), cos_sin.sin().to(f16)
        self.h = torch.empty((m, d), device=dev, dtype=f16)
        self.h2 = torch.empty((m, d), device=dev, dtype=f16)
        self.normed = torch.empty((m, d), device=dev, dtype=f16)
        self.o = torch.empty((m, d), device=dev, dtype=f16)
        self.attn = torch.empty((m, d), device=dev, dtype=f16)
        self.qx = torch.empty((m, 8192), device=dev, dtype=i8)
        self.sx = torch.empty(m, device=dev, dtype=f32)
        self.qkv = torch.empty((m, 6144), device=dev, dtype=f16)
        self.rq = torch.empty((m, DEC_HEADS, 64), device=dev, dtype=f16)
        self.rk = torch.empty((m, DEC_HEADS, 64), device=dev, dtype=f16)
        self.gate_up = torch.empty((m, 16384), device=dev, dtype=f16)
        self.final = torch.empty((m, d), device=dev, dtype=f16)
        self.conv_events = None
        torch.cuda.synchronize()

    # -- raw C-ABI helpers ---------------------------------------------------------------
    def _p(self, t):
        return self.hip.ptr(t)

    def norm_conv(self, x, layer, out, h, w, stream, pre_bias=None):
        cin, cout, _, _ = self.enc_layers[layer]
        qw, ws, bias, gamma, beta = self.enc_w[layer]
        call, p = self.hip.call, self._p
        t = self.t
        call("h3v_gn_norm_pack_i8", p(x), p(pre_bias), p(gamma), p(beta), 1e-6, cin, t, h, w, p(self.q),
             p(self.qscale), p(self.stats), p(self.gn_ws), p(self.amax), stream)
        ev = self.conv_events is not None and cin == 128 and cout == 128
        if ev:
            e0, e1 = self.torch.cuda.Event(enable_timing=True), self.torch.cuda.Event(enable_timing=True)
            e0.record()
        call("h3v_conv3d_i8", p(self.q), p(self.qscale), p(qw), p(ws), p(bias), p(out), 1, cin, t + 2, h + 2, w + 2,
             cout, 3, 3, 3, 1, 1, 1, 1, stream)
        if ev:
            e1.record()
            self.conv_events.append((e0, e1))

    def encode_call(self, stream):
        """One prefix call: 8 fused norm + INT8 conv layers (stage 0 then stage 1)."""
        b = [w[2] for w in self.enc_w]
        self.norm_conv(self.x0, 0, self.a0, 256, 256, stream)
        self.norm_conv(self.a0, 1, self.a1, 256, 256, stream, pre_bias=b[0])
        self.norm_conv(self.a1, 2, self.a0, 256, 256, stream)
        self.norm_conv(self.a0, 3, self.a1, 256, 256, stream, pre_bias=b[2])
        self.norm_conv(self.x1, 4, self.b0, 128, 128, stream)
        self.norm_conv(self.b0, 5, self.b1, 128, 128, stream, pre_bias=b[4])
        self.norm_conv(self.b1, 6, self.b0, 128, 128, stream)
        self.norm_conv(self.b0, 7, self.b1, 128, 128, stream, pre_bias=b[6])

    def decode_call(self, stream):
        """One B4 decoder call: 36 blocks of the INT8 path + the final LayerNorm."""
        call, p = self.hip.call, self._p
        m, d = DEC_M, DEC_D
        h, h2 = self.h, self.h2
        self.h.copy_(self.tokens0)
        for i, blk in enumerate(self.blocks):
            if i == 0:
                call("h3v_rms_fp16", p(h), p(blk["g1"]), 9.999999747378752e-06, m, d, p(self.normed), stream)
                call("h3v_row_quant", p(self.normed), m, d, p(self.qx), p(self.sx), stream)
            else:
                # h <- fp16(h + o * scale2_prev), norm1, row quant (in place on h)
                call("h3v_residual_norm1_quant", p(h), p(self.o), p(self.blocks[i - 1]["scale2"]), p(blk["g1"]),
                     1e-5, m, d, p(h), p(self.qx), p(self.sx), stream)
            call("h3v_gemm_i8_dequant", p(self.qx), p(self.sx), p(blk["qkv"]), p(blk["qkv_s"]), p(blk["qkv_b"]),
                 p(self.qkv), m, 6144, d, stream)
            call("h3v_qk_rope", p(self.qkv), p(self.cos), p(self.sin), m, DEC_HEADS, 64, 48, 1e-6, p(self.rq),
                 p(self.rk), stream)
            # attention itself (SDPA) is outside the INT8 path; its output is a resident stand-in
            call("h3v_row_quant", p(self.attn_y), m, d, p(self.qx), p(self.sx), stream)
            call("h3v_gemm_i8_dequant", p(self.qx), p(self.sx), p(blk["out"]), p(blk["out_s"]), p(blk["out_b"]),
                 p(self.attn), m, d, d, stream)
            call("h3v_residual_rms_quant", p(h), p(self.attn), p(blk["scale1"]), p(blk["g2"]), 1e-5, m, d, p(h2),
                 p(self.qx), p(self.sx), stream)
            # FFN-up + SwiGLU + requant: dequant GEMM over the 16384 [gate | up] weight rows, then the
            # SwiGLU row quantizer (bit-identical to the fused-epilogue GEMM + row quant, and faster)
            call("h3v_gemm_i8_dequant", p(self.qx), p(self.sx), p(blk["up"]), p(blk["up_s"]), p(blk["up_b"]),
                 p(self.gate_up), m, 16384, d, stream)
            call("h3v_swiglu_row_quant", p(self.gate_up), m, 8192, p(self.qx), p(self.sx), stream)
            call("h3v_gemm_i8_dequant", p(self.qx), p(self.sx), p(blk["down"]), p(blk["down_s"]), p(blk["down_b"]),
                 p(self.o), m, d, 8192, stream)
            h, h2 = h2, h
        call("h3v_residual_layernorm", p(h), p(self.o), p(self.blocks[-1]["scale2"]), p(self.ln_g), p(self.ln_b),
             9.999999747378752e-06, m, d, p(self.final), stream)


def mfma_ceiling(torch, hip, wl, stream):
    """Measured INT8 MFMA ceiling for the stage-0 conv's own operands (h3v_probe_mfma_rate).

    The published peak assumes the top shader clock; under a matrix load the part holds a clock that
    depends on the power the MFMAs draw, i.e. on the data.  One stage-0 fused layer leaves its quantized
    input in `wl.q`; the probe multiplies those bytes with the layer's quantized weights from registers
    (no memory traffic), one workgroup of 8 waves per CU, and reports the rate and the mean clock.
    """
    props = torch.cuda.get_device_properties(wl.dev)
    blocks = int(props.multi_processor_count)
    wl.norm_conv(wl.x0, 0, wl.a0, 256, 256, stream)
    a = wl.q[: (wl.t + 2) * 258 * 258 * 128]
    b = wl.enc_w[0][0]
    sink = torch.empty(blocks * 512, device=wl.dev, dtype=torch.int32)
    clocks = torch.empty(2 * blocks, device=wl.dev, dtype=torch.int64)
    iters = 4000
    ops = blocks * int(hip.lib().h3v_probe_mfma_ops_per_block(iters))
    args = (hip.ptr(a), a.numel(), hip.ptr(b), b.numel(), blocks, iters, hip.ptr(sink), hip.ptr(clocks), stream)
    for _ in range(20):                     # ~0.1 s at the sustained clock before timing
        hip.call("h3v_probe_mfma_rate", *args)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 10
    e0.record()
    for _ in range(reps):
        hip.call("h3v_probe_mfma_rate", *args)
    e1.record()
    torch.cuda.synchronize()
    sec = e0.elapsed_time(e1) / 1e3 / reps
    ticks = clocks.view(blocks, 2).double().sum(0).tolist()
    tops = ops / sec / 1e12
    return {
        "kernel": "h3v_probe_mfma_rate: register-resident v_mfma_i32_32x32x32_i8, 8 waves per CU, no memory traffic",
        "data": "stage-0 conv operands: the fused producer's int8 activations x the layer's int8 kaiming weights",
        "tops": round(tops, 1),
        "frac_of_peak": round(tops / INT8_PEAK_TOPS, 4),
        "clock_mhz": round(ticks[0] / ticks[1] * 100.0, 0),
        "blocks": blocks,
    }


def config_measurements(torch, hip, kitchen, enc, stream, reps=20, vs_torch=False):
    """BASELINE.json configs 1-4 on their own shapes: mean kernel time and roofline fraction each.

    Every entry is timed with HIP events on the launch stream over `reps` launches after 3 warm-up
    launches; `frac` is achieved INT8 ops / the INT8 dense peak (MFMA-bound kernels) or algorithmic
    bytes / 8 TB/s (memory-bound kernels).
    """
    import torch.nn.functional as F
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(20261002)
    f16, i8, f32 = torch.float16, torch.int8, torch.float32
    call, p = hip.call, hip.ptr

    def randn(*shape, scale=1.0):
        return (torch.randn(*shape, generator=g, device=dev, dtype=f32) * scale).to(f16)

    def timed(fn):
        for _ in range(3):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        e1.synchronize()
        return e0.elapsed_time(e1) * 1e3 / reps          # microseconds

    def mfma(us, ops):
        return {"us": round(us, 2), "tops": round(ops / us / 1e6, 1), "frac": round(ops / us / 1e6 / INT8_PEAK_TOPS, 4),
                "bound": "mfma", "ops": ops}

    def fp16_mfma(us, flops):
        return {"us": round(us, 2), "tflops": round(flops / us / 1e6, 1),
                "frac": round(flops / us / 1e6 / FP16_PEAK_TFLOPS, 4), "bound": "mfma", "flops": flops}

    def hbm(us, nbytes):
        return {"us": round(us, 2), "gbs": round(nbytes / us / 1e3, 1), "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4),
                "bound": "hbm", "bytes": nbytes}

    out = {}
    with torch.inference_mode():
        # cfg1: causal conv3d C128 -> 128 on [1,128,9,64,64]: per-tensor quant of the padded input + INT8 conv
        x = randn(1, 128, 9, 64, 64)
        xp = F.pad(x.float(), (1, 1, 1, 1, 0, 0), mode="reflect").to(f16)
        xp = F.pad(xp, (0, 0, 0, 0, 2, 0))                                   # two zero causal frames
        xn = xp[0].permute(1, 2, 3, 0).contiguous()                           # [11, 66, 66, 128]
        qw, ws, _ = enc.prepare_int8_weight(randn(128, 128, 3, 3, 3, scale=3456 ** -0.5))
        bias = randn(128, scale=0.1)
        qx = torch.empty(xn.numel(), device=dev, dtype=i8)
        xs = torch.empty(1, device=dev, dtype=f32)
        amax = torch.empty(1, device=dev, dtype=torch.int32)
        y = torch.empty((9, 64, 64, 128), device=dev, dtype=f16)
        t_q = timed(lambda: call("h3v_tensor_quant_i8", p(xn), xn.numel(), p(qx), p(xs), p(amax), stream))
        t_c = timed(lambda: call("h3v_conv3d_i8", p(qx), p(xs), p(qw), p(ws), p(bias), p(y), 1, 128, 11, 66, 66, 128,
                                 3, 3, 3, 1, 1, 1, 1, stream))
        useful = 2 * 36864 * 128 * 3456 * 8 // 9
        out["cfg1_causal_conv3d_c128_9x64x64"] = {"tensor_quant": hbm(t_q, xn.numel() * 3),
                                                   "conv": mfma(t_c, useful)}
        del x, xp, xn, qx, y

        # cfg2: residual + norm1 (RMS, W16 tree) + row quant, then QKV GEMM 1024 -> 3072, M = 16384
        m, d = 16384, 1024
        h, o = randn(m, d), randn(m, d)
        gate, gam, beta = randn(d, scale=0.1), (1 + 0.1 * torch.randn(d, generator=g, device=dev)).to(f16), randn(d, scale=0.02)
        h_out = torch.empty_like(h)
        q = torch.empty((m, 8192), device=dev, dtype=i8)
        sx = torch.empty(m, device=dev, dtype=f32)
        wq, wqs = kitchen.quantize_int8_rowwise(randn(3072, d, scale=0.02))
        wqs = wqs.reshape(-1).contiguous()
        bq = randn(3072, scale=0.02)
        qkv = torch.empty((m, 3072), device=dev, dtype=f16)
        t_n = timed(lambda: call("h3v_residual_norm1_quant", p(h), p(o), p(gate), p(gam), 1e-5, m, d, p(h_out), p(q),
                                 p(sx), stream))
        t_ln = timed(lambda: call("h3v_residual_layernorm", p(h), p(o), p(gate), p(gam), p(beta), 1e-5, m, d, p(h_out),
                                  stream))
        t_g = timed(lambda: call("h3v_gemm_i8_dequant", p(q), p(sx), p(wq), p(wqs), p(bq), p(qkv), m, 3072, d, stream))
        out["cfg2_norm1_qkv_m16384_d1024"] = {"residual_rms_quant": hbm(t_n, m * d * 7 + m * 4),
                                              "residual_layernorm": hbm(t_ln, m * d * 6),
                                              "qkv_gemm": mfma(t_g, 2 * m * 3072 * d)}

        # cfg3: FFN-up GEMM over [gate | up] (1024 -> 2 x 4096) + SwiGLU row quant + down GEMM 4096 -> 1024
        xq = randn(m, d)
        t_rq = timed(lambda: call("h3v_row_quant", p(xq), m, d, p(q), p(sx), stream))
        wu, wus = kitchen.quantize_int8_rowwise(randn(8192, d, scale=0.02))
        wd, wds = kitchen.quantize_int8_rowwise(randn(d, 4096, scale=0.02))
        wus, wds = wus.reshape(-1).contiguous(), wds.reshape(-1).contiguous()
        bu, bd = randn(8192, scale=0.02), randn(d, scale=0.02)
        gu = torch.empty((m, 8192), device=dev, dtype=f16)
        q2 = torch.empty((m, 4096), device=dev, dtype=i8)
        s2 = torch.empty(m, device=dev, dtype=f32)
        yo = torch.empty((m, d), device=dev, dtype=f16)
        t_up = timed(lambda: call("h3v_gemm_i8_dequant", p(q), p(sx), p(wu), p(wus), p(bu), p(gu), m, 8192, d, stream))
        t_sw = timed(lambda: call("h3v_swiglu_row_quant", p(gu), m, 4096, p(q2), p(s2), stream))
        t_dn = timed(lambda: call("h3v_gemm_i8_dequant", p(q2), p(s2), p(wd), p(wds), p(bd), p(yo), m, d, 4096, stream))
        out["cfg3_ffn_m16384_d1024_h4096"] = {"row_quant": hbm(t_rq, m * d * 3 + m * 4),
                                              "up_gemm": mfma(t_up, 2 * m * 8192 * d),
                                              "swiglu_row_quant": hbm(t_sw, m * 8192 * 2 + m * 4096 + m * 4),
                                              "down_gemm": mfma(t_dn, 2 * m * d * 4096)}
        del gu

        # cfg4: QK-RMSNorm-RoPE on [16384, 16 heads x (q|k|v)], attention-out row quant + GEMM 1024 -> 1024
        heads = 16
        qkv4 = randn(m, heads * 192)
        ang = torch.rand(m, 48, generator=g, device=dev) * 6.283
        cos, sin = ang.cos().to(f16), ang.sin().to(f16)
        rq = torch.empty((m, heads, 64), device=dev, dtype=f16)
        rk = torch.empty((m, heads, 64), device=dev, dtype=f16)
        t_r = timed(lambda: call("h3v_qk_rope", p(qkv4), p(cos), p(sin), m, heads, 64, 48, 1e-6, p(rq), p(rk), stream))
        ya = randn(m, d)
        wo, wos = kitchen.quantize_int8_rowwise(randn(d, d, scale=0.02))
        wos = wos.reshape(-1).contiguous()
        bo = randn(d, scale=0.02)
        t_oq = timed(lambda: call("h3v_row_quant", p(ya), m, d, p(q), p(sx), stream))
        t_og = timed(lambda: call("h3v_gemm_i8_dequant", p(q), p(sx), p(wo), p(wos), p(bo), p(yo), m, d, d, stream))
        rope_bytes = m * heads * 128 * 2 * 2 + 2 * m * 48 * 2
        out["cfg4_qk_rope_out_proj_16384tok_16x64"] = {"qk_rope": hbm(t_r, rope_bytes),
                                                       "out_row_quant": hbm(t_oq, m * d * 3 + m * 4),
                                                       "out_gemm": mfma(t_og, 2 * m * d * d)}

        # decoder edge (opt/fp16_finalize.py): one B4 decoder call's tiles [4, 3, 28, 256, 256] fp16 -> fp32
        import ctypes
        px = randn(4, 3, 28, 256, 256)
        pstd = torch.tensor([0.229, 0.224, 0.225], device=dev, dtype=f32)
        pmean = torch.tensor([0.485, 0.456, 0.406], device=dev, dtype=f32)
        pout = torch.empty(px.shape, device=dev, dtype=f32)
        pstrides = (ctypes.c_int64 * 5)(*px.stride())
        t_f = timed(lambda: call("h3v_finalize_pixels", p(px), 1, 4, 28, 256, 256,
                                 ctypes.cast(pstrides, ctypes.c_void_p), p(pstd), p(pmean), p(pout), stream))
        out["edge_finalize_pixels_4x3x28x256x256"] = {"finalize_pixels": hbm(t_f, px.numel() * 6)}

        # decoder attention (head_dim 64): h3v_attention_d64 and torch's SDPA on the same inputs, q/k from the
        # QK-RoPE layout [B, N, H, 64] and v the strided slice of the QKV projection
        def attention_case(b, n, heads):
            qkv_t = randn(b, n, heads * 192)
            qa, ka = randn(b, n, heads, 64), randn(b, n, heads, 64)
            va = qkv_t.view(b, n, heads, 192)[..., 128:]
            oa = torch.empty((b, n, heads, 64), device=dev, dtype=f16)
            t_a = timed(lambda: call("h3v_attention_d64", p(qa), qa.stride(1), qa.stride(2), p(ka), ka.stride(1),
                                     ka.stride(2), p(va), va.stride(1), va.stride(2), p(oa), oa.stride(1), oa.stride(2),
                                     b, n, heads, 0.125, stream))
            qt, kt, vt = qa.transpose(1, 2), ka.transpose(1, 2), va.transpose(1, 2)
            t_s = timed(lambda: F.scaled_dot_product_attention(qt, kt, vt.contiguous(), scale=0.125))
            flops = 4 * b * heads * n * n * 64
            return {"h3v_attention_d64": fp16_mfma(t_a, flops), "torch_sdpa_incl_v_copy": fp16_mfma(t_s, flops)}

        out["attention_h3_4x1797x32x64"] = attention_case(4, 1797, 32)
        out["attention_cfg4_1x16384x16x64"] = attention_case(1, 16384, 16)

        # FP16 encoder convs outside the INT8 path (h3v_conv3d_f16; with --vs-torch also the model's F.conv3d on
        # the same padded channels-last operands and on an NCDHW copy): suffix 3x3x3 convs of a staged batch of 4
        # clips after the producer (two causal zero frames per clip: the kernel skips those taps; flops count the
        # dense reduction), the two prefix downsample convs and a nin_shortcut projection
        def fp16_conv_case(b, cin, cout, dp, hp, wp, k, stride, causal):
            xs = randn(b, cin, dp, hp, wp).contiguous(memory_format=torch.channels_last_3d)
            if causal:
                xs[:, :, :2] = 0
            ws = randn(cout, cin, k, k, k, scale=(k ** 3 * cin) ** -0.5)
            wsp = ws.permute(0, 2, 3, 4, 1).reshape(cout, -1).contiguous()
            bs = randn(cout, scale=0.1)
            do, ho, wo = (dp - k) // stride[0] + 1, (hp - k) // stride[1] + 1, (wp - k) // stride[2] + 1
            ys = torch.empty((b, cout, do, ho, wo), device=dev, dtype=f16).contiguous(
                memory_format=torch.channels_last_3d)
            t_c = timed(lambda: call("h3v_conv3d_f16", p(xs), p(wsp), p(bs), None, p(ys), b, cin, dp, hp, wp, cout, k, k,
                                     k, *stride, int(causal), stream))
            flops = 2 * b * do * ho * wo * cout * k ** 3 * cin
            res = {"h3v_conv3d_f16": fp16_mfma(t_c, flops)}
            if vs_torch:
                res["torch_conv3d"] = fp16_mfma(timed(lambda: F.conv3d(xs, ws, bs, stride=stride)), flops)
                xn = xs.contiguous()
                res["torch_conv3d_ncdhw"] = fp16_mfma(timed(lambda: F.conv3d(xn, ws, bs, stride=stride)), flops)
            return res

        out["suffix_conv_f16_4x256x9x64x64"] = fp16_conv_case(4, 256, 256, 11, 66, 66, 3, (1, 1, 1), True)
        out["suffix_conv_f16_4x512x5x32x32"] = fp16_conv_case(4, 512, 512, 7, 34, 34, 3, (1, 1, 1), True)
        out["suffix_conv_f16_4x1024x5x16x16"] = fp16_conv_case(4, 1024, 1024, 7, 18, 18, 3, (1, 1, 1), True)
        out["downsample0_f16_128x17x256x256_s122"] = fp16_conv_case(1, 128, 128, 19, 258, 258, 3, (1, 2, 2), False)
        out["downsample1_f16_256x17x128x128_s222"] = fp16_conv_case(1, 256, 256, 19, 129, 129, 3, (2, 2, 2), False)
        out["nin_shortcut_f16_128to256x17x128x128"] = fp16_conv_case(1, 128, 256, 17, 128, 128, 1, (1, 1, 1), False)

        # conv_in 3 -> 128 of one clip: tap-folded pack (3x3 taps x 3 channels -> 32, reflect border, two causal
        # zero frames) + the 3x1x1 conv over 32 channels; flops count the 81 real taps x channels
        xin = randn(1, 3, 17, 256, 256).contiguous(memory_format=torch.channels_last_3d)
        xf = torch.empty((1, 32, 19, 256, 256), device=dev, dtype=f16).contiguous(memory_format=torch.channels_last_3d)
        wf = randn(128, 96, scale=81 ** -0.5)
        bf = randn(128, scale=0.1)
        yf = torch.empty((1, 128, 17, 256, 256), device=dev, dtype=f16).contiguous(memory_format=torch.channels_last_3d)

        def conv_in():
            call("h3v_tap_fold_pack", p(xin), p(xf), 1, 3, 17, 256, 256, 2, 32, stream)
            call("h3v_conv3d_f16", p(xf), p(wf), p(bf), None, p(yf), 1, 32, 19, 256, 256, 128, 3, 1, 1, 1, 1, 1, 1,
                 stream)

        t_in = timed(conv_in)
        out["conv_in_f16_3to128x17x256x256"] = {"tap_fold_pack_and_conv3d_f16":
                                                fp16_mfma(t_in, 2 * 17 * 256 * 256 * 128 * 81)}
    torch.cuda.synchronize()
    return out


def enc_ops_per_call():
    """Useful (non-causal-zero) and dense INT8 ops of the 8 convs of one prefix call."""
    useful = dense = 0
    t = 17
    for cin, cout, h, w in [(128, 128, 256, 256)] * 4 + [(128, 256, 128, 128)] + [(256, 256, 128, 128)] * 3:
        per_frame = 2 * h * w * cout * 27 * cin
        dense += t * per_frame
        useful += t * per_frame - per_frame * (2 + 1) // 3     # frame 0 skips 2 of 3 taps, frame 1 skips 1
    return useful, dense


def dec_ops_per_call():
    m, d = DEC_M, DEC_D
    return 2 * m * DEC_BLOCKS * (6144 * d + d * d + 16384 * d + d * 8192)


def cpu_baseline(budget_s: float):
    """The CPU oracle on a bounded sample of the same work, extrapolated by op count."""
    import numpy as np
    import oracle

    threads = len(os.sched_getaffinity(0))
    oracle.set_threads(threads)
    rng = np.random.default_rng(20261002)
    # sample 1: a stage-0 fused layer (norm producer + conv) on 3 frames of 64x256 pixels
    x = rng.standard_normal((3, 64, 256, 128)).astype(np.float16)
    gamma = np.ones(128, np.float16)
    beta = np.zeros(128, np.float16)
    qw = rng.integers(-127, 128, (128, 3456)).astype(np.int8)
    ws = np.full(128, 1e-4, np.float32)
    bias = np.zeros(128, np.float16)
    # sample 2: one decoder block's GEMM work on 64 of 7188 rows
    mrow = 64
    a = rng.integers(-127, 128, (mrow, DEC_D)).astype(np.int8)
    wq = rng.integers(-127, 128, (6144, DEC_D)).astype(np.int8)
    wu = rng.integers(-127, 128, (16384, DEC_D)).astype(np.int8)
    wd = rng.integers(-127, 128, (DEC_D, 8192)).astype(np.int8)
    wo = rng.integers(-127, 128, (DEC_D, DEC_D)).astype(np.int8)
    sx = np.full(mrow, 1e-2, np.float32)
    t_enc = t_dec = 0.0
    n_enc = n_dec = 0
    start = time.perf_counter()
    while time.perf_counter() - start < budget_s or n_enc == 0 or n_dec == 0:
        t0 = time.perf_counter()
        oracle.norm_conv3d(x, gamma, beta, 1e-6, qw, ws, bias)      # out: [3, 64, 256, 128]
        t_enc += time.perf_counter() - t0
        n_enc += 1
        t0 = time.perf_counter()
        qkv = oracle.gemm_dequant(oracle.gemm_acc(a, wq), sx, np.full(6144, 1e-3, np.float32))
        oracle.gemm_dequant(oracle.gemm_acc(a, wo), sx, np.full(DEC_D, 1e-3, np.float32))
        act = oracle.gemm_swiglu(oracle.gemm_acc(a, wu), sx, np.full(16384, 1e-3, np.float32))
        q2, s2 = oracle.row_quant(act)
        oracle.gemm_dequant(oracle.gemm_acc(q2, wd), s2, np.full(DEC_D, 1e-3, np.float32))
        del qkv
        t_dec += time.perf_counter() - t0
        n_dec += 1
    enc_sample_ops = 3 * 64 * 256 * 2 * 128 * 3456          # dense conv ops of the sample (3 frames)
    dec_sample_ops = 2 * mrow * (6144 * DEC_D + DEC_D * DEC_D + 16384 * DEC_D + DEC_D * 8192)
    useful, dense = enc_ops_per_call()
    enc_total = ENC_CALLS * dense
    dec_total = DEC_CALLS * dec_ops_per_call()
    enc_s = (t_enc / n_enc) * enc_total / enc_sample_ops
    dec_s = (t_dec / n_dec) * dec_total / dec_sample_ops
    return {
        "value": round(enc_s + dec_s, 1),
        "unit": "s (extrapolated)",
        "cores": threads,
        "kind": "port",
        "sample": (f"CPU oracle (C, OpenMP {threads} threads): {n_enc}x one fused stage-0 norm+conv on a "
                   f"3x64x256x128 input ({enc_sample_ops / 1e9:.1f} GOP) and {n_dec}x one decoder block's four "
                   f"INT8 GEMMs + SwiGLU + requant on {mrow} of 7188 rows ({dec_sample_ops / 1e9:.1f} GOP); "
                   f"extrapolated by op count to the full step (encode {enc_s:.0f} s + decode {dec_s:.0f} s)"),
    }


TRAFFIC_PROFILE = ROOT / "profiles" / "stage0_conv_traffic_pmc.md"


def stage0_conv_traffic():
    """HBM (L2-miss) bytes per stage-0 conv launch from the committed FETCH_SIZE/WRITE_SIZE summary.

    The summary holds one line `traffic_bytes_per_launch: N`, derived from two rocprofv3 --pmc runs of
    `bench.py --traffic-sample`, each scaled by the counter's reading for a copy of known size.
    """
    try:
        for line in TRAFFIC_PROFILE.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1].strip())
    except OSError:
        pass
    return None


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: the H3 hot path runs per GPU and multi-GPU sharding is not "
              "part of this build (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    import torch
    import __graft_entry__

    pkg = __graft_entry__.load_package()
    import importlib
    hip = importlib.import_module(f"{pkg.__name__}._hip")
    hip.require_gfx950("cuda:0", "bench")
    kitchen = importlib.import_module(f"{pkg.__name__}.opt.kitchen_int8")
    enc = importlib.import_module(f"{pkg.__name__}.opt.encoder_int8")
    wl = Workload(torch, hip, kitchen, enc)
    stream = hip.stream(wl.dev)
    enc_calls, dec_calls = args.enc_calls, args.dec_calls

    if args.configs_only:
        print(json.dumps(config_measurements(torch, hip, kitchen, enc, stream, vs_torch=args.vs_torch)), flush=True)
        return

    if args.traffic_sample:
        # Counter calibration + the dominant kernel in pipeline context.  FETCH_SIZE/WRITE_SIZE of the
        # copy (1 GiB read + 1 GiB written) give the counter's scale; the stage-0 conv launches follow
        # their producer exactly as in a step.
        with torch.inference_mode():
            src = torch.ones(1 << 29, device=wl.dev, dtype=torch.float16)   # 1 GiB
            dst = torch.empty_like(src)
            for _ in range(3):
                torch.neg(src, out=dst)
            for _ in range(3):
                wl.norm_conv(wl.x0, 0, wl.a0, 256, 256, stream)
            torch.cuda.synchronize()
        print("[bench] traffic sample done: 3 x neg(1 GiB fp16), 3 x stage-0 producer + conv", file=sys.stderr)
        return

    def step(timings=None):
        t0 = time.perf_counter()
        for _ in range(enc_calls):
            wl.encode_call(stream)
        if timings is not None:
            torch.cuda.synchronize()
            timings["enc"] += time.perf_counter() - t0
            t0 = time.perf_counter()
        for _ in range(dec_calls):
            wl.decode_call(stream)
        if timings is not None:
            torch.cuda.synchronize()
            timings["dec"] += time.perf_counter() - t0

    def log(msg):
        print(f"[bench] {msg}", file=sys.stderr, flush=True)

    with torch.inference_mode():
        for i in range(args.warmup):
            step()
            torch.cuda.synchronize()
            log(f"warmup step {i + 1}/{args.warmup} done")
        split = {"enc": 0.0, "dec": 0.0}
        step(split)                      # one extra untimed step for the encode/decode split
        log(f"split step: encode {split['enc']:.3f} s, decode {split['dec']:.3f} s")
        wl.conv_events = []
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        log(f"timed {args.steps} steps: {elapsed / args.steps:.3f} s/step")
        conv_ms = [e0.elapsed_time(e1) for e0, e1 in wl.conv_events]
        wl.conv_events = None

    sec_per_step = elapsed / args.steps
    useful, dense = enc_ops_per_call()
    enc_ops = enc_calls * useful
    dec_ops = dec_calls * dec_ops_per_call()
    conv_avg_s = sum(conv_ms) / len(conv_ms) / 1e3
    conv_useful = 17 * 2 * 256 * 256 * 128 * 27 * 128 - 3 * 2 * 256 * 256 * 128 * 9 * 128
    achieved = conv_useful / conv_avg_s / 1e12
    result = {
        "metric": "H3 VAE encode/decode s @768x1344x124 tile256; INT8 MFMA % of peak",
        "value": round(sec_per_step, 4),
        "unit": "s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec_per_step * 1e3, 2),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": ("synthetic, seeded: random-init H3-shaped weights (linears N(0,0.02), kaiming-normal convs, unit norm "
                 "affines) quantized by the build's INT8 weight quantizers; N(0,1) fp16 activations; all resident in HBM"),
        "config": {
            "workload": "h3vae_int8_hot_path_encode_decode_1x3x124x768x1344_tile256",
            "encode_prefix_calls": enc_calls,
            "encode_int8_convs": 8 * enc_calls,
            "decode_calls": dec_calls,
            "decode_blocks": DEC_BLOCKS,
            "decode_tokens_per_call": DEC_M,
            "excluded": "FP16 layers outside the INT8 path: conv_in, downsample/suffix convs, SDPA, output head",
        },
        "encode_s": round(split["enc"], 4),
        "decode_s": round(split["dec"], 4),
        "int8_tops_step": round((enc_ops + dec_ops) / sec_per_step / 1e12, 1),
        "int8_mfma_frac_step": round((enc_ops + dec_ops) / sec_per_step / 1e12 / INT8_PEAK_TOPS, 4),
        "roofline": {
            "kernel": "conv3_halo_i8<256,Dequant> (stage-0 conv C128->128, [1,128,19,258,258] int8)",
            "bound": "mfma",
            "achieved": round(achieved, 1),
            "peak": INT8_PEAK_TOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / INT8_PEAK_TOPS, 4),
            "traffic": stage0_conv_traffic(),
            "launches_timed": len(conv_ms),
            "avg_us": round(conv_avg_s * 1e6, 1),
            "algorithmic_ops_per_launch": conv_useful,
        },
    }
    log("measuring the MFMA ceiling for the stage-0 conv operands")
    with torch.inference_mode():
        ceiling = mfma_ceiling(torch, hip, wl, stream)
    ceiling["conv_frac_of_ceiling"] = round(achieved / ceiling["tops"], 4)
    result["mfma_ceiling"] = ceiling
    if not args.no_configs:
        log("timing BASELINE configs 1-4 on their own shapes")
        result["configs"] = config_measurements(torch, hip, kitchen, enc, stream, vs_torch=args.vs_torch)
    if not args.no_cpu_baseline:
        log("timing the CPU oracle baseline sample")
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
