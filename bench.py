"""Benchmark: full-VAE encode + decode of the H3 video VAE on one MI355X.

One step = ``runtime.encode`` of a synthetic fp16 1x3x124x768x1344 clip, then
``runtime.decode`` of its latents into a preallocated fp32 pixel buffer, through
``H3VAEPyOptRuntime`` in the modes of the reference's headline numbers
(README.md:43,53-54: INT8 encode, INT8 fused decode, tile 256, staged batch 4,
tile batch 4).  The model is a random-init reconstruction of the H3
architecture (``reconstructed_h3``; the MiniMax model code is not available).
Nothing is excluded: conv_in, every encoder stage, the blends, every decoder
block with its attention, the output head and the pixel finalisation run.

* encode: 28 spatial tiles (4 x 7 at 256 px) x 8 clips of 17 frames: 224
  prefix calls (8 INT8 convs each), 56 clip-batched suffix calls, stitching;
* decode: 7 temporal chunks x 28 tiles = 196 tiles in 49 calls of 4
  (M = 4 x 1797 = 7188 tokens, width 2048, 36 blocks), blending, finalisation.

The dominant kernel's roofline (stage-0 INT8 conv) and the FFN-up GEMM's are
timed with HIP events around their launches inside the timed steps.  BASELINE.json
configs 1-4 are timed on their own shapes afterwards, then a CPU baseline.

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
REF_ENCODE_S = 8.458108    # reference, RTX PRO 5000, INT8 encode (README.md:43,53)
REF_DECODE_S = 6.440266    # reference, RTX PRO 5000, INT8 fused decode (README.md:43,54)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=3)
    p.add_argument("--warmup", type=int, default=1)
    p.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU baseline sample")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-configs", action="store_true", help="skip the per-config (BASELINE.json configs 1-4) kernel timings")
    p.add_argument("--vs-torch", action="store_true",
                   help="also time the model's F.conv3d (MIOpen) on the FP16 conv configs; its first call per shape "
                        "runs MIOpen's solver search, which takes minutes")
    p.add_argument("--configs-only", action="store_true",
                   help="run only the per-config kernel timings and print them as JSON (for rocprofv3 kernel traces)")
    p.add_argument("--traffic-sample", action="store_true",
                   help="run only a 1 GiB elementwise copy and the step's and configs' INT8 convs and GEMMs, "
                        "3 launches each (for rocprofv3 --pmc)")
    p.add_argument("--frames", type=int, default=124, help=argparse.SUPPRESS)
    p.add_argument("--depth", type=int, default=DEC_BLOCKS, help=argparse.SUPPRESS)
    return p.parse_args()


def synthetic_clip(torch, dev, seed=20261002, shape=(1, 3, 124, 768, 1344)):
    """fp16 clip = clamp(U(-1, 1) + bilinearly upsampled coarse noise, -1, 1) (seeded, generated on the GPU)."""
    import torch.nn.functional as F
    g = torch.Generator(device=dev).manual_seed(seed)
    b, c, t, h, w = shape
    fine = torch.rand(shape, generator=g, device=dev) * 2 - 1
    coarse = torch.randn((b * t, c, h // 32, w // 32), generator=g, device=dev)
    smooth = F.interpolate(coarse, size=(h, w), mode="bilinear", align_corners=False)
    smooth = smooth.view(b, t, c, h, w).transpose(1, 2)
    return (fine + smooth).clamp_(-1, 1).half()


class LaunchTimer:
    """HIP events around selected C-ABI launches, recorded on torch's current stream (the stream every op
    of the package launches on: one of the runtime's tile streams inside a step).  Wraps ``_hip.call``;
    off until ``arm()``, which also records a reference event that dates every launch on one clock."""

    def __init__(self, torch, hip, selectors):
        self.torch, self.hip, self.selectors = torch, hip, selectors
        self.events = {name: [] for name in selectors}
        self.armed = False
        self.ref = None
        self._call = hip.call
        hip.call = self

    def reset(self):
        self.events = {name: [] for name in self.selectors}

    def arm(self):
        self.ref = self.torch.cuda.Event(enable_timing=True)
        self.ref.record()
        self.armed = True

    def union_us(self, keys):
        """Length of the union of the selected launches' [start, end] intervals: the time in which at least
        one of them ran.  Launches on different tile streams overlap; without overlap this is the sum of
        their durations."""
        spans = sorted((self.ref.elapsed_time(e0), self.ref.elapsed_time(e1))
                       for key in keys for e0, e1 in self.events[key])
        total, cur0, cur1 = 0.0, None, None
        for a, b in spans:
            if cur1 is None or a > cur1:
                if cur1 is not None:
                    total += cur1 - cur0
                cur0, cur1 = a, b
            else:
                cur1 = max(cur1, b)
        if cur1 is not None:
            total += cur1 - cur0
        return total * 1e3

    def __call__(self, name, *args):
        if self.armed:
            for key, (entry, match) in self.selectors.items():
                if name == entry and match(args):
                    e0 = self.torch.cuda.Event(enable_timing=True)
                    e1 = self.torch.cuda.Event(enable_timing=True)
                    e0.record()
                    self._call(name, *args)
                    e1.record()
                    self.events[key].append((e0, e1))
                    return
        self._call(name, *args)

    def mean_us(self, key):
        spans = [e0.elapsed_time(e1) * 1e3 for e0, e1 in self.events[key]]
        return (sum(spans) / len(spans) if spans else float("nan")), len(spans)

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
        words = int(hip.lib().h3v_tensor_quant_scratch_words())
        amax = torch.empty(words, device=dev, dtype=torch.int32)
        y = torch.empty((9, 64, 64, 128), device=dev, dtype=f16)
        t_q = timed(lambda: call("h3v_tensor_quant_i8", p(xn), xn.numel(), p(qx), p(xs), p(amax), words, stream))
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

        # The INT8 GEMMs of the step (H3 decoder call, M = 7188) and of configs 2-4 (M = 16384) next to the
        # vendor library's INT8 GEMM on the same operands: torch._int_mm (hipBLASLt, int32 output, no
        # epilogue; it needs M, N, K multiples of 8, so it runs M = 7192 where ours runs 7188).  Activations
        # are row-quantized N(0, 1), weights row-quantized N(0, 0.02), as in the step.
        vs = {}
        for label, mm, nn, kk in [("h3_qkv", 7188, 6144, 2048), ("h3_attn_out", 7188, 2048, 2048),
                                  ("h3_ffn_up", 7188, 16384, 2048), ("h3_ffn_down", 7188, 2048, 8192),
                                  ("cfg2_qkv", 16384, 3072, 1024), ("cfg3_up", 16384, 8192, 1024),
                                  ("cfg3_down", 16384, 1024, 4096), ("cfg4_out", 16384, 1024, 1024)]:
            xa = randn(mm, kk)
            qa = torch.empty((mm, kk), device=dev, dtype=i8)
            sa = torch.empty(mm, device=dev, dtype=f32)
            call("h3v_row_quant", p(xa), mm, kk, p(qa), p(sa), stream)
            wb, wbs = kitchen.quantize_int8_rowwise(randn(nn, kk, scale=0.02))
            wbs = wbs.reshape(-1).contiguous()
            bb = randn(nn, scale=0.02)
            yb = torch.empty((mm, nn), device=dev, dtype=f16)
            t_ours = timed(lambda: call("h3v_gemm_i8_dequant", p(qa), p(sa), p(wb), p(wbs), p(bb), p(yb), mm, nn, kk,
                                        stream))
            m8 = (mm + 7) // 8 * 8
            qa8 = torch.zeros((m8, kk), device=dev, dtype=i8)
            qa8[:mm] = qa
            wbt = wb.t()
            t_lib = timed(lambda: torch._int_mm(qa8, wbt))
            vs[f"{label}_{mm}x{nn}x{kk}"] = {"h3v_gemm_i8_dequant": mfma(t_ours, 2 * mm * nn * kk),
                                             "hipblaslt_int_mm_int32_out": mfma(t_lib, 2 * m8 * nn * kk)}
            del xa, qa, qa8, wb, yb
        out["int8_gemm_vs_hipblaslt"] = vs

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
            floats = int(hip.lib().h3v_conv3d_f16_workspace_floats(b, cin, dp, hp, wp, cout, k, k, k, *stride))
            wsf = torch.empty(max(floats, 1), device=dev, dtype=torch.float32)
            t_c = timed(lambda: call("h3v_conv3d_f16_ws", p(xs), p(wsp), p(bs), None, p(ys), b, cin, dp, hp, wp, cout, k,
                                     k, k, *stride, int(causal), p(wsf), floats, stream))
            flops = 2 * b * do * ho * wo * cout * k ** 3 * cin
            if k == 1:   # a 1x1x1 projection does 2 * Cin flops per output value: far below the fp16 ridge, HBM-bound
                nbytes = 2 * (b * dp * hp * wp * cin + b * do * ho * wo * cout + cout * cin)
                res = {"h3v_conv3d_f16": dict(hbm(t_c, nbytes), tflops=round(flops / t_c / 1e6, 1), flops=flops)}
            else:
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
        # convs that fill under half of the CUs: K split over a workspace (suffix downsamples, conv_out)
        out["suffix_downsample2_f16_4x256x9x64x64_s222"] = fp16_conv_case(4, 256, 256, 11, 65, 65, 3, (2, 2, 2), False)
        out["suffix_downsample3_f16_4x512x5x32x32_s122"] = fp16_conv_case(4, 512, 512, 7, 33, 33, 3, (1, 2, 2), False)
        out["conv_out_f16_4x1024to48x5x16x16"] = fp16_conv_case(4, 1024, 48, 7, 18, 18, 3, (1, 1, 1), True)

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
        # 2 * 81 flops per output value against its 2-byte store: HBM-bound.  Bytes: the 3-channel input read, the
        # folded input written and read back, the weights, the fp16 output written
        in_bytes = 2 * (17 * 256 * 256 * 3 + 2 * 19 * 256 * 256 * 32 + 128 * 96 + 17 * 256 * 256 * 128)
        in_flops = 2 * 17 * 256 * 256 * 128 * 81
        out["conv_in_f16_3to128x17x256x256"] = {"tap_fold_pack_and_conv3d_f16":
                                                dict(hbm(t_in, in_bytes), tflops=round(in_flops / t_in / 1e6, 1),
                                                     flops=in_flops)}
    torch.cuda.synchronize()
    return out


def stage0_conv_useful_ops():
    """Useful INT8 ops of one stage-0 conv (C128 -> 128, 17 x 256 x 256): frame 0 skips 2 of 3 depth
    taps, frame 1 skips 1 (the causal zero frames)."""
    per_frame_tap = 2 * 256 * 256 * 128 * 9 * 128
    return 17 * 3 * per_frame_tap - 3 * per_frame_tap


def enc_ops_per_call():
    """Useful (non-causal-zero) and dense INT8 ops of the 8 INT8 convs of one prefix call (one clip, one tile)."""
    useful = dense = 0
    t = 17
    for cin, cout, h, w in [(128, 128, 256, 256)] * 4 + [(128, 256, 128, 128)] + [(256, 256, 128, 128)] * 3:
        per_frame = 2 * h * w * cout * 27 * cin
        dense += t * per_frame
        useful += t * per_frame - per_frame * (2 + 1) // 3     # frame 0 skips 2 of 3 taps, frame 1 skips 1
    return useful, dense


def dec_ops_per_call():
    """INT8 GEMM ops of one B4 decoder call (36 blocks: QKV, attention-out, FFN-up, FFN-down)."""
    m, d = DEC_M, DEC_D
    return 2 * m * DEC_BLOCKS * (6144 * d + d * d + 16384 * d + d * 8192)

def _host_cpu():
    """Model, sockets and cores of the host CPU (lscpu), with the threads this process may use."""
    import subprocess
    info = {"threads_available": len(os.sched_getaffinity(0)), "os_cpu_count": os.cpu_count()}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            key, _, value = line.partition(":")
            if key.strip() in ("Model name", "Socket(s)", "Core(s) per socket", "Thread(s) per core"):
                info[key.strip().lower().replace("(s)", "s").replace(" ", "_")] = value.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return info


def _median_s(fn, runs=5):
    """Median wall time of ``runs`` calls after one warm-up call."""
    import statistics
    fn()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times)


def cpu_configs(rng, threads):
    """BASELINE.json configs 1-4 through the CPU oracle (C, OpenMP): config 1 in full; configs 2-4, whose work is
    independent per token row, on a row sample scaled to the full M (stated per entry).  Median of 5 runs
    after a warm-up.  Attention (config 4) is torch's CPU SDPA in fp32 on a query sample."""
    import numpy as np
    import oracle
    import torch
    out = {}
    # cfg1: per-tensor quant of the padded [11, 66, 66, 128] input + causal conv C128 -> 128 + dequant epilogue
    xp = np.zeros((1, 11, 66, 66, 128), np.float16)
    xp[0, 2:] = rng.standard_normal((9, 66, 66, 128)).astype(np.float16)
    qw = rng.integers(-127, 128, (128, 3456)).astype(np.int8)
    ws = np.full(128, 1e-4, np.float32)
    b = np.zeros(128, np.float16)

    def cfg1():
        s = oracle.tensor_scale(xp)
        acc = oracle.conv3d_acc(oracle.tensor_quant(xp, s), qw, (3, 3, 3), (1, 1, 1))
        oracle.gemm_dequant(acc.reshape(-1, 128), np.float32(s), ws, b)

    out["cfg1_causal_conv3d_c128_9x64x64"] = {"s": round(_median_s(cfg1), 4), "sample": "full"}

    def rows(m):
        return rng.standard_normal((m, 1024)).astype(np.float16)

    # cfg2: residual + norm1 (W16 tree) + row quant, QKV GEMM 1024 -> 3072; M = 16384, sample 2048 rows
    ms = 2048
    h, o = rows(ms), rows(ms)
    g, gam = (0.1 * rng.standard_normal(1024)).astype(np.float16), np.ones(1024, np.float16)
    wq = rng.integers(-31, 32, (3072, 1024)).astype(np.int8)
    sq = np.full(3072, 1e-3, np.float32)
    bq = np.zeros(3072, np.float16)

    def cfg2():
        _, q, sx = oracle.residual_rms_quant(h, o, g, gam, 1e-5, recipe=1)
        oracle.gemm_dequant(oracle.gemm_acc(q, wq), sx, sq, bq)

    out["cfg2_norm1_qkv_m16384_d1024"] = {"s": round(_median_s(cfg2) * 16384 / ms, 4),
                                          "sample": f"{ms} of 16384 rows, scaled"}
    # cfg3: row quant + FFN-up 1024 -> 2 x 4096 + SwiGLU requant + down 4096 -> 1024; sample 1024 rows
    ms = 1024
    x3 = rows(ms)
    wu = rng.integers(-31, 32, (8192, 1024)).astype(np.int8)
    wd = rng.integers(-31, 32, (1024, 4096)).astype(np.int8)
    su, sd = np.full(8192, 1e-3, np.float32), np.full(1024, 1e-3, np.float32)

    def cfg3():
        q, sx = oracle.row_quant(x3)
        hidden = oracle.gemm_dequant(oracle.gemm_acc(q, wu), sx, su, np.zeros(8192, np.float16))
        q2, s2 = oracle.swiglu_row_quant(hidden)
        oracle.gemm_dequant(oracle.gemm_acc(q2, wd), s2, sd, np.zeros(1024, np.float16))

    out["cfg3_ffn_m16384_d1024_h4096"] = {"s": round(_median_s(cfg3) * 16384 / ms, 4),
                                          "sample": f"{ms} of 16384 rows, scaled"}
    # cfg4: QK-RMSNorm-RoPE + SDPA (16 heads x 64, 16384 keys) + out row quant + GEMM 1024 -> 1024;
    # sample 1024 query rows (every key is kept)
    ms, n, heads = 1024, 16384, 16
    qkv = rng.standard_normal((ms, heads * 192)).astype(np.float16)
    ang = rng.uniform(0, 6.283, (ms, 48))
    cos, sin = np.cos(ang).astype(np.float16), np.sin(ang).astype(np.float16)
    kv = torch.randn(1, heads, n, 64)
    wo = rng.integers(-31, 32, (1024, 1024)).astype(np.int8)
    so = np.full(1024, 1e-3, np.float32)

    def cfg4():
        rq, _ = oracle.qk_rope(qkv, cos, sin, heads, 1e-6)
        qt = torch.from_numpy(np.asarray(rq, np.float32).reshape(1, ms, heads, 64)).transpose(1, 2)
        y = torch.nn.functional.scaled_dot_product_attention(qt, kv, kv)
        ya = y.transpose(1, 2).reshape(ms, 1024).half().numpy()
        q, sx = oracle.row_quant(ya)
        oracle.gemm_dequant(oracle.gemm_acc(q, wo), sx, so, np.zeros(1024, np.float16))

    out["cfg4_qk_rope_sdpa_out_proj_16384tok_16x64"] = {"s": round(_median_s(cfg4) * 16384 / ms, 4),
                                                        "sample": f"{ms} of 16384 query rows, scaled"}
    return out


def _cpu_row_quant(x):
    """Q1 per-row quant on the CPU (CK quantize_int8_rowwise): s = max|x| / 127 per row (1 for a zero row),
    q = round(x / s) clamped to +-127."""
    import torch
    xf = x.float()
    s = xf.abs().amax(dim=-1, keepdim=True) / 127.0
    s = torch.where(s > 0, s, torch.ones_like(s))
    return torch.round(xf / s).clamp_(-127, 127).to(torch.int8), s


def _cpu_tensor_quant(x):
    """E3 per-tensor quant on the CPU (reference opt/encoder_int8.py:591-610): half-away rounding."""
    import torch
    xf = x.float()
    s = xf.abs().amax() / 127.0
    s = torch.where(s > 0, s, torch.ones_like(s))
    y = xf / s
    q = torch.where(y >= 0, torch.floor(y + 0.5), -torch.floor(-y + 0.5))
    return q.clamp_(-127, 127).to(torch.int8), s


def _cpu_int8_linear(q, s, w_t, ws, bias):
    """int8 [M, K] x int8 [K, N] -> exact int32 (torch._int_mm) -> fp16(acc * sx * sw + b)."""
    import torch
    acc = torch._int_mm(q, w_t)
    return (acc.float() * s * ws + bias.float()).half()


def _cpu_conv3x3x3(qx, qw_t, d, h, w):
    """Valid 3x3x3 conv of an int8 NDHWC [d + 2, h + 2, w + 2, C] input as im2col + torch._int_mm (exact int32),
    one output frame per GEMM: -> int32 [d, h * w, Cout]."""
    import torch
    out = []
    for t in range(d):
        cols = torch.cat([qx[t + kd, kh:kh + h, kw:kw + w] for kd in range(3) for kh in range(3) for kw in range(3)],
                         dim=-1).reshape(h * w, -1)
        out.append(torch._int_mm(cols, qw_t))
    return torch.stack(out)


def torch_cpu_configs(threads):
    """BASELINE.json configs 1-4 in full through a PyTorch CPU restatement of the reference arithmetic (exact int32
    GEMMs with torch._int_mm, convs as im2col + _int_mm, quantizers and norms in fp32): median of 5 runs after a
    warm-up each."""
    import torch
    g = torch.Generator().manual_seed(20261002)
    randn = lambda *shape, scale=1.0: (torch.randn(*shape, generator=g) * scale).half()
    qweight = lambda n, k: torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    out = {}
    # cfg1: per-tensor quant of the padded input, causal 3x3x3 conv C128 -> 128 (dense reduction), dequant
    xp = torch.zeros(11, 66, 66, 128, dtype=torch.float16)
    xp[2:] = randn(9, 66, 66, 128)
    w1 = qweight(128, 3456).t()
    ws1, b1 = torch.full((128,), 1e-4), torch.zeros(128, dtype=torch.float16)

    def cfg1():
        q, s = _cpu_tensor_quant(xp)
        acc = _cpu_conv3x3x3(q, w1, 9, 64, 64)
        return (acc.float() * s * ws1 + b1.float()).half()

    m, d = 16384, 1024
    h, o = randn(m, d), randn(m, d)
    gate, gam, beta = randn(d, scale=0.1), (1 + 0.1 * torch.randn(d, generator=g)).half(), randn(d, scale=0.02)
    wq, sq, bq = qweight(3072, d).t(), torch.full((3072,), 1e-3), randn(3072, scale=0.02)

    def cfg2():   # residual + RMSNorm (fp32) + row quant, QKV GEMM 1024 -> 3072
        hn = (h.float() + o.float() * gate.float()).half()
        n = (hn.float() * torch.rsqrt(hn.float().pow(2).mean(-1, keepdim=True) + 1e-5) * gam.float()).half()
        q, s = _cpu_row_quant(n)
        return _cpu_int8_linear(q, s, wq, sq, bq)

    x3 = randn(m, d)
    wu, su, bu = qweight(8192, d).t(), torch.full((8192,), 1e-3), randn(8192, scale=0.02)
    wd, sd, bd = qweight(d, 4096).t(), torch.full((d,), 1e-3), randn(d, scale=0.02)

    def cfg3():   # row quant, FFN-up 1024 -> 2 x 4096, SwiGLU (fp32) + row quant, down 4096 -> 1024
        q, s = _cpu_row_quant(x3)
        gu = _cpu_int8_linear(q, s, wu, su, bu).float()
        act = (torch.nn.functional.silu(gu[:, :4096]) * gu[:, 4096:]).half()
        q2, s2 = _cpu_row_quant(act)
        return _cpu_int8_linear(q2, s2, wd, sd, bd)

    heads = 16
    qkv = randn(1, m, heads, 192)
    ang = torch.rand(m, 1, 24, generator=g) * 6.283
    cos, sin = torch.cat([ang.cos()] * 2, -1), torch.cat([ang.sin()] * 2, -1)
    wo, so, bo = qweight(d, d).t(), torch.full((d,), 1e-3), randn(d, scale=0.02)

    def rope(t):   # RMS (fp32, no affine) then rotate-half on the first 48 dims
        t = t.float()
        t = (t * torch.rsqrt(t.pow(2).mean(-1, keepdim=True) + 1e-6)).half().float()
        r = t[..., :48]
        rot = torch.cat([-r[..., 24:], r[..., :24]], -1)
        return torch.cat([r * cos + rot * sin, t[..., 48:]], -1)

    def cfg4():   # QK-RMSNorm-RoPE, SDPA over 16384 tokens (fp32 on the CPU), out row quant + GEMM 1024 -> 1024
        qh, kh, vh = rope(qkv[..., :64]), rope(qkv[..., 64:128]), qkv[..., 128:].float()
        y = torch.nn.functional.scaled_dot_product_attention(qh.transpose(1, 2), kh.transpose(1, 2),
                                                             vh.transpose(1, 2), scale=0.125)
        q, s = _cpu_row_quant(y.transpose(1, 2).reshape(m, d).half())
        return _cpu_int8_linear(q, s, wo, so, bo)

    for key, fn in (("cfg1_causal_conv3d_c128_9x64x64", cfg1), ("cfg2_norm1_qkv_m16384_d1024", cfg2),
                    ("cfg3_ffn_m16384_d1024_h4096", cfg3), ("cfg4_qk_rope_sdpa_out_proj_16384tok_16x64", cfg4)):
        out[key] = {"s": round(_median_s(fn), 4), "sample": "full"}
    return out


def torch_cpu_step_sample():
    """The INT8 hot path of the step on the CPU, sampled: one output frame of a stage-0 fused layer (GroupNorm
    statistics, SiLU, pad, per-tensor quant, dense 3x3x3 conv C128 -> 128 on 256 x 256 pixels as im2col +
    _int_mm, dequant) and one decoder block at the B4 shape M = 7188 (norm1 + row quant + QKV GEMM, QK-RMSNorm-
    RoPE, SDPA fp32 over 4 x 32 heads x 1797 tokens, out GEMM, norm2 + row quant, FFN-up, SwiGLU + row quant,
    FFN-down).  -> (encoder seconds per dense op, decoder seconds per block)."""
    import torch
    g = torch.Generator().manual_seed(20261002)
    randn = lambda *shape, scale=1.0: (torch.randn(*shape, generator=g) * scale).half()
    qweight = lambda n, k: torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    # encoder: the producer over the 3 input frames one output frame reads, then that frame's conv
    x = randn(3, 256, 256, 128)
    w0 = qweight(128, 3456).t()
    ws0, b0 = torch.full((128,), 1e-4), torch.zeros(128, dtype=torch.float16)

    def enc():
        xf = x.float().view(3, 256 * 256, 32, 4)
        mean = xf.mean(dim=(1, 3), keepdim=True)
        var = xf.var(dim=(1, 3), keepdim=True, unbiased=False)
        y = torch.nn.functional.silu((xf - mean) * torch.rsqrt(var + 1e-6)).view(3, 256, 256, 128).half()
        yp = torch.nn.functional.pad(y.permute(0, 3, 1, 2).float(), (1, 1, 1, 1), mode="reflect").permute(0, 2, 3, 1)
        q, s = _cpu_tensor_quant(yp.half())
        acc = _cpu_conv3x3x3(q, w0, 1, 256, 256)
        return (acc.float() * s * ws0 + b0.float()).half()

    enc_s = _median_s(enc, runs=3)
    enc_ops = 2 * 256 * 256 * 128 * 3456
    # decoder block at M = 7188 (4 x 1797 tokens), width 2048, 32 heads
    m, dd, heads = DEC_M, DEC_D, DEC_HEADS
    h = randn(m, dd)
    gam = (1 + 0.1 * torch.randn(dd, generator=g)).half()
    w_qkv, w_o, w_u, w_d = qweight(3 * dd, dd).t(), qweight(dd, dd).t(), qweight(16384, dd).t(), qweight(dd, 8192).t()
    sc = lambda n: torch.full((n,), 1e-3)
    zb = lambda n: torch.zeros(n, dtype=torch.float16)
    ang = torch.rand(m, 1, 24, generator=g) * 6.283
    cos, sin = torch.cat([ang.cos()] * 2, -1), torch.cat([ang.sin()] * 2, -1)

    def rms(t, w):
        return (t.float() * torch.rsqrt(t.float().pow(2).mean(-1, keepdim=True) + 1e-5) * w.float()).half()

    def rope(t):
        t = t.float()
        t = (t * torch.rsqrt(t.pow(2).mean(-1, keepdim=True) + 1e-6)).half().float()
        r = t[..., :48]
        rot = torch.cat([-r[..., 24:], r[..., :24]], -1)
        return torch.cat([r * cos + rot * sin, t[..., 48:]], -1)

    def dec():
        q, s = _cpu_row_quant(rms(h, gam))
        qkv = _cpu_int8_linear(q, s, w_qkv, sc(3 * dd), zb(3 * dd)).view(m, heads, 192)
        qh, kh, vh = rope(qkv[..., :64]), rope(qkv[..., 64:128]), qkv[..., 128:].float()
        split = lambda t: t.view(4, 1797, heads, 64).transpose(1, 2)
        y = torch.nn.functional.scaled_dot_product_attention(split(qh), split(kh), split(vh), scale=0.125)
        q, s = _cpu_row_quant(y.transpose(1, 2).reshape(m, dd).half())
        h2 = (h.float() + _cpu_int8_linear(q, s, w_o, sc(dd), zb(dd)).float()).half()
        q, s = _cpu_row_quant(rms(h2, gam))
        gu = _cpu_int8_linear(q, s, w_u, sc(16384), zb(16384)).float()
        q, s = _cpu_row_quant((torch.nn.functional.silu(gu[:, :8192]) * gu[:, 8192:]).half())
        return _cpu_int8_linear(q, s, w_d, sc(dd), zb(dd))

    dec_s = _median_s(dec, runs=3)
    return enc_s / enc_ops, dec_s


def cpu_baseline(budget_s: float):
    """The reference arithmetic on the host CPU: BASELINE.json configs 1-4 in full through PyTorch (torch._int_mm,
    median of 5), the full step extrapolated from one stage-0 conv frame and one decoder block; the scalar C oracle
    beside it (configs 1-4 on row samples, labelled)."""
    import numpy as np
    import oracle
    import torch

    threads = len(os.sched_getaffinity(0))
    oracle.set_threads(threads)
    torch.set_num_threads(threads)
    configs = torch_cpu_configs(threads)
    enc_s_per_op, dec_block_s = torch_cpu_step_sample()
    _, dense = enc_ops_per_call()
    enc_s = enc_s_per_op * ENC_CALLS * dense
    dec_s = dec_block_s * DEC_BLOCKS * DEC_CALLS
    rng = np.random.default_rng(20261002)
    return {
        "value": round(enc_s + dec_s, 1),
        "unit": "s (extrapolated)",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"PyTorch CPU restatement of the reference arithmetic ({torch.get_num_threads()} threads; exact int32 "
                   f"GEMMs with torch._int_mm, convs as im2col + _int_mm, quantizers and norms in fp32): one output "
                   f"frame of a stage-0 fused layer (producer + dense 3x3x3 conv on 256x256x128) and one decoder block "
                   f"at M = 7188 (GEMMs, row quants, norms, QK-RoPE, fp32 SDPA), median of 3 each, extrapolated by "
                   f"dense conv op count to the {ENC_CALLS} prefix calls and x{DEC_BLOCKS} blocks x{DEC_CALLS} calls: "
                   f"encode {enc_s:.0f} s + decode {dec_s:.0f} s (the encoder's FP16 layers are not included, so this "
                   f"is a lower bound)"),
        "host": _host_cpu(),
        "torch_threads": torch.get_num_threads(),
        "configs": configs,
        "c_oracle_configs": {"kind": "port (scalar C oracle, OpenMP)", **cpu_configs(rng, threads)},
    }


TRAFFIC_PROFILE = ROOT / "profiles" / "stage0_conv_traffic_pmc.md"
GEMM_TRAFFIC_PROFILE = ROOT / "profiles" / "int8_gemm_decoder_traffic_pmc.md"
GEMM_KERNEL = ("gemm_i8_pingpong<Dequant> (every decoder INT8 GEMM: QKV, attention-out and FFN-up with K = 2048, "
               "FFN-down with K = 8192; 256x256x128 tiles, two wave groups alternating MFMA and fragment-read phases)")


def _profile_number(path, key):
    """The integer after `key:` in a committed profile summary, or None."""
    try:
        for line in path.read_text().splitlines():
            if line.startswith(key + ":"):
                return int(line.split(":", 1)[1].strip())
    except (OSError, ValueError):
        pass
    return None


def stage0_conv_traffic():
    """HBM (L2-miss) bytes per stage-0 conv launch from the committed FETCH_SIZE/WRITE_SIZE summary.

    The summary holds one line `traffic_bytes_per_launch: N`, derived from two rocprofv3 --pmc runs of
    `bench.py --traffic-sample`, each scaled by the counter's reading for a copy of known size.
    """
    return _profile_number(TRAFFIC_PROFILE, "traffic_bytes_per_launch")


def gemm_traffic():
    """HBM (L2-miss) bytes per launch of the decoder GEMM kernel (mean over the QKV, attention-out, FFN-up and
    FFN-down launches of a block), from the committed FETCH_SIZE/WRITE_SIZE summary of `bench.py --traffic-sample`."""
    return _profile_number(GEMM_TRAFFIC_PROFILE, "traffic_bytes_per_launch")


def build_runtime(torch, pkg, args):
    """The reconstructed H3 core (random init, built on the GPU) wrapped by H3VAEPyOptRuntime in the INT8
    encode + fused INT8 decode modes of the reference's headline numbers (README.md:43,53-54)."""
    import importlib
    rec = importlib.import_module(f"{pkg.__name__}.reconstructed_h3")
    rt = importlib.import_module(f"{pkg.__name__}.h3vae_runtime")
    dev = torch.device("cuda:0")
    with torch.device(dev):
        core, config = rec.build_core(depth=args.depth)
    runtime = rt.H3VAEPyOptRuntime(device="cuda", dtype=torch.float16, decoder_tile_size=256, tile_batch=4,
                                   encoder_staged_batch=4, encoder_tile_size=0, int8_encode=True, int8_decode=True,
                                   decode_fusions=True, log_calls=False, core=core, config=config,
                                   tile_streams=2)
    return runtime


PMC_SAMPLE_ORDER = [
    # (label, entry point, shape) in dispatch order; each runs 3 times (the first one warms L2 and the clock)
    ("copy_1GiB", "torch.neg fp16 [2^29]", None),
    ("stage0_conv", "h3v_conv3d_i8", "[1,128,19,258,258] -> 128, causal, after the fused producer"),
    ("stage1_conv_c256", "h3v_conv3d_i8", "[1,256,19,130,130] -> 256, causal"),
    ("stage1_conv_c128_256", "h3v_conv3d_i8", "[1,128,19,130,130] -> 256, causal"),
    ("h3_qkv", "h3v_gemm_i8_dequant", "7188 x 6144 x 2048"),
    ("h3_attn_out", "h3v_gemm_i8_dequant", "7188 x 2048 x 2048"),
    ("h3_ffn_up", "h3v_gemm_i8_dequant", "7188 x 16384 x 2048"),
    ("h3_ffn_down", "h3v_gemm_i8_dequant", "7188 x 2048 x 8192"),
    ("cfg2_qkv", "h3v_gemm_i8_dequant", "16384 x 3072 x 1024"),
    ("cfg3_up", "h3v_gemm_i8_dequant", "16384 x 8192 x 1024"),
    ("cfg3_down", "h3v_gemm_i8_dequant", "16384 x 1024 x 4096"),
    ("cfg4_out", "h3v_gemm_i8_dequant", "16384 x 1024 x 1024"),
    ("cfg1_conv", "h3v_conv3d_i8", "[1,128,11,66,66] -> 128, causal"),
]


def traffic_sample(torch, pkg):
    """The INT8 matrix kernels of the step and of configs 1-4, each launched 3 times in PMC_SAMPLE_ORDER, for
    rocprofv3 --pmc passes (HBM bytes, MFMA busy cycles): a 1 GiB elementwise copy first (FETCH_SIZE / WRITE_SIZE
    scale), then the stage-0 fused layer (producer + conv) and the other convs and GEMMs on their step shapes with
    the step's data distributions (row-quantized N(0, 1) activations, N(0, 0.02) weights; fused-producer int8
    activations and kaiming-like weights for the convs)."""
    import importlib
    integ = importlib.import_module(f"{pkg.__name__}.opt.encoder_int8_integration")
    enc = importlib.import_module(f"{pkg.__name__}.opt.encoder_int8")
    kitchen = importlib.import_module(f"{pkg.__name__}.opt.kitchen_int8")
    hip = importlib.import_module(f"{pkg.__name__}._hip")
    dev = torch.device("cuda:0")
    stream = hip.stream(dev)
    call, p = hip.call, hip.ptr
    g = torch.Generator(device=dev).manual_seed(20261002)

    def randn(*shape, scale=1.0):
        return (torch.randn(*shape, generator=g, device=dev) * scale).half()

    def conv(cin, cout, d, h, w):
        x = randn(1, cin, d, h, w).contiguous(memory_format=torch.channels_last_3d)
        qx, xs = enc.quantize_activation_tensor(F.pad(x, (1, 1, 1, 1, 2, 0)))
        qw, ws, _ = enc.prepare_int8_weight(randn(cout, cin, 3, 3, 3, scale=(27 * cin) ** -0.5))
        bias = randn(cout, scale=0.1)
        y = torch.empty((d, h, w, cout), device=dev, dtype=torch.float16)
        for _ in range(3):
            call("h3v_conv3d_i8", p(qx), p(xs), p(qw), p(ws), p(bias), p(y), 1, cin, d + 2, h + 2, w + 2, cout,
                 3, 3, 3, 1, 1, 1, 1, stream)

    def gemm(m, n, k):
        xa = randn(m, k)
        qa = torch.empty((m, k), device=dev, dtype=torch.int8)
        sa = torch.empty(m, device=dev, dtype=torch.float32)
        call("h3v_row_quant", p(xa), m, k, p(qa), p(sa), stream)
        wb, wbs = kitchen.quantize_int8_rowwise(randn(n, k, scale=0.02))
        wbs = wbs.reshape(-1).contiguous()
        bb = randn(n, scale=0.02)
        yb = torch.empty((m, n), device=dev, dtype=torch.float16)
        for _ in range(3):
            call("h3v_gemm_i8_dequant", p(qa), p(sa), p(wb), p(wbs), p(bb), p(yb), m, n, k, stream)

    import torch.nn.functional as F
    with torch.inference_mode():
        src = torch.ones(1 << 29, device=dev, dtype=torch.float16)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)
        del src, dst
        x = torch.randn((1, 128, 17, 256, 256), generator=g, device=dev).half().contiguous(
            memory_format=torch.channels_last_3d)
        gamma, beta = torch.ones(128, device=dev, dtype=torch.float16), torch.zeros(128, device=dev, dtype=torch.float16)
        qw, ws, _ = enc.prepare_int8_weight(torch.randn((128, 128, 3, 3, 3), generator=g, device=dev).half() * 3456 ** -0.5)
        bias = torch.zeros(128, device=dev, dtype=torch.float16)
        for _ in range(3):
            integ.int8_norm_conv3d(x, gamma, beta, None, 1e-6, qw, ws, bias)
        del x
        conv(256, 256, 17, 128, 128)
        conv(128, 256, 17, 128, 128)
        for m, n, k in [(DEC_M, 3 * DEC_D, DEC_D), (DEC_M, DEC_D, DEC_D), (DEC_M, 16384, DEC_D), (DEC_M, DEC_D, 8192),
                        (16384, 3072, 1024), (16384, 8192, 1024), (16384, 1024, 4096), (16384, 1024, 1024)]:
            gemm(m, n, k)
        conv(128, 128, 9, 64, 64)
        torch.cuda.synchronize()
    print("[bench] traffic / PMC sample done: " + "; ".join(f"{label}: {entry} {shape or ''}".strip()
                                                              for label, entry, shape in PMC_SAMPLE_ORDER),
          file=sys.stderr)


def mfma_ceiling(torch, hip, runtime, clip):
    """Measured INT8 MFMA ceiling for the stage-0 conv's own operands (h3v_probe_mfma_rate).

    The published peak assumes the top shader clock; under a matrix load the part holds a clock that
    depends on the power the MFMAs draw, i.e. on the data.  The runtime's own first stage-0 layer
    operands are taken: conv_in of the clip's first tile, the block's fused producer (int8 activations)
    and the block's int8 weights; the probe multiplies those bytes from registers (no memory traffic),
    one workgroup of 8 waves per CU, and reports the rate and the mean clock."""
    import importlib
    norm = importlib.import_module(f"{hip.__name__.rsplit('.', 1)[0]}.opt.encoder_int8_norm")
    dev = torch.device("cuda:0")
    block = runtime.prefix.stages[0].block[0]
    tile = runtime._normalize_pixels(clip[:, :, :17, :256, :256]).contiguous(memory_format=torch.channels_last_3d)
    h = runtime.prefix.conv_in(tile)
    a, _ = norm.quantized_temporal_norm_pad(h, block.first.norm_weight, block.first.norm_bias, block.first.eps)
    a = a.permute(0, 2, 3, 4, 1).reshape(-1)                          # channels-last bytes
    b = block.int8_first.qweight.reshape(-1)
    blocks = int(torch.cuda.get_device_properties(dev).multi_processor_count)
    sink = torch.empty(blocks * 512, device=dev, dtype=torch.int32)
    clocks = torch.empty(2 * blocks, device=dev, dtype=torch.int64)
    iters = 4000
    ops = blocks * int(hip.lib().h3v_probe_mfma_ops_per_block(iters))
    stream = hip.stream(dev)
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
        "data": "stage-0 conv operands of the runtime: the fused producer's int8 activations of the first tile x "
                "the block's int8 weights",
        "tops": round(tops, 1),
        "frac_of_peak": round(tops / INT8_PEAK_TOPS, 4),
        "clock_mhz": round(ticks[0] / ticks[1] * 100.0, 0),
        "blocks": blocks,
    }


GEMM_SHAPES = {"qkv": (3 * DEC_D, DEC_D), "attn_out": (DEC_D, DEC_D), "ffn_up": (16384, DEC_D),
               "ffn_down": (DEC_D, 8192)}   # (N, K) of the decoder linears, M = DEC_M


def launch_stats(timer):
    """Roofline figures of the timed launches: the decoder GEMM family per shape and together, and the
    stage-0 conv.  avg_us = the union of the launches' HIP-event intervals per launch (the time in which at
    least one of them ran; the plain mean duration when no two overlap), launch_avg_us_shared = the mean of
    the individual durations; achieved = algorithmic ops over the union."""
    per_gemm = {}
    for key, (n_, k_) in GEMM_SHAPES.items():
        shared, n = timer.mean_us(key)
        us = timer.union_us([key]) / n
        ops = 2 * DEC_M * n_ * k_
        per_gemm[key] = {"avg_us": round(us, 2), "launch_avg_us_shared": round(shared, 2), "launches_timed": n,
                         "ops_per_launch": ops, "tops": round(ops / us / 1e6, 1),
                         "frac": round(ops / us / 1e6 / INT8_PEAK_TOPS, 4)}
    fam = tuple(GEMM_SHAPES)
    fam_n = sum(per_gemm[k]["launches_timed"] for k in fam)
    fam_us = timer.union_us(fam) / fam_n
    fam_shared = sum(per_gemm[k]["launch_avg_us_shared"] * per_gemm[k]["launches_timed"] for k in fam) / fam_n
    fam_ops = sum(per_gemm[k]["ops_per_launch"] * per_gemm[k]["launches_timed"] for k in fam) / fam_n
    conv_shared, conv_n = timer.mean_us("stage0_conv")
    conv_us = timer.union_us(["stage0_conv"]) / conv_n
    conv_ops = stage0_conv_useful_ops()
    return {"per_gemm": per_gemm, "fam_n": fam_n, "fam_us": fam_us, "fam_shared": fam_shared, "fam_ops": fam_ops,
            "gemm_achieved": fam_ops / fam_us / 1e6, "conv_n": conv_n, "conv_us": conv_us, "conv_shared": conv_shared,
            "conv_ops": conv_ops, "conv_achieved": conv_ops / conv_us / 1e6}


def in_step_summary(st, which):
    """The timed steps' figures of one roofline kernel (two tile streams: launches overlap)."""
    if which == "gemm":
        us, shared, n, achieved = st["fam_us"], st["fam_shared"], st["fam_n"], st["gemm_achieved"]
    else:
        us, shared, n, achieved = st["conv_us"], st["conv_shared"], st["conv_n"], st["conv_achieved"]
    out = {"launches_timed": n, "avg_us": round(us, 2), "launch_avg_us_shared": round(shared, 2),
           "achieved": round(achieved, 1), "frac": round(achieved / INT8_PEAK_TOPS, 4),
           "timing": "timed steps, two tile streams: avg_us = the union of the launches' HIP-event intervals per "
                     "launch (time in which at least one ran), launch_avg_us_shared = the mean individual duration "
                     "(includes time shared with the other stream's kernels); achieved = ops / union"}
    if which == "gemm":
        out["per_gemm"] = st["per_gemm"]
    return out


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: the H3 VAE runs per GPU and multi-GPU sharding is not "
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
    stream = hip.stream(torch.device("cuda:0"))

    def log(msg):
        print(f"[bench] {msg}", file=sys.stderr, flush=True)

    if args.configs_only:
        print(json.dumps(config_measurements(torch, hip, kitchen, enc, stream, vs_torch=args.vs_torch)), flush=True)
        return
    if args.traffic_sample:
        traffic_sample(torch, pkg)
        return

    # the decoder's INT8 GEMMs (h3v_gemm_i8_dequant args: ..., m, n, k, stream) and the stage-0 conv (C128 -> 128
    # on the padded [19, 258, 258] int8 input, no residual; h3v_conv3d_i8_gn args: qx, xs, qw, ws, bias, residual,
    # out, cin, d, h, w, cout, ...: the blocks' first convs, which also write the next norm's tile statistics)
    timer = LaunchTimer(torch, hip, {
        "qkv": ("h3v_gemm_i8_dequant", lambda a: a[7] == 3 * DEC_D and a[8] == DEC_D),
        "attn_out": ("h3v_gemm_i8_dequant", lambda a: a[7] == DEC_D and a[8] == DEC_D),
        "ffn_up": ("h3v_gemm_i8_dequant", lambda a: a[7] == 16384 and a[8] == DEC_D),
        "ffn_down": ("h3v_gemm_i8_dequant", lambda a: a[7] == DEC_D and a[8] == 8192),
        "stage0_conv": ("h3v_conv3d_i8_gn",
                        lambda a: a[5] is None and a[7] == 128 and a[11] == 128 and a[10] == 258 and a[8] == 19),
    })
    log("building the reconstructed H3 VAE (random init) and the runtime")
    runtime = build_runtime(torch, pkg, args)
    clip = synthetic_clip(torch, torch.device("cuda:0"), shape=(1, 3, args.frames, 768, 1344))
    out = torch.empty(runtime.decode_output_shape((1, 24, runtime._tokens_from_frames(args.frames), 48, 84)),
                      device="cuda:0", dtype=torch.float32)

    def step(split=None):
        t0 = time.perf_counter()
        latents = runtime.encode(clip)
        if split is not None:
            torch.cuda.synchronize()
            split["enc"] += time.perf_counter() - t0
            t0 = time.perf_counter()
        runtime.decode(latents.half(), output_buffer=out)
        if split is not None:
            torch.cuda.synchronize()
            split["dec"] += time.perf_counter() - t0
        return latents

    with torch.inference_mode():
        for i in range(args.warmup):
            step()
            torch.cuda.synchronize()
            log(f"warmup step {i + 1}/{args.warmup} done")
        split = {"enc": 0.0, "dec": 0.0}
        latents = step(split)               # one extra untimed step for the encode/decode split
        log(f"split step: encode {split['enc']:.3f} s, decode {split['dec']:.3f} s; latents {tuple(latents.shape)}")
        finite = bool(torch.isfinite(latents).all()) and bool(torch.isfinite(out).all())
        torch.cuda.synchronize()
        timer.arm()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        timer.armed = False
        log(f"timed {args.steps} steps: {elapsed / args.steps:.3f} s/step")

    sec_per_step = elapsed / args.steps
    in_step = launch_stats(timer)

    # The timed steps run encoder tiles and decoder tile groups on two streams at once, so a launch shares
    # the GPU with the other stream's kernels for part of its time and its duration no longer describes the
    # kernel.  One more step with a single tile stream times the same launches alone: `roofline` and
    # `roofline_stage0_conv` come from it, their `in_step` objects from the timed steps.
    with torch.inference_mode():
        streams = runtime.tile_streams.count
        runtime.tile_streams.count = 1
        timer.reset()
        torch.cuda.synchronize()
        timer.arm()
        t0 = time.perf_counter()
        step()
        torch.cuda.synchronize()
        one_stream_s = time.perf_counter() - t0
        timer.armed = False
        runtime.tile_streams.count = streams
    alone = launch_stats(timer)
    log(f"one-stream step for the launch timings: {one_stream_s:.3f} s")
    clips = -(-args.frames // 17)
    enc_calls = 28 * clips
    dec_calls = 7 * 28 // 4 if args.frames == 124 else None
    conv_ops, fam_ops = alone["conv_ops"], alone["fam_ops"]
    achieved, gemm_achieved = alone["conv_achieved"], alone["gemm_achieved"]
    ref_s = REF_ENCODE_S + REF_DECODE_S
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
        "vs_baseline": round(sec_per_step / ref_s, 4) if args.frames == 124 and args.depth == DEC_BLOCKS else None,
        "dtype": "int8",
        "data": ("synthetic, seeded: fp16 clip clamp(U(-1,1) + upsampled coarse noise); random-init RECONSTRUCTED "
                 "H3 VAE (the MiniMax model code is not available): linears N(0,0.02), kaiming-uniform convs, "
                 "norm affines 1+N(0,0.1); INT8 weights from the build's quantizers"),
        "config": {
            "workload": f"cfg5_full_vae_encode_decode_1x3x{args.frames}x768x1344_tile256_batch4",
            "step": "runtime.encode(clip) then runtime.decode(latents, output_buffer) through H3VAEPyOptRuntime, "
                    "int8_encode + int8_decode + decode_fusions, staged batch 4, tile batch 4, two tile streams "
                    "(encoder tiles and decoder tile groups run two at a time)",
            "encode_tiles": 28, "clips": clips, "encode_prefix_calls": enc_calls,
            "decode_calls": dec_calls, "decode_blocks": args.depth, "decode_tokens_per_call": DEC_M,
        },
        "encode_s": round(split["enc"], 4),
        "decode_s": round(split["dec"], 4),
        "reference_rtx_pro_5000": {"encode_s": REF_ENCODE_S, "decode_s": REF_DECODE_S,
                                   "source": "reference README.md:43,53-54"},
        "outputs_finite": finite,
        "roofline": {
            "kernel": GEMM_KERNEL,
            "bound": "mfma",
            "achieved": round(gemm_achieved, 1),
            "peak": INT8_PEAK_TOPS,
            "unit": "TFLOP/s",
            "frac": round(gemm_achieved / INT8_PEAK_TOPS, 4),
            "traffic": gemm_traffic(),
            "launches_timed": alone["fam_n"],
            "avg_us": round(alone["fam_us"], 2),
            "timing": f"HIP events around every launch of one extra step run with a single tile stream "
                      f"({one_stream_s:.3f} s), so that no launch shares the GPU; achieved = mean ops per launch / "
                      "mean launch time",
            "algorithmic_ops_per_launch": round(fam_ops),
            "launch_mix": "per decoder block: QKV 7188x6144x2048, attention-out 7188x2048x2048, FFN-up "
                          "7188x16384x2048, FFN-down 7188x2048x8192 (one of each)",
            "per_gemm": alone["per_gemm"],
            "in_step": in_step_summary(in_step, "gemm"),
        },
        "roofline_stage0_conv": {
            "kernel": "conv3_halo_i8<256,Dequant,SP,64> (stage-0 conv C128->128, strided pixels on 64-pixel column blocks, "
                      "[1,128,19,258,258] int8, no residual, with the GroupNorm tile statistics of its output)",
            "bound": "mfma",
            "achieved": round(achieved, 1),
            "peak": INT8_PEAK_TOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / INT8_PEAK_TOPS, 4),
            "traffic": stage0_conv_traffic(),
            "launches_timed": alone["conv_n"],
            "avg_us": round(alone["conv_us"], 1),
            "timing": "as roofline: the one-stream step",
            "algorithmic_ops_per_launch": conv_ops,
            "in_step": in_step_summary(in_step, "conv"),
        },
    }
    log("measuring the MFMA ceiling for the stage-0 conv operands")
    with torch.inference_mode():
        ceiling = mfma_ceiling(torch, hip, runtime, clip)
    ceiling["conv_frac_of_ceiling"] = round(achieved / ceiling["tops"], 4)
    ceiling["gemm_frac_of_ceiling"] = round(gemm_achieved / ceiling["tops"], 4)
    result["mfma_ceiling"] = ceiling
    del runtime, clip, out
    torch.cuda.empty_cache()
    if not args.no_configs:
        log("timing BASELINE.json configs 1-4 on their own shapes")
        result["configs"] = config_measurements(torch, hip, kitchen, enc, stream, vs_torch=args.vs_torch)
    if not args.no_cpu_baseline:
        log("timing the CPU oracle baseline sample")
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
