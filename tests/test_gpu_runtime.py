"""GPU: the runtime's encoder wiring end to end on a reconstructed H3 core (tests/h3_arch.py).

H3VAEPyOptRuntime is built around the core exactly as for the real model: internal-padding stage-0
downsample, bias-fused prefix with the residual-pack downsample, INT8 prefix convolutions (int8_encode),
the clip-batched fused suffix (all stages) and staged clip batching.  Its encode must match the model's own
modules run through the same staged routine: within FP16 reduction-order differences in FP16 mode, within
the INT8 quantisation error in INT8 mode.  One, two and three 17-frame clips cover suffix batches 1, 2, 3.
"""
from __future__ import annotations

import copy
import importlib

import pytest
import torch
import torch.nn as nn

import h3_arch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


class _Core(nn.Module):
    """The parts of the klvae core the runtime touches on encode (decode is not called here)."""

    def __init__(self):
        super().__init__()
        self.encoder = h3_arch.H3Encoder()
        self.quant_conv = nn.Conv3d(48, 48, 1)
        self.decoder = h3_arch.H3Decoder(dim=256, hidden=512, depth=1)
        self.clip_length, self.token_drop, self.vae_ratio, self.tile_overlap_min = 17, 3, 16, 64
        self.tile_size, self.decoder_tile_size, self.stack_tiling = 672, 256, False

    def _run_tile_tasks(self, tiles, indices, forward_fn, stack_tiling, cls_agg=None):
        raise AssertionError("decode is not part of this test")

    def blend(self, a, b, extent, dim):
        raise AssertionError("a single spatial tile needs no blend")


def _config():
    return {"latents_mean": [0.05 * i for i in range(24)], "latents_std": [1.0 + 0.02 * i for i in range(24)]}


@pytest.fixture(scope="module")
def rt(pkg):
    return importlib.import_module(f"{pkg.__name__}.h3vae_runtime")


@pytest.mark.parametrize("int8_encode,clips", [(False, 1), (False, 2), (True, 3), (True, 2)])
def test_runtime_encode_matches_model_modules(rt, pkg, int8_encode, clips):
    print(f"runtime encode int8_encode={int8_encode} clips={clips}", flush=True)
    staged = importlib.import_module(f"{pkg.__name__}.opt.encoder_staged_batch")
    torch.manual_seed(11)
    core = _Core().eval()
    ref_enc = copy.deepcopy(core.encoder).half().to(DEV).eval().to(memory_format=torch.channels_last_3d)
    ref_quant = copy.deepcopy(core.quant_conv).half().to(DEV).eval().to(memory_format=torch.channels_last_3d)
    # the INT8 two-clip case builds the runtime under inference mode (its weights become inference tensors)
    with torch.inference_mode(int8_encode and clips == 2):
        runtime = rt.H3VAEPyOptRuntime(device="cuda", dtype=torch.float16, int8_encode=int8_encode,
                                       encoder_staged_batch=4, log_calls=False, core=core, config=_config())
    gen = torch.Generator().manual_seed(clips)
    x = (torch.rand(1, 3, 17 * clips, 64, 64, generator=gen) * 2 - 1).half().to(DEV)
    with torch.inference_mode():
        latents = runtime.encode(x)
        normed = runtime._normalize_pixels(x)
        moments = staged.encode_staged(normed, staged.EncoderPrefix(ref_enc, 2), staged.EncoderSuffix(ref_enc, ref_quant, 2),
                                       clip_length=17, token_drop=3, batch_size=4, cut=2)
        want = (moments.float()[:, :24] - runtime.latents_mean.float()) / runtime.latents_std.float()
        torch.cuda.synchronize()
    assert latents.shape == want.shape == (1, 24, 9 * clips - 3, 16, 16)
    assert torch.isfinite(latents).all()
    rel = float((latents - want).norm() / want.norm())
    assert rel < (0.1 if int8_encode else 1e-2), rel
