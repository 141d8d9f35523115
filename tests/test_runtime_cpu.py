"""CPU contracts of the runtime (encode/decode callers) and the ComfyUI loader node.

Golden vectors from the reference's tests/test_runtime_tiling.py:17-24 and
tests/test_fp16_finalize.py:30-46 pin the tile planner and the decode
padding/output-buffer rules; closed-form invariants cover the rest of the
planner's domain.  Model code is faked: only the runtime's own logic runs.
"""
from __future__ import annotations

import importlib
import inspect
import math
import sys
import types

import pytest
import torch
import torch.nn.functional as F


@pytest.fixture(scope="module")
def rt(pkg):
    return importlib.import_module(f"{pkg.__name__}.h3vae_runtime")


@pytest.fixture(scope="module")
def nodes(pkg):
    return importlib.import_module(f"{pkg.__name__}.h3vae_nodes")


# -- C1 tile planner --------------------------------------------------------------------------------------

def test_encoder_tile_choice_golden(rt):
    choose = rt.H3VAEPyOptRuntime._select_encoder_tile
    assert choose(0, 672, 672) == 672
    assert choose(0, 768, 1344) == 256
    assert choose(672, 768, 1344) == 672


def test_encoder_split_golden(rt):
    split = rt.H3VAEPyOptRuntime._split_encoder_tiles
    assert split(672, 672, 64, 16) == ([0], [672], [])
    assert split(768, 256, 64, 16) == ([0, 160, 336, 512], [256] * 4, [96, 80, 80])
    assert split(1344, 256, 64, 16) == ([0, 176, 352, 528, 704, 896, 1088], [256] * 7, [80, 80, 80, 80, 64, 64])
    with pytest.raises(ValueError):
        split(768, 64, 64, 16)


@pytest.mark.parametrize("tile,overlap", [(256, 64), (672, 64), (128, 32)])
def test_encoder_split_invariants(rt, tile, overlap):
    split = rt.H3VAEPyOptRuntime._split_encoder_tiles
    for length in range(16, 4097, 16):
        starts, lengths, overlaps = split(length, tile, overlap, 16)
        if tile >= length:
            assert (starts, lengths, overlaps) == ([0], [length], [])
            continue
        n = len(starts)
        assert lengths == [tile] * n and len(overlaps) == n - 1
        assert starts[-1] + tile == length                      # exact cover for lengths on the 16-pixel grid
        assert all(o >= overlap and o % 16 == 0 for o in overlaps)
        assert max(overlaps) - min(overlaps) <= 16              # slack spread round-robin
        assert all(b - a == tile - o for a, b, o in zip(starts, starts[1:], overlaps))
        # minimal count: one tile fewer cannot cover the length with minimum overlaps
        assert tile * (n - 1) - overlap * (n - 2) < length


# -- C2 frames <-> tokens, decode padding and output buffer ------------------------------------------------

def test_frames_tokens_closed_form(rt):
    R = rt.H3VAEPyOptRuntime
    assert R._frames_from_tokens(37) == 124 and R._tokens_from_frames(124) == 37
    assert R._frames_from_tokens(1) == 1 and R._tokens_from_frames(1) == 1
    for k in range(40):
        assert R._frames_from_tokens(5 * k + 2) == 17 * k + 5
        assert R._tokens_from_frames(17 * k + 5) == 5 * k + 2


class _DecodeCore(torch.nn.Module):
    def decode(self, z):
        return z[:, :3]

    def decode_base(self, z, frame_num):
        self.last_frame_num = frame_num
        return self.decode(z)


def _bare_runtime(rt, core):
    r = rt.H3VAEPyOptRuntime.__new__(rt.H3VAEPyOptRuntime)
    torch.nn.Module.__init__(r)
    r.core = core
    r.latents_mean = torch.zeros((1, 24, 1, 1, 1), dtype=torch.float16)
    r.latents_std = torch.ones_like(r.latents_mean)
    r.int8_decode = r.int8_encode = False
    r.decode_fusions = False
    r.log_calls = False
    r.tile_streams = rt._TileStreams(2)
    r._img_mean = torch.tensor(rt._IMG_MEAN).reshape(1, 3, 1, 1, 1)
    r._img_std = torch.tensor(rt._IMG_STD).reshape(1, 3, 1, 1, 1)
    return r


def test_decode_padding_and_output_buffer_contract(rt):
    r = _bare_runtime(rt, _DecodeCore())
    with torch.inference_mode():
        for t in (1, 2, 7):
            z = torch.randn((1, 24, t, 2, 4), dtype=torch.float16)
            if t == 1:
                raw = z[:, :3, -1:]
            else:
                zp = torch.cat([z, z[:, :, -1:].repeat(1, 1, 7 - t, 1, 1)], dim=2) if t < 7 else z
                raw = zp[:, :3]
            expected = (raw.float() * r._img_std + r._img_mean).clamp(0, 1)
            got = r.decode(z)
            assert torch.equal(got, expected)
            if t > 1:
                assert r.core.last_frame_num == rt.H3VAEPyOptRuntime._frames_from_tokens(t)
            for out in (torch.empty_like(expected), torch.empty_like(expected).half(),
                        torch.empty((*expected.shape[:-2], 4, 2)).transpose(-1, -2)):
                assert r.decode(z, output_buffer=out) is out
                assert torch.equal(out, expected.to(out.dtype))
    r.int8_decode = True
    with pytest.raises(RuntimeError, match="FP16 latent"):
        r.decode(torch.zeros((1, 24, 2, 2, 4)))


def test_decode_fusions_finalize_path_matches_eager(rt, pkg, monkeypatch):
    """Reference tests/test_fp16_finalize.py:30-46: with decode_fusions the pixel finalisation goes
    through opt.fp16_finalize.finalize_pixels (patched here with the eager formula, as the reference
    test does), and both paths give the same pixels and honour the output-buffer contract."""
    fin = importlib.import_module(f"{pkg.__name__}.opt.fp16_finalize")
    calls = []

    def eager(x, std, mean, out=None):
        calls.append(out is not None)
        y = (x.float() * std + mean).clamp_(0, 1)
        if out is not None:
            out.copy_(y)
            return out
        return y

    monkeypatch.setattr(fin, "finalize_pixels", eager)
    r = _bare_runtime(rt, _DecodeCore())
    with torch.inference_mode():
        for int8, t in ((i, t) for i in (False, True) for t in (1, 2, 7)):
            r.int8_decode = int8
            z = torch.randn((1, 24, t, 2, 4), dtype=torch.float16)
            r.decode_fusions = False
            reference = r.decode(z)
            r.decode_fusions = True
            actual = r.decode(z)
            assert torch.equal(actual, reference)
            for out in (torch.empty_like(reference), torch.empty_like(reference).half(),
                        torch.empty((*reference.shape[:-2], 4, 2)).transpose(-1, -2)):
                assert r.decode(z, output_buffer=out) is out
                assert torch.equal(out, reference.to(out.dtype))
    # a matching contiguous fp32 buffer is written in place by the kernel; others get a copy
    assert True in calls and False in calls


def test_finalize_guards(pkg):
    """Reference tests/test_fp16_finalize.py:21-28: metadata guards raise ValueError before any launch,
    and a CPU tensor is refused (there is no eager fallback)."""
    fin = importlib.import_module(f"{pkg.__name__}.opt.fp16_finalize")
    x = torch.zeros((1, 3, 2, 4, 4), dtype=torch.float16)
    v = torch.ones(3)
    fin.validate(x, v, v)
    with pytest.raises(ValueError, match="gfx950"):
        fin.finalize_pixels(x, v, v)
    for a, b, c, o in [(x[:, :2], v, v, None), (x.double(), v, v, None), (x, v.half(), v, None),
                       (x, v, v, torch.empty_like(x)), (x[:, :, :0], v, v, None),
                       (x, v, v, torch.empty((1, 3, 2, 4, 4)).transpose(-1, -2))]:
        with pytest.raises(ValueError):
            fin.validate(a, b, c, o)


def test_decode_output_shape(rt):
    r = _bare_runtime(rt, _DecodeCore())
    r.core.decoder = torch.nn.Module()
    assert r.decode_output_shape((2, 24, 37, 48, 84)) == (2, 3, 124, 768, 1344)


# -- C1 encode orchestration (spatial tiles, clips, blend, posterior mean, normalisation) -------------------

class _EncodeCore:
    clip_length, token_drop, tile_overlap_min, vae_ratio = 17, 3, 64, 16

    @staticmethod
    def blend(a, b, overlap, dim):
        """Linear cross-fade of the overlap (a textbook stand-in for the model's blend)."""
        b = b.clone()
        n = overlap
        shape = [1] * b.ndim
        shape[dim] = n
        w = (torch.arange(n, dtype=b.dtype) / n).view(shape)
        a_tail = a.narrow(dim, a.shape[dim] - n, n)
        b.narrow(dim, 0, n).copy_(a_tail * (1 - w) + b.narrow(dim, 0, n) * w)
        return b


def _prefix(x):
    # 16x spatial average, 17 -> 5 frames, 3 -> 48 channels: translation-equivariant on the 16-pixel grid
    y = F.avg_pool3d(x.double(), (1, 16, 16))[:, :, ::4]
    return y.repeat(1, 16, 1, 1, 1)


def test_encode_tiled_equals_untiled_for_equivariant_model(rt, pkg):
    staged = importlib.import_module(f"{pkg.__name__}.opt.encoder_staged_batch")
    r = _bare_runtime(rt, _EncodeCore())
    r.latents_mean = torch.linspace(-0.5, 0.5, 24, dtype=torch.float64).view(1, 24, 1, 1, 1)
    r.latents_std = torch.linspace(0.5, 1.5, 24, dtype=torch.float64).view(1, 24, 1, 1, 1)
    r.prefix, r.suffix = _prefix, (lambda h: h)
    r._encode_staged, r.encoder_staged_batch, r.encoder_tile_size = staged.encode_staged, 4, 0
    gen = torch.Generator().manual_seed(1)
    # smooth content: any 16x16 cell average is what the untiled pass sees too
    base = torch.rand(1, 3, 34, 512 // 16, 768 // 16, generator=gen, dtype=torch.float64) * 2 - 1
    x = base.repeat_interleave(16, dim=3).repeat_interleave(16, dim=4)
    tiled = r.encode(x)
    assert tiled.shape == (1, 24, 2 * 5 - 3, 32, 48)
    untiled_moments = r._encode_moments(r._normalize_pixels(x))
    untiled = (untiled_moments.float()[:, :24] - r.latents_mean.float()) / r.latents_std.float()
    assert torch.allclose(tiled, untiled, rtol=0, atol=1e-5)
    # the posterior mean is the first half of the moments, then (mean - latents_mean) / latents_std
    x01 = (x.float() + 1) * 0.5
    normed = ((x01 - r._img_mean) / r._img_std).double()
    frames = torch.cat([normed, normed[:, :, -1:].repeat(1, 1, 0, 1, 1)], dim=2)
    moments = torch.cat([_prefix(frames[:, :, 0:17]), _prefix(frames[:, :, 17:34])], dim=2)[:, :, :-3]
    want = (moments.float()[:, :24] - r.latents_mean.float()) / r.latents_std.float()
    assert torch.allclose(untiled, want, rtol=0, atol=1e-6)
    r.int8_encode = True
    with pytest.raises(RuntimeError, match="FP16 pixel"):
        r.encode(x.float())


# -- option policy ---------------------------------------------------------------------------------------

def _supported(**overrides):
    values = dict(enabled=True, fast_linear=False, device="cuda", dtype=torch.float16, hip="7.0", available=True,
                  arch="gfx950", library_loads=True)
    values.update(overrides)
    return values


def test_int8_decode_option_policy(rt):
    v = rt._validate_int8_decode_options
    v(enabled=False, fast_linear=True, device="cpu", dtype=torch.float32)
    v(**_supported())
    with pytest.raises(ValueError, match="mutually exclusive"):
        v(**_supported(fast_linear=True))
    for override, message in ((dict(device="cpu"), "GPU device"), (dict(dtype=torch.float32), "fp16"),
                              (dict(hip=None), "ROCm"), (dict(available=False), "available"),
                              (dict(arch="gfx942"), "gfx950"), (dict(library_loads=False), "libh3vae_hip")):
        with pytest.raises(RuntimeError, match=message):
            v(**_supported(**override))


def test_int8_encode_and_fusion_option_policy(rt):
    e = rt._validate_int8_encode_options
    kwargs = _supported()
    del kwargs["fast_linear"]
    e(**kwargs)
    with pytest.raises(RuntimeError, match="gfx950"):
        e(**{**kwargs, "arch": "gfx90a"})
    f = rt._validate_decode_fusions_options
    f(enabled=False, int8_decode=False, fast_linear=True)
    f(enabled=True, int8_decode=True, fast_linear=False)
    with pytest.raises(ValueError, match="int8_decode"):
        f(enabled=True, int8_decode=False, fast_linear=False)
    with pytest.raises(ValueError, match="mutually exclusive"):
        f(enabled=True, int8_decode=True, fast_linear=True)


def test_runtime_rejects_before_loading(rt):
    params = inspect.signature(rt.H3VAEPyOptRuntime).parameters
    assert params["int8_decode"].default is False and params["int8_encode"].default is False
    assert params["decode_fusions"].default is False and params["fast_linear"].default is False
    with pytest.raises(RuntimeError, match="fast_linear"):
        rt.H3VAEPyOptRuntime(fast_linear=True)
    with pytest.raises(RuntimeError):
        rt.H3VAEPyOptRuntime(device="cpu", int8_decode=True)
    with pytest.raises(ValueError, match="model_code_dir"):
        rt.H3VAEPyOptRuntime(model_code_dir="", device="cpu")
    assert params["tile_streams"].default == 2
    with pytest.raises(ValueError, match="tile_streams"):
        rt.H3VAEPyOptRuntime(device="cpu", tile_streams=0)


def test_tile_streams_run_jobs_in_order_off_gpu(rt):
    """Off the GPU (and with one stream) the tile jobs run in order on the caller's stream."""
    seen = []
    jobs = [lambda k=k: seen.append(k) or torch.full((1,), float(k)) for k in range(5)]
    out = rt._TileStreams(3).run(jobs, torch.device("cpu"))
    assert seen == [0, 1, 2, 3, 4] and [float(t) for t in out] == [0.0, 1.0, 2.0, 3.0, 4.0]
    seen.clear()
    assert [float(t) for t in rt._TileStreams(1).run(jobs, torch.device("cpu"))] == [0.0, 1.0, 2.0, 3.0, 4.0]


# -- ComfyUI node -----------------------------------------------------------------------------------------

REQUIRED = ["vae_name", "dtype", "decoder_tile_size", "tile_batch", "compile_decoder", "compile_encoder",
            "encoder_staged_batch", "cudnn_benchmark", "warmup", "warmup_frames", "warmup_width", "warmup_height",
            "log_calls"]
OPTIONAL = ["encoder_tile_size", "fast_linear", "decode_fusions", "int8_decode", "int8_encode", "model_code_dir",
            "weights_path"]


def test_node_interface(pkg, nodes):
    assert pkg.NODE_CLASS_MAPPINGS == {"H3VAEPyOptLoader": nodes.H3VAEPyOptLoader}
    assert pkg.NODE_DISPLAY_NAME_MAPPINGS == {"H3VAEPyOptLoader": "MiniMax H3 VAE Load (PyTorch Optimized)"}
    spec = nodes.H3VAEPyOptLoader.INPUT_TYPES()
    assert list(spec["required"]) == REQUIRED and list(spec["optional"]) == OPTIONAL
    defaults = {name: opts[1].get("default") for part in spec.values() for name, opts in part.items()
                if len(opts) > 1}
    assert defaults == {"vae_name": "use default", "dtype": "fp16", "decoder_tile_size": 256, "tile_batch": 2,
                        "compile_decoder": True, "compile_encoder": True, "encoder_staged_batch": 4,
                        "cudnn_benchmark": True, "warmup": "none", "warmup_frames": 124, "warmup_width": 1344,
                        "warmup_height": 768, "log_calls": True, "encoder_tile_size": 0, "fast_linear": False,
                        "decode_fusions": False, "int8_decode": False, "int8_encode": False,
                        "model_code_dir": nodes.DEFAULT_MODEL_CODE_DIR, "weights_path": ""}
    assert spec["required"]["dtype"][0] == ["fp16", "fp32"]
    assert spec["required"]["encoder_staged_batch"][0] == [1, 2, 4]
    assert spec["required"]["warmup"][0] == ["none", "decode", "encode", "both"]
    assert nodes.H3VAEPyOptLoader.RETURN_TYPES == ("VAE",) and nodes.H3VAEPyOptLoader.FUNCTION == "load"
    params = list(inspect.signature(nodes.H3VAEPyOptLoader.load).parameters)[1:]
    assert params == REQUIRED + ["model_code_dir", "weights_path", "encoder_tile_size", "fast_linear",
                                 "int8_decode", "int8_encode", "decode_fusions"]


def test_node_rejects_before_loading(nodes, monkeypatch):
    loader = nodes.H3VAEPyOptLoader()
    args = dict(vae_name="use default", dtype="fp16", decoder_tile_size=256, tile_batch=2, compile_decoder=True,
                compile_encoder=True, encoder_staged_batch=4, cudnn_benchmark=True, warmup="none", warmup_frames=124,
                warmup_width=1344, warmup_height=768, log_calls=True)
    with pytest.raises(ValueError, match="mutually exclusive"):
        loader.load(**args, fast_linear=True, int8_decode=True)
    monkeypatch.setattr(nodes, "DEFAULT_WEIGHTS_FALLBACK", "")
    with pytest.raises(ValueError, match="H3_VAE_WEIGHTS_PATH"):
        loader.load(**args)
    assert nodes._resolve_weights("x.safetensors", "/direct/path") == "/direct/path"


def test_build_comfy_vae_configuration(rt, monkeypatch):
    comfy = types.ModuleType("comfy")
    sd = types.ModuleType("comfy.sd")
    mm = types.ModuleType("comfy.model_management")
    mp = types.ModuleType("comfy.model_patcher")

    class VAE:
        def model_size(self):
            self.size = 1000

    sd.VAE = VAE
    mm.vae_device = lambda: torch.device("cpu")
    mm.vae_offload_device = lambda: torch.device("cpu")
    mm.vae_dtype = lambda device, dtypes: dtypes[0]
    mm.intermediate_device = lambda: torch.device("cpu")
    mm.dtype_size = lambda dtype: torch.empty((), dtype=dtype).element_size()
    mp.CoreModelPatcher = lambda model, load_device, offload_device: ("patcher", model)
    comfy.sd, comfy.model_management, comfy.model_patcher = sd, mm, mp
    for name, module in (("comfy", comfy), ("comfy.sd", sd), ("comfy.model_management", mm),
                         ("comfy.model_patcher", mp)):
        monkeypatch.setitem(sys.modules, name, module)
    runtime = types.SimpleNamespace(int8_decode=True, int8_encode=False)
    vae = rt.build_comfy_vae(runtime)
    assert vae.first_stage_model is runtime and vae.latent_channels == 24 and vae.handles_tiling
    assert vae.upscale_ratio[0](37) == 124 and vae.upscale_ratio[1:] == (16, 16)
    assert vae.downscale_ratio[0](124) == 37 and vae.downscale_ratio[0](1) == 1
    assert vae.working_dtypes == [torch.float16] and vae.vae_dtype == torch.float16
    x = torch.rand(3)
    assert torch.equal(vae.process_input(x), x * 2.0 - 1.0) and vae.process_output(x) is x
    enc = vae.memory_used_encode((1, 3, 124, 768, 1344), torch.float16)
    dec = vae.memory_used_decode((1, 24, 37, 48, 84), torch.float16)
    assert enc == int(1000 + (1000 * 17 * 768 * 1344 + 1_100_000_000) * 2 / 2 * 1.15)
    assert dec == int(1000 + (3 * 124 * 768 * 1344 * 2 * 2.5 + 1_100_000_000) * 2 / 2 * 1.1)
    with pytest.raises(RuntimeError, match="FP16 VAE dtype"):
        rt.build_comfy_vae(runtime, dtype=torch.float32)
    fp = rt.build_comfy_vae(types.SimpleNamespace(int8_decode=False, int8_encode=False))
    assert fp.working_dtypes == [torch.float16, torch.float32]
    assert math.isclose(vae.memory_used_decode((1, 24, 1, 1, 1), torch.float16),
                        int(1000 + (3 * 1 * 16 * 16 * 2 * 2.5 + 1_100_000_000) * 1.1))


def test_encoder_wiring_on_a_reconstructed_core(rt, pkg):
    """The runtime's encoder wiring (reference h3vae_runtime.py:389-395, plus conv_in): conv_in and
    down.0.downsample.conv through the internal-padding wrapper, the bias-fused prefix with the residual
    pack downsample, and the clip-batched fused suffix over every suffix stage."""
    import h3_arch
    import torch.nn as nn

    class _Core(nn.Module):
        def __init__(self):
            super().__init__()
            self.encoder = h3_arch.H3Encoder()
            self.quant_conv = nn.Conv3d(48, 48, 1)
            self.decoder = h3_arch.H3Decoder(dim=128, hidden=256, depth=1)
            self.clip_length, self.token_drop, self.vae_ratio, self.tile_overlap_min = 17, 3, 16, 64
            self.tile_size, self.decoder_tile_size, self.stack_tiling = 672, 256, False

        def _run_tile_tasks(self, *args, **kwargs):
            raise AssertionError("not called")

    config = {"latents_mean": [0.0] * 24, "latents_std": [1.0] * 24}
    # a conv_in without a reflect border is refused before any conv of the caller's core is swapped
    bad = _Core().eval()
    bad.encoder.conv_in.pad_mode = "constant"
    down, conv_in = bad.encoder.down[0].downsample.conv, bad.encoder.conv_in
    with pytest.raises(ValueError, match="conv_in: .*pad_mode='constant'"):
        rt.H3VAEPyOptRuntime(device="cpu", dtype=torch.float32, log_calls=False, core=bad, config=config)
    assert bad.encoder.down[0].downsample.conv is down and bad.encoder.conv_in is conv_in
    runtime = rt.H3VAEPyOptRuntime(device="cpu", dtype=torch.float32, log_calls=False, core=_Core().eval(),
                                   config=config)
    assert type(runtime.prefix.conv_in).__name__ == "ImplicitTemporalPadConv3d"
    assert type(runtime.prefix.stages[0].downsample.conv).__name__ == "ImplicitTemporalPadConv3d"
    assert [type(b).__name__ for b in runtime.prefix.stages[0].block] == ["BiasFusedResidualBlock"] * 2
    assert type(runtime.prefix.stages[1].block[-1]).__name__ == "ResidualDownsampleBlock"
    assert type(runtime.suffix).__name__ == "BatchedSuffix"
    assert type(runtime.suffix.stages[0].block[0]).__name__ == "BatchedResidualBlock"
    assert runtime.suffix.final is not None
