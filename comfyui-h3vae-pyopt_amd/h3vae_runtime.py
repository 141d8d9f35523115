"""H3 video-VAE runtime (ComfyUI ``first_stage_model``) over the gfx950 INT8 hot path.

Counterpart of h3vae_runtime.py in fishelegs/ComfyUI-H3VAE-PyOpt
(``H3VAEPyOptRuntime``, :283-728; ``build_comfy_vae``, :731-806).  It loads
the MiniMax H3 klvae model code and weights, rewires the decoder and the
encoder prefix onto this package's operator modules, and serves the
interface ComfyUI's ``comfy.sd.VAE`` expects:

  decode: z [B,24,t,h,w] normalised latents -> fp32 pixels [B,3,F,16h,16w] in [0,1]
  encode: x [B,3,T,H,W] in [-1,1]           -> normalised latents [B,24,t,H/16,W/16]

Decoder wiring (``int8_decode``): INT8 FFNs; with ``decode_fusions`` also
INT8 QKV and attention-out, the fused norm2/FFN-up/SwiGLU/requant/down chain
and the residual carry protocol with the fused norm1/QKV producer.  Fused
QK-RMSNorm/RoPE is always installed.  Encoder wiring (``int8_encode``): the
eight INT8 3x3x3 convolutions of prefix stages 0-1 with the fused
GroupNorm/SiLU/pad/quant producer, staged clip batching of the suffix.

Differences from the reference runtime, all deliberate:

* The platform gate is an AMD MI355X (gfx950) ROCm build instead of NVIDIA
  SM80+/SM120 CUDA; ``fast_linear`` (comfy-kitchen FP16 linears) and the FP16
  ``decode_fusions`` variant are not part of this build and are rejected.
* No tracing compiler: ``compile_decoder`` / ``compile_encoder`` are accepted
  and recorded but nothing is handed to torch.compile; the hot operators are
  already single hand-written kernels.
* The FP16 encoder suffix is the reference's clip-batched ``fused_suffix``
  (all stages): per-frame GroupNorm/SiLU/pad producers as
  ``h3v_gn_norm_pack_f16`` and the 3x3x3 stride-1 convolutions that fit as
  ``h3v_conv3d_f16``.
* The other FP16 encoder convolutions (conv_in, the prefix downsamples, the
  ``nin_shortcut`` projections, conv_out) also run as ``h3v_conv3d_f16``
  where the reference calls cuDNN; conv_in is routed through the same
  internal-padding wrapper as ``down.0.downsample.conv``.
"""
from __future__ import annotations

import json
import logging
import math
import os
import sys
import time
from pathlib import Path

import torch

from . import _hip

logger = logging.getLogger("ComfyUI_H3VAE_PyOpt")

DEFAULT_MODEL_CODE_DIR = os.environ.get("H3_VAE_MODEL_CODE_DIR", "")
DEFAULT_WEIGHTS_FALLBACK = os.environ.get("H3_VAE_WEIGHTS_PATH", "")

_PROBE = object()   # "not given": probe the platform
_IMG_MEAN = (0.485, 0.456, 0.406)
_IMG_STD = (0.229, 0.224, 0.225)


def _platform(device, *, hip=_PROBE, available=_PROBE, arch=_PROBE):
    """(device type, ROCm version, GPU available, gcn arch); arguments not given are probed."""
    try:
        device = torch.device(device)
    except (TypeError, RuntimeError):
        return None, hip, available, arch
    if hip is _PROBE:
        hip = torch.version.hip
    if available is _PROBE:
        available = torch.cuda.is_available()
    if arch is _PROBE:
        arch = None
        if device.type == "cuda" and hip is not None and available:
            index = torch.cuda.current_device() if device.index is None else device.index
            arch = str(torch.cuda.get_device_properties(index).gcnArchName).split(":")[0]
    return device.type, hip, available, arch


def _validate_platform(what, device, dtype, *, hip=_PROBE, available=_PROBE, arch=_PROBE):
    device_type, hip, available, arch = _platform(device, hip=hip, available=available, arch=arch)
    if device_type != "cuda":
        raise RuntimeError(f"{what} requires an AMD MI355X GPU device, got {device!r}")
    if dtype != torch.float16:
        raise RuntimeError(f"{what} requires dtype=fp16")
    if hip is None:
        raise RuntimeError(f"{what} requires a ROCm PyTorch build (AMD MI355X, gfx950)")
    if not available:
        raise RuntimeError(f"{what} requires an available AMD MI355X GPU")
    if arch != "gfx950":
        raise RuntimeError(f"{what} requires an AMD MI355X (gfx950) GPU; got {arch}")


def _validate_int8_decode_options(*, enabled, fast_linear, device, dtype, hip=_PROBE, available=_PROBE, arch=_PROBE,
                                  library_loads=_PROBE):
    """The explicit INT8 decoder contract, checked before any model is built (reference :66-128)."""
    if not enabled:
        return
    if fast_linear:
        raise ValueError("int8_decode and fast_linear are mutually exclusive; choose one")
    _validate_platform("int8_decode", device, dtype, hip=hip, available=available, arch=arch)
    _require_library("int8_decode", library_loads)


def _validate_int8_encode_options(*, enabled, device, dtype, hip=_PROBE, available=_PROBE, arch=_PROBE,
                                  library_loads=_PROBE):
    """The explicit INT8 encoder contract (reference :131-163)."""
    if not enabled:
        return
    _validate_platform("int8_encode", device, dtype, hip=hip, available=available, arch=arch)
    _require_library("int8_encode", library_loads)


def _validate_decode_fusions_options(*, enabled, int8_decode, fast_linear):
    """decode_fusions selects the fused INT8 decoder chain (reference :47-63)."""
    if not enabled:
        return
    if fast_linear:
        raise ValueError("decode_fusions and fast_linear are mutually exclusive")
    if not int8_decode:
        raise ValueError("decode_fusions on this build fuses the INT8 decoder; set int8_decode=true")
    if os.environ.get("MINIMAX_H3_VAE_DECODER_VIT_FP32_NORM", "1").lower() not in ("1", "true", "yes", "on"):
        raise ValueError("decode_fusions requires FP32 decoder normalization")


def _require_library(what, library_loads):
    if library_loads is _PROBE:
        try:
            _hip.lib()
        except RuntimeError as exc:
            raise RuntimeError(f"{what} requires libh3vae_hip.so: {exc}") from exc
    elif not library_loads:
        raise RuntimeError(f"{what} requires libh3vae_hip.so")


def _load_klvae_core(model_code_dir: str):
    """Build the MiniMax klvae ``AutoencoderKLLegacy`` from its code bundle (reference :208-257)."""
    if not model_code_dir:
        raise ValueError("Set H3_VAE_MODEL_CODE_DIR or pass model_code_dir")
    model_code_dir = Path(model_code_dir)
    if not (model_code_dir / "config.json").is_file():
        raise FileNotFoundError(f"MiniMax VAE config.json not found in {model_code_dir}")
    pkg_parent = str(model_code_dir.parent)
    if pkg_parent not in sys.path:
        sys.path.insert(0, pkg_parent)
    cfg = json.loads((model_code_dir / "config.json").read_text())
    from video_vae.parallel import get_parallel_state
    state = get_parallel_state()
    if isinstance(state, dict) and not state:
        # single-process inference: one rank, no sequence/tensor parallel groups
        state.update({"group_size": 1, "group_rank": 0, "local_process_group": None, "sp_size": 1, "sp_rank": 0,
                      "sp_enabled": False, "sp_process_group": None, "tp_size": 1, "tp_rank": 0})
    from video_vae.klvae import AutoencoderKLLegacy
    keys = ("clip_length", "token_drop", "encoder_tiling", "decoder_tiling", "parallel_tiling", "tile_size",
            "tile_overlap_min", "encoder_parallel", "decoder_parallel", "chunk_dim")
    load_kwargs = {key: int(cfg[f"vae_{key}"]) for key in keys}
    source_config = AutoencoderKLLegacy.load_config(str(model_code_dir / cfg["source_path"]))
    core, _ = AutoencoderKLLegacy.from_config(source_config, return_unused_kwargs=True, **load_kwargs)
    core.eval()
    return core, cfg


def _load_weights(core, weights_path: str):
    """Strict state-dict load; only the latent statistics may be extra (reference :260-280)."""
    if not weights_path:
        raise ValueError("Set H3_VAE_WEIGHTS_PATH or select a VAE file")
    if not Path(weights_path).is_file():
        raise FileNotFoundError(weights_path)
    weights_path = str(weights_path)
    if weights_path.endswith(".safetensors"):
        import safetensors.torch
        sd = safetensors.torch.load_file(weights_path)
    else:
        sd = torch.load(weights_path, map_location="cpu", weights_only=True)
    missing, unexpected = core.load_state_dict(sd, strict=False)
    bad_unexpected = set(unexpected) - {"latents_mean", "latents_std"}
    if missing or bad_unexpected:
        raise RuntimeError(f"weight mismatch for {weights_path}: missing={list(missing)[:8]} "
                           f"unexpected={sorted(bad_unexpected)[:8]}")
    if unexpected:
        logger.info("[H3VAE-PyOpt] ignored non-model buffer keys: %s", sorted(unexpected))


class H3VAEPyOptRuntime(torch.nn.Module):
    """ComfyUI first_stage_model over the gfx950 hot path."""

    comfy_has_chunked_io = True

    def __init__(self, model_code_dir: str = DEFAULT_MODEL_CODE_DIR, weights_path: str = DEFAULT_WEIGHTS_FALLBACK,
                 device: str = "cuda", dtype: torch.dtype = torch.float16, decoder_tile_size: int = 256,
                 tile_batch: int = 2, compile_decoder: bool = True, compile_encoder: bool = True, qk_rows: int = 8,
                 encoder_staged_batch: int = 4, log_calls: bool = True, encoder_tile_size: int = 0,
                 fast_linear: bool = False, int8_decode: bool = False, int8_encode: bool = False,
                 decode_fusions: bool = False, *, core=None, config=None):
        super().__init__()
        int8_decode, int8_encode = bool(int8_decode), bool(int8_encode)
        if fast_linear:
            raise RuntimeError("fast_linear (comfy-kitchen FP16 linears) is not part of this build")
        _validate_decode_fusions_options(enabled=bool(decode_fusions), int8_decode=int8_decode,
                                         fast_linear=bool(fast_linear))
        _validate_int8_decode_options(enabled=int8_decode, fast_linear=bool(fast_linear), device=device, dtype=dtype)
        _validate_int8_encode_options(enabled=int8_encode, device=device, dtype=dtype)
        if encoder_tile_size < 0 or encoder_tile_size % 16:
            raise ValueError("encoder_tile_size must be 0 (auto) or a positive multiple of 16")
        if int(tile_batch) < 0:
            raise ValueError("tile_batch must be non-negative")
        from .opt.decoder_fused_qk_rope import clone_with_qk_fusion
        from .opt.encoder_fused_norm_next import next_fused_prefix
        from .opt.encoder_internal_padding import replace_selected
        from .opt.encoder_fused_batched_norm import fused_suffix
        from .opt.encoder_staged_batch import encode_staged
        self._encode_staged = encode_staged

        if core is None:
            core, config = _load_klvae_core(model_code_dir)
            if encoder_tile_size and encoder_tile_size <= core.tile_overlap_min:
                raise ValueError("encoder_tile_size must exceed encoder tile overlap")
            _load_weights(core, weights_path)
        elif config is None:
            raise ValueError("a prebuilt core needs its config (latents_mean / latents_std)")
        core.to(device=device, dtype=dtype)
        self.core = core
        self.config = config
        self.encoder_tile_size = int(encoder_tile_size)
        core.tile_size = self.encoder_tile_size or 672

        # ---- decoder -------------------------------------------------------------------------------
        new_dec = clone_with_qk_fusion(core.decoder, qk_rows)
        if int8_decode:
            from .opt.kitchen_int8 import install_kitchen_int8_ffn
            try:
                count = install_kitchen_int8_ffn(new_dec, mode="INT8both", require_cuda=True)
            except Exception as exc:  # noqa: BLE001 - an explicit option has no fallback
                raise RuntimeError("int8_decode installation failed; no fallback was applied") from exc
            logger.info("[H3VAE-PyOpt] INT8 FFNs: %d", count)
            if decode_fusions:
                from .opt.int8_attention_out import from_raw_decoder
                from .opt.int8_norm1_quant import clone_norm1_quant_decoder, supports_norm1_quant
                new_dec = from_raw_decoder(new_dec, warps=8)
                if supports_norm1_quant(device) and not getattr(new_dec, "spatial_parallel", False):
                    new_dec = clone_norm1_quant_decoder(new_dec, enabled=True)
        core.decoder = new_dec
        core.decoder_tile_size = int(decoder_tile_size)
        core.stack_tiling = False
        if int(tile_batch) == 0 or int(tile_batch) > 1:
            self._install_batched_tiles(core, int(tile_batch))

        # ---- encoder -------------------------------------------------------------------------------
        enc = core.encoder.to(memory_format=torch.channels_last_3d)
        quant = core.quant_conv.to(memory_format=torch.channels_last_3d)
        replace_selected(enc, ["down.0.downsample.conv"])
        try:
            # conv_in (3 channels) through the tap-folded native conv; a conv_in that is not a causal
            # reflect-padded CausalConv3d stays the model's
            replace_selected(enc, ["conv_in"])
        except ValueError:
            pass
        prefix = next_fused_prefix(enc, "extend_bias_pack")
        suffix = fused_suffix(enc, quant, all_stages=True)
        metadata = None
        if int8_encode:
            from .opt.encoder_int8_integration import install_int8_encoder_prefix
            try:
                metadata = install_int8_encoder_prefix(prefix, require_cuda=True, tile_variant="auto")
            except Exception as exc:  # noqa: BLE001 - an explicit option has no fallback
                raise RuntimeError("int8_encode installation failed; no fallback was applied") from exc
            logger.info("[H3VAE-PyOpt] INT8 encoder convolutions: %d", metadata["count"])
        self.prefix, self.suffix = prefix, suffix
        self.encoder_staged_batch = int(encoder_staged_batch)
        self.fast_linear = bool(fast_linear)
        self.int8_decode, self.int8_encode = int8_decode, int8_encode
        self.decode_fusions = bool(decode_fusions)
        self.compile_decoder, self.compile_encoder = bool(compile_decoder), bool(compile_encoder)
        self.int8_encoder_metadata = metadata

        # ---- normalisation constants ---------------------------------------------------------------
        self.latents_mean = torch.tensor(config["latents_mean"], dtype=dtype, device=device).view(1, -1, 1, 1, 1)
        self.latents_std = torch.tensor(config["latents_std"], dtype=dtype, device=device).view(1, -1, 1, 1, 1)
        self._img_mean = torch.tensor(_IMG_MEAN, dtype=torch.float32, device=device).view(1, 3, 1, 1, 1)
        self._img_std = torch.tensor(_IMG_STD, dtype=torch.float32, device=device).view(1, 3, 1, 1, 1)

        self.log_calls = bool(log_calls)
        self._dec_calls, self._dec_total_ms = 0, 0.0
        self._enc_calls, self._enc_total_ms = 0, 0.0
        logger.info("[H3VAE-PyOpt] runtime ready: decoder_tile=%d encoder_tile=%s tile_batch=%d staged_batch=%d "
                    "int8_decode=%s int8_encode=%s decode_fusions=%s", core.decoder_tile_size,
                    self.encoder_tile_size or "auto", tile_batch, self.encoder_staged_batch, self.int8_decode,
                    self.int8_encode, self.decode_fusions)

    # ---- helpers ------------------------------------------------------------------------------------

    @staticmethod
    def _install_batched_tiles(core, batch: int):
        """Batch decoder tiles per forward; zero picks 1 or 2 from free memory (reference :452-483)."""
        original = core._run_tile_tasks

        def batched(tiles, indices, forward_fn, stack_tiling, cls_agg=None):
            if (cls_agg is not None or not tiles or tiles[0].shape[1] != 24 or tiles[0].shape[0] != 1
                    or torch.is_grad_enabled()):
                return original(tiles, indices, forward_fn, stack_tiling, cls_agg)
            current = batch
            if batch == 0:
                free, _ = torch.cuda.mem_get_info(tiles[0].device)
                # keep room for the decoded video and other users of the GPU before pairing tiles
                current = max(1, min(2, (free - 12 * 1024**3) // (4 * 1024**3)))
            core._last_tile_batch = current
            if current == 1:
                return original(tiles, indices, forward_fn, stack_tiling, cls_agg)
            outputs = []
            for start in range(0, len(indices), current):
                selected = indices[start:start + current]
                pixels = forward_fn(torch.cat([tiles[i] for i in selected], dim=0))
                outputs.extend(pixels.split(1, dim=0))
            return outputs

        core._run_tile_tasks = batched

    def _device(self):
        return self.latents_mean.device

    @staticmethod
    def _frames_from_tokens(t: int) -> int:
        """Latent frames -> pixel frames: 5k+2 -> 17k+5 (reference :485-488)."""
        return 1 if t <= 1 else max(1, (t - 2) // 5 * 17 + 5)

    @staticmethod
    def _tokens_from_frames(frames: int) -> int:
        """Pixel frames -> latent frames: 17k+5 -> 5k+2 (reference :490-493)."""
        return 1 if frames <= 1 else max(1, (frames - 5) // 17 * 5 + 2)

    def _log_call(self, kind: str, t0: float):
        if not self.log_calls:
            return
        if self._device().type == "cuda":
            torch.cuda.synchronize()
        dt = (time.monotonic() - t0) * 1000.0
        if kind == "decode":
            self._dec_calls += 1
            self._dec_total_ms += dt
            calls, total = self._dec_calls, self._dec_total_ms
        else:
            self._enc_calls += 1
            self._enc_total_ms += dt
            calls, total = self._enc_calls, self._enc_total_ms
        logger.info("[H3VAE-PyOpt] %s #%d: %.1f ms (running mean %.1f ms)", kind, calls, dt, total / calls)

    # ---- comfy first_stage_model interface -----------------------------------------------------------

    def decode_output_shape(self, input_shape):
        b, _, t, h, w = input_shape
        channels = getattr(self.core.decoder, "out_channels", 3)
        return (b, channels, self._frames_from_tokens(t), h * 16, w * 16)

    def decode(self, z, output_buffer=None, **kwargs):
        """Normalised latents -> fp32 pixels in [0, 1] (reference :514-564)."""
        t0 = time.monotonic()
        if self.int8_decode and z.dtype != torch.float16:
            raise RuntimeError("int8_decode requires FP16 latent input; use the FP16 VAE dtype")
        z = z.to(device=self._device())
        zn = z * self.latents_std + self.latents_mean
        t = zn.shape[2]
        if t == 1:
            dec = self.core.decode(zn)[:, :, -1:, :, :]
        else:
            if t < 7:
                # fewer latent frames than one temporal chunk: repeat the last one
                zn = torch.cat([zn, zn[:, :, -1:, :, :].repeat(1, 1, 7 - t, 1, 1)], dim=2)
            dec = self.core.decode_base(zn, frame_num=self._frames_from_tokens(t))
        # raw decoder output -> fp32 pixels in [0, 1] (reference :543-563)
        if self.decode_fusions:
            from .opt.fp16_finalize import finalize_pixels
            direct = (output_buffer is not None and output_buffer.shape == dec.shape
                      and output_buffer.dtype == torch.float32 and output_buffer.device == dec.device
                      and output_buffer.is_contiguous())
            pixels = finalize_pixels(dec, self._img_std, self._img_mean, output_buffer if direct else None)
        else:
            pixels = dec.float() * self._img_std + self._img_mean
            pixels = pixels.clamp_(0.0, 1.0)
        if output_buffer is not None:
            if pixels is not output_buffer:
                output_buffer.copy_(pixels)
            out = output_buffer
        else:
            out = pixels
        self._log_call("decode", t0)
        return out

    def _normalize_pixels(self, x):
        # [-1, 1] ComfyUI pixels -> ImageNet-normalised [0, 1] pixels in the model dtype
        x01 = (x.float() + 1.0) * 0.5
        normed = (x01 - self._img_mean.to(x01.dtype)) / self._img_std.to(x01.dtype)
        return normed.to(self.latents_mean.dtype)

    def _encode_moments(self, normed):
        if normed.shape[2] == 1:
            moments = self.suffix(self.prefix(normed.contiguous(memory_format=torch.channels_last_3d)))
            return moments[:, :, -1:, :, :]
        return self._encode_staged(normed, self.prefix, self.suffix, clip_length=self.core.clip_length,
                                   token_drop=self.core.token_drop, batch_size=self.encoder_staged_batch, cut=2)

    @staticmethod
    def _split_encoder_tiles(length, tile_size, overlap_min, ratio):
        """Tile starts/lengths/overlaps along one axis (reference :584-603).

        The smallest tile count whose minimum overlaps cover ``length``; the
        slack is spread round-robin over the overlaps in steps of ``ratio``.
        """
        if tile_size <= overlap_min:
            raise ValueError("encoder tile must exceed its minimum overlap")
        if tile_size >= length:
            return [0], [length], []
        count = math.ceil(length / tile_size)
        while True:
            overlaps = [overlap_min] * (count - 1)
            remaining = tile_size * count - sum(overlaps) - length
            if remaining >= 0:
                break
            count += 1
        for i in range(remaining // ratio):
            overlaps[i % (count - 1)] += ratio
        starts = [0]
        for overlap in overlaps:
            starts.append(starts[-1] + tile_size - overlap)
        return starts, [tile_size] * count, overlaps

    @staticmethod
    def _select_encoder_tile(configured, height, width):
        return configured or (672 if max(height, width) <= 672 else 256)

    def _encode_spatial_tiled(self, x, tile_size):
        core = self.core

        def split(length):
            return self._split_encoder_tiles(length, tile_size, core.tile_overlap_min, core.vae_ratio)

        y_idx, y_len, y_overlap = split(x.shape[-2])
        x_idx, x_len, x_overlap = split(x.shape[-1])
        rows = [[self._encode_moments(self._normalize_pixels(x[..., yp:yp + hh, xp:xp + ww]))
                 for xp, ww in zip(x_idx, x_len)] for yp, hh in zip(y_idx, y_len)]
        y_overlap = [o // core.vae_ratio for o in y_overlap]
        x_overlap = [o // core.vae_ratio for o in x_overlap]
        result_rows = []
        for i, row in enumerate(rows):
            result_row = []
            for j, tile in enumerate(row):
                if i:
                    tile = core.blend(rows[i - 1][j], tile, y_overlap[i - 1], dim=-2)
                if j:
                    tile = core.blend(row[j - 1], tile, x_overlap[j - 1], dim=-1)
                if i < len(rows) - 1:
                    tile = tile[..., :-y_overlap[i], :]
                if j < len(row) - 1:
                    tile = tile[..., :, :-x_overlap[j]]
                result_row.append(tile)
            result_rows.append(torch.cat(result_row, dim=-1))
        return torch.cat(result_rows, dim=-2)

    def encode(self, x, device=None):
        """[-1, 1] pixels -> normalised latent means (reference :641-661)."""
        t0 = time.monotonic()
        if self.int8_encode and x.dtype != torch.float16:
            raise RuntimeError("int8_encode requires FP16 pixel input; use the FP16 VAE dtype")
        x = x.to(device=self._device())
        if x.ndim == 4:
            x = x.unsqueeze(2)
        tile_size = self._select_encoder_tile(self.encoder_tile_size, x.shape[-2], x.shape[-1])
        if x.shape[-2] > tile_size or x.shape[-1] > tile_size:
            moments = self._encode_spatial_tiled(x, tile_size)
        else:
            moments = self._encode_moments(self._normalize_pixels(x))
        mean = moments.float()[:, :moments.shape[1] // 2]
        latents = (mean - self.latents_mean.float()) / self.latents_std.float()
        self._log_call("encode", t0)
        return latents

    def decode_tiled(self, z, **kwargs):
        return self.decode(z)

    def encode_tiled(self, x, **kwargs):
        return self.encode(x)

    @torch.no_grad()
    def warmup(self, frames: int, width: int, height: int, mode: str = "both"):
        """Run one dummy decode and/or encode of the given shape (first-call costs leave the first request)."""
        dev = self._device()
        is_gpu = dev.type == "cuda"
        results = {}
        if mode in ("decode", "both"):
            z = torch.randn((1, 24, self._tokens_from_frames(frames), height // 16, width // 16), device=dev,
                            dtype=self.latents_mean.dtype)
            if is_gpu:
                torch.cuda.synchronize()
            t0 = time.monotonic()
            self.decode(z)
            if is_gpu:
                torch.cuda.synchronize()
            results["decode_first_s"] = round(time.monotonic() - t0, 3)
        if mode in ("encode", "both"):
            x = torch.rand((1, 3, frames, height, width), device=dev, dtype=self.latents_mean.dtype) * 2.0 - 1.0
            if is_gpu:
                torch.cuda.synchronize()
            t0 = time.monotonic()
            self.encode(x)
            if is_gpu:
                torch.cuda.synchronize()
            results["encode_first_s"] = round(time.monotonic() - t0, 3)
        if is_gpu:
            torch.cuda.empty_cache()
        self._dec_calls, self._dec_total_ms = 0, 0.0
        self._enc_calls, self._enc_total_ms = 0, 0.0
        logger.info("[H3VAE-PyOpt] warmup %s (%d frames, %dx%d): %s", mode, frames, width, height, results)
        return results


def build_comfy_vae(runtime: H3VAEPyOptRuntime, dtype=None):
    """Wrap the runtime in a ``comfy.sd.VAE`` configured like ComfyUI's H3 branch (reference :731-806)."""
    import comfy.model_management as model_management
    import comfy.model_patcher
    import comfy.sd

    int8 = bool(getattr(runtime, "int8_decode", False) or getattr(runtime, "int8_encode", False))

    class H3VAEPyOptVAE(comfy.sd.VAE):
        def __init__(self, first_stage_model, device=None, dtype=None):
            # configured directly: the parent constructor would sniff a state dict
            self.first_stage_model = first_stage_model
            self.latent_channels = 24
            self.latent_dim = 3
            self.output_channels = 3
            self.upscale_ratio = (H3VAEPyOptRuntime._frames_from_tokens, 16, 16)
            self.upscale_index_formula = (4, 16, 16)
            self.downscale_ratio = (H3VAEPyOptRuntime._tokens_from_frames, 16, 16)
            self.downscale_index_formula = (4, 16, 16)
            self.working_dtypes = [torch.float16] if int8 else [torch.float16, torch.float32]
            self.handles_tiling = True
            self.process_output = lambda image: image
            self.process_input = lambda image: image * 2.0 - 1.0
            self.pad_channel_value = None
            self.disable_offload = False
            self.not_video = False
            self.size = None
            self.extra_1d_channel = None
            self.crop_input = True
            self.format_encoded = None
            if device is None:
                device = model_management.vae_device()
            self.device = device
            offload_device = model_management.vae_offload_device()
            if dtype is None:
                dtype = model_management.vae_dtype(self.device, self.working_dtypes)
            if int8 and dtype != torch.float16:
                raise RuntimeError("INT8 VAE mode requires ComfyUI to select an FP16 VAE dtype")
            self.vae_dtype = dtype
            self.output_device = model_management.intermediate_device()

            def estimate_encode_memory(shape, dtype_):
                _, _, t, h, w = shape
                dsize = model_management.dtype_size(dtype_)
                act = 1000 * min(t, 17) * h * w          # staged prefix activations, about 1 kB per clip pixel
                return int(self.size + (act + 1_100_000_000) * dsize / 2 * 1.15)

            def estimate_decode_memory(shape, dtype_):
                _, _, t, h, w = shape
                dsize = model_management.dtype_size(dtype_)
                out = 3 * self.upscale_ratio[0](t) * (h * 16) * (w * 16) * 2 * 2.5   # canvas + tiles + blend
                return int(self.size + (out + 1_100_000_000) * dsize / 2 * 1.1)

            self.memory_used_encode = estimate_encode_memory
            self.memory_used_decode = estimate_decode_memory
            self.patcher = comfy.model_patcher.CoreModelPatcher(first_stage_model, load_device=self.device,
                                                                offload_device=offload_device)
            self.model_size()

    return H3VAEPyOptVAE(runtime, dtype=dtype)
