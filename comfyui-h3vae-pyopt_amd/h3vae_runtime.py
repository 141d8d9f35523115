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


# ---- planning and stitching of spatial tiles ------------------------------------------------------------

def axis_tiles(length, tile, overlap_min, step):
    """Starts, lengths and overlaps of the tiles that cover one axis of ``length`` pixels.

    The fewest tiles of ``tile`` pixels whose overlaps are all at least ``overlap_min`` (n tiles
    cover n * tile - (n - 1) * overlap_min pixels); the surplus coverage is handed out in ``step``
    pixel units, one unit per overlap in turn from the first.  One tile if it already covers the axis.
    """
    if tile <= overlap_min:
        raise ValueError("encoder tile must exceed its minimum overlap")
    if tile >= length:
        return [0], [length], []
    count = -(-(length - overlap_min) // (tile - overlap_min))
    units = (count * tile - (count - 1) * overlap_min - length) // step
    each, extra = divmod(units, count - 1)
    overlaps = [overlap_min + step * (each + (k < extra)) for k in range(count - 1)]
    starts = [0]
    for overlap in overlaps:
        starts.append(starts[-1] + tile - overlap)
    return starts, [tile] * count, overlaps


def stitch_tiles(grid, y_overlaps, x_overlaps, blend):
    """Row-major grid of equally shaped tiles [..., h, w] -> one tensor.

    Each tile is cross-faded with the untouched tile above it over their vertical overlap, then
    with the untouched tile to its left over their horizontal overlap (``blend``); the part it
    shares with the tile below / to the right is cut, and the rest is placed on the canvas."""
    rows, cols = len(grid), len(grid[0])
    keep_h = [grid[i][0].shape[-2] - (y_overlaps[i] if i < rows - 1 else 0) for i in range(rows)]
    keep_w = [grid[0][j].shape[-1] - (x_overlaps[j] if j < cols - 1 else 0) for j in range(cols)]
    canvas = grid[0][0].new_empty((*grid[0][0].shape[:-2], sum(keep_h), sum(keep_w)))
    top = 0
    for i in range(rows):
        left = 0
        for j in range(cols):
            tile = grid[i][j]
            if i:
                tile = blend(grid[i - 1][j], tile, y_overlaps[i - 1], dim=-2)
            if j:
                tile = blend(grid[i][j - 1], tile, x_overlaps[j - 1], dim=-1)
            canvas[..., top:top + keep_h[i], left:left + keep_w[j]] = tile[..., :keep_h[i], :keep_w[j]]
            left += keep_w[j]
        top += keep_h[i]
    return canvas


class _TileStreams:
    """Runs independent tile jobs on ``count`` side streams in turn (default priority), so that one tile's
    memory-bound kernels and the partial last rounds of its matrix kernels overlap another tile's work.
    Each side stream first waits for the caller's stream; the caller's stream waits for every side stream
    before it goes on, and each result is marked as used on the caller's stream (``record_stream``), so
    the caching allocator never hands its memory out while a later kernel may still read it.  The tiles
    compute exactly what they compute one after another; only their kernels interleave.  count <= 1 (or
    a CPU device) runs the jobs in order on the caller's stream."""

    def __init__(self, count: int):
        self.count = max(1, int(count))
        self._streams = {}

    def run(self, jobs, device):
        if self.count == 1 or device.type != "cuda":
            return [job() for job in jobs]
        streams = self._streams.get(device)
        if streams is None:
            streams = self._streams[device] = [torch.cuda.Stream(device=device) for _ in range(self.count)]
        main = torch.cuda.current_stream(device)
        results = []
        for k, job in enumerate(jobs):
            side = streams[k % self.count]
            side.wait_stream(main)
            with torch.cuda.stream(side):
                out = job()
            out.record_stream(main)
            results.append(out)
        for side in streams:
            main.wait_stream(side)
        return results


class _TileBatcher:
    """Replacement for the core's ``_run_tile_tasks``: decoder tiles go through ``forward_fn`` in
    groups of ``batch`` (0: 1 or 2 by free GPU memory).  Anything it does not batch (class-token
    aggregation, batch > 1 or non-24-channel tiles, autograd) goes to the core's own routine."""

    RESERVE = 12 * 1024 ** 3      # kept free for the decoded video and other GPU users
    PER_TILE = 4 * 1024 ** 3

    def __init__(self, core, own, batch, streams=None):
        self.core, self.own, self.batch = core, own, int(batch)
        self.streams = streams if streams is not None else _TileStreams(1)

    def _group_size(self, device):
        if self.batch:
            return self.batch
        free, _ = torch.cuda.mem_get_info(device)
        return max(1, min(2, (free - self.RESERVE) // self.PER_TILE))

    def __call__(self, tiles, indices, forward_fn, stack_tiling, cls_agg=None):
        plain = bool(tiles) and tiles[0].shape[0] == 1 and tiles[0].shape[1] == 24
        if cls_agg is not None or not plain or torch.is_grad_enabled():
            return self.own(tiles, indices, forward_fn, stack_tiling, cls_agg)
        size = self._group_size(tiles[0].device)
        self.core._last_tile_batch = size
        if size == 1:
            return self.own(tiles, indices, forward_fn, stack_tiling, cls_agg)
        groups = [[tiles[i] for i in indices[first:first + size]] for first in range(0, len(indices), size)]
        outs = self.streams.run([lambda g=g: forward_fn(torch.cat(g, dim=0)) for g in groups], tiles[0].device)
        return [tile for out in outs for tile in out.split(1, dim=0)]


class _CallTimer:
    """Wall time of encode / decode calls with a running mean (logged when ``log_calls`` is on)."""

    def __init__(self):
        self.count, self.total_ms = {"encode": 0, "decode": 0}, {"encode": 0.0, "decode": 0.0}

    def reset(self):
        self.__init__()

    def record(self, kind, started, device):
        if device.type == "cuda":
            torch.cuda.synchronize(device)
        ms = (time.monotonic() - started) * 1e3
        self.count[kind] += 1
        self.total_ms[kind] += ms
        logger.info("[H3VAE-PyOpt] %s #%d: %.1f ms (running mean %.1f ms)", kind, self.count[kind], ms,
                    self.total_ms[kind] / self.count[kind])


class H3VAEPyOptRuntime(torch.nn.Module):
    """ComfyUI first_stage_model over the gfx950 hot path."""

    comfy_has_chunked_io = True

    def __init__(self, model_code_dir: str = DEFAULT_MODEL_CODE_DIR, weights_path: str = DEFAULT_WEIGHTS_FALLBACK,
                 device: str = "cuda", dtype: torch.dtype = torch.float16, decoder_tile_size: int = 256,
                 tile_batch: int = 2, compile_decoder: bool = True, compile_encoder: bool = True, qk_rows: int = 8,
                 encoder_staged_batch: int = 4, log_calls: bool = True, encoder_tile_size: int = 0,
                 fast_linear: bool = False, int8_decode: bool = False, int8_encode: bool = False,
                 decode_fusions: bool = False, *, core=None, config=None, tile_streams: int = 2):
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
        if int(tile_streams) < 1:
            raise ValueError("tile_streams must be at least 1")
        # independent encoder tiles and decoder tile groups run on this many streams at once
        self.tile_streams = _TileStreams(tile_streams)
        if core is None:
            core, config = _load_klvae_core(model_code_dir)
            if encoder_tile_size and encoder_tile_size <= core.tile_overlap_min:
                raise ValueError("encoder_tile_size must exceed encoder tile overlap")
            _load_weights(core, weights_path)
        elif config is None:
            raise ValueError("a prebuilt core needs its config (latents_mean / latents_std)")
        core.to(device=device, dtype=dtype)
        self.core, self.config = core, config
        self.encoder_tile_size = int(encoder_tile_size)
        core.tile_size = self.encoder_tile_size or 672
        self.encoder_staged_batch = int(encoder_staged_batch)
        self.fast_linear = False
        self.int8_decode, self.int8_encode = int8_decode, int8_encode
        self.decode_fusions = bool(decode_fusions)
        self.compile_decoder, self.compile_encoder = bool(compile_decoder), bool(compile_encoder)
        if self.compile_decoder or self.compile_encoder:
            logger.debug("[H3VAE-PyOpt] compile_decoder / compile_encoder are accepted but not used: the hot "
                         "operators are hand-written kernels, nothing is traced")
        self._wire_decoder(core, qk_rows, int(decoder_tile_size), int(tile_batch), device)
        self._wire_encoder(core)
        stats = {name: torch.tensor(config[name], dtype=dtype, device=device).view(1, -1, 1, 1, 1)
                 for name in ("latents_mean", "latents_std")}
        self.latents_mean, self.latents_std = stats["latents_mean"], stats["latents_std"]
        self._img_mean = torch.tensor(_IMG_MEAN, dtype=torch.float32, device=device).view(1, 3, 1, 1, 1)
        self._img_std = torch.tensor(_IMG_STD, dtype=torch.float32, device=device).view(1, 3, 1, 1, 1)
        self.log_calls = bool(log_calls)
        self._timer = _CallTimer()
        logger.info("[H3VAE-PyOpt] runtime ready: decoder_tile=%d encoder_tile=%s tile_batch=%d staged_batch=%d "
                    "int8_decode=%s int8_encode=%s decode_fusions=%s", core.decoder_tile_size,
                    self.encoder_tile_size or "auto", tile_batch, self.encoder_staged_batch, self.int8_decode,
                    self.int8_encode, self.decode_fusions)

    # ---- wiring ---------------------------------------------------------------------------------------

    def _wire_decoder(self, core, qk_rows, tile_size, tile_batch, device):
        """Fused QK-RMSNorm/RoPE always; INT8 FFNs with int8_decode; with decode_fusions also INT8 QKV and
        attention-out linears and the residual carry chain (reference h3vae_runtime.py:346-377)."""
        from .opt.decoder_fused_qk_rope import clone_with_qk_fusion
        decoder = clone_with_qk_fusion(core.decoder, qk_rows)
        if self.int8_decode:
            from .opt.kitchen_int8 import install_kitchen_int8_ffn
            try:
                count = install_kitchen_int8_ffn(decoder, mode="INT8both", require_cuda=True)
            except Exception as exc:  # noqa: BLE001 - an explicit option has no fallback
                raise RuntimeError("int8_decode installation failed; no fallback was applied") from exc
            logger.info("[H3VAE-PyOpt] INT8 FFNs: %d", count)
            if self.decode_fusions:
                from .opt.int8_attention_out import from_raw_decoder
                from .opt.int8_norm1_quant import clone_norm1_quant_decoder, supports_norm1_quant
                decoder = from_raw_decoder(decoder, warps=8)
                if supports_norm1_quant(device) and not getattr(decoder, "spatial_parallel", False):
                    decoder = clone_norm1_quant_decoder(decoder, enabled=True)
        core.decoder = decoder
        core.decoder_tile_size = tile_size
        core.stack_tiling = False
        if tile_batch != 1:
            self._install_batched_tiles(core, tile_batch, self.tile_streams)

    def _wire_encoder(self, core):
        """conv_in and every downsample conv with packed padding; the bias-fused prefix (residual-pack
        downsample) with INT8 convolutions under int8_encode; the clip-batched native suffix."""
        from .opt.encoder_fused_batched_norm import fused_suffix
        from .opt.encoder_fused_norm_next import next_fused_prefix
        from .opt.encoder_internal_padding import replace_selected, restore_selected
        from .opt.encoder_staged_batch import encode_staged
        self._encode_staged = encode_staged
        encoder = core.encoder.to(memory_format=torch.channels_last_3d)
        quant = core.quant_conv.to(memory_format=torch.channels_last_3d)
        # checked as a whole before anything is swapped; a later failure puts the model's convs back
        swaps = replace_selected(encoder, ["down.0.downsample.conv", "conv_in"])
        try:
            prefix = next_fused_prefix(encoder, "extend_bias_pack")
            suffix = fused_suffix(encoder, quant, all_stages=True)
            self.int8_encoder_metadata = None
            if self.int8_encode:
                from .opt.encoder_int8_integration import install_int8_encoder_prefix
                try:
                    self.int8_encoder_metadata = install_int8_encoder_prefix(prefix, require_cuda=True,
                                                                             tile_variant="auto")
                except Exception as exc:  # noqa: BLE001 - an explicit option has no fallback
                    raise RuntimeError("int8_encode installation failed; no fallback was applied") from exc
                logger.info("[H3VAE-PyOpt] INT8 encoder convolutions: %d", self.int8_encoder_metadata["count"])
        except BaseException:
            restore_selected(swaps)
            raise
        self.prefix, self.suffix = prefix, suffix

    @staticmethod
    def _install_batched_tiles(core, batch: int, streams=None):
        """Batch decoder tiles per forward call (0 picks 1 or 2 from free memory; reference :452-483); the
        groups run on ``streams`` (a _TileStreams) in turn."""
        core._run_tile_tasks = _TileBatcher(core, core._run_tile_tasks, batch, streams)

    # ---- small helpers --------------------------------------------------------------------------------

    def _device(self):
        return self.latents_mean.device

    @staticmethod
    def _frames_from_tokens(t: int) -> int:
        """Latent frames -> pixel frames, 5k+2 -> 17k+5 (reference :485-488)."""
        return 1 if t <= 1 else max(1, 17 * ((t - 2) // 5) + 5)

    @staticmethod
    def _tokens_from_frames(frames: int) -> int:
        """Pixel frames -> latent frames, 17k+5 -> 5k+2 (reference :490-493)."""
        return 1 if frames <= 1 else max(1, 5 * ((frames - 5) // 17) + 2)

    @staticmethod
    def _split_encoder_tiles(length, tile_size, overlap_min, ratio):
        return axis_tiles(length, tile_size, overlap_min, ratio)

    @staticmethod
    def _select_encoder_tile(configured, height, width):
        """The configured encoder tile, or 672 when the frame fits one, else 256."""
        if configured:
            return configured
        return 672 if max(height, width) <= 672 else 256

    def _record(self, kind, started):
        if self.log_calls:
            self._timer.record(kind, started, self._device())

    # ---- decode ---------------------------------------------------------------------------------------

    def decode_output_shape(self, input_shape):
        b, _, t, h, w = input_shape
        return (b, getattr(self.core.decoder, "out_channels", 3), self._frames_from_tokens(t), 16 * h, 16 * w)

    def _decode_raw(self, latents):
        """Denormalised latents -> the model's raw decoder output (reference :533-541): one latent
        frame is decoded alone and its last frame kept; fewer than 7 latent frames repeat the last one
        up to a whole temporal chunk."""
        t = latents.shape[2]
        if t == 1:
            return self.core.decode(latents)[:, :, -1:]
        if t < 7:
            latents = torch.cat([latents, latents[:, :, -1:].expand(-1, -1, 7 - t, -1, -1)], dim=2)
        return self.core.decode_base(latents, frame_num=self._frames_from_tokens(t))

    def _finalize(self, raw, output_buffer):
        """Raw pixels -> fp32 in [0, 1]: x * std + mean, then clamp.  A contiguous fp32 output_buffer of
        the output's shape on its device is written in place; any other buffer receives a copy."""
        direct = (output_buffer is not None and tuple(output_buffer.shape) == tuple(raw.shape)
                  and output_buffer.dtype == torch.float32 and output_buffer.device == raw.device
                  and output_buffer.is_contiguous())
        if self.decode_fusions:
            from .opt.fp16_finalize import finalize_pixels
            pixels = finalize_pixels(raw, self._img_std, self._img_mean, output_buffer if direct else None)
        else:
            pixels = (raw.float() * self._img_std + self._img_mean).clamp_(0.0, 1.0)
        if output_buffer is None:
            return pixels
        if pixels is not output_buffer:
            output_buffer.copy_(pixels)
        return output_buffer

    def decode(self, z, output_buffer=None, **kwargs):
        """Normalised latents [B, 24, t, h, w] -> fp32 pixels [B, 3, F, 16h, 16w] in [0, 1] (reference :514-564)."""
        started = time.monotonic()
        if self.int8_decode and z.dtype != torch.float16:
            raise RuntimeError("int8_decode requires FP16 latent input; use the FP16 VAE dtype")
        latents = z.to(device=self._device()) * self.latents_std + self.latents_mean
        out = self._finalize(self._decode_raw(latents), output_buffer)
        self._record("decode", started)
        return out

    # ---- encode ---------------------------------------------------------------------------------------

    def _normalize_pixels(self, x):
        """[-1, 1] pixels -> ImageNet-normalised [0, 1] pixels in the model dtype (fp32 arithmetic)."""
        unit = (x.float() + 1.0) * 0.5
        return ((unit - self._img_mean) / self._img_std).to(self.latents_mean.dtype)

    def _encode_moments(self, normed):
        """Moments of one spatial tile: clip-staged (reference :566-579); a single frame runs prefix and
        suffix directly and keeps the last latent frame."""
        if normed.shape[2] == 1:
            single = self.suffix(self.prefix(normed.contiguous(memory_format=torch.channels_last_3d)))
            return single[:, :, -1:]
        return self._encode_staged(normed, self.prefix, self.suffix, clip_length=self.core.clip_length,
                                   token_drop=self.core.token_drop, batch_size=self.encoder_staged_batch, cut=2)

    def _encode_spatial_tiled(self, x, tile_size):
        """Tiles of ``tile_size`` pixels encoded one by one and stitched with the core's blend
        (reference :609-639); x is normalised once for the whole video."""
        core = self.core
        ys, hs, y_over = axis_tiles(x.shape[-2], tile_size, core.tile_overlap_min, core.vae_ratio)
        xs, ws, x_over = axis_tiles(x.shape[-1], tile_size, core.tile_overlap_min, core.vae_ratio)
        normed = self._normalize_pixels(x)
        jobs = [lambda y=y, h=h, x0=x0, w=w: self._encode_moments(normed[..., y:y + h, x0:x0 + w])
                for y, h in zip(ys, hs) for x0, w in zip(xs, ws)]
        flat = self.tile_streams.run(jobs, normed.device)
        grid = [flat[i * len(xs):(i + 1) * len(xs)] for i in range(len(ys))]
        r = core.vae_ratio
        return stitch_tiles(grid, [o // r for o in y_over], [o // r for o in x_over], core.blend)

    def encode(self, x, device=None):
        """[-1, 1] pixels [B, 3, T, H, W] -> normalised latent means [B, 24, t, H/16, W/16] (reference :641-661)."""
        started = time.monotonic()
        if self.int8_encode and x.dtype != torch.float16:
            raise RuntimeError("int8_encode requires FP16 pixel input; use the FP16 VAE dtype")
        x = x.to(device=self._device())
        if x.ndim == 4:
            x = x.unsqueeze(2)
        tile = self._select_encoder_tile(self.encoder_tile_size, x.shape[-2], x.shape[-1])
        if max(x.shape[-2], x.shape[-1]) > tile:
            moments = self._encode_spatial_tiled(x, tile)
        else:
            moments = self._encode_moments(self._normalize_pixels(x))
        mean = moments.float()[:, :moments.shape[1] // 2]
        latents = (mean - self.latents_mean.float()) / self.latents_std.float()
        self._record("encode", started)
        return latents

    def decode_tiled(self, z, **kwargs):
        return self.decode(z)

    def encode_tiled(self, x, **kwargs):
        return self.encode(x)

    @torch.no_grad()
    def warmup(self, frames: int, width: int, height: int, mode: str = "both"):
        """One dummy decode and/or encode of the given shape, so first-call costs leave the first request."""
        dev = self._device()
        results = {}
        runs = []
        if mode in ("decode", "both"):
            z = torch.randn((1, 24, self._tokens_from_frames(frames), height // 16, width // 16), device=dev,
                            dtype=self.latents_mean.dtype)
            runs.append(("decode_first_s", self.decode, z))
        if mode in ("encode", "both"):
            x = torch.rand((1, 3, frames, height, width), device=dev, dtype=self.latents_mean.dtype) * 2.0 - 1.0
            runs.append(("encode_first_s", self.encode, x))
        for key, fn, arg in runs:
            if dev.type == "cuda":
                torch.cuda.synchronize(dev)
            started = time.monotonic()
            fn(arg)
            if dev.type == "cuda":
                torch.cuda.synchronize(dev)
            results[key] = round(time.monotonic() - started, 3)
        del runs
        if dev.type == "cuda":
            torch.cuda.empty_cache()
        self._timer.reset()
        logger.info("[H3VAE-PyOpt] warmup %s (%d frames, %dx%d): %s", mode, frames, width, height, results)
        return results


# ---- ComfyUI VAE wrapper ------------------------------------------------------------------------------

def _encode_memory(vae, shape, dtype):
    """Bytes ComfyUI reserves for an encode: the staged prefix holds about 1 kB per pixel of one clip."""
    import comfy.model_management as mm
    _, _, t, h, w = shape
    return int(vae.size + (1000 * min(t, 17) * h * w + 1_100_000_000) * mm.dtype_size(dtype) / 2 * 1.15)


def _decode_memory(vae, shape, dtype):
    """Bytes ComfyUI reserves for a decode: the whole fp16 video canvas, tile outputs and blend temporaries."""
    import comfy.model_management as mm
    _, _, t, h, w = shape
    canvas = 3 * vae.upscale_ratio[0](t) * (16 * h) * (16 * w) * 2 * 2.5
    return int(vae.size + (canvas + 1_100_000_000) * mm.dtype_size(dtype) / 2 * 1.1)


def _comfy_fields(int8):
    """The attributes ComfyUI's VAE reads, as its H3 branch sets them (reference :731-806)."""
    return {
        "latent_channels": 24, "latent_dim": 3, "output_channels": 3,
        "upscale_ratio": (H3VAEPyOptRuntime._frames_from_tokens, 16, 16), "upscale_index_formula": (4, 16, 16),
        "downscale_ratio": (H3VAEPyOptRuntime._tokens_from_frames, 16, 16), "downscale_index_formula": (4, 16, 16),
        "working_dtypes": [torch.float16] if int8 else [torch.float16, torch.float32],
        # the runtime tiles internally and returns finalised [0, 1] pixels; it wants [-1, 1] input
        "handles_tiling": True,
        "process_output": lambda image: image,
        "process_input": lambda image: image * 2.0 - 1.0,
        # defaults of the base class, whose constructor is not run
        "pad_channel_value": None, "disable_offload": False, "not_video": False, "size": None,
        "extra_1d_channel": None, "crop_input": True, "format_encoded": None,
    }


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
            for name, value in _comfy_fields(int8).items():
                setattr(self, name, value)
            self.device = model_management.vae_device() if device is None else device
            if dtype is None:
                dtype = model_management.vae_dtype(self.device, self.working_dtypes)
            if int8 and dtype != torch.float16:
                raise RuntimeError("INT8 VAE mode requires ComfyUI to select an FP16 VAE dtype")
            self.vae_dtype = dtype
            self.output_device = model_management.intermediate_device()
            self.memory_used_encode = lambda shape, dtype_: _encode_memory(self, shape, dtype_)
            self.memory_used_decode = lambda shape, dtype_: _decode_memory(self, shape, dtype_)
            self.patcher = comfy.model_patcher.CoreModelPatcher(
                first_stage_model, load_device=self.device, offload_device=model_management.vae_offload_device())
            self.model_size()

    return H3VAEPyOptVAE(runtime, dtype=dtype)
