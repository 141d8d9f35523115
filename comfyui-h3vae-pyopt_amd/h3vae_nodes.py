"""ComfyUI loader node for the H3 video VAE on MI355X.

Counterpart of h3vae_nodes.py in fishelegs/ComfyUI-H3VAE-PyOpt
(``H3VAEPyOptLoader``, :34-191; mappings :194-197): the same node class name,
display name, option names, types and defaults, returning ``("VAE",)`` for
the stock VAEDecode / VAEEncode nodes.  ComfyUI's ``folder_paths`` is
imported when the node is used, so the package also imports without ComfyUI.
"""
from __future__ import annotations

import logging

import torch

from .h3vae_runtime import DEFAULT_MODEL_CODE_DIR, DEFAULT_WEIGHTS_FALLBACK, H3VAEPyOptRuntime, build_comfy_vae

logger = logging.getLogger("ComfyUI_H3VAE_PyOpt")

# Built VAEs per option set, so re-queueing a workflow does not reload the weights.
_VAE_CACHE: dict[tuple, object] = {}


def _folder_paths():
    import folder_paths
    return folder_paths


def _resolve_weights(vae_name: str, weights_path: str) -> str:
    if weights_path:
        return weights_path
    if vae_name == "use default":
        if not DEFAULT_WEIGHTS_FALLBACK:
            raise ValueError("Set H3_VAE_WEIGHTS_PATH or select a VAE file")
        return DEFAULT_WEIGHTS_FALLBACK
    return _folder_paths().get_full_path_or_raise("vae", vae_name)


class H3VAEPyOptLoader:
    """Load the MiniMax H3 video VAE with the MI355X INT8 hot path."""

    @classmethod
    def INPUT_TYPES(cls):
        try:
            vae_files = _folder_paths().get_filename_list("vae")
        except Exception:  # noqa: BLE001 - no ComfyUI model folders: offer the default only
            vae_files = []
        choices = ["use default"] + vae_files
        return {
            "required": {
                "vae_name": (choices, {"default": "use default",
                             "tooltip": "VAE safetensors from ComfyUI's vae folder; 'use default' reads "
                                        "H3_VAE_WEIGHTS_PATH."}),
                "dtype": (["fp16", "fp32"], {"default": "fp16"}),
                "decoder_tile_size": ("INT", {"default": 256, "min": 128, "max": 1024, "step": 16,
                                      "tooltip": "Spatial tile of the decoder in pixels."}),
                "tile_batch": ("INT", {"default": 2, "min": 0, "max": 8, "step": 1,
                               "tooltip": "Decoder tiles per forward call; 0 picks 1 or 2 from free GPU memory."}),
                "compile_decoder": ("BOOLEAN", {"default": True,
                                    "tooltip": "Accepted for workflow compatibility; the decoder hot path is "
                                               "hand-written HIP kernels and is not traced."}),
                "compile_encoder": ("BOOLEAN", {"default": True,
                                    "tooltip": "Accepted for workflow compatibility; the encoder hot path is "
                                               "hand-written HIP kernels and is not traced."}),
                "encoder_staged_batch": ([1, 2, 4], {"default": 4,
                                         "tooltip": "17-frame clips batched per encoder suffix call."}),
                "cudnn_benchmark": ("BOOLEAN", {"default": True,
                                    "tooltip": "Process-wide torch.backends.cudnn.benchmark (MIOpen search for the "
                                               "FP16 convolutions)."}),
                "warmup": (["none", "decode", "encode", "both"], {"default": "none",
                           "tooltip": "Run one dummy pass of the warmup shape at load."}),
                "warmup_frames": ("INT", {"default": 124, "min": 1, "max": 1000}),
                "warmup_width": ("INT", {"default": 1344, "min": 64, "max": 4096, "step": 16}),
                "warmup_height": ("INT", {"default": 768, "min": 64, "max": 4096, "step": 16}),
                "log_calls": ("BOOLEAN", {"default": True,
                              "tooltip": "Log each decode/encode latency with a running mean."}),
            },
            "optional": {
                "encoder_tile_size": ("INT", {"default": 0, "min": 0, "max": 1024, "step": 16,
                                      "tooltip": "0 = 672 up to 672x672 inputs, else 256."}),
                "fast_linear": ("BOOLEAN", {"default": False,
                                "tooltip": "comfy-kitchen FP16 linears; not available on this build."}),
                "decode_fusions": ("BOOLEAN", {"default": False,
                                   "tooltip": "With int8_decode: INT8 QKV/attention-out, fused norm/FFN chain and "
                                              "the residual carry between blocks."}),
                "int8_decode": ("BOOLEAN", {"default": False,
                                "tooltip": "INT8 decoder linears on MI355X (gfx950); FP16 only; no fallback."}),
                "int8_encode": ("BOOLEAN", {"default": False,
                                "tooltip": "INT8 3x3x3 convolutions of encoder prefix stages 0-1 with the fused "
                                           "GroupNorm/SiLU/pad/quant producer; FP16 only; no fallback."}),
                "model_code_dir": ("STRING", {"default": DEFAULT_MODEL_CODE_DIR,
                                   "tooltip": "MiniMax video_vae code bundle (klvae + source config)."}),
                "weights_path": ("STRING", {"default": "",
                                 "tooltip": "Direct path to the VAE safetensors (overrides vae_name)."}),
            },
        }

    RETURN_TYPES = ("VAE",)
    FUNCTION = "load"
    CATEGORY = "MiniMax_H3/Acceleration"
    DESCRIPTION = ("Load the MiniMax H3 video VAE on AMD MI355X: INT8 encoder prefix convolutions and INT8 decoder "
                   "blocks as hand-written gfx950 kernels; feeds the stock VAEDecode / VAEEncode nodes.")

    def load(self, vae_name, dtype, decoder_tile_size, tile_batch, compile_decoder, compile_encoder,
             encoder_staged_batch, cudnn_benchmark, warmup, warmup_frames, warmup_width, warmup_height, log_calls,
             model_code_dir=DEFAULT_MODEL_CODE_DIR, weights_path="", encoder_tile_size=0, fast_linear=False,
             int8_decode=False, int8_encode=False, decode_fusions=False):
        if bool(fast_linear) and bool(int8_decode):
            raise ValueError("int8_decode and fast_linear are mutually exclusive; choose one")
        key = (vae_name, weights_path, dtype, int(decoder_tile_size), int(encoder_tile_size), int(tile_batch),
               bool(compile_decoder), bool(compile_encoder), int(encoder_staged_batch), model_code_dir,
               bool(log_calls), bool(fast_linear), bool(int8_decode), bool(int8_encode), bool(decode_fusions))
        vae = _VAE_CACHE.get(key)
        if vae is None:
            weights = _resolve_weights(vae_name, weights_path)
            torch.backends.cudnn.benchmark = bool(cudnn_benchmark)
            torch.backends.cudnn.benchmark_limit = 5
            runtime = H3VAEPyOptRuntime(
                model_code_dir=model_code_dir, weights_path=weights, device="cuda",
                dtype=torch.float16 if dtype == "fp16" else torch.float32,
                decoder_tile_size=int(decoder_tile_size), encoder_tile_size=int(encoder_tile_size),
                tile_batch=int(tile_batch), compile_decoder=bool(compile_decoder),
                compile_encoder=bool(compile_encoder), encoder_staged_batch=int(encoder_staged_batch),
                fast_linear=bool(fast_linear), int8_decode=bool(int8_decode), int8_encode=bool(int8_encode),
                decode_fusions=bool(decode_fusions), log_calls=bool(log_calls))
            vae = build_comfy_vae(runtime)
            _VAE_CACHE[key] = vae
            logger.info("[H3VAE-PyOpt] loaded %s (%s, tile=%d, batch=%d)", weights, dtype, decoder_tile_size,
                        tile_batch)
        runtime = vae.first_stage_model
        if warmup != "none" and not getattr(runtime, "_warmed_up", False):
            try:
                runtime.warmup(int(warmup_frames), int(warmup_width), int(warmup_height), mode=warmup)
                runtime._warmed_up = True
            except Exception as exc:  # noqa: BLE001 - warmup is best effort outside the INT8 modes
                if (getattr(runtime, "int8_decode", False) or getattr(runtime, "int8_encode", False)
                        or getattr(runtime, "decode_fusions", False)):
                    raise RuntimeError("explicit optimized VAE warmup failed; no fallback was applied") from exc
                logger.warning("[H3VAE-PyOpt] warmup failed (%s: %s)", type(exc).__name__, exc)
        return (vae,)


NODE_CLASS_MAPPINGS = {"H3VAEPyOptLoader": H3VAEPyOptLoader}
NODE_DISPLAY_NAME_MAPPINGS = {"H3VAEPyOptLoader": "MiniMax H3 VAE Load (PyTorch Optimized)"}
