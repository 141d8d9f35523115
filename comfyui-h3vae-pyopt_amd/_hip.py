"""ctypes boundary to libh3vae_hip.so (the gfx950 kernels).

The library is built in-tree next to this file (``make -C csrc``).  There is
no fallback: if the library is missing or the device is not an MI355X
(gfx950), the ops raise instead of computing anything elsewhere.

Every kernel call passes raw device pointers, sizes and the current HIP
stream of the tensor's device.  Non-zero return codes become exceptions:
H3V_EINVAL -> ValueError (contract violation, nothing was queued),
anything else -> RuntimeError.
"""
from __future__ import annotations

import ctypes
import functools
import os
from pathlib import Path

import torch

LIB_NAME = "libh3vae_hip.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME
ABI_VERSION = 5
EINVAL = 1

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float

# name -> argtypes (every entry point returns int)
SIGNATURES: dict[str, list] = {
    "h3v_row_quant": [_P, _I64, _I64, _P, _P, _P],
    "h3v_swiglu_row_quant": [_P, _I64, _I64, _P, _P, _P],
    "h3v_gemm_i8_dequant": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P],
    "h3v_gemm_i8_swiglu": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P],
    "h3v_gemm_i8_i32": [_P, _P, _P, _I64, _I64, _I64, _P],
    "h3v_conv3d_i8_residual": [_P] * 7 + [_I] * 13 + [_P],
    "h3v_conv3d_i8_residual_padded": [_P] * 8 + [_I] * 12 + [_P],
    "h3v_conv3d_i8_gn": [_P] * 7 + [_I] * 6 + [_P, _P, _P],
    "h3v_conv3d_i8": [_P, _P, _P, _P, _P, _P] + [_I] * 13 + [_P],
    "h3v_conv3d_i8_i32": [_P, _P, _P] + [_I] * 13 + [_P],
    "h3v_tensor_quant_i8": [_P, _I64, _P, _P, _P, _I64, _P],
    "h3v_gn_norm_pack_i8": [_P, _P, _P, _P, _F, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P],
    "h3v_gn_norm_pack_i8_noalloc": [_P, _P, _P, _P, _F, _I, _I, _I, _I, _P, _P, _P, _P],
    "h3v_gn_norm_pack_i8_partials": [_P, _P, _P, _P, _F, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P],
    "h3v_residual_norm1_quant": [_P, _P, _P, _P, _F, _I64, _I64, _P, _P, _P, _P],
    "h3v_residual_rms_quant": [_P, _P, _P, _P, _F, _I64, _I64, _P, _P, _P, _P],
    "h3v_rms_fp16": [_P, _P, _F, _I64, _I64, _P, _P],
    "h3v_residual_layernorm": [_P, _P, _P, _P, _P, _F, _I64, _I64, _P, _P],
    "h3v_qk_rope": [_P, _P, _P, _I64, _I, _I, _I, _F, _P, _P, _P],
    "h3v_residual_downsample_pack": [_P, _P, _P, _P, _I, _I, _I, _I, _P],
    "h3v_selftest_fast_div": [_P, _P],
    "h3v_probe_mfma_rate": [_P, _I64, _P, _I64, _I, _I, _P, _P, _P],
    "h3v_finalize_pixels": [_P, _I, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P],
    "h3v_causal_reflect_pack": [_P, _P] + [_I] * 10 + [_P],
    "h3v_tap_fold_pack": [_P, _P] + [_I] * 7 + [_P],
    "h3v_conv3d_f16": [_P, _P, _P, _P, _P] + [_I] * 13 + [_P],
    "h3v_conv3d_f16_ws": [_P, _P, _P, _P, _P] + [_I] * 13 + [_P, _I64, _P],
    "h3v_conv3d_f16_gn": [_P, _P, _P, _P] + [_I] * 12 + [_P, _P],
    "h3v_gn_norm_pack_f16": [_P, _P, _P, _P, _F, _I, _I, _I, _I, _I, _P, _P, _P, _P],
    "h3v_attention_d64": [_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _I64, _I64, _I64, _F, _P],
}
# entry points with a non-int result
SPECIAL: dict[str, tuple] = {
    "h3v_abi_version": (ctypes.c_int, []),
    "h3v_last_error": (ctypes.c_char_p, []),
    "h3v_gn_norm_pack_workspace_floats": (ctypes.c_int64, [_I, _I, _I]),
    "h3v_tensor_quant_scratch_words": (ctypes.c_int64, []),
    "h3v_probe_mfma_ops_per_block": (ctypes.c_int64, [_I]),
    "h3v_gn_norm_pack_f16_workspace_floats": (ctypes.c_int64, [_I, _I, _I, _I, _I]),
    "h3v_conv3d_f16_workspace_floats": (ctypes.c_int64, [_I] * 12),
}


@functools.lru_cache(maxsize=1)
def lib() -> ctypes.CDLL:
    """Load the in-tree library once; raise if it is missing or stale."""
    path = Path(os.environ.get("H3VAE_HIP_LIB", str(LIB_PATH)))
    if not path.is_file():
        raise RuntimeError(
            f"{LIB_NAME} not found at {path}; build it with `make -C csrc` in the "
            "package directory (or __graft_entry__.build()). There is no fallback path.")
    handle = ctypes.CDLL(str(path))
    for name, args in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = ctypes.c_int
        fn.argtypes = args
    for name, (res, args) in SPECIAL.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    version = handle.h3v_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"{LIB_NAME} ABI version {version} != expected {ABI_VERSION}; rebuild it")
    return handle


def call(name: str, *args) -> None:
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        msg = lib().h3v_last_error().decode(errors="replace")
        raise (ValueError if rc == EINVAL else RuntimeError)(msg or f"{name} failed with code {rc}")


def ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


@functools.lru_cache(maxsize=8)
def _device_arch(index: int) -> str:
    return str(torch.cuda.get_device_properties(index).gcnArchName)


def is_gfx950(device) -> bool:
    device = torch.device(device)
    if device.type != "cuda" or torch.version.hip is None or not torch.cuda.is_available():
        return False
    index = torch.cuda.current_device() if device.index is None else device.index
    return _device_arch(index).split(":")[0] == "gfx950"


def require_gfx950(device, what: str) -> None:
    """Platform gate: the kernels are built for MI355X (gfx950) only."""
    device = torch.device(device)
    if device.type != "cuda":
        raise RuntimeError(f"{what} requires an AMD MI355X (gfx950) GPU tensor, got device {device}")
    if torch.version.hip is None:
        raise RuntimeError(f"{what} requires a ROCm PyTorch build")
    if not is_gfx950(device):
        raise RuntimeError(f"{what} requires an AMD MI355X (gfx950) GPU")
    lib()
