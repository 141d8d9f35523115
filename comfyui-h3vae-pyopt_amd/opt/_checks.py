"""Shared argument checks for the operator modules (raise before any launch)."""
from __future__ import annotations

import torch

ROW_WIDTHS = (1024, 2048, 4096)


def same_device_contiguous(tensors, device) -> bool:
    return all(t.device == device and t.is_contiguous() for t in tensors if t is not None)


def require_fp16(name: str, *tensors) -> None:
    for t in tensors:
        if t is not None and t.dtype != torch.float16:
            raise ValueError(f"{name}: FP16 tensors required, got {t.dtype}")


def require_grad_off(what: str) -> None:
    if torch.is_grad_enabled():
        raise RuntimeError(f"{what} requires inference/no_grad")
