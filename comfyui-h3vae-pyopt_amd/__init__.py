"""ComfyUI H3 VAE INT8 hot path for AMD MI355X (gfx950).

Drop-in counterpart of the ComfyUI-H3VAE-PyOpt plugin's INT8 hot path: the
same operator modules (``opt/``) and op names, running hand-written CDNA4
kernels from ``libh3vae_hip.so`` through a C ABI (``_hip.py``).

ComfyUI loads custom-node directories with ``spec_from_file_location`` on this
file, which makes the directory a package; the modules use relative imports.
"""
import os

__version__ = "0.1.0"

# Same process-wide defaults as the reference plugin entry (__init__.py:23-24).
os.environ.setdefault("MINIMAX_H3_TORCH_SDPA_BACKEND", "auto")
os.environ.setdefault("MINIMAX_H3_VAE_DECODER_VIT_FP32_NORM", "1")

from .h3vae_nodes import NODE_CLASS_MAPPINGS, NODE_DISPLAY_NAME_MAPPINGS  # noqa: E402

__all__ = ["NODE_CLASS_MAPPINGS", "NODE_DISPLAY_NAME_MAPPINGS"]
