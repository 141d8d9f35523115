"""Reconstructed H3 video-VAE modules for the tests (test infrastructure).

The modules live in the package's ``reconstructed_h3`` (a random-init
reconstruction of the MiniMax H3 architecture, which the reference repository
does not contain).  Tests build a lighter encoder by default: stages 0 and 1 as
in H3 (they are the INT8 prefix) and one 256-wide suffix stage, 64 x 64 clips
-> 16 x 16 x 9-frame moments per clip.
"""
from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import torch

_ROOT = Path(__file__).resolve().parents[1]
if str(_ROOT) not in sys.path:
    sys.path.insert(0, str(_ROOT))
import __graft_entry__  # noqa: E402

_pkg = __graft_entry__.load_package()
_rec = importlib.import_module(f"{_pkg.__name__}.reconstructed_h3")

CausalConv3d = _rec.CausalConv3d
TemporalIsolatedSpatialParallelGroupNorm = _rec.TemporalIsolatedSpatialParallelGroupNorm
ResnetBlock3D = _rec.ResnetBlock3D
Downsample = _rec.Downsample
H3Attention = _rec.H3Attention
GatedFFN = _rec.GatedFFN
H3Block = _rec.H3Block
H3Decoder = _rec.H3Decoder
H3Core = _rec.H3Core
H3_ENCODER_STAGES = _rec.H3_ENCODER_STAGES
build_core = _rec.build_core

# stages 0-1 of H3 (the INT8 prefix) and one 256-wide suffix stage without a downsample
TEST_ENCODER_STAGES = (H3_ENCODER_STAGES[0], H3_ENCODER_STAGES[1], (256, None))


def H3Encoder(stages=TEST_ENCODER_STAGES, blocks_per_stage=2):
    return _rec.H3Encoder(stages, blocks_per_stage)


def rope_tables(batch, tokens, rot=48, base=10000.0, dtype=torch.float16):
    """cos/sin [B, N, 1, rot] for a 1-D token grid (the layout the fused op reads)."""
    inv = 1.0 / base ** (torch.arange(0, rot // 2, dtype=torch.float64) * 2 / rot)
    ang = torch.outer(torch.arange(tokens, dtype=torch.float64), inv)
    ang = torch.cat([ang, ang], dim=-1)
    cos = ang.cos().to(dtype).view(1, tokens, 1, rot).expand(batch, -1, -1, -1).contiguous()
    sin = ang.sin().to(dtype).view(1, tokens, 1, rot).expand(batch, -1, -1, -1).contiguous()
    return cos, sin
