"""CPU: the reconstructed core's decode planner (temporal chunks, spatial tiles, blends).

A decoder whose pixels depend only on the latent value under them (each latent
voxel -> a 4 x 16 x 16 block of its own value plus a per-frame offset) is
equivariant to tiling: overlapping tiles agree on their overlaps, every blend
is then a lerp of equal values, and ``decode_base`` must equal that decoder
applied to the whole latent, with the pre-padding frames taken out.  A dropped
or shifted tile, a wrong tail, a misplaced chunk or a wrong trim breaks the
equality.  In time each group of 5 latent frames decodes to 20 frames of
which 17 are kept (the next group's 3 pre-padding frames are dropped).  Output lengths follow the latent <-> frame formula 5k+2 <-> 17k+5
(h3vae_runtime.py:485-493 in the reference), and the planner constants those
of bench_h3vae_trt.py:175-259.
"""
from __future__ import annotations

import pytest
import torch

import h3_arch


class _BlockDecoder(torch.nn.Module):
    def forward(self, z):
        b, c, t, h, w = z.shape
        pix = z[:, :3].repeat_interleave(4, 2).repeat_interleave(16, 3).repeat_interleave(16, 4)
        frame = torch.arange(4 * t, dtype=z.dtype).remainder(4).view(1, 1, -1, 1, 1)
        return pix + 0.125 * frame


def _core(tile=256):
    core = h3_arch.H3Core(torch.nn.Identity(), _BlockDecoder())
    core.decoder_tile_size = tile
    return core


def test_planner_constants_and_tiles():
    core = _core()
    assert (core.chunk_tokens, core.token_overlap, core.frame_pre_padding) == (5, 2, 3)
    # the H3 video: 768 x 1344 at tile 256 -> 4 x 7 tiles
    assert core.split_tiles(768, 256) == ([0, 160, 336, 512], [256] * 4, [96, 80, 80])
    assert core.split_tiles(1344, 256) == ([0, 176, 352, 528, 704, 896, 1088], [256] * 7, [80, 80, 80, 80, 64, 64])
    assert core.split_tiles(200, 256) == ([0], [200], [])
    assert core.temporal_chunks(37) == (0, 7)      # 124 frames: 7 chunks of 7 tokens
    assert core.temporal_chunks(2) == (5, 1)


@pytest.mark.parametrize("t", [2, 7, 8, 12, 17, 22])
@pytest.mark.parametrize("hw,tile", [((16, 16), 256), ((8, 12), 128), ((10, 21), 96)])
def test_decode_base_equals_untiled_for_an_equivariant_decoder(t, hw, tile):
    core = _core(tile)
    gen = torch.Generator().manual_seed(t * 100 + hw[0])
    z = torch.randn(1, 24, t, *hw, generator=gen, dtype=torch.float64)
    frames = h3_arch._rec.frames_for_tokens(t)
    got = core.decode_base(z, frame_num=frames)
    pad, _ = core.temporal_chunks(t)
    zp = torch.cat([z, z[:, :, -1:].expand(-1, -1, pad, -1, -1)], dim=2) if pad else z
    # each 5-token group (20 decoder frames) keeps its frames 3..19; the 3 pre-padding frames of the next
    # group are dropped: output frame f comes from decoder frame 20 * (f // 17) + 3 + f % 17
    keep = torch.tensor([20 * (f // 17) + 3 + f % 17 for f in range(frames)])
    want = _BlockDecoder()(zp)[:, :, keep]
    assert got.shape == (1, 3, frames, 16 * hw[0], 16 * hw[1])
    torch.testing.assert_close(got, want, rtol=0, atol=1e-12)


def test_blend_is_a_linear_crossfade():
    a = torch.zeros(1, 1, 1, 1, 6, dtype=torch.float64)
    b = torch.ones(1, 1, 1, 1, 6, dtype=torch.float64)
    out = h3_arch.H3Core.blend(a, b, 4, dim=-1)
    assert out.flatten().tolist() == [0.0, 0.25, 0.5, 0.75, 1.0, 1.0]
    assert h3_arch.H3Core.blend(a, b, 0, dim=-1) is b


def test_reconstructed_shapes():
    torch.manual_seed(0)
    core = h3_arch.H3Core(h3_arch._rec.H3Encoder(), h3_arch.H3Decoder(dim=128, hidden=256, depth=1)).eval()
    with torch.no_grad():
        moments = core.quant_conv(core.encoder(torch.randn(1, 3, 17, 64, 64)))
        pixels = core.decoder(torch.randn(2, 24, 7, 2, 3))
        one = core.decode(torch.randn(1, 24, 1, 2, 2))
    assert moments.shape == (1, 48, 5, 4, 4)          # /4 in time (17 -> 5), /16 in space
    assert pixels.shape == (2, 3, 28, 32, 48)
    assert one.shape == (1, 3, 1, 32, 32)
