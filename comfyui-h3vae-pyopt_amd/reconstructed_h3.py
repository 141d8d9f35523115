"""A random-init RECONSTRUCTION of the MiniMax H3 video VAE (klvae) for tests and the benchmark.

The runtime drives the MiniMax model code (``video_vae.klvae.AutoencoderKLLegacy``,
loaded by ``_load_klvae_core`` in fishelegs/ComfyUI-H3VAE-PyOpt
h3vae_runtime.py:208-257).  That code and its weights are not part of the
reference repository and are not available here, so this module rebuilds the
architecture from the evidence the reference holds, with random weights.  It is
not the MiniMax model; nothing in the product path imports it.

What it reproduces, and where each fact comes from:

* Encoder (``H3Encoder``).  Causal 3x3x3 convs with two zero leading frames and
  a reflect spatial border (opt/encoder_internal_padding.py:14-35), per-frame
  GroupNorm(32) (opt/encoder_fused_temporal_norm.py), residual blocks with a
  1x1x1 ``nin_shortcut`` where the width changes.  conv_in 3 -> 128; stage 0:
  two C128 blocks at 17x256x256, downsample stride (1,2,2); stage 1: 128->256,
  256->256, downsample stride (2,2,2) with right/bottom reflect
  (opt/encoder_fused_residual_pack.py:58-63); suffix stages 2-4 at C 256, 512,
  1024 (the widths opt/encoder_fused_batched_norm.py:49 accepts) down to
  5x16x16; norm_out + SiLU + conv_out -> 48; a 1x1x1 quant_conv
  (opt/encoder_staged_batch.py:32-36).  One 17-frame 256x256 clip gives
  [1, 48, 5, 16, 16] (bench_h3vae_trt.py:35-37).
* Decoder (``H3Decoder``).  A [B, 24, 7, 16, 16] latent tile becomes 1792
  patch tokens of width 2048 plus 5 learned register tokens (1797 rows per
  item, the B4 shape [4, 1797, 2048] of opt/int8_norm1_quant.py); 36 blocks of
  RMSNorm -> QKV -> QK-RMSNorm + rotary on 48 of 64 dims -> attention over 32
  heads -> out -> ``h + attn * scale1`` -> RMSNorm -> gated SiLU FFN 2048 ->
  2 x 8192 -> 2048 -> ``h + ffn * scale2`` (opt/int8_norm_quant.py:106-124,
  opt/int8_norm1_quant.py:218-252, opt/decoder_fused_qk_rope.py:56-74); a final
  LayerNorm (opt/decoder_final_norm.py) and a linear head to 3 x 4 x 16 x 16
  pixels per patch token: [B, 3, 28, 256, 256] (bench_h3vae_trt.py:34-36).
  The 3-D rotary table gives each of t, y, x eight frequencies of the 24
  rotated pairs; register tokens sit at position zero.
* Core (``H3Core``).  The planner constants clip_length 17, token_drop 3,
  spatial ratio 16, temporal ratio 4, minimum tile overlap 64
  (bench_h3vae_trt.py:175-185); ``blend`` (:317-330); ``decode_base``: 7-token
  temporal chunks with 2 tokens of overlap, spatial tiles of
  ``decoder_tile_size`` pixels blended across their overlaps, the chunk
  split/blend in time and the tail trim (:338-442); ``_run_tile_tasks``, the
  hook the runtime batches tiles through (h3vae_runtime.py:452-479).

Initialisation: linears N(0, 0.02) with N(0, 0.02) biases, convs PyTorch's
default kaiming-uniform, norm scales 1 + N(0, 0.1) and shifts N(0, 0.1),
residual gates 0.1 * N(0, 1); ``build_core(seed=...)`` makes it reproducible.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

LATENT_CHANNELS = 24

# (output width, downsample) per encoder stage; downsample = (stride, padding, right/bottom-only reflect)
H3_ENCODER_STAGES = (
    (128, ((1, 2, 2), (1, 1, 1), False)),
    (256, ((2, 2, 2), (1, 0, 0), True)),
    (256, ((2, 2, 2), (1, 0, 0), True)),
    (512, ((1, 2, 2), (1, 0, 0), True)),
    (1024, None),
)


# -- encoder ------------------------------------------------------------------------------------

class CausalConv3d(nn.Module):
    """Conv3d after a reflect spatial border and left-only zero frames in time.

    ``padding = (pt, ph, pw)``: 2*pt zero frames in front (kd - 1 for a single-frame input), a reflect
    border of ph/pw; ``right_bottom_only`` reflects one row and one column at the far edges instead."""

    def __init__(self, cin, cout, kernel=3, stride=(1, 1, 1), padding=(1, 1, 1), bias=True):
        super().__init__()
        k = (kernel,) * 3 if isinstance(kernel, int) else tuple(kernel)
        self.weight = nn.Parameter(torch.empty(cout, cin, *k))
        self.bias = nn.Parameter(torch.empty(cout)) if bias else None
        nn.init.kaiming_uniform_(self.weight, a=5 ** 0.5)
        if self.bias is not None:
            nn.init.uniform_(self.bias, -0.1, 0.1)
        self.kernel_size, self.stride, self.padding = k, tuple(stride), tuple(padding)
        self.causal, self.pad_mode, self.pad_mode_t, self.spatial_parallel = True, "reflect", "constant", False
        self.groups, self.dilation = 1, (1, 1, 1)
        self.right_bottom_only = False

    def forward(self, x):
        pt, ph, pw = self.padding
        if self.right_bottom_only:
            x = F.pad(x, (0, 1, 0, 1, 0, 0), mode="reflect")
        elif ph or pw:
            x = F.pad(x, (pw, pw, ph, ph, 0, 0), mode="reflect")
        if pt:
            front = 2 * pt if x.shape[2] > 1 else self.kernel_size[0] - 1
            x = F.pad(x, (0, 0, 0, 0, front, 0))
        return F.conv3d(x, self.weight, self.bias, stride=self.stride)


class TemporalIsolatedSpatialParallelGroupNorm(nn.GroupNorm):
    """GroupNorm whose statistics are taken per frame (fp32 statistics, output in the input dtype)."""

    def forward(self, x):
        b, c, d, h, w = x.shape
        y = x.transpose(1, 2).reshape(b * d, c, h, w)
        y = F.group_norm(y.float(), self.num_groups, self.weight.float(), self.bias.float(), self.eps)
        return y.to(x.dtype).reshape(b, d, c, h, w).transpose(1, 2)


def _init_norm(norm):
    nn.init.normal_(norm.weight, 1.0, 0.1)
    nn.init.normal_(norm.bias, 0.0, 0.1)


class ResnetBlock3D(nn.Module):
    def __init__(self, cin, cout, eps=1e-6):
        super().__init__()
        self.norm1 = TemporalIsolatedSpatialParallelGroupNorm(32, cin, eps=eps)
        self.conv1 = CausalConv3d(cin, cout)
        self.norm2 = TemporalIsolatedSpatialParallelGroupNorm(32, cout, eps=eps)
        self.conv2 = CausalConv3d(cout, cout)
        if cin != cout:
            self.nin_shortcut = nn.Conv3d(cin, cout, 1)
        self.use_fused_norm = False
        _init_norm(self.norm1)
        _init_norm(self.norm2)

    def forward(self, x, zq=None):
        h = self.conv1(F.silu(self.norm1(x)))
        h = self.conv2(F.silu(self.norm2(h)))
        return (self.nin_shortcut(x) if hasattr(self, "nin_shortcut") else x) + h


class Downsample(nn.Module):
    def __init__(self, c, stride, padding, right_bottom=False):
        super().__init__()
        self.conv = CausalConv3d(c, c, 3, stride=stride, padding=padding)
        self.conv.right_bottom_only = right_bottom

    def forward(self, x):
        return self.conv(x)


class H3Encoder(nn.Module):
    """conv_in -> stages of residual blocks (+ downsample) -> norm_out / SiLU / conv_out (2 x latent channels)."""

    def __init__(self, stages=H3_ENCODER_STAGES, blocks_per_stage=2, latent=LATENT_CHANNELS, base=128):
        super().__init__()
        self.conv_in = CausalConv3d(3, base)
        self.down = nn.ModuleList()
        cin = base
        for cout, down in stages:
            stage = nn.Module()
            stage.block = nn.ModuleList([ResnetBlock3D(cin if i == 0 else cout, cout)
                                         for i in range(blocks_per_stage)])
            if down is not None:
                stride, padding, right_bottom = down
                stage.downsample = Downsample(cout, stride, padding, right_bottom)
            self.down.append(stage)
            cin = cout
        self.norm_out = TemporalIsolatedSpatialParallelGroupNorm(32, cin, eps=1e-6)
        _init_norm(self.norm_out)
        self.conv_out = CausalConv3d(cin, 2 * latent)
        self.gradient_checkpointing = False
        self.use_fused_norm = False

    def forward(self, x):
        h = self.conv_in(x)
        for stage in self.down:
            for block in stage.block:
                h = block(h)
            if hasattr(stage, "downsample"):
                h = stage.downsample(h)
        return self.conv_out(F.silu(self.norm_out(h)))


# -- decoder ------------------------------------------------------------------------------------

def _init_linear(lin, std=0.02):
    nn.init.normal_(lin.weight, 0.0, std)
    if lin.bias is not None:
        nn.init.normal_(lin.bias, 0.0, 0.02)


class H3Attention(nn.Module):
    """QKV projection (per head [q | k | v]), unaffined QK RMSNorm, rotary on the first ``rot`` dims,
    attention, out projection.  ``mix = "sum"`` swaps the softmax attention for the elementwise fp16
    ``(q + k) + v`` (a test hook: it keeps a decoder chain checkable bit for bit)."""

    def __init__(self, dim, dim_head=64, eps=1e-6, rot=48):
        super().__init__()
        self.heads, self.dim_head, self.rot = dim // dim_head, dim_head, rot
        self.to_qkv = nn.Linear(dim, 3 * dim)
        self.to_out = nn.Linear(dim, dim)
        self.norm_q = nn.RMSNorm(dim_head, eps=eps, elementwise_affine=False)
        self.norm_k = nn.RMSNorm(dim_head, eps=eps, elementwise_affine=False)
        self.spatial_parallel = False
        self.mix = "sdpa"
        _init_linear(self.to_qkv)
        _init_linear(self.to_out)

    def _rope(self, x, cos, sin):
        half = self.rot // 2
        xr = x[..., :self.rot]
        rotated = torch.cat([-xr[..., half:], xr[..., :half]], dim=-1)
        return torch.cat([xr * cos + rotated * sin, x[..., self.rot:]], dim=-1)

    def perform_attention(self, q, k, v, pack_info):
        if self.mix == "sum":
            return (q + k) + v
        y = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2).contiguous())
        return y.transpose(1, 2)

    def forward(self, x, rotary_pos_emb=None, pack_info=None):
        b, n, _ = x.shape
        qkv = self.to_qkv(x).view(b, n, self.heads, 3 * self.dim_head)
        q, k, v = qkv.split(self.dim_head, dim=-1)
        q = self.norm_q(q.float()).to(x.dtype)
        k = self.norm_k(k.float()).to(x.dtype)
        if rotary_pos_emb is not None:
            cos, sin = rotary_pos_emb
            q, k = self._rope(q, cos, sin), self._rope(k, cos, sin)
        y = self.perform_attention(q, k, v, pack_info or {})
        return self.to_out(y.reshape(b, n, -1))


class GatedFFN(nn.Module):
    def __init__(self, dim, hidden):
        super().__init__()
        self.use_gated = True
        self.act_fn = nn.SiLU()
        self.w1 = nn.Linear(dim, 2 * hidden)
        self.w2 = nn.Linear(hidden, dim)
        _init_linear(self.w1)
        _init_linear(self.w2)

    def forward(self, x):
        gate, up = self.w1(x).chunk(2, dim=-1)
        return self.w2(self.act_fn(gate) * up)


class H3Block(nn.Module):
    def __init__(self, dim, hidden):
        super().__init__()
        self.norm1 = nn.RMSNorm(dim, eps=1e-5)
        self.attn = H3Attention(dim)
        self.norm2 = nn.RMSNorm(dim, eps=1e-5)
        self.ff = GatedFFN(dim, hidden)
        self.scale1 = nn.Parameter(0.1 * torch.randn(dim))
        self.scale2 = nn.Parameter(0.1 * torch.randn(dim))
        self.use_scale = True
        nn.init.normal_(self.norm1.weight, 1.0, 0.1)
        nn.init.normal_(self.norm2.weight, 1.0, 0.1)

    def forward(self, h, rotary_pos_emb=None, pack_info=None):
        normed = self.norm1(h.float()).to(h.dtype)
        h = h + self.attn(normed, rotary_pos_emb, pack_info or {}) * self.scale1
        normed = self.norm2(h.float()).to(h.dtype)
        return h + self.ff(normed) * self.scale2


def rotary_table_3d(t, h, w, extra, rot=48, base=10000.0):
    """fp64 (cos, sin) [t*h*w + extra, rot] for patch tokens in (t, y, x) order, then ``extra`` tokens at 0.

    Rotated pair i (dims i and i + rot/2) belongs to axis i // (rot/6) with frequency index i % (rot/6)."""
    per_axis = rot // 6
    inv = 1.0 / base ** (torch.arange(per_axis, dtype=torch.float64) / per_axis)
    grid = torch.stack(torch.meshgrid(torch.arange(t), torch.arange(h), torch.arange(w), indexing="ij"), -1)
    pos = torch.cat([grid.reshape(-1, 3).double(), torch.zeros(extra, 3, dtype=torch.float64)])
    ang = torch.cat([pos[:, a:a + 1] * inv for a in range(3)], dim=-1)         # [N, rot/2]
    ang = torch.cat([ang, ang], dim=-1)
    return ang.cos(), ang.sin()


class H3Decoder(nn.Module):
    """Latent tile [B, 24, T, h, w] -> pixels [B, 3, 4T, 16h, 16w] through a ViT of ``depth`` blocks.

    ``forward`` also takes token rows directly: ``decoder(states [B, N, dim], (cos, sin), pack_info)`` runs
    the blocks, the unpad hook and the final LayerNorm (the part the INT8 wrappers replace)."""

    def __init__(self, dim=2048, hidden=8192, depth=36, latent=LATENT_CHANNELS, registers=5, patch=(4, 16, 16),
                 out_channels=3):
        super().__init__()
        self.transformer_blocks = nn.ModuleList([H3Block(dim, hidden) for _ in range(depth)])
        self.norm_out = nn.LayerNorm(dim, eps=1e-5)
        nn.init.normal_(self.norm_out.weight, 1.0, 0.1)
        nn.init.normal_(self.norm_out.bias, 0.0, 0.02)
        self.proj_in = nn.Linear(latent, dim)
        _init_linear(self.proj_in, std=latent ** -0.5)
        self.registers = nn.Parameter(torch.randn(registers, dim))
        self.proj_out = nn.Linear(dim, out_channels * patch[0] * patch[1] * patch[2])
        _init_linear(self.proj_out)
        self.patch, self.out_channels, self.spatial_parallel = tuple(patch), out_channels, False
        self.rot = self.transformer_blocks[0].attn.rot if depth else 48
        self._rope_cache = {}

    def _unpad_for_sp(self, states, pad_len):
        return states if pad_len == 0 else states[:, :-pad_len]

    def set_mix(self, mix):
        for block in self.transformer_blocks:
            block.attn.mix = mix

    def rotary(self, batch, t, h, w, device, dtype):
        key = (batch, t, h, w, device, dtype)
        if key not in self._rope_cache:
            cos, sin = rotary_table_3d(t, h, w, self.registers.shape[0], self.rot)
            n = cos.shape[0]
            self._rope_cache[key] = tuple(v.to(dtype).view(1, n, 1, -1).expand(batch, -1, -1, -1).contiguous()
                                          .to(device) for v in (cos, sin))
        return self._rope_cache[key]

    def run_tokens(self, states, rotary_pos_emb=None, pack_info=None):
        pack_info = {} if pack_info is None else pack_info
        for block in self.transformer_blocks:
            states = block(states, rotary_pos_emb, pack_info)
        return self.norm_out(self._unpad_for_sp(states, 0))

    def forward(self, x, rotary_pos_emb=None, pack_info=None):
        if x.ndim == 3:
            return self.run_tokens(x, rotary_pos_emb, pack_info)
        b, c, t, h, w = x.shape
        tokens = self.proj_in(x.permute(0, 2, 3, 4, 1).reshape(b, t * h * w, c))
        states = torch.cat([tokens, self.registers.to(tokens.dtype).expand(b, -1, -1)], dim=1).contiguous()
        states = self.run_tokens(states, self.rotary(b, t, h, w, x.device, x.dtype), {})
        pixels = self.proj_out(states[:, :t * h * w])
        pt, ph, pw = self.patch
        pixels = pixels.view(b, t, h, w, self.out_channels, pt, ph, pw).permute(0, 4, 1, 5, 2, 6, 3, 7)
        return pixels.reshape(b, self.out_channels, t * pt, h * ph, w * pw)


# -- core: planners, tiled decode ------------------------------------------------------------------

class H3Core(nn.Module):
    """The klvae core surface the runtime uses: encoder, quant_conv, decoder, planners, blend, decode_base."""

    def __init__(self, encoder, decoder, latent=LATENT_CHANNELS):
        super().__init__()
        self.encoder, self.decoder = encoder, decoder
        self.quant_conv = nn.Conv3d(2 * latent, 2 * latent, 1)
        self.clip_length, self.token_drop = 17, 3
        self.vae_ratio, self.vae_ratio_t = 16, 4
        self.tile_overlap_min = 64
        self.tile_size, self.decoder_tile_size, self.stack_tiling = 672, 256, False

    # temporal plan of one decode (bench_h3vae_trt.py:175-200)
    @property
    def chunk_tokens(self):
        return -(-self.clip_length // self.vae_ratio_t)

    @property
    def token_overlap(self):
        return (-self.token_drop) % self.chunk_tokens

    @property
    def frame_pre_padding(self):
        return (-self.clip_length) % self.vae_ratio_t

    def temporal_chunks(self, z_len):
        """(padding tokens, chunk count) for z_len latent frames."""
        total = z_len + self.token_drop
        pad = (-total) % self.chunk_tokens
        count = (total + pad) // self.chunk_tokens - int(self.token_drop > 0)
        if count < 1:
            pad, count = pad + self.chunk_tokens, count + 1
        return pad, count

    def pad_frames(self, z_len_padded, pad_tokens):
        """Pixel frames that the padding tokens add at the end (bench_h3vae_trt.py:202-213)."""
        if pad_tokens <= 0:
            return 0
        tail = self.clip_length % self.vae_ratio_t
        if tail == 0:
            return pad_tokens * self.vae_ratio_t
        before = z_len_padded - pad_tokens
        return sum(tail if (before + k) % self.chunk_tokens == 0 else self.vae_ratio_t for k in range(pad_tokens))

    def split_tiles(self, length, tile):
        """Tile starts / lengths / overlaps along one pixel axis (bench_h3vae_trt.py:243-259)."""
        if tile >= length:
            return [0], [length], []
        n = -(-length // tile)
        while tile * n - self.tile_overlap_min * (n - 1) < length:
            n += 1
        overlaps = [self.tile_overlap_min] * (n - 1)
        for i in range((tile * n - sum(overlaps) - length) // self.vae_ratio):
            overlaps[i % (n - 1)] += self.vae_ratio
        starts = [0]
        for o in overlaps:
            starts.append(starts[-1] + tile - o)
        return starts, [tile] * n, overlaps

    @staticmethod
    def blend(a, b, blend_extent, dim):
        """Linear cross-fade of a's tail into b's head over blend_extent positions along dim."""
        extent = min(a.shape[dim], b.shape[dim], blend_extent)
        if extent <= 0:
            return b
        shape = [1] * a.ndim
        shape[dim] = extent
        weight = (torch.arange(extent, device=b.device, dtype=b.dtype) / extent).view(shape)
        head = torch.lerp(a.narrow(dim, a.shape[dim] - extent, extent), b.narrow(dim, 0, extent), weight)
        if extent == b.shape[dim]:
            return head
        return torch.cat([head, b.narrow(dim, extent, b.shape[dim] - extent)], dim=dim)

    def _run_tile_tasks(self, tiles, indices, forward_fn, stack_tiling, cls_agg=None):
        """Decode the selected tiles one by one (the runtime may replace this to batch them)."""
        return [forward_fn(tiles[i]) for i in indices]

    def _decode_tile(self, tile):
        return self.decoder(tile)

    def decode_spatial(self, z):
        """One temporal chunk [B, 24, T, h, w] -> raw pixels [B, 3, 4T, 16h, 16w], tiles blended."""
        r = self.vae_ratio
        height, width = z.shape[-2] * r, z.shape[-1] * r
        ys, yl, yo = self.split_tiles(height, self.decoder_tile_size)
        xs, xl, xo = self.split_tiles(width, self.decoder_tile_size)
        tiles = [z[..., y // r:(y + hh) // r, x // r:(x + ww) // r] for y, hh in zip(ys, yl) for x, ww in zip(xs, xl)]
        outs = self._run_tile_tasks(tiles, list(range(len(tiles))), self._decode_tile, self.stack_tiling)
        canvas = None
        above = [None] * len(xs)
        oy = 0
        for i in range(len(ys)):
            left, ox = None, 0
            for j in range(len(xs)):
                tile = outs[i * len(xs) + j]
                raw = tile
                if i:
                    tile = self.blend(above[j], tile, yo[i - 1], dim=-2)
                if j:
                    tile = self.blend(left, tile, xo[j - 1], dim=-1)
                left = raw[..., :, -xo[j]:] if j < len(xs) - 1 else None
                above[j] = raw[..., -yo[i]:, :] if i < len(ys) - 1 else None
                if i < len(ys) - 1:
                    tile = tile[..., :-yo[i], :]
                if j < len(xs) - 1:
                    tile = tile[..., :, :-xo[j]]
                if canvas is None:
                    canvas = tile.new_zeros((*tile.shape[:-2], height, width))
                canvas[..., oy:oy + tile.shape[-2], ox:ox + tile.shape[-1]] = tile
                ox += tile.shape[-1]
            oy += tile.shape[-2]
        return canvas

    def decode_base(self, z, frame_num=None):
        """Latents [B, 24, t, h, w] (t >= 2) -> raw pixels [B, 3, F, 16h, 16w] (bench_h3vae_trt.py:396-431)."""
        pad, count = self.temporal_chunks(z.shape[2])
        if pad:
            z = torch.cat([z, z[:, :, -1:].expand(-1, -1, pad, -1, -1)], dim=2)
        span = self.chunk_tokens * self.vae_ratio_t
        parts, carry = [], None
        for i in range(count):
            start = i * self.chunk_tokens
            dec = self.decode_spatial(z[:, :, start:start + self.chunk_tokens + self.token_overlap])
            head = dec[:, :, self.frame_pre_padding:span]
            if carry is not None:
                head = self.blend(carry, head, max(self.token_overlap * self.vae_ratio_t - self.frame_pre_padding, 0),
                                  dim=-3)
            parts.append(head)
            carry = dec[:, :, span + self.frame_pre_padding:] if self.token_drop > 0 else None
        if carry is not None and carry.shape[2]:
            parts.append(carry)
        out = torch.cat(parts, dim=2)
        trim = self.pad_frames(z.shape[2], pad)
        if trim:
            out = out[:, :, :-trim]
        return out if frame_num is None else out[:, :, :frame_num]

    def decode(self, z):
        """Any t: short inputs repeat their last latent frame up to one chunk."""
        t = z.shape[2]
        need = self.chunk_tokens + self.token_overlap
        if t < need:
            z = torch.cat([z, z[:, :, -1:].expand(-1, -1, need - t, -1, -1)], dim=2)
        frames = 1 if t <= 1 else max(1, (t - 2) // 5 * 17 + 5)
        return self.decode_base(z, frame_num=frames)


def build_core(*, dim=2048, hidden=8192, depth=36, encoder_stages=H3_ENCODER_STAGES, blocks_per_stage=2,
               seed=20261002):
    """-> (core, config): a random-init reconstructed H3 core and the config dict the runtime reads
    (latent statistics zero mean / unit std)."""
    state = torch.random.get_rng_state()
    torch.manual_seed(seed)
    try:
        core = H3Core(H3Encoder(encoder_stages, blocks_per_stage), H3Decoder(dim, hidden, depth)).eval()
    finally:
        torch.random.set_rng_state(state)
    config = {"latents_mean": [0.0] * LATENT_CHANNELS, "latents_std": [1.0] * LATENT_CHANNELS,
              "reconstruction": True}
    return core, config


def frames_for_tokens(t):
    return 1 if t <= 1 else max(1, (t - 2) // 5 * 17 + 5)


def tokens_for_frames(frames):
    return 1 if frames <= 1 else max(1, (frames - 5) // 17 * 5 + 2)


__all__ = ["H3Core", "H3Encoder", "H3Decoder", "H3Block", "H3Attention", "GatedFFN", "ResnetBlock3D", "Downsample",
           "CausalConv3d", "TemporalIsolatedSpatialParallelGroupNorm", "H3_ENCODER_STAGES", "build_core",
           "rotary_table_3d", "frames_for_tokens", "tokens_for_frames"]
