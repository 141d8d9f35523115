"""Reconstructed H3 video-VAE modules for the caller tests (test infrastructure).

The MiniMax H3 model code (``video_vae`` / klvae) is not part of the reference
repository and is not available here.  These modules reproduce only the
attribute surface and forward semantics that the reference's wrappers read
(opt/encoder_fused_temporal_norm.py:101-118, opt/encoder_fused_norm_bias.py:121-140,
opt/encoder_fused_residual_pack.py:63-85, opt/int8_norm_quant.py:87-124,
opt/int8_norm1_quant.py:185-343, opt/decoder_fused_qk_rope.py:56-89), with
random initialisation:

* encoder: causal 3x3x3 convs (2 zero leading frames, reflect spatial pad),
  per-frame GroupNorm(32), residual blocks, stage-0/1 downsamples;
* decoder: RMSNorm / QKV / QK-RMSNorm + partial RoPE / attention / out /
  RMSNorm / gated SiLU FFN blocks with ``scale1``/``scale2`` residual gates and
  a final LayerNorm.

``H3Attention.mix = "sum"`` replaces the softmax attention by the elementwise
fp16 ``(q + k) + v``: attention is outside the INT8 path, and the stand-in
keeps every value of a decoder chain checkable bit for bit against the oracle.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn


# -- encoder ------------------------------------------------------------------------------------

class CausalConv3d(nn.Module):
    """Conv3d with left-only zero temporal padding and reflect spatial padding."""

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
            left = 2 * pt if x.shape[2] > 1 else self.kernel_size[0] - 1
            x = F.pad(x, (0, 0, 0, 0, left, 0))
        return F.conv3d(x, self.weight, self.bias, stride=self.stride)


class TemporalIsolatedSpatialParallelGroupNorm(nn.GroupNorm):
    """GroupNorm whose statistics are taken per frame."""

    def forward(self, x):
        b, c, d, h, w = x.shape
        y = x.transpose(1, 2).reshape(b * d, c, h, w)
        y = F.group_norm(y.float(), self.num_groups, self.weight.float(), self.bias.float(), self.eps)
        return y.to(x.dtype).reshape(b, d, c, h, w).transpose(1, 2)


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
        for norm in (self.norm1, self.norm2):
            nn.init.normal_(norm.weight, 1.0, 0.1)
            nn.init.normal_(norm.bias, 0.0, 0.1)

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
    """conv_in 3->128; stage 0: 2 x C128 + spatial /2; stage 1: 128->256, 256->256 + /2 x3; suffix stage."""

    def __init__(self, latent=24, suffix_channels=256):
        super().__init__()
        self.conv_in = CausalConv3d(3, 128)
        stage0, stage1, stage2 = nn.Module(), nn.Module(), nn.Module()
        stage0.block = nn.ModuleList([ResnetBlock3D(128, 128), ResnetBlock3D(128, 128)])
        stage0.downsample = Downsample(128, (1, 2, 2), (1, 1, 1))
        stage1.block = nn.ModuleList([ResnetBlock3D(128, 256), ResnetBlock3D(256, 256)])
        stage1.downsample = Downsample(256, (2, 2, 2), (1, 0, 0), right_bottom=True)
        stage2.block = nn.ModuleList([ResnetBlock3D(256, suffix_channels)])
        self.down = nn.ModuleList([stage0, stage1, stage2])
        self.norm_out = TemporalIsolatedSpatialParallelGroupNorm(32, suffix_channels, eps=1e-6)
        self.conv_out = CausalConv3d(suffix_channels, 2 * latent)
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

class H3Attention(nn.Module):
    def __init__(self, dim, dim_head=64, eps=1e-6, rot=48):
        super().__init__()
        self.heads, self.dim_head, self.rot = dim // dim_head, dim_head, rot
        self.to_qkv = nn.Linear(dim, 3 * dim)
        self.to_out = nn.Linear(dim, dim)
        self.norm_q = nn.RMSNorm(dim_head, eps=eps, elementwise_affine=False)
        self.norm_k = nn.RMSNorm(dim_head, eps=eps, elementwise_affine=False)
        self.spatial_parallel = False
        self.mix = "sdpa"
        for lin in (self.to_qkv, self.to_out):
            nn.init.normal_(lin.weight, 0.0, 0.02)
            nn.init.normal_(lin.bias, 0.0, 0.02)

    def _rope(self, x, cos, sin):
        half = self.rot // 2
        xr = x[..., :self.rot]
        rotated = torch.cat([-xr[..., half:], xr[..., :half]], dim=-1)
        out = xr * cos + rotated * sin
        return torch.cat([out, x[..., self.rot:]], dim=-1)

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
        for lin in (self.w1, self.w2):
            nn.init.normal_(lin.weight, 0.0, 0.02)
            nn.init.normal_(lin.bias, 0.0, 0.02)

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
        for norm in (self.norm1, self.norm2):
            nn.init.normal_(norm.weight, 1.0, 0.1)

    def forward(self, h, rotary_pos_emb=None, pack_info=None):
        normed = self.norm1(h.float()).to(h.dtype)
        h = h + self.attn(normed, rotary_pos_emb, pack_info or {}) * self.scale1
        normed = self.norm2(h.float()).to(h.dtype)
        return h + self.ff(normed) * self.scale2


class H3Decoder(nn.Module):
    def __init__(self, dim=2048, hidden=8192, depth=36):
        super().__init__()
        self.transformer_blocks = nn.ModuleList([H3Block(dim, hidden) for _ in range(depth)])
        self.norm_out = nn.LayerNorm(dim, eps=1e-5)
        nn.init.normal_(self.norm_out.weight, 1.0, 0.1)
        nn.init.normal_(self.norm_out.bias, 0.0, 0.02)
        self.spatial_parallel = False

    def _unpad_for_sp(self, states, pad_len):
        if pad_len == 0:
            return states
        return states[:, :-pad_len]

    def forward(self, x, rotary_pos_emb=None, pack_info=None):
        states = x
        for block in self.transformer_blocks:
            states = block(states, rotary_pos_emb, pack_info)
        return self.norm_out(self._unpad_for_sp(states, 0))

    def set_mix(self, mix):
        for block in self.transformer_blocks:
            block.attn.mix = mix


def rope_tables(batch, tokens, rot=48, base=10000.0, dtype=torch.float16):
    """cos/sin [B, N, 1, rot] for a 1-D token grid (the layout the fused op reads)."""
    inv = 1.0 / base ** (torch.arange(0, rot // 2, dtype=torch.float64) * 2 / rot)
    pos = torch.arange(tokens, dtype=torch.float64)
    ang = torch.outer(pos, inv)
    ang = torch.cat([ang, ang], dim=-1)
    cos = ang.cos().to(dtype).view(1, tokens, 1, rot).expand(batch, -1, -1, -1).contiguous()
    sin = ang.sin().to(dtype).view(1, tokens, 1, rot).expand(batch, -1, -1, -1).contiguous()
    return cos, sin
