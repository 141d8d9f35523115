"""Staged encode of a batch-one video: the prefix clip by clip, the suffix on groups of clips.

Counterpart of opt/encoder_staged_batch.py in fishelegs/ComfyUI-H3VAE-PyOpt
(``EncoderPrefix`` :6-22, ``EncoderSuffix`` :25-38, ``encode_staged`` :41-57).
The encoder is causal per 17-frame clip, so clips are independent.  The prefix
(conv_in and the stages before ``cut``, where the INT8 convolutions are) runs
on one clip at a time; the prefix outputs of up to ``batch_size`` clips then go
through one suffix call as a batch.  A video whose length is not a whole number
of clips has its last clip completed by repeating its last frame, and the last
``token_drop`` latent frames are removed.

Memory: no padded copy of the video is made (only the last, incomplete clip is
gathered with its repeated frame), and every suffix output is written straight
into its place in the preallocated moments tensor.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

_VALIDATED = ((1, 1), (1, 2), (2, 1), (2, 2), (2, 4))
_CL3D = torch.channels_last_3d


def _reads_partials(stage):
    """Whether the first block of ``stage`` normalises its input through the INT8 producer, which can take the
    input's GroupNorm statistics from the conv that wrote it instead of its own statistics pass."""
    blocks = getattr(stage, "block", None)
    if not blocks or getattr(blocks[0], "forward_partials", None) is None:
        return False
    first = getattr(blocks[0], "int8_first", None)
    return first is not None and bool(getattr(first, "fuse_norm", False))


def _run_stages(stages, h, partials=None):
    """Every residual block of each stage in order, then the stage's downsample if it has one.  Blocks with
    ``forward_partials`` (the INT8 prefix blocks) hand the GroupNorm statistics of their output, written by
    their last conv, to the next block's first norm.  ``partials``: the statistics of ``h`` (written by
    conv_in) for the first block; a downsample conv forms those of its output when the next stage's first
    block reads them."""
    for i, stage in enumerate(stages):
        for block in stage.block:
            step = getattr(block, "forward_partials", None)
            if step is not None:
                h, partials = step(h, partials)
            else:
                h, partials = block(h), None
        partials = None
        downsample = getattr(stage, "downsample", None)
        if downsample is not None:
            request = getattr(getattr(downsample, "conv", None), "partials_requested", None)
            if request is not None and i + 1 < len(stages) and _reads_partials(stages[i + 1]):
                with request() as slot:
                    h = downsample(h)
                partials = slot.partials
            else:
                h = downsample(h)
    return h


class EncoderPrefix(torch.nn.Module):
    """conv_in and encoder stages [0, cut) on one clip."""

    def __init__(self, encoder, cut):
        super().__init__()
        if cut not in (1, 2):
            raise ValueError("Only validated split locations 1 and 2 supported")
        if encoder.gradient_checkpointing or encoder.use_fused_norm:
            raise ValueError("Expected inference encoder without fused-norm flag")
        self.conv_in = encoder.conv_in
        self.stages = torch.nn.ModuleList(encoder.down[i] for i in range(cut))

    def forward(self, x):
        x = x.contiguous(memory_format=_CL3D)
        step = getattr(self.conv_in, "forward_partials", None)
        if step is not None and len(self.stages) and _reads_partials(self.stages[0]):
            h, partials = step(x)
        else:
            h, partials = self.conv_in(x), None
        return _run_stages(self.stages, h, partials)


class EncoderSuffix(torch.nn.Module):
    """Encoder stages [cut, end), then norm_out / SiLU / conv_out and quant_conv: -> moments."""

    def __init__(self, encoder, quant_conv, cut):
        super().__init__()
        self.stages = torch.nn.ModuleList(encoder.down[i] for i in range(cut, len(encoder.down)))
        self.norm_out, self.conv_out, self.quant_conv = encoder.norm_out, encoder.conv_out, quant_conv

    def head(self, h):
        return self.quant_conv(self.conv_out(F.silu(self.norm_out(h))))

    def forward(self, h):
        return self.head(_run_stages(self.stages, h))


def _clip(video, index, clip_length):
    """Frames [index * L, (index + 1) * L) of the video; frames past its end repeat its last frame."""
    first, frames = index * clip_length, video.shape[2]
    if first + clip_length <= frames:
        return video[:, :, first:first + clip_length]
    taken = torch.arange(first, first + clip_length, device=video.device).clamp_(max=frames - 1)
    return video.index_select(2, taken).contiguous(memory_format=_CL3D)


def encode_staged(normalized_video, prefix, suffix, *, clip_length, token_drop, batch_size, cut):
    """Moments [1, 2 * latent, t, h, w] of a batch-one normalised video (t = 5 per clip - token_drop)."""
    if normalized_video.ndim != 5 or normalized_video.shape[0] != 1:
        raise ValueError("Expected batch-one video")
    if (cut, batch_size) not in _VALIDATED:
        raise ValueError("Unsupported combination; avoid large int32-indexed tensors")
    video = normalized_video.contiguous(memory_format=_CL3D)
    clips = -(-video.shape[2] // clip_length)
    moments, per_clip = None, 0
    for group in range(0, clips, batch_size):
        members = range(group, min(group + batch_size, clips))
        features = [prefix(_clip(video, i, clip_length)) for i in members]
        batch = features[0] if len(features) == 1 else torch.cat(features, dim=0)
        out = suffix(batch.contiguous(memory_format=_CL3D))
        del features, batch
        if moments is None:
            per_clip = out.shape[2]
            moments = torch.empty((1, out.shape[1], clips * per_clip, *out.shape[3:]), dtype=out.dtype,
                                  device=out.device, memory_format=_CL3D)
        for k, i in enumerate(members):
            moments[0, :, i * per_clip:(i + 1) * per_clip].copy_(out[k])
        del out
    return moments[:, :, :moments.shape[2] - token_drop] if token_drop else moments
