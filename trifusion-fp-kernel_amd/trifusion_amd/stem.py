"""Front and head of the benchmark encoder on the gfx950 kernels.

``frame_audio`` mixes each clip's channels and frames the zero-padded signal
for the strided Conv1d stem, which is then one GEMM (``tf_frame_audio``);
``frames_mask`` turns sample lengths into valid frame counts and the row mask
(``tf_frames_mask``; the hop-count lengths of the reference front end,
``src/trifusion_l4/front.py:62-67,90``, and ``time_mask``,
``src/trifusion_l4/masking.py:6-7``); ``small_linear`` is the bf16 head layer of
an autocast forward (``tf_small_linear``). Each replaces a run of tiny torch
launches of the graph-replayed forward with one kernel.
"""

import torch

from . import _lib
from .ops import ops


def frame_audio(audio, channels, kernel, stride, pad, width=None):
    """``[B, C, N]`` fp32 audio -> bf16 ``[B, T, width]`` frames of the channel
    mean (``sum_{c < channels[b]} audio[b, c] / channels[b]``), zero-padded by
    ``pad`` samples each side; columns ``kernel <= k < width`` are 0
    (``trifusion_amd::frame_audio``)."""
    return ops.frame_audio(audio, channels, int(kernel), int(stride), int(pad), int(width or kernel))


def launch_frame_audio(audio, channels, kernel, stride, pad, width):
    lib = _lib.load()
    _lib.require_cuda(audio, channels, what="frame_audio")
    if audio.dim() != 3 or audio.dtype != torch.float32:
        raise TypeError("frame_audio: audio must be float32 [B, C, N]")
    b, c, n = audio.shape
    if tuple(channels.shape) != (b,) or channels.dtype != torch.int64:
        raise ValueError("frame_audio: channels must be an int64 tensor of shape [B]")
    if width < kernel or width % 8:
        raise ValueError("frame_audio: width must be >= kernel and a multiple of 8")
    frames = (n + 2 * pad - kernel) // stride + 1
    if frames < 1:
        raise ValueError("frame_audio: clip shorter than one frame")
    audio = audio.contiguous()
    channels = channels.contiguous()
    out = torch.empty((b, frames, width), device=audio.device, dtype=torch.bfloat16)
    status = lib.tf_frame_audio(
        audio.data_ptr(), channels.data_ptr(), out.data_ptr(), b, c, n, frames, kernel, width, stride, pad,
        _lib.stream_of(audio),
    )
    _lib.check(status, "frame_audio")
    return out


def frames_mask(lengths, stride, time):
    """``frames = clamp(lengths // stride, 1, time)`` (int64 ``[B]``) and the row
    mask ``t < frames`` (bool ``[B, time]``) (``trifusion_amd::frames_mask``)."""
    return ops.frames_mask(lengths, int(stride), int(time))


def launch_frames_mask(lengths, stride, time):
    lib = _lib.load()
    _lib.require_cuda(lengths, what="frames_mask")
    lengths = lengths.to(torch.int64).contiguous()
    b = lengths.shape[0]
    frames = torch.empty((b,), device=lengths.device, dtype=torch.int64)
    mask = torch.empty((b, time), device=lengths.device, dtype=torch.bool)
    status = lib.tf_frames_mask(lengths.data_ptr(), stride, frames.data_ptr(), mask.data_ptr(), b, time,
                                _lib.stream_of(lengths))
    _lib.check(status, "frames_mask")
    return frames, mask


def small_linear(x, weight, bias=None):
    """``bf16(bf16(x) @ bf16(weight).T + bf16(bias))`` as fp32, the autocast
    linear layer on an fp32 ``[B, D]`` input (``trifusion_amd::small_linear``)."""
    return ops.small_linear(x, weight, bias)


def launch_small_linear(x, weight, bias=None):
    lib = _lib.load()
    _lib.require_cuda(x, weight, bias, what="small_linear")
    if x.dim() != 2 or x.dtype != torch.float32:
        raise TypeError("small_linear: x must be float32 [B, D]")
    o, d = weight.shape
    if x.shape[1] != d or (bias is not None and (tuple(bias.shape) != (o,) or bias.dtype != weight.dtype)):
        raise ValueError("small_linear: shapes or bias dtype do not match")
    x = x.contiguous()
    weight = weight.contiguous()
    bias = bias.contiguous() if bias is not None else None
    y = torch.empty((x.shape[0], o), device=x.device, dtype=torch.float32)
    status = lib.tf_small_linear(
        x.data_ptr(), weight.data_ptr(), bias.data_ptr() if bias is not None else None,
        _lib.dtype_code(weight, "small_linear"), y.data_ptr(), x.shape[0], o, d, _lib.stream_of(x),
    )
    _lib.check(status, "small_linear")
    return y
