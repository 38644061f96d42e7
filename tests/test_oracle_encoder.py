"""Pins the oracle's encoder front and head (no GPU): the framing against the
library Conv1d, the frame counts against integer floor division in Python, and
the head against an explicit bf16 computation."""

import math

import torch
import torch.nn.functional as F

from oracle import encoder as O


def test_framing_matches_conv1d_on_the_channel_mean():
    g = torch.Generator().manual_seed(0)
    audio = torch.randn(3, 2, 2000, generator=g)
    channels = torch.tensor([2, 1, 2])
    k, s, p = 400, 160, 120
    framed = O.frame_audio(audio, channels, k, s, p).float()
    w = torch.randn(8, 1, k, generator=g).to(torch.bfloat16).float()
    mono = torch.stack([audio[0].mean(0), audio[1, 0], audio[2].mean(0)])
    conv = F.conv1d(mono.to(torch.bfloat16).float()[:, None], w, stride=s, padding=p).transpose(1, 2)
    assert framed.shape == (3, (2000 + 2 * p - k) // s + 1, k)
    assert torch.allclose(framed @ w[:, 0].t(), conv, rtol=1e-5, atol=1e-4)
    wide = O.frame_audio(audio, channels, k, s, p, width=448)
    assert torch.equal(wide[..., :k], framed.to(torch.bfloat16)) and not wide[..., k:].any()


def test_valid_frames_floor_division():
    lengths = torch.tensor([64000, 159, 160, 0, -5, 10**6, 32001])
    got = O.valid_frames(lengths, 160, 400).tolist()
    want = [min(max(math.floor(n / 160), 1), 400) for n in lengths.tolist()]
    assert got == want


def test_small_linear_is_the_bf16_layer():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(4, 512, generator=g)
    w = torch.randn(5, 512, generator=g).to(torch.bfloat16)
    b = torch.randn(5, generator=g).to(torch.bfloat16)
    y = O.small_linear(x, w, b)
    ref = (x.to(torch.bfloat16).double() @ w.double().t() + b.double()).to(torch.bfloat16).float()
    assert y.dtype == torch.float32 and (y - ref).abs().max() <= 2 ** -7 * ref.abs().max()
