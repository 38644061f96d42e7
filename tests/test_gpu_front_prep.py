"""Front-end preparation kernels on MI355X against the reference's torch
formulations (as the oracle restates them): waveform masking and the stage
length chain bit for bit, the pooled grid (lengths, masks, neighbours and the
fp32 interpolation weight) bit for bit against oracle/trifusion.py:grids, and
the log power from the same complex spectrum within 2e-6 (fp32 log on two
libraries)."""

import pytest
import torch

from oracle import trifusion as O
from oracle.elementwise import time_mask
from trifusion_amd.kernels.block import front_lengths, grids, log_power, mask_audio

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_mask_audio_and_lengths():
    g = torch.Generator().manual_seed(0)
    audio = torch.randn(3, 2, 4001, generator=g)
    lengths = torch.tensor([4001, 1999, 0])
    channels = torch.tensor([2, 1, 2])
    y = mask_audio(audio.to(DEV), lengths.to(DEV), channels.to(DEV)).cpu()
    keep = time_mask(lengths, 4001)[:, None, :] & (torch.arange(2)[None, :] < channels[:, None])[..., None]
    assert torch.equal(y, audio.masked_fill(~keep, 0).reshape(6, 4001))
    n = torch.tensor([64000, 63999, 1, 0, 160, 161, 32000])
    counts = front_lengths(n.to(DEV), 160, [1, 2, 2]).cpu()
    want = [n // 160 + 1]
    for s in (1, 2, 2):
        want.append((want[-1] + s - 1) // s)
    assert torch.equal(counts, torch.stack(want))


@pytest.mark.parametrize("channels", [[1, 1, 1], [2, 1, 2]])
def test_log_power(channels):
    g = torch.Generator().manual_seed(len(channels) + sum(channels))
    c = max(channels)
    channels = torch.tensor(channels)
    n = torch.tensor([64000, 33333, 160])
    wave = torch.randn(3 * c, 64000, generator=g) * 0.1
    spec = torch.stft(wave.to(DEV), n_fft=512, hop_length=160, win_length=400,
                      window=torch.hann_window(400, periodic=True, device=DEV), center=True, pad_mode="constant",
                      return_complex=True)
    y = log_power(spec, channels.to(DEV), n.to(DEV), 160).cpu()
    sc = spec.cpu()
    power = (sc.real.square() + sc.imag.square()).reshape(3, c, 257, -1).sum(1) / channels[:, None, None]
    ref = torch.log(1e-6 + power).transpose(1, 2)
    ref = ref.masked_fill(~time_mask(n // 160 + 1, ref.shape[1])[..., None], 0)
    assert y.shape == ref.shape
    assert (y - ref).abs().max().item() <= 2e-6 * max(ref.abs().max().item(), 1.0)
    assert not y[2, 2:].any()


@pytest.mark.parametrize("t,lengths", [(101, [101, 57, 4, 1]), (26, [26, 25, 9]), (1, [1])])
def test_grids(t, lengths):
    lengths = torch.tensor(lengths)
    mask, low, low_mask, left, right, alpha = (x.cpu() for x in grids(lengths.to(DEV), t))
    r_low, r_left, r_right, r_alpha = O.grids(lengths, t)
    assert torch.equal(mask, time_mask(lengths, t))
    assert torch.equal(low, r_low) and torch.equal(low_mask, time_mask(r_low, (t + 3) // 4))
    assert torch.equal(left, r_left) and torch.equal(right, r_right)
    assert torch.equal(alpha, r_alpha)
