"""Encoder front, first norm, paired B/C norm and head kernels (MI355X) against
the oracle: framing, frame counts and the masked residual bit-exact; norms and
the head within float tolerance."""

import pytest
import torch

from oracle import elementwise as E
from oracle import encoder as O
from trifusion_amd.kernels.native import mask_rms, rms_pair
from trifusion_amd.stem import frame_audio, frames_mask, small_linear

pytestmark = pytest.mark.gpu
DEV = "cuda"


FRAMING = [
    # chans, width, samples, kernel, stride, pad
    (1, 400, 4000, 400, 160, 120),   # staged blocks, float4 span loads
    (2, 400, 4000, 400, 160, 120),
    (2, 448, 4000, 400, 160, 120),   # zero columns past the kernel
    (2, 448, 3999, 400, 160, 120),   # samples % 4 != 0: scalar span loads
    (2, 408, 4000, 401, 160, 122),   # kernel % 8 != 0 (a chunk straddles it), pad % 4 != 0
    (1, 448, 64000, 400, 160, 120),  # the encoder's 4 s clip: 400 frames, 50 blocks of 8
    (2, 400, 3000, 400, 100, 120),   # stride % 8 != 0: one workgroup per frame
    (1, 64, 300, 64, 16, 0),         # fewer frames than a block's last one needs
]


@pytest.mark.parametrize("chans,width,n,kernel,stride,pad", FRAMING)
def test_frame_audio_is_exact(chans, width, n, kernel, stride, pad):
    """Bitwise equal to the oracle for the staged block form (vector and scalar
    span loads, a kernel that is not a multiple of 8, zero columns) and the
    per-frame form (stride not a multiple of 8)."""
    g = torch.Generator().manual_seed(chans * 7 + n)
    audio = torch.randn(3, chans, n, generator=g)
    channels = torch.tensor([chans, 1, chans])
    print(f"case frame_audio chans={chans} width={width} n={n} kernel={kernel} stride={stride} pad={pad}", flush=True)
    got = frame_audio(audio.to(DEV), channels.to(DEV), kernel, stride, pad, width).cpu()
    assert torch.equal(got, O.frame_audio(audio, channels, kernel, stride, pad, width))


def test_frames_mask_is_exact():
    lengths = torch.tensor([64000, 159, 160, 0, -5, 10**6, 32001])
    frames, mask = frames_mask(lengths.to(DEV), 160, 400)
    want = O.valid_frames(lengths, 160, 400)
    assert torch.equal(frames.cpu(), want)
    assert torch.equal(mask.cpu(), E.time_mask(want, 400))


@pytest.mark.parametrize("d", [512, 100])
def test_mask_rms_matches_masked_then_norm(d):
    g = torch.Generator().manual_seed(d)
    x = torch.randn(37, d, generator=g).to(torch.bfloat16)
    w = torch.rand(d, generator=g) + 0.5
    mask = torch.rand(37, generator=g) > 0.3
    s, y = mask_rms(x.to(DEV), mask.to(DEV), w.to(DEV))
    ref_s = E.mask_rows(x.float(), mask)
    assert torch.equal(s.cpu(), ref_s)
    assert (y.cpu().float() - E.rms_norm(ref_s, w).to(torch.bfloat16).float()).abs().max() <= 0.02


@pytest.mark.parametrize("d,rows", [(64, 50), (64, 3), (128, 7), (8, 33), (48, 11)])
def test_rms_pair_matches_two_norms_on_strided_rows(d, rows):
    """Vector path (power-of-two d, several rows per wave, a partial last
    wave) and the scalar path (d = 48)."""
    g = torch.Generator().manual_seed(3 + d)
    p = torch.randn(2, rows, 2304, generator=g).to(torch.bfloat16)
    w0 = torch.rand(d, generator=g) + 0.5
    w1 = torch.rand(d, generator=g) + 0.5
    kq = p[..., 2048 : 2048 + 2 * d]
    y = rms_pair(p.to(DEV)[..., 2048 : 2048 + 2 * d], w0.to(DEV), w1.to(DEV)).cpu()
    assert y.shape == (2, rows, 2, d)
    for grp, w in ((0, w0), (1, w1)):
        ref = E.rms_norm(kq[..., d * grp : d * grp + d], w)
        assert (y[:, :, grp].float() - ref.float()).abs().max() <= 0.02
        assert (y[:, :, grp] != ref).float().mean() < 0.02  # bf16 outputs agree but for rare ties


def test_small_linear_matches_bf16_layer():
    g = torch.Generator().manual_seed(4)
    x = torch.randn(16, 512, generator=g)
    w = (torch.randn(5, 512, generator=g) * 0.05).to(torch.bfloat16)
    b = torch.randn(5, generator=g).to(torch.bfloat16)
    y = small_linear(x.to(DEV), w.to(DEV), b.to(DEV)).cpu()
    ref = O.small_linear(x, w, b)
    assert (y - ref).abs().max() <= 2 ** -7 * ref.abs().max()
