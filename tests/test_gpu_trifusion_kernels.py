"""TriFusion block and front-end kernels on MI355X against the oracle's unfused
reference formulations. Tolerances: fp32 outputs within 1e-5 relative to the
largest magnitude (1e-4 for the sums of the convolution); bf16 outputs within
one bf16 rounding (rtol 1/128) of the oracle's bf16 result."""

from types import SimpleNamespace

import pytest
import torch

from oracle import trifusion as O
from oracle.elementwise import rms_norm
from trifusion_amd.kernels import gated_concat
from trifusion_amd.kernels.buffers import Pool4, RotaryQKV, depthwise_masked, front_norm
from trifusion_amd.kernels import RMSNorm
from trifusion_amd.kernels.block import interpolate_rmsnorm
from trifusion_amd.kernels.native import bands, evidence_norm, interpolate

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16


def close(y, ref, dtype):
    y, ref = y.float().cpu(), ref.float().cpu()
    scale = ref.abs().max().clamp_min(1e-30)
    if dtype == BF:
        torch.testing.assert_close(y, ref, rtol=2 ** -7, atol=2 ** -7 * scale.item())
    else:
        assert ((y - ref).abs().max() / scale).item() <= 1e-5


def gen(seed):
    return torch.Generator().manual_seed(seed)


@pytest.mark.parametrize("dtype", [torch.float32, BF])
def test_depthwise_masked(dtype):
    g = gen(0)
    x = torch.randn(3, 101, 1024, generator=g).to(dtype)
    layer = torch.nn.Conv1d(1024, 1024, 7, padding=3, groups=1024)
    weight, bias = layer.weight.detach().to(dtype).clone(), layer.bias.detach().to(dtype).clone()
    lengths = torch.tensor([101, 40, 1])
    y = depthwise_masked(x.to(DEV), layer.to(DEV).to(dtype), lengths.to(DEV))
    ref = O.depthwise_masked(x, weight, bias, lengths)
    y, ref = y.float().cpu(), ref.float()
    scale = ref.abs().max()
    tol = 2 ** -7 if dtype == BF else 1e-4
    assert ((y - ref).abs().max() / scale).item() <= tol
    assert not y[1, 40:].any() and not y[2, 1:].any()


@pytest.mark.parametrize("dtype", [torch.float32, BF])
def test_pool4_and_interpolate(dtype):
    g = gen(1)
    lengths = torch.tensor([101, 57, 4])
    x = torch.randn(3, 101, 512, generator=g).to(dtype)
    low = Pool4.apply(x.to(DEV), lengths.to(DEV))
    ref_low = O.pool4(x, lengths)
    close(low, ref_low, dtype)
    low_lengths, left, right, alpha = O.grids(lengths, 101)
    grids = SimpleNamespace(left=left.to(DEV), right=right.to(DEV), alpha=alpha.to(DEV), lengths=lengths.to(DEV))
    y = interpolate(ref_low.to(DEV), grids)
    close(y, O.interpolate(ref_low, left, right, alpha, lengths), dtype)


@pytest.mark.parametrize("d", [36, 1024])
def test_interpolate_widths(d):
    """The 8-wide vector form (d % 8 == 0) and the per-element form (d = 36)."""
    g = gen(7)
    lengths = torch.tensor([101, 57, 4])
    low_lengths, left, right, alpha = O.grids(lengths, 101)
    low = torch.randn(3, left.max().item() + 1, d, generator=g).to(BF)
    grids = SimpleNamespace(left=left.to(DEV), right=right.to(DEV), alpha=alpha.to(DEV), lengths=lengths.to(DEV))
    y = interpolate(low.to(DEV), grids)
    ref = O.interpolate(low, left, right, alpha, lengths)
    close(y, ref, BF)
    assert not y[1, 57:].float().any() and not y[2, 4:].float().any()


@pytest.mark.parametrize("dtype", [torch.float32, BF])
@pytest.mark.parametrize("d", [1024, 520])
def test_interpolate_rmsnorm(d, dtype):
    """One pass equals interpolate then the RMSNorm launch bit for bit (same
    rounding of the interpolated row, same summation order), and the oracle's
    composition within one rounding."""
    g = gen(8)
    lengths = torch.tensor([101, 57, 4])
    low_lengths, left, right, alpha = O.grids(lengths, 101)
    low = torch.randn(3, 26, d, generator=g).to(dtype)
    norm = RMSNorm(d)
    with torch.no_grad():
        norm.weight.copy_(torch.rand(d, generator=g) + 0.5)
    grids = SimpleNamespace(left=left.to(DEV), right=right.to(DEV), alpha=alpha.to(DEV), lengths=lengths.to(DEV))
    dn = norm.to(DEV)
    y = interpolate_rmsnorm(low.to(DEV), grids, dn)
    two = dn(interpolate(low.to(DEV), grids))
    torch.cuda.synchronize()
    assert torch.equal(y.cpu(), two.cpu())
    mid = O.interpolate(low, left, right, alpha, lengths)
    ref = rms_norm(mid, norm.weight.detach().cpu(), norm.eps)
    close(y, ref, dtype)
    assert not y[1, 57:].float().any() and not y[2, 4:].float().any()


@pytest.mark.parametrize("t,lengths", [(1, [1, 1]), (5, [5, 1, 3]), (7, [2, 7])])
def test_interpolate_rmsnorm_short(t, lengths):
    """Grids of one or two pooled rows: one pass equals interpolate then the
    RMSNorm launch bit for bit, rows past each length zero."""
    g = gen(40 + t)
    d = 264
    lens = torch.tensor(lengths)
    low_lengths, left, right, alpha = O.grids(lens, t)
    low = torch.randn(len(lengths), (t + 3) // 4, d, generator=g).to(BF)
    norm = RMSNorm(d)
    with torch.no_grad():
        norm.weight.copy_(torch.rand(d, generator=g) + 0.5)
    grids = SimpleNamespace(left=left.to(DEV), right=right.to(DEV), alpha=alpha.to(DEV), lengths=lens.to(DEV))
    dn = norm.to(DEV)
    print(f"case interpolate_rmsnorm short t={t} lengths={lengths}", flush=True)
    y = interpolate_rmsnorm(low.to(DEV), grids, dn)
    two = dn(interpolate(low.to(DEV), grids))
    torch.cuda.synchronize()
    assert torch.equal(y.cpu(), two.cpu())
    ref = rms_norm(O.interpolate(low, left, right, alpha, lens), norm.weight.detach().cpu(), norm.eps)
    close(y, ref, BF)
    for i, length in enumerate(lengths):
        assert not y[i, length:].float().any()


@pytest.mark.parametrize("dtype", [torch.float32, BF])
def test_rotary_qkv(dtype):
    g = gen(2)
    b, t, h, d = 2, 26, 16, 64
    x = torch.randn(b, t, 3 * h * d, generator=g).to(dtype)
    phase = torch.arange(t).float()[:, None] * 10000.0 ** (-torch.arange(0, d, 2).float() / d)[None, :]
    y = RotaryQKV.apply(x.to(DEV), phase.cos().to(DEV), phase.sin().to(DEV), h)
    close(y, O.rotary_qkv(x, phase.cos(), phase.sin(), h), dtype)


@pytest.mark.parametrize("silu", [False, True])
@pytest.mark.parametrize("channels_last", [False, True])
def test_front_norm(silu, channels_last):
    g = gen(3)
    x = torch.randn(2, 64, 51, 65, generator=g).to(BF)
    if channels_last:
        x = x.contiguous(memory_format=torch.channels_last)
    lengths = torch.tensor([51, 20])
    norm = SimpleNamespace(weight=(torch.rand(64, generator=g) + 0.5).to(DEV), eps=1e-5)
    y = front_norm(x.to(DEV), lengths.to(DEV), norm, silu=silu)
    assert y.shape == x.shape
    ref = O.front_norm(x, lengths, norm.weight.cpu(), silu=silu).permute(0, 3, 1, 2)
    close(y, ref, BF)


@pytest.mark.parametrize("channels_last", [False, True])
def test_bands(channels_last):
    g = gen(4)
    x = torch.randn(2, 128, 26, 33, generator=g).to(BF)
    if channels_last:
        x = x.contiguous(memory_format=torch.channels_last)
    close(bands(x.to(DEV)), O.bands(x), BF)


def test_evidence_norm_and_gated_concat():
    g = gen(5)
    x = torch.randn(2, 101, 1024, generator=g)
    value = torch.randn(2, 101, 1024, generator=g).to(BF)
    gate = torch.randn(2, 101, 1024, generator=g).to(BF)
    w = torch.rand(1024, generator=g) + 0.5
    mask = torch.rand(2, 101, generator=g) > 0.2
    y = evidence_norm(x.to(DEV), value.to(DEV), gate.to(DEV), w.to(DEV), mask.to(DEV))
    close(y, O.evidence_norm(x, value, gate, w, mask), torch.float32)
    s = torch.randn(2, 101, 3072, generator=g).to(BF)
    sg = torch.randn(2, 101, 3, generator=g).to(BF)
    close(gated_concat(s.to(DEV), sg.to(DEV)), O.gated_concat(s, sg), BF)
