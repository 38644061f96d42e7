"""Fused front-end CNN stage kernels (``tf_front_conv1`` + ``tf_front_conv2``) on
MI355X against the oracle's stage: bf16-rounded operands, the library's fp32
convolution rounded to bf16, the channel norms, the 1x1 skip, the bf16 residual
and SiLU. The kernels sum the convolution in another order, which can move a
bf16 rounding by one step and, through the norms, a value by a few; tolerance:
|y - ref| <= 2^-6 (|ref| + max|ref|), mean |y - ref| <= 1e-3 max|ref|. Rows past
each length are exactly 0 and repeated calls give the same bits."""

import pytest
import torch

from oracle import trifusion as O
from oracle.elementwise import time_mask
from trifusion_amd.kernels.block import front_stage
from trifusion_amd.trifusion import CNNStage

pytestmark = pytest.mark.gpu
DEV = "cuda"

# (cin, cout, stride, time, freq): the three stages of the front end, short clips
CASES = [(1, 32, 1, 57, 257), (32, 64, 2, 57, 129), (64, 128, 2, 29, 65)]


def make_stage(cin, cout, stride, g):
    stage = CNNStage(cin, cout, stride)
    with torch.no_grad():
        for conv in (stage.conv1, stage.conv2, stage.skip):
            conv.weight.copy_(torch.randn(conv.weight.shape, generator=g) / (conv.weight[0].numel() ** 0.5))
        stage.norm1.weight.copy_(torch.rand(cout, generator=g) + 0.5)
        stage.norm2.weight.copy_(torch.rand(cout, generator=g) + 0.5)
    return stage


@pytest.mark.parametrize("cin,cout,stride,t,f", CASES)
def test_front_stage_matches_oracle(cin, cout, stride, t, f):
    g = torch.Generator().manual_seed(cin + cout)
    stage = make_stage(cin, cout, stride, g)
    in_lengths = torch.tensor([t, t // 2, 1])
    x = torch.randn(3, cin, t, f, generator=g) * (4.0 if cin == 1 else 1.0)
    x = x.masked_fill(~time_mask(in_lengths, t)[:, None, :, None], 0)
    if cin > 1:
        x = x.to(torch.bfloat16).contiguous(memory_format=torch.channels_last)
    lengths = (in_lengths + stride - 1) // stride
    ref = O.front_stage(x.float(), lengths, stage.conv1.weight.detach(), stage.conv2.weight.detach(),
                        stage.skip.weight.detach(), stage.norm1.weight.detach(), stage.norm2.weight.detach(),
                        stride).float()
    stage = stage.to(DEV)
    y = front_stage(stage, x.to(DEV), lengths.to(DEV))
    y2 = front_stage(stage, x.to(DEV), lengths.to(DEV))
    assert y.dtype == torch.bfloat16 and y.is_contiguous(memory_format=torch.channels_last)
    y = y.permute(0, 2, 3, 1).float().cpu()
    assert torch.equal(y, y2.permute(0, 2, 3, 1).float().cpu())
    assert y.shape == ref.shape
    scale = ref.abs().max().item()
    err = (y - ref).abs()
    print(f"stage {cin}->{cout}: max err {err.max().item():.3e} mean {err.mean().item():.3e} scale {scale:.3f}")
    assert bool((err <= 2 ** -6 * (ref.abs() + scale)).all())
    assert err.mean().item() <= 1e-3 * scale
    valid = time_mask(lengths, y.shape[1])
    assert not y[~valid].any()
