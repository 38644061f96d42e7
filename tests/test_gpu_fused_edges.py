"""Edge cases of the fused front-stage and block kernels on MI355X against the
oracle: one time step, time steps that do not fill a 4-step pool group or a
depthwise tile, zero and one valid steps, the smallest widths and widths that
leave lanes idle. Tolerances as in test_gpu_block_fused.py and
test_gpu_front_conv.py; rows past each length are exactly 0. A pooled row with
no valid key has no defined softmax: the kernel returns 0 there (the oracle's
SDPA returns NaN), and the test checks that."""

from types import SimpleNamespace

import pytest
import torch
import torch.nn.functional as F

from oracle import trifusion as O
from oracle.elementwise import time_mask
from trifusion_amd.kernels import RMSNorm
from trifusion_amd.kernels.block import (
    block_pre,
    front_stage,
    glu_depthwise,
    merge_conv,
    merge_gate,
    norm_silu,
    pooled_attention,
)
from trifusion_amd.trifusion import CNNStage

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16


def close_bf16(y, ref, steps=2):
    y, ref = y.float().cpu(), ref.float().cpu()
    tol = steps * 2 ** -7
    torch.testing.assert_close(y, ref, rtol=tol, atol=tol * max(ref.abs().max().item(), 1e-6))


def norm(d, g):
    n = RMSNorm(d)
    with torch.no_grad():
        n.weight.copy_(torch.rand(d, generator=g) + 0.5)
    return n


@pytest.mark.parametrize("t,d,lengths", [(1, 8, [1]), (5, 136, [5, 0, 2]), (7, 1024, [7, 4]), (3, 16, [0, 3])])
def test_block_pre_edges(t, d, lengths):
    g = torch.Generator().manual_seed(t * d)
    lengths = torch.tensor(lengths)
    x = torch.randn(len(lengths), t, d, generator=g)
    n = norm(d, g)
    xm, h, p = block_pre(x.to(DEV), lengths.to(DEV), n.to(DEV))
    rm, rh, rp = O.block_pre(x, lengths, n.weight.detach().cpu())
    assert torch.equal(xm.cpu(), rm)
    close_bf16(h, rh, 1)
    close_bf16(p, rp, 1)
    assert not p.cpu()[lengths == 0].any()


@pytest.mark.parametrize("k", [3, 7])
@pytest.mark.parametrize("t,d,lengths", [(1, 8, [1]), (3, 24, [3, 0]), (9, 520, [9, 1, 5])])
def test_glu_depthwise_and_norm_silu_edges(k, t, d, lengths):
    g = torch.Generator().manual_seed(k * t + d)
    lengths = torch.tensor(lengths)
    up = torch.randn(len(lengths), t, 2 * d, generator=g).to(BF)
    layer = torch.nn.Conv1d(d, d, k, padding=k // 2, groups=d)
    w, b = layer.weight.detach().clone(), layer.bias.detach().clone()
    y = glu_depthwise(up.to(DEV), layer.to(DEV), lengths.to(DEV))
    ref = O.glu_depthwise(up, w, b, lengths)
    close_bf16(y, ref)
    assert not y.cpu()[~time_mask(lengths, t)].any()
    n = norm(d, g)
    close_bf16(norm_silu(ref.to(DEV), n.to(DEV)), O.norm_silu(ref, n.weight.detach().cpu()))


@pytest.mark.parametrize("t,heads,hd,low", [(1, 1, 32, [1]), (17, 2, 64, [17, 0, 3]), (70, 3, 32, [70, 65, 64])])
def test_pooled_attention_edges(t, heads, hd, low):
    g = torch.Generator().manual_seed(t + heads)
    low = torch.tensor(low)
    qkv = torch.randn(len(low), t, 3 * heads * hd, generator=g).to(BF)
    phase = torch.arange(t).float()[:, None] * 10000.0 ** (-torch.arange(0, hd, 2).float() / hd)[None, :]
    grids = SimpleNamespace(rope_cos=phase.cos().to(DEV), rope_sin=phase.sin().to(DEV), low_lengths=low.to(DEV))
    y = pooled_attention(qkv.to(DEV), grids, heads).cpu()
    ref = O.pooled_attention(qkv, phase.cos(), phase.sin(), low, heads)
    some = low > 0
    close_bf16(y[some], ref[some])
    assert not y[~some].any()


@pytest.mark.parametrize("t,d,lengths", [(1, 8, [1]), (6, 24, [6, 0]), (13, 520, [13, 2])])
def test_merge_kernels_edges(t, d, lengths):
    g = torch.Generator().manual_seed(t * 7 + d)
    lengths = torch.tensor(lengths)
    b = len(lengths)
    valid = time_mask(lengths, t)[..., None]
    cn, an, mf, mb = ((torch.randn(b, t, d, generator=g) * valid).to(BF) for _ in range(4))
    n = norm(d, g)
    gate = torch.nn.Linear(3 * d, 3)
    with torch.no_grad():
        gate.weight.normal_(std=0.05, generator=g)
        gate.bias.normal_(generator=g)
    mn, gg = merge_gate(cn.to(DEV), mf.to(DEV), mb.to(DEV), an.to(DEV), n.to(DEV), gate.to(DEV))
    rmn, rg = O.merge_gate(cn, mf, mb, an, n.weight.detach().cpu(), gate.weight.detach().cpu(),
                           gate.bias.detach().cpu())
    assert (mn.cpu() - rmn).abs().max().item() <= 1e-5 * max(rmn.abs().max().item(), 1e-6)
    close_bf16(gg, rg)
    layer = torch.nn.Conv1d(3 * d, 3 * d, 3, padding=1, groups=3 * d)
    y = merge_conv(cn.to(DEV), rmn.to(DEV), an.to(DEV), rg.to(DEV), layer.to(DEV), lengths.to(DEV))
    ref = O.merge_conv(cn, rmn, an, rg, layer.weight.detach().cpu(), layer.bias.detach().cpu(), lengths)
    close_bf16(y, ref, 1)


@pytest.mark.parametrize("cin,cout,stride", [(1, 32, 1), (32, 64, 2), (64, 128, 2)])
@pytest.mark.parametrize("t,f,lengths", [(1, 3, [1]), (4, 17, [4, 0, 1]), (9, 8, [9, 6])])
def test_front_stage_edges(cin, cout, stride, t, f, lengths):
    g = torch.Generator().manual_seed(cin + t + f)
    stage = CNNStage(cin, cout, stride)
    with torch.no_grad():
        for conv in (stage.conv1, stage.conv2, stage.skip):
            conv.weight.copy_(torch.randn(conv.weight.shape, generator=g) / (conv.weight[0].numel() ** 0.5))
        stage.norm1.weight.copy_(torch.rand(cout, generator=g) + 0.5)
        stage.norm2.weight.copy_(torch.rand(cout, generator=g) + 0.5)
    in_lengths = torch.tensor(lengths)
    x = torch.randn(len(lengths), cin, t, f, generator=g)
    x = x.masked_fill(~time_mask(in_lengths, t)[:, None, :, None], 0)
    if cin > 1:
        x = x.to(BF).contiguous(memory_format=torch.channels_last)
    out_lengths = (in_lengths + stride - 1) // stride
    ref = O.front_stage(x.float(), out_lengths, stage.conv1.weight.detach(), stage.conv2.weight.detach(),
                        stage.skip.weight.detach(), stage.norm1.weight.detach(), stage.norm2.weight.detach(),
                        stride).float()
    y = front_stage(stage.to(DEV), x.to(DEV), out_lengths.to(DEV)).permute(0, 2, 3, 1).float().cpu()
    assert y.shape == ref.shape
    err = (y - ref).abs()
    scale = max(ref.abs().max().item(), 1e-6)
    assert bool((err <= 2 ** -6 * (ref.abs() + scale)).all())
    assert not y[~time_mask(out_lengths, y.shape[1])].any()
