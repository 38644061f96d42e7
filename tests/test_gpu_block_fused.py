"""Fused TriFusion block kernels on MI355X against the oracle's compositions of
the unfused reference ops (bf16 autocast values), and against the unfused GPU
kernels the block otherwise runs. Tolerances: bf16 outputs within one bf16 step
of the oracle (rtol 2^-7 plus 2^-7 of the largest magnitude; two steps where a
bf16 value feeds a second rounding), fp32 outputs within 1e-5 of the largest
magnitude. Against the unfused GPU kernels, outputs with the same per-element
arithmetic are bit-identical; the gate dot product and the attention sum in a
different order and are held to the oracle's tolerance."""

from types import SimpleNamespace

import pytest
import torch
import torch.nn.functional as F

from oracle import trifusion as O
from oracle.elementwise import mean_norm as o_mean_norm
from oracle.elementwise import time_mask
from trifusion_amd.kernels import RMSNorm, gated_concat
from trifusion_amd.kernels.block import (
    Pool4,
    block_pre,
    block_pre_add,
    depthwise_masked,
    evidence_down,
    evidence_norm,
    glu_depthwise,
    glu_norm_silu,
    merge_conv,
    merge_gate,
    norm_silu,
    pooled_attention,
    query_read,
)
from trifusion_amd.kernels.buffers import mask_buffer
from trifusion_amd.kernels.native import add, mean_norm

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16
LENGTHS = torch.tensor([101, 57, 4])


def gen(seed):
    return torch.Generator().manual_seed(seed)


def close_bf16(y, ref, steps=1):
    y, ref = y.float().cpu(), ref.float().cpu()
    tol = steps * 2 ** -7
    torch.testing.assert_close(y, ref, rtol=tol, atol=tol * ref.abs().max().item())


def norm(d, g):
    n = RMSNorm(d)
    with torch.no_grad():
        n.weight.copy_(torch.rand(d, generator=g) + 0.5)
    return n


def test_block_pre():
    g = gen(0)
    x = torch.randn(3, 101, 1024, generator=g)
    n = norm(1024, g)
    xm, h, p = block_pre(x.to(DEV), LENGTHS.to(DEV), n.to(DEV))
    rm, rh, rp = O.block_pre(x, LENGTHS, n.weight.detach().cpu())
    assert torch.equal(xm.cpu(), rm)
    close_bf16(h, rh)
    close_bf16(p, rp)
    # the unfused GPU ops: mask, fp32 norm, casts, fp32 pooling
    mask = time_mask(LENGTHS, 101).to(DEV)
    um = mask_buffer(x.to(DEV), mask)
    uh = n(um)
    assert torch.equal(h, uh.to(BF))
    assert torch.equal(p, Pool4.apply(uh, LENGTHS.to(DEV)).to(BF))


@pytest.mark.parametrize("d", [1024, 128])
def test_block_pre_add_equals_add_then_block_pre(d):
    """The previous block's closing masked add applied by the start kernel: the
    values of tf_add then tf_block_pre, bit for bit."""
    g = gen(21)
    r = torch.randn(3, 101, d, generator=g).to(DEV)
    down = torch.randn(3, 101, d, generator=g).to(BF).to(DEV)
    n = norm(d, g).to(DEV)
    mask = time_mask(LENGTHS, 101).to(DEV)
    print(f"case block_pre_add d={d}", flush=True)
    with torch.inference_mode():
        fused = block_pre_add(r, down, LENGTHS.to(DEV), n)
        two = block_pre(add(r, down, mask), LENGTHS.to(DEV), n)
    torch.cuda.synchronize()
    for a, b in zip(fused, two):
        assert torch.equal(a, b)


@pytest.mark.parametrize("k", [3, 7])
def test_glu_depthwise_and_norm_silu(k):
    g = gen(k)
    up = torch.randn(3, 101, 2048, generator=g).to(BF)
    layer = torch.nn.Conv1d(1024, 1024, k, padding=k // 2, groups=1024)
    w, b = layer.weight.detach().clone(), layer.bias.detach().clone()
    y = glu_depthwise(up.to(DEV), layer.to(DEV), LENGTHS.to(DEV))
    ref = O.glu_depthwise(up, w, b, LENGTHS)
    close_bf16(y, ref, steps=2)
    assert not y[1, 57:].any() and not y[2, 4:].any()
    with torch.autocast("cuda", dtype=BF):
        unfused = depthwise_masked(F.glu(up.to(DEV), dim=-1), layer, LENGTHS.to(DEV))
    assert torch.equal(y, unfused)
    n = norm(1024, g)
    s = norm_silu(ref.to(DEV), n.to(DEV))
    close_bf16(s, O.norm_silu(ref, n.weight.detach().cpu()))
    assert torch.equal(s, F.silu(n(ref.to(DEV))))


@pytest.mark.parametrize("k", [3, 7])
@pytest.mark.parametrize("d", [1024, 520, 128])
def test_glu_norm_silu_equals_two_launches(d, k):
    """GLU + depthwise + RMSNorm + SiLU in one launch gives the values of
    glu_depthwise then norm_silu, bit for bit (rows past the length included)."""
    g = gen(10 + k)
    up = (torch.randn(3, 101, 2 * d, generator=g) * 2).to(BF).to(DEV)
    layer = torch.nn.Conv1d(d, d, k, padding=k // 2, groups=d).to(DEV)
    n = norm(d, g).to(DEV)
    lengths = LENGTHS.to(DEV)
    print(f"case glu_norm_silu d={d} k={k}", flush=True)
    with torch.inference_mode():
        y = glu_norm_silu(up, layer, lengths, n)
        two = norm_silu(glu_depthwise(up, layer, lengths), n)
    torch.cuda.synchronize()
    assert y.shape == two.shape and torch.equal(y, two)


@pytest.mark.parametrize("t,lengths", [(1, [1, 0]), (5, [5, 3]), (9, [9, 0, 6])])
def test_block_pre_add_short(t, lengths):
    """Fewer rows than a pooling group, a partial last group and zero-length
    rows: the start kernel with the previous block's add equals tf_add then
    tf_block_pre bit for bit, and the oracle's block start."""
    g = gen(30 + t)
    d = 256
    lens = torch.tensor(lengths)
    r = torch.randn(len(lengths), t, d, generator=g)
    down = torch.randn(len(lengths), t, d, generator=g).to(BF)
    n = norm(d, g).to(DEV)
    mask = time_mask(lens, t).to(DEV)
    print(f"case block_pre_add short t={t} lengths={lengths}", flush=True)
    with torch.inference_mode():
        fused = block_pre_add(r.to(DEV), down.to(DEV), lens.to(DEV), n)
        summed = add(r.to(DEV), down.to(DEV), mask)
        two = block_pre(summed, lens.to(DEV), n)
    torch.cuda.synchronize()
    for a, b in zip(fused, two):
        assert torch.equal(a, b)
    rm, rh, rp = O.block_pre(summed.cpu(), lens, n.weight.detach().cpu())
    assert torch.equal(fused[0].cpu(), rm)
    close_bf16(fused[1], rh)
    close_bf16(fused[2], rp)


@pytest.mark.parametrize("k", [3, 7])
@pytest.mark.parametrize("t,lengths", [(1, [1, 0]), (3, [3, 2]), (6, [6, 1])])
def test_glu_short_sequences(t, lengths, k):
    """Sequences shorter than the kernels' time tiles and the conv halo: GLU
    rows outside [0, T) are zero (their clamped loads dropped). glu_depthwise
    against the oracle, the one-launch form bitwise against the two launches,
    rows past each length exactly zero."""
    g = gen(20 + 3 * t + k)
    d = 520
    up = torch.randn(len(lengths), t, 2 * d, generator=g).to(BF)
    layer = torch.nn.Conv1d(d, d, k, padding=k // 2, groups=d)
    w, b = layer.weight.detach().clone(), layer.bias.detach().clone()
    n = norm(d, g).to(DEV)
    lens = torch.tensor(lengths)
    print(f"case glu short t={t} lengths={lengths} k={k}", flush=True)
    with torch.inference_mode():
        y = glu_depthwise(up.to(DEV), layer.to(DEV), lens.to(DEV))
        one = glu_norm_silu(up.to(DEV), layer.to(DEV), lens.to(DEV), n)
        two = norm_silu(y, n)
    torch.cuda.synchronize()
    close_bf16(y, O.glu_depthwise(up, w, b, lens), steps=2)
    assert torch.equal(one, two)
    for i, length in enumerate(lengths):
        assert not y[i, length:].any() and not one[i, length:].any()


@pytest.mark.parametrize("t,heads,hd", [(26, 16, 64), (101, 8, 32)])
def test_pooled_attention(t, heads, hd):
    g = gen(t)
    qkv = torch.randn(3, t, 3 * heads * hd, generator=g).to(BF)
    low = torch.tensor([t, (t + 1) // 2, 1])
    phase = torch.arange(t).float()[:, None] * 10000.0 ** (-torch.arange(0, hd, 2).float() / hd)[None, :]
    grids = SimpleNamespace(rope_cos=phase.cos().to(DEV), rope_sin=phase.sin().to(DEV), low_lengths=low.to(DEV))
    y = pooled_attention(qkv.to(DEV), grids, heads)
    ref = O.pooled_attention(qkv, phase.cos(), phase.sin(), low, heads)
    assert y.shape == ref.shape
    close_bf16(y, ref, steps=2)


def test_merge_gate_and_conv():
    g = gen(11)
    d = 1024
    cn, an = (torch.randn(3, 101, d, generator=g).to(BF) for _ in range(2))
    mf, mb = (torch.randn(3, 101, d, generator=g).to(BF) for _ in range(2))
    n = norm(d, g)
    gate = torch.nn.Linear(3 * d, 3)
    with torch.no_grad():
        gate.weight.copy_(torch.randn(3, 3 * d, generator=g) * 0.02)
        gate.bias.copy_(torch.randn(3, generator=g))
    dev = [t.to(DEV) for t in (cn, mf, mb, an)]
    mn, gg = merge_gate(*dev, n.to(DEV), gate.to(DEV))
    rmn, rg = O.merge_gate(cn, mf, mb, an, n.weight.detach().cpu(), gate.weight.detach().cpu(),
                           gate.bias.detach().cpu())
    scale = rmn.abs().max().item()
    assert ((mn.cpu() - rmn).abs().max().item()) <= 1e-5 * scale
    assert torch.equal(mn, mean_norm(dev[1], dev[2], n.weight, n.eps))
    close_bf16(gg, rg, steps=2)
    layer = torch.nn.Conv1d(3 * d, 3 * d, 3, padding=1, groups=3 * d)
    w, b = layer.weight.detach().clone(), layer.bias.detach().clone()
    lengths = LENGTHS.to(DEV)
    # zero-preserved inputs: rows past each length are 0 in the block
    valid = time_mask(LENGTHS, 101)[..., None]
    cn, an, rmn = cn * valid, an * valid, rmn * valid
    y = merge_conv(cn.to(DEV), rmn.to(DEV), an.to(DEV), rg.to(DEV), layer.to(DEV), lengths)
    close_bf16(y, O.merge_conv(cn, rmn, an, rg, w, b, LENGTHS))
    s = torch.cat((cn.to(DEV).float(), rmn.to(DEV), an.to(DEV).float()), -1)
    v = gated_concat(s, rg.to(DEV).float())
    with torch.autocast("cuda", dtype=BF):
        conv = depthwise_masked(v, layer, lengths)
    assert torch.equal(y, add(v, conv, bf16=True))


@pytest.mark.parametrize("rows, d, r", [(3 * 101, 1024, 64), (101, 128, 16), (37, 256, 48), (1, 384, 32), (0, 128, 64),
                                        (1616, 1024, 64), (70, 640, 48), (45, 1536, 64), (33, 1280, 16)])
def test_evidence_down(rows, d, r):
    """silu(e_down(cat(cn, an))) in one launch: the oracle's composition, and the
    unfused GPU composition under autocast, within two bf16 steps (the linear's
    output and the SiLU are each rounded; the sums run in another order). d up
    to 1024 runs the LDS-staged kernel, wider d the direct-load kernel."""
    g = gen(5)
    cn = (torch.randn(rows, d, generator=g) * 1.5).to(BF)
    an = (torch.randn(rows, d, generator=g) * 0.5).to(BF)
    layer = torch.nn.Linear(2 * d, r)
    with torch.no_grad():
        layer.bias.uniform_(-0.5, 0.5, generator=g)
    print(f"case evidence_down rows={rows} d={d} r={r}", flush=True)
    dl = torch.nn.Linear(2 * d, r).to(DEV)
    dl.load_state_dict(layer.state_dict())
    with torch.inference_mode():
        z = evidence_down(cn.to(DEV), an.to(DEV), dl)
        with torch.autocast("cuda", torch.bfloat16):
            unfused = F.silu(dl(torch.cat((cn.to(DEV), an.to(DEV)), -1)))
    torch.cuda.synchronize()
    assert z.shape == (rows, r) and z.dtype == BF
    if rows == 0:
        return
    ref = O.evidence_down(cn, an, layer.weight.detach(), layer.bias.detach())
    close_bf16(z, ref, steps=2)
    close_bf16(z, unfused, steps=2)


def test_evidence_down_3d_rows():
    """[B, T, d] inputs: one row per (b, t), the output [B, T, r]."""
    g = gen(6)
    cn, an = (torch.randn(2, 70, 1024, generator=g).to(BF) for _ in range(2))
    layer = torch.nn.Linear(2048, 64)
    print("case evidence_down 3d", flush=True)
    dl = torch.nn.Linear(2048, 64).to(DEV)
    dl.load_state_dict(layer.state_dict())
    with torch.inference_mode():
        z = evidence_down(cn.to(DEV), an.to(DEV), dl)
    torch.cuda.synchronize()
    assert z.shape == (2, 70, 64)
    close_bf16(z, O.evidence_down(cn, an, layer.weight.detach(), layer.bias.detach()), steps=2)


def test_evidence_norm_bf16_out():
    g = gen(12)
    x = torch.randn(2, 101, 1024, generator=g).to(DEV)
    value = torch.randn(2, 101, 1024, generator=g).to(BF).to(DEV)
    gate = torch.randn(2, 101, 1024, generator=g).to(BF).to(DEV)
    w = (torch.rand(1024, generator=g) + 0.5).to(DEV)
    mask = (torch.rand(2, 101, generator=g) > 0.2).to(DEV)
    y32 = evidence_norm(x, value, gate, w, mask)
    y16 = evidence_norm(x, value, gate, w, mask, bf16_out=True)
    assert y16.dtype == BF and torch.equal(y16, y32.to(BF))


@pytest.mark.parametrize("t,lengths", [(101, [101, 57, 4]), (1608, [1608, 800, 8]), (70, [0, 1])])
def test_query_read(t, lengths):
    g = gen(t)
    lengths = torch.tensor(lengths)
    q = (torch.randn(10, 256, generator=g) * 0.5).to(BF)
    kv = torch.randn(len(lengths), t, 512, generator=g).to(BF)
    y = query_read(q.to(DEV), kv.to(DEV), lengths.to(DEV)).cpu()
    some = lengths > 0
    close_bf16(y[some], O.query_read(q, kv, lengths)[some], steps=2)
    assert not y[~some].any()
