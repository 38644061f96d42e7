"""Pins the oracle of the TriFusion block and front-end kernels (no GPU) against
explicit loops and library routines on small inputs."""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import trifusion as O


def test_depthwise_masked_matches_loop():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(2, 9, 5, generator=g)
    w = torch.randn(5, 1, 7, generator=g)
    bias = torch.randn(5, generator=g)
    lengths = torch.tensor([9, 4])
    y = O.depthwise_masked(x, w, bias, lengths)
    for b in range(2):
        for t in range(9):
            for c in range(5):
                want = 0.0
                if t < lengths[b]:
                    want = bias[c].item() + sum(
                        x[b, t + k - 3, c].item() * w[c, 0, k].item() for k in range(7) if 0 <= t + k - 3 < 9
                    )
                assert abs(y[b, t, c].item() - want) < 1e-5


def test_pool4_matches_loop():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(3, 10, 4, generator=g)
    lengths = torch.tensor([10, 5, 1])
    y = O.pool4(x, lengths)
    assert y.shape == (3, 3, 4)
    for b in range(3):
        for j in range(3):
            rows = [4 * j + k for k in range(4) if 4 * j + k < lengths[b]]
            want = x[b, rows].sum(0) / max(len(rows), 1) if rows else torch.zeros(4)
            assert torch.allclose(y[b, j], want, atol=1e-6)


def test_interpolate_matches_loop_and_grids():
    g = torch.Generator().manual_seed(2)
    lengths = torch.tensor([13, 6])
    low_lengths, left, right, alpha = O.grids(lengths, 13)
    assert low_lengths.tolist() == [4, 2]
    assert ((0 <= alpha) & (alpha < 1)).all() and (right >= left).all()
    low = torch.randn(2, 4, 3, generator=g)
    y = O.interpolate(low, left, right, alpha, lengths)
    for b in range(2):
        for t in range(13):
            if t >= lengths[b]:
                assert not y[b, t].any()
                continue
            a, z, al = low[b, left[b, t]], low[b, right[b, t]], alpha[b, t]
            assert torch.allclose(y[b, t], a + (z - a) * al, atol=1e-6)


def test_rotary_qkv_matches_loop_and_keeps_pair_norms():
    g = torch.Generator().manual_seed(3)
    b, t, h, d = 2, 5, 3, 4
    x = torch.randn(b, t, 3 * h * d, generator=g)
    phase = torch.rand(t, d // 2, generator=g) * 6
    y = O.rotary_qkv(x, phase.cos(), phase.sin(), h)
    assert y.shape == (3, b, h, t, d)
    raw = x.view(b, t, 3, h, d)
    for q in range(3):
        for i in range(b):
            for j in range(h):
                for s in range(t):
                    for c in range(d // 2):
                        a, z = raw[i, s, q, j, 2 * c].item(), raw[i, s, q, j, 2 * c + 1].item()
                        co, si = math.cos(phase[s, c]), math.sin(phase[s, c])
                        want = (a * co - z * si, a * si + z * co) if q < 2 else (a, z)
                        got = (y[q, i, j, s, 2 * c].item(), y[q, i, j, s, 2 * c + 1].item())
                        assert abs(got[0] - want[0]) < 1e-5 and abs(got[1] - want[1]) < 1e-5


def test_front_norm_matches_rms_norm_per_row():
    g = torch.Generator().manual_seed(4)
    x = torch.randn(2, 6, 5, 3, generator=g)
    w = torch.rand(6, generator=g) + 0.5
    lengths = torch.tensor([5, 2])
    y = O.front_norm(x, lengths, w, silu=False)
    ys = O.front_norm(x, lengths, w, silu=True)
    assert y.shape == (2, 5, 3, 6)
    for b in range(2):
        for t in range(5):
            for f in range(3):
                if t >= lengths[b]:
                    assert not y[b, t, f].any() and not ys[b, t, f].any()
                    continue
                want = F.rms_norm(x[b, :, t, f], (6,), w, eps=1e-5)
                assert torch.allclose(y[b, t, f], want, atol=1e-6)
                assert torch.allclose(ys[b, t, f], F.silu(want), atol=1e-6)


def test_bands_are_the_adaptive_pool_windows():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 3, 4, 21, generator=g)
    y = O.bands(x)
    assert y.shape == (2, 4, 8, 3)
    for i in range(8):
        start, end = (i * 21) // 8, -(-((i + 1) * 21) // 8)
        want = x[..., start:end].mean(-1).permute(0, 2, 1)
        assert torch.allclose(y[:, :, i], want, atol=1e-6)


def test_evidence_norm_and_gated_concat():
    g = torch.Generator().manual_seed(6)
    x = torch.randn(4, 16, generator=g)
    value = torch.randn(4, 16, generator=g)
    gate = torch.randn(4, 16, generator=g)
    w = torch.rand(16, generator=g) + 0.5
    mask = torch.tensor([True, False, True, True])
    y = O.evidence_norm(x, value, gate, w, mask)
    want = F.rms_norm(x + value * 2 / (1 + torch.exp(-gate)), (16,), w, eps=1e-5)
    assert torch.allclose(y[mask], want[mask], atol=1e-5) and not y[1].any()
    gx = torch.randn(4, 12, generator=g)
    gg = torch.randn(4, 3, generator=g)
    gy = O.gated_concat(gx, gg)
    for r in range(4):
        for k in range(3):
            assert torch.allclose(gy[r, 4 * k : 4 * k + 4], gx[r, 4 * k : 4 * k + 4] * 2 * torch.sigmoid(gg[r, k]))


def _bf_values(*shape, g):
    return torch.randn(*shape, generator=g).to(torch.bfloat16).float()


@pytest.mark.parametrize("s", [1, 2])
def test_front_stage_matches_direct_loops(s):
    """A CNN stage against direct float64 loops over taps: 3x3 conv of stride
    (s, 2) with zero padding 1, norm, SiLU, second conv, norm, 1x1 strided skip,
    residual, SiLU, rows past the length 0. The oracle rounds to bf16 at five
    points, so values agree within a few bf16 steps; a wrong stride axis, padding
    or weight orientation moves them by O(1)."""
    g = torch.Generator().manual_seed(7)
    b, cin, cout, t, f = 2, 3, 4, 7, 9
    x = _bf_values(b, cin, t, f, g=g)
    w1, w2, ws = _bf_values(cout, cin, 3, 3, g=g), _bf_values(cout, cout, 3, 3, g=g), _bf_values(cout, cin, 1, 1, g=g)
    n1, n2 = torch.rand(cout, generator=g) + 0.5, torch.rand(cout, generator=g) + 0.5
    lengths = torch.tensor([4, 2])
    y = O.front_stage(x, lengths, w1, w2, ws, n1, n2, s).double()
    to, fo = (t - 1) // s + 1, (f - 1) // 2 + 1
    assert y.shape == (b, to, fo, cout)
    xd = x.double()

    def conv3(src, w, st, sf, ti_max, fi_max, i, tt, ff):
        acc = torch.zeros(w.shape[0], dtype=torch.float64)
        for dy in range(3):
            for dx in range(3):
                ti, fi = tt * st + dy - 1, ff * sf + dx - 1
                if 0 <= ti < ti_max and 0 <= fi < fi_max:
                    acc += w[:, :, dy, dx].double() @ src[i, :, ti, fi]
        return acc

    def rms(v, w):
        return v / torch.sqrt((v * v).mean() + 1e-5) * w.double()

    h = torch.zeros(b, cout, to, fo, dtype=torch.float64)
    for i in range(b):
        for tt in range(int(lengths[i])):
            for ff in range(fo):
                h[i, :, tt, ff] = F.silu(rms(conv3(xd, w1, s, 2, t, f, i, tt, ff), n1))
    for i in range(b):
        for tt in range(to):
            for ff in range(fo):
                if tt >= lengths[i]:
                    assert not y[i, tt, ff].any()
                    continue
                main = rms(conv3(h, w2, 1, 1, to, fo, i, tt, ff), n2)
                skip = ws[:, :, 0, 0].double() @ xd[i, :, tt * s, ff * 2]
                want = F.silu(main + skip)
                assert torch.allclose(y[i, tt, ff], want, rtol=0.03, atol=0.03), (i, tt, ff)


def test_evidence_down_matches_loop():
    """``evidence_down`` against an explicit float64 loop over rows and output
    columns of the concatenated bf16 row, with the bf16 roundings of the
    linear's result and of the SiLU; and the concatenation order matters."""
    g = torch.Generator().manual_seed(31)
    rows, d, r = 5, 12, 4
    cn, an = torch.randn(rows, d, generator=g), torch.randn(rows, d, generator=g)
    w, b = torch.randn(r, 2 * d, generator=g) / 4, torch.randn(r, generator=g)
    y = O.evidence_down(cn, an, w, b).double()
    bf = lambda t: t.to(torch.bfloat16).double()  # noqa: E731
    ref = torch.empty(rows, r, dtype=torch.float64)
    for i in range(rows):
        s = torch.cat((bf(cn[i]), bf(an[i])))
        for o in range(r):
            z = bf(torch.tensor(sum(float(s[k]) * float(bf(w[o, k])) for k in range(2 * d)) + float(bf(b[o]))))
            ref[i, o] = bf(z / (1 + torch.exp(-z)))
    torch.testing.assert_close(y, ref, rtol=2 ** -7, atol=2 ** -7 * ref.abs().max().item())
    assert not torch.allclose(O.evidence_down(an, cn, w, b).double(), ref, rtol=2 ** -6, atol=0)
