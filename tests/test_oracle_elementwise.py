"""Pins the CPU oracle of the bandwidth ops against library routines and
hand-evaluated cases (no GPU)."""

import torch
import torch.nn.functional as F

from oracle import elementwise as E


def test_rms_norm_matches_torch_rms_norm():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(37, 512, generator=g)
    w = torch.rand(512, generator=g) + 0.5
    expect = F.rms_norm(x, (512,), w, eps=1e-5)
    assert torch.allclose(E.rms_norm(x, w), expect, rtol=1e-5, atol=1e-6)
    xb = x.to(torch.bfloat16)
    assert E.rms_norm(xb, w).dtype == torch.bfloat16
    assert torch.allclose(E.rms_norm(xb, w).float(), F.rms_norm(xb.float(), (512,), w, eps=1e-5), atol=0.02)


def test_swiglu_matches_silu_times_up():
    g = torch.Generator().manual_seed(1)
    gate = torch.randn(9, 1365, generator=g)
    up = torch.randn(9, 1365, generator=g)
    x = torch.cat((gate, up), -1)
    assert torch.allclose(E.swiglu(x), gate * torch.sigmoid(gate) * up, rtol=1e-6, atol=1e-6)


def test_time_mask_and_mask_rows():
    lengths = torch.tensor([3, 0, 5])
    m = E.time_mask(lengths, 5)
    assert m.tolist() == [[1, 1, 1, 0, 0], [0, 0, 0, 0, 0], [1, 1, 1, 1, 1]]
    x = torch.arange(30.0).reshape(3, 5, 2)
    y = E.mask_rows(x, m)
    assert torch.equal(y, torch.where(m[..., None], x, torch.zeros(())))


def test_add_masked_and_dtype():
    a = torch.randn(4, 6, 8)
    b = torch.randn(4, 6, 8).to(torch.bfloat16)
    mask = torch.rand(4, 6) > 0.5
    y = E.add(a, b, mask)
    assert y.dtype == torch.float32
    assert torch.equal(y, torch.where(mask[..., None], a + b.float(), torch.zeros(())))
    assert E.add(a, b, bf16=True).dtype == torch.bfloat16


def test_mamba_controls_special_cases():
    # a >= 0: control = -(a + 1); a < 0: control = -1/(1 - a); floored at -1e-4
    a = torch.tensor([[[0.0, 2.0, -1.0, -1e9]]])
    ddt = torch.tensor([[[0.0, 25.0, -30.0, 1.0]]])
    bias = torch.tensor([0.5, 0.0, 0.0, -1.0])
    adt, dt = E.mamba_controls(a, ddt, bias)
    assert adt.shape == (1, 4, 1) and dt.shape == (1, 4, 1)
    sp = F.softplus(torch.tensor([0.5, 25.0, -30.0, 0.0]))  # threshold 20 like the reference
    assert torch.allclose(dt[0, :, 0], sp)
    control = torch.tensor([-1.0, -3.0, -0.5, -1e-4])
    assert torch.allclose(adt[0, :, 0], control * sp, rtol=1e-6)


def test_masked_mean_matches_loop():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(3, 11, 5, generator=g).to(torch.bfloat16)
    lengths = torch.tensor([11, 4, 1])
    y = E.masked_mean(x, lengths)
    for b in range(3):
        n = int(lengths[b])
        expect = sum(x[b, t].float() for t in range(n)) / n
        assert torch.allclose(y[b], expect, atol=1e-6)


def _reverse_loop(x, lengths):
    b, t, _ = x.shape
    y = torch.zeros_like(x)
    for i in range(b):
        n = max(0, min(int(lengths[i]), t))
        for s in range(n):
            y[i, s] = x[i, n - 1 - s]
    return y


def test_reverse_valid_matches_loop_flip_and_squares_to_mask():
    g = torch.Generator().manual_seed(7)
    x = torch.randn(5, 9, 3, generator=g)
    lengths = torch.tensor([9, 4, 0, 1, 12])  # full, ragged, empty, single, past T
    y = E.reverse_valid(x, lengths)
    assert torch.equal(y, _reverse_loop(x, lengths))
    assert torch.equal(y[0], torch.flip(x[0], (0,)))
    assert torch.equal(y[4], torch.flip(x[4], (0,)))
    assert not y[2].any() and torch.equal(y[3, 0], x[3, 0]) and not y[3, 1:].any()
    mask = E.time_mask(lengths.clamp(0, 9), 9)
    assert torch.equal(E.reverse_valid(y, lengths), E.mask_rows(x, mask))


def test_mean_norm_matches_rms_norm_of_the_mean():
    g = torch.Generator().manual_seed(8)
    a = torch.randn(11, 512, generator=g)
    b = torch.randn(11, 512, generator=g)
    w = torch.rand(512, generator=g) + 0.5
    expect = F.rms_norm((a + b) / 2, (512,), w, eps=1e-5)
    assert torch.allclose(E.mean_norm(a, b, w), expect, rtol=1e-5, atol=1e-6)
    assert torch.allclose(E.mean_norm(a, a, w), F.rms_norm(a, (512,), w, eps=1e-5), rtol=1e-5, atol=1e-6)
    ab = a.to(torch.bfloat16)
    assert E.mean_norm(ab, ab, w).dtype == torch.float32
    assert not E.mean_norm(torch.zeros(2, 512), torch.zeros(2, 512), w).any()
