"""Pins the CPU oracle of the recurrence (no GPU).

Each check compares two independent formulations or a closed form, chosen so
that plausible mistakes (dropped halo term, wrong rotation sign, half-split
instead of interleaved pairs, diagonal included, exp instead of exp2, missing
phase carry, wrong head mapping) fail at least one of them; the planted-mistake
tests at the bottom verify exactly that.
"""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import recurrence as R
from trifusion_amd.synthetic import clip_inputs, reference_test_inputs


def f32(args):
    return tuple(a.float() for a in args)


# (B, T, H) shapes of the reference test, tests/test_recurrence.py:34-37 (the
# T=1501 case is covered at smaller H to keep the CPU suite fast)
REF_SHAPES = [(1, 1, 4), (2, 26, 4), (1, 63, 32), (1, 64, 32), (2, 65, 4), (1, 255, 8), (1, 1501, 2)]


@pytest.mark.parametrize("batch,time,heads", REF_SHAPES)
def test_chunked_fp32_matches_f64_loop_reference_shapes(batch, time, heads):
    args = f32(reference_test_inputs(batch, time, heads))
    ref = R.fused_mamba_f64(*args)
    out = R.fused_mamba_chunked(*args)
    assert R.rel_fro(out, ref) < 1e-5
    assert R.max_rel(out, ref) < 2e-5


@pytest.mark.parametrize(
    "b,t,h,p,n,r,hq",
    [(2, 256, 4, 32, 16, 4, 1), (2, 100, 4, 64, 64, 16, 1), (1, 70, 4, 64, 32, 8, 4), (1, 140, 2, 32, 128, 64, 2)],
)
def test_chunked_fp32_matches_f64_loop_clip_distributions(b, t, h, p, n, r, hq):
    args = clip_inputs(b, t, heads=h, head_dim=p, state=n, rotary=r, qk_heads=hq, dtype=torch.float32, seed=3)
    ref = R.fused_mamba_f64(*args)
    out = R.fused_mamba_chunked(*args)
    assert R.max_rel(out, ref) < 2e-5


@pytest.mark.parametrize("t", [50, 150])
def test_chunked_clamps_positive_decay_within_chunks(t):
    """Steps with adt > 0: the chunked form equals the FP64 attention form whose
    weights are capped at 1 inside a 64-step chunk and uncapped across chunks
    (mamba_fused.py:143-152). The unclamped closed form (the true recurrence)
    is far away on the same inputs, so a form without the clamp fails here."""
    args = list(clip_inputs(2, t, heads=4, head_dim=32, state=32, rotary=8, dtype=torch.float32, seed=9))
    g = torch.Generator().manual_seed(19)
    flip = torch.rand(args[3].shape, generator=g) < 0.3
    args[3] = torch.where(flip, -0.5 * args[3], args[3])
    assert (args[3] > 0).sum() > 10
    out = R.fused_mamba_chunked(*args)
    clamped = R.fused_mamba_attention_f64(*args, clamp_chunk=R.CHUNK)
    assert R.max_rel(out, clamped) < 2e-5
    unclamped = R.fused_mamba_attention_f64(*args)
    assert R.max_rel(unclamped, clamped) > 1e-2
    # with adt <= 0 the clamp is the identity
    neg = list(args)
    neg[3] = -args[3].abs()
    assert R.max_rel(R.fused_mamba_attention_f64(*neg, clamp_chunk=R.CHUNK), R.fused_mamba_attention_f64(*neg)) < 1e-12


@pytest.mark.parametrize("b,t,h,n,r,hq", [(1, 17, 4, 128, 32, 1), (2, 40, 4, 16, 4, 2), (1, 90, 3, 64, 16, 3)])
def test_f64_loop_matches_attention_form(b, t, h, n, r, hq):
    args = clip_inputs(b, t, heads=h, head_dim=32, state=n, rotary=r, qk_heads=hq, dtype=torch.float64, seed=5)
    loop = R.fused_mamba_f64(*args)
    attn = R.fused_mamba_attention_f64(*args)
    assert R.max_rel(loop, attn) < 1e-10


def test_single_step_closed_form():
    # T=1: no history, y = silu(z) * (D + dt*sigmoid(trap) * (q+qb).(k+kb)) * v
    args = clip_inputs(
        3, 1, heads=4, head_dim=32, state=16, rotary=4, dtype=torch.float64, ctrl_dtype=torch.float64, seed=11
    )
    q, k, v, adt, dt, trap, qb, kb, angles, d, z = args
    gamma = dt[:, :, 0] * torch.sigmoid(trap[:, :, 0])
    dot = ((q[:, 0] + qb) * (k[:, 0] + kb)).sum(-1)  # Hq=1 broadcast over heads
    expect = F.silu(z[:, 0]) * (d + gamma * dot)[..., None] * v[:, 0]
    for fn in (R.fused_mamba_f64, R.fused_mamba_attention_f64):
        assert R.max_rel(fn(*args)[:, 0], expect) < 1e-12
    # the chunked oracle computes in fp32
    assert R.max_rel(R.fused_mamba_chunked(*args)[:, 0], expect) < 1e-6


def test_causal_linear_attention_special_case():
    # adt=0 (no decay), theta=0 (no rotation), trap=+inf (gamma = s = dt), dt=1,
    # zero biases, D=0 and z large (silu(z) ~ z): y = z * sum_{u<=t} (q_t.k_u) v_u
    g = torch.Generator().manual_seed(4)
    b, t, h, p, n = 2, 50, 3, 8, 16
    q = torch.randn(b, t, 1, n, generator=g, dtype=torch.float64)
    k = torch.randn(b, t, 1, n, generator=g, dtype=torch.float64)
    v = torch.randn(b, t, h, p, generator=g, dtype=torch.float64)
    z = torch.full((b, t, h, p), 40.0, dtype=torch.float64)
    adt = torch.zeros(b, h, t, dtype=torch.float64)
    dt = torch.ones(b, h, t, dtype=torch.float64)
    trap = torch.full((b, h, t), 1e4, dtype=torch.float64)
    qb = torch.zeros(h, n, dtype=torch.float64)
    kb = torch.zeros(h, n, dtype=torch.float64)
    angles = torch.zeros(b, t, h, 4, dtype=torch.float64)
    d = torch.zeros(h, dtype=torch.float64)
    scores = torch.einsum("btn,bun->btu", q[:, :, 0], k[:, :, 0]).tril()
    expect = torch.einsum("btu,buhp->bthp", scores, v) * 40.0
    args = (q, k, v, adt, dt, trap, qb, kb, angles, d, z)
    assert R.max_rel(R.fused_mamba_f64(*args), expect) < 1e-12
    assert R.max_rel(R.fused_mamba_chunked(*f32(args)), expect) < 1e-5


@pytest.mark.parametrize("chunk", [16, 32, 128])
def test_chunk_size_independence(chunk):
    args = clip_inputs(2, 300, heads=3, head_dim=32, state=32, dtype=torch.float32, seed=9)
    base = R.fused_mamba_chunked(*args, chunk=64)
    other = R.fused_mamba_chunked(*args, chunk=chunk)
    assert R.max_rel(other, base) < 1e-5


def test_causality():
    args = list(clip_inputs(1, 150, heads=2, head_dim=32, state=16, dtype=torch.float32, seed=12))
    base = R.fused_mamba_chunked(*args)
    cut = 97
    q, k, v, adt, dt, trap, qb, kb, angles, d, z = args
    pert = [x.clone() for x in args]
    for idx in (0, 1, 2, 8, 10):  # q, k, v, angles, z: time dim 1
        pert[idx][:, cut + 1 :] += 1.0
    for idx in (3, 4, 5):  # adt, dt, trap: time dim 2
        pert[idx][:, :, cut + 2 :] *= 0.5
    out = R.fused_mamba_chunked(*pert)
    # rows <= cut only see t' <= cut+1 through the trapezoid halo of step cut
    assert torch.equal(out[:, : cut + 1], base[:, : cut + 1])
    assert not torch.equal(out[:, cut + 2 :], base[:, cut + 2 :])


def test_phase_matches_f64_cumsum():
    g = torch.Generator().manual_seed(21)
    b, t, h, r = 2, 700, 3, 8
    angles = torch.randn(b, t, h, r, generator=g) * 3
    dt = torch.rand(b, h, t, generator=g) * 2  # large steps: many wraps of 2*pi
    ph = R.phase_chunked(angles, dt, pairs=12)
    assert ph.shape == (b, t, h, 12)
    assert torch.all(ph[..., r:] == 0)
    assert torch.all((ph >= 0) & (ph < 2 * math.pi + 1e-6))
    exact = (angles.double().tanh() * math.pi * dt.double().transpose(1, 2)[..., None]).cumsum(1)
    assert torch.allclose(ph[..., :r].double().cos(), exact.cos(), atol=2e-4)
    assert torch.allclose(ph[..., :r].double().sin(), exact.sin(), atol=2e-4)


def test_fp32_phase_arithmetic_against_closed_form():
    """The reference-arithmetic phase option: a constant increment c per step has
    phase (t + 1) c mod 2 pi. The fp64 form meets it to its final fp32 rounding;
    the fp32 form drifts, since the rounding of the increment and of each carry
    has one sign at every step here (7.8e-4 rad after 7200 steps; random
    increments, as at the long-clip workload, drift ~6e-6), but stays within
    2e-3 rad. A dropped carry or a missing reduction misses by whole radians."""
    t, theta, step = 7200, 0.7, 0.37
    angles = torch.full((1, t, 1, 2), theta)
    dt = torch.full((1, 1, t), step)
    theta32, step32 = (float(torch.tensor(x, dtype=torch.float32)) for x in (theta, step))
    c = math.pi * math.tanh(theta32) * step32
    exact = torch.tensor([((i + 1) * c) % (2 * math.pi) for i in range(t)], dtype=torch.float64)

    def wrapped_gap(ph):
        d = (ph[0, :, 0, 0].double() - exact).abs()
        return torch.minimum(d, 2 * math.pi - d).max().item()

    ph64 = R.phase_chunked(angles, dt, pairs=2)
    ph32 = R.phase_chunked(angles, dt, pairs=2, accumulate=torch.float32)
    assert wrapped_gap(ph64) <= 1e-6  # the final fp32 rounding of a value below 2 pi
    assert 1e-5 <= wrapped_gap(ph32) <= 2e-3
    assert not torch.equal(ph32, ph64)
    assert torch.all((ph32 >= 0) & (ph32 <= 2 * math.pi))


def test_rotation_is_interleaved_and_norm_preserving():
    x = torch.tensor([[1.0, 2.0, 3.0, 4.0]])
    c = torch.tensor([[0.0, 1.0]])
    s = torch.tensor([[1.0, 0.0]])
    # pair (x0, x1) rotated by +90 degrees, pair (x2, x3) unchanged
    assert torch.equal(R.rotate_pairs(x, c, s), torch.tensor([[-2.0, 1.0, 3.0, 4.0]]))
    g = torch.Generator().manual_seed(1)
    y = torch.randn(5, 16, generator=g, dtype=torch.float64)
    ang = torch.rand(5, 8, generator=g, dtype=torch.float64) * 6
    assert torch.allclose(R.rotate_pairs(y, ang.cos(), ang.sin()).norm(dim=-1), y.norm(dim=-1))


def test_bf16_rounded_oracle_within_reference_tolerance_of_f64():
    # tests/test_recurrence.py:86 bounds the fused kernel at rel-Frobenius < 0.012 vs FP64
    args = reference_test_inputs(1, 17, 4)
    ref = R.fused_mamba_f64(*args)
    out = R.fused_mamba_chunked(*args, out_dtype=torch.bfloat16)
    assert R.rel_fro(out, ref) < 0.012
    args = clip_inputs(2, 200, heads=4, head_dim=64, state=64, seed=2)
    out = R.fused_mamba_chunked(*args)
    assert R.rel_fro(out, R.fused_mamba_f64(*args)) < 0.012


def test_lengths_mask_rows_only():
    args = clip_inputs(3, 130, heads=2, head_dim=32, state=16, dtype=torch.float32, seed=8)
    lengths = torch.tensor([130, 64, 5])
    full = R.fused_mamba_chunked(*args)
    masked = R.fused_mamba_chunked(*args, lengths=lengths)
    for b, n in enumerate(lengths.tolist()):
        assert torch.equal(masked[b, :n], full[b, :n])
        assert torch.all(masked[b, n:] == 0)


def _flip_t(args):
    q, k, v, adt, dt, trap, qb, kb, angles, d, z = args

    def f(x):
        return torch.flip(x, (1,))

    def g(x):
        return torch.flip(x, (2,))

    return (f(q), f(k), f(v), g(adt), g(dt), g(trap), qb, kb, f(angles), d, f(z))


def _truncate(args, b, n):
    q, k, v, adt, dt, trap, qb, kb, angles, d, z = args

    def s(x):
        return x[b : b + 1, :n]

    def u(x):
        return x[b : b + 1, :, :n]

    return (s(q), s(k), s(v), u(adt), u(dt), u(trap), qb, kb, s(angles), d, s(z))


def test_reversed_is_per_row_flip_of_the_valid_prefix():
    """The gather-based reversed oracle against its definition taken another way:
    each row cut to its length, flipped with torch.flip, run, flipped back."""
    args = clip_inputs(3, 150, heads=2, head_dim=32, state=16, dtype=torch.float32, seed=13)
    lengths = torch.tensor([150, 77, 1])
    out = R.fused_mamba_reversed(*args, lengths=lengths)
    for b, n in enumerate(lengths.tolist()):
        ref = torch.flip(R.fused_mamba_chunked(*_flip_t(_truncate(args, b, n))), (1,))
        assert R.max_rel(out[b : b + 1, :n], ref) <= 1e-5
        assert not out[b, n:].any()
    full = R.fused_mamba_reversed(*args)
    assert R.max_rel(full, torch.flip(R.fused_mamba_chunked(*_flip_t(args)), (1,))) <= 1e-5


def test_planted_off_by_one_reversal_is_caught():
    """A reversal that starts one row early (x[L - t] instead of x[L-1-t])
    fails the per-row flip check."""
    args = clip_inputs(2, 90, heads=2, head_dim=32, state=16, dtype=torch.float32, seed=14)
    lengths = torch.tensor([90, 41])
    out = R.fused_mamba_reversed(*args, lengths=lengths - 1)  # planted: one row short
    b, n = 1, 41
    ref = torch.flip(R.fused_mamba_chunked(*_flip_t(_truncate(args, b, n))), (1,))
    assert R.max_rel(out[b : b + 1, :n], ref) > 1e-3


# --- planted mistakes: each variant must be caught by the checks above -------


def _mutated_chunked(monkeypatch, **patches):
    # the chunked oracle runs in fp32, the FP64 forms in float64: a planted
    # mistake applies to fp32 arguments only, so the FP64 reference stays intact
    for name, fn in patches.items():
        orig = getattr(R, name)

        def dispatch(*a, _fn=fn, _orig=orig, **kw):
            return _fn(*a, **kw) if a[0].dtype == torch.float32 else _orig(*a, **kw)

        monkeypatch.setattr(R, name, dispatch)
    args = clip_inputs(1, 150, heads=2, head_dim=32, state=16, dtype=torch.float32, seed=31)
    return R.fused_mamba_chunked(*args), R.fused_mamba_attention_f64(*args)


def test_planted_no_halo_is_caught(monkeypatch):
    def no_halo(dt, trap):
        gamma = dt * torch.sigmoid(trap)
        return gamma, gamma

    out, ref = _mutated_chunked(monkeypatch, step_controls=no_halo)
    assert R.max_rel(out, ref) > 1e-3


def test_planted_rotation_sign_is_caught(monkeypatch):
    orig = R.rotate_pairs

    def wrong(x, cos, sin):
        return orig(x, cos, -sin)

    out, ref = _mutated_chunked(monkeypatch, rotate_pairs=wrong)
    assert R.max_rel(out, ref) > 1e-3


def test_planted_half_split_pairs_is_caught(monkeypatch):
    def half_split(x, cos, sin):
        h = x.shape[-1] // 2
        x0, x1 = x[..., :h], x[..., h:]
        return torch.cat((x0 * cos - x1 * sin, x0 * sin + x1 * cos), -1)

    out, ref = _mutated_chunked(monkeypatch, rotate_pairs=half_split)
    assert R.max_rel(out, ref) > 1e-3


def test_planted_missing_phase_carry_is_caught(monkeypatch):
    def no_carry(angles, dt, pairs, chunk=R.CHUNK, accumulate=None):
        vals = (torch.tanh(angles.float()) * math.pi) * dt.float().transpose(1, 2)[..., None]
        out = torch.cat([torch.cumsum(vals[:, c : c + chunk], 1) for c in range(0, vals.shape[1], chunk)], 1)
        return F.pad(out, (0, pairs - angles.shape[-1]))

    out, ref = _mutated_chunked(monkeypatch, phase_chunked=no_carry)
    assert R.max_rel(out, ref) > 1e-3


def test_planted_exp_instead_of_exp2_is_caught(monkeypatch):
    monkeypatch.setattr(R, "LOG2E", 1.0)
    out, ref = _mutated_chunked(monkeypatch)
    assert R.max_rel(out, ref) > 1e-3
