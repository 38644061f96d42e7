"""The oracle against the committed known-answer cases (``tests/golden/``),
whose expected outputs come from float64 closed forms written without the
oracle (``tests/golden/make_golden.py``)."""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import recurrence as R

KAT = Path(__file__).parent / "golden" / "recurrence_kat.npz"
ORDER = ("q", "k", "v", "adt", "dt", "trap", "qb", "kb", "angles", "d", "z")
CASES = ["single_step", "linear_attention", "shift", "mixed_trap", "segmented", "mixed_trap_n64"]


def load_case(name):
    """``(args, expected)``: the fused_mamba operands in reference order (float32;
    q, k, v, z hold bf16-exact values) and the float64 expected output."""
    with np.load(KAT, allow_pickle=False) as f:
        args = tuple(torch.from_numpy(np.array(f[f"{name}/{key}"])) for key in ORDER)
        expected = torch.from_numpy(np.array(f[f"{name}/expected"]))
    return args, expected


@pytest.mark.parametrize("name", CASES)
def test_fixture_inputs_are_bf16_exact(name):
    args, _ = load_case(name)
    for i in (0, 1, 2, 10):
        assert torch.equal(args[i].to(torch.bfloat16).float(), args[i])


@pytest.mark.parametrize("name", CASES)
def test_oracle_matches_known_answers(name):
    args, expected = load_case(name)
    assert R.max_rel(R.fused_mamba_f64(*(a.double() for a in args)), expected) < 1e-10
    assert R.max_rel(R.fused_mamba_chunked(*args), expected) < 1e-5
    # with the reference's bf16 rounding points: within its own FP64 bound
    bf = tuple(a.to(torch.bfloat16) if i in (0, 1, 2, 10) else a for i, a in enumerate(args))
    assert R.rel_fro(R.fused_mamba_chunked(*bf, out_dtype=torch.float32), expected) < 0.012


HALO_CASES = ["shift", "mixed_trap", "segmented", "mixed_trap_n64"]


def _sig(trap):
    return torch.sigmoid(trap)


# Plausible ways to get the trapezoid step wrong (mamba_fused.py:96-101). Each
# replaces the oracle's step_controls; the known answers must reject every one.
PLANTED_STEPS = {
    "sigma_for_one_minus_sigma": lambda dt, trap: dt * _sig(trap)
    + torch.nn.functional.pad(dt[..., 1:], (0, 1)) * torch.nn.functional.pad(_sig(trap[..., 1:]), (0, 1)),
    "dt_t_for_dt_t_plus_1": lambda dt, trap: dt * _sig(trap)
    + dt * (1 - torch.nn.functional.pad(_sig(trap[..., 1:]), (0, 1))),
    "sigma_t_for_sigma_t_plus_1": lambda dt, trap: dt * _sig(trap)
    + torch.nn.functional.pad(dt[..., 1:], (0, 1)) * (1 - _sig(trap)),
    "no_halo": lambda dt, trap: dt * _sig(trap),
}


@pytest.mark.parametrize("mistake", sorted(PLANTED_STEPS))
def test_planted_trapezoid_mistakes_are_caught(mistake, monkeypatch):
    wrong = PLANTED_STEPS[mistake]
    original = R.step_controls
    monkeypatch.setattr(R, "step_controls", lambda dt, trap: (original(dt, trap)[0], wrong(dt, trap)))
    worst = 0.0
    for name in HALO_CASES:
        args, expected = load_case(name)
        worst = max(worst, R.max_rel(R.fused_mamba_f64(*(a.double() for a in args)), expected))
    assert worst > 0.05, f"{mistake} passed the known answers (max_rel {worst:.2e})"


def test_last_step_is_gamma():
    # the step past the sequence loads 0 for dt and trap, so s_{T-1} = gamma_{T-1}
    # exactly, whatever trap_{T-1} is (mamba_fused.py:97,99)
    g = torch.Generator().manual_seed(9)
    dt = torch.rand(2, 3, 7, generator=g, dtype=torch.float64) + 0.5
    trap = torch.randn(2, 3, 7, generator=g, dtype=torch.float64) * 3
    gamma, s = R.step_controls(dt, trap)
    assert torch.equal(s[..., -1], gamma[..., -1])
    assert torch.equal(gamma, dt * torch.sigmoid(trap))
    # and interior steps take the next step's (dt, 1 - sigmoid(trap)) exactly
    assert torch.allclose(s[..., :-1] - gamma[..., :-1], dt[..., 1:] * torch.sigmoid(-trap[..., 1:]), rtol=1e-14)
