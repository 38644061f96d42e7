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
CASES = ["single_step", "linear_attention"]


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
