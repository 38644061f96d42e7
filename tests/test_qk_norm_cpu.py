"""Inputs of the fused B/C norm tests, and the oracle-side sensitivity of
their tolerance.

``norm_inputs`` gives raw B/C rows (bf16) whose RMS spans four decades with a
few rows below the norm's eps, and distinct q and k norm weights;
``normalised`` applies the oracle's ``rms_norm`` (pinned against
``torch.nn.functional.rms_norm`` in ``tests/test_oracle_elementwise.py``), the
reference's C/B norms (``src/trifusion_l4/mamba.py:56-57``). The GPU tests in
``tests/test_gpu_qk_norm.py`` hold the kernels' fused norms to the oracle run
on ``normalised`` inputs at ``MAX_REL``; the test here shows that the raw rows,
or swapped weights, miss that oracle by far more than ``MAX_REL``.
"""

import torch

from oracle.elementwise import rms_norm
from oracle.recurrence import fused_mamba_chunked, max_rel
from trifusion_amd.synthetic import clip_inputs

MAX_REL = 1e-3
EPS = 1e-5


def raw_rows(x, seed):
    """bf16 rows of ``x`` at per-row scales 10^U(-2, 2); 2% of rows at 1e-3
    (mean square ~1e-6, below eps)."""
    g = torch.Generator().manual_seed(seed)
    shape = x.shape[:-1] + (1,)
    scale = 10.0 ** (4 * torch.rand(shape, generator=g) - 2)
    tiny = torch.rand(shape, generator=g) < 0.02
    scale = torch.where(tiny, torch.full_like(scale, 1e-3), scale)
    return (x.float() * scale).to(torch.bfloat16)


def norm_inputs(b, t, h, n=64, p=64, r=None, seed=5):
    args = list(clip_inputs(b, t, heads=h, state=n, head_dim=p, rotary=r, seed=seed))
    args[0] = raw_rows(args[0], seed + 1)
    args[1] = raw_rows(args[1], seed + 2)
    g = torch.Generator().manual_seed(seed + 3)
    wq = 0.5 + torch.rand(n, generator=g)
    wk = 0.5 + torch.rand(n, generator=g)
    return tuple(args), wq, wk


def normalised(args, wq, wk):
    args = list(args)
    args[0] = rms_norm(args[0], wq, EPS)
    args[1] = rms_norm(args[1], wk, EPS)
    assert args[0].dtype == torch.bfloat16
    return tuple(args)


def test_unnormalised_rows_are_far_from_the_oracle():
    """The raw rows, or the weights swapped, give an oracle far outside the
    tolerance the fused kernels are held to."""
    args, wq, wk = norm_inputs(2, 300, 8)
    ref = fused_mamba_chunked(*normalised(args, wq, wk))
    assert max_rel(fused_mamba_chunked(*args), ref) > 50 * MAX_REL
    assert max_rel(fused_mamba_chunked(*normalised(args, wk, wq)), ref) > 10 * MAX_REL
