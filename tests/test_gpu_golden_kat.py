"""The HIP recurrence against the committed known-answer cases
(``tests/golden/recurrence_kat.npz``: float64 closed forms, no oracle in
between), for every kernel variant that takes the shape. bf16 q, k, v, z
(exact: the fixture values are bf16), fp32 controls and fp32 output.

Tolerances: the single step has no bf16 rounding point on its path (the skip
term is formed in fp32 from the unrotated operands), so max relative error
<= 1e-4; the linear-attention case goes through the reference's bf16
rounding of qr, kr, the scores and the state, so it is held to the
reference's own bound against FP64, rel-Frobenius < 0.012
(``tests/test_recurrence.py:86``)."""

import pytest
import torch

from oracle.recurrence import max_rel, rel_fro
from test_golden_kat import load_case
from trifusion_amd.mamba_fused import fused_mamba, selected_variant

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("variant", ["generic", "mfma"])
@pytest.mark.parametrize("name", ["single_step", "linear_attention"])
def test_known_answers(name, variant):
    args, expected = load_case(name)
    dargs = tuple((a.to(torch.bfloat16) if i in (0, 1, 2, 10) else a).to("cuda") for i, a in enumerate(args))
    try:
        selected_variant(*dargs, variant=variant)
    except ValueError:
        pytest.skip(f"{variant} kernel does not take this shape")
    print(f"case {name} variant={variant}", flush=True)
    out = torch.empty(dargs[2].shape, device="cuda", dtype=torch.float32)
    with torch.inference_mode():
        fused_mamba(*dargs, out=out, variant=variant)
    torch.cuda.synchronize()
    y = out.cpu().double()
    print(f"  max_rel={max_rel(y, expected):.3e} rel_fro={rel_fro(y, expected):.3e}", flush=True)
    if name == "single_step":
        assert max_rel(y, expected) <= 1e-4
    else:
        assert rel_fro(y, expected) < 0.012
