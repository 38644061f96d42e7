"""The HIP recurrence against the committed known-answer cases
(``tests/golden/recurrence_kat.npz``: float64 closed forms, no oracle in
between), for every kernel variant that takes the shape. bf16 q, k, v, z
(exact: the fixture values are bf16), fp32 controls and fp32 output.

Tolerances: the single step has no bf16 rounding point on its path (the skip
term is formed in fp32 from the unrotated operands), so max relative error
<= 1e-4; the linear-attention case goes through the reference's bf16
rounding of qr, kr, the scores and the state, so it is held to the
reference's own bound against FP64, rel-Frobenius < 0.012
(``tests/test_recurrence.py:86``), and so are the trapezoid-step cases
(``shift``, ``mixed_trap``, ``segmented``: trap = +-40, see
``tests/golden/make_golden.py``). Those also run backwards: the reversed
operands with ``reverse=True`` must give the reversed known answer. The
``segmented`` case has one (batch, head) unit, so the MFMA kernel takes its
chunk-parallel form with a segment boundary at t = 256."""

import pytest
import torch

from oracle.recurrence import max_rel, rel_fro
from test_golden_kat import load_case
from trifusion_amd.mamba_fused import fused_mamba, selected_variant

pytestmark = pytest.mark.gpu


TIME_AXIS = {0: 1, 1: 1, 2: 1, 3: 2, 4: 2, 5: 2, 8: 1, 10: 1}  # operand index -> time dim


@pytest.mark.parametrize("reverse", [False, True])
@pytest.mark.parametrize("variant", ["generic", "mfma", "pipe"])
@pytest.mark.parametrize("name", ["single_step", "linear_attention", "shift", "mixed_trap", "segmented", "mixed_trap_n64"])
def test_known_answers(name, variant, reverse):
    args, expected = load_case(name)
    if reverse:
        args = tuple(a.flip(TIME_AXIS[i]) if i in TIME_AXIS else a for i, a in enumerate(args))
        expected = expected.flip(1)
    dargs = tuple((a.to(torch.bfloat16) if i in (0, 1, 2, 10) else a).contiguous().to("cuda") for i, a in enumerate(args))
    try:
        selected_variant(*dargs, variant=variant)
    except ValueError:
        pytest.skip(f"{variant} kernel does not take this shape")
    print(f"case {name} variant={variant} reverse={reverse}", flush=True)
    out = torch.empty(dargs[2].shape, device="cuda", dtype=torch.float32)
    with torch.inference_mode():
        fused_mamba(*dargs, out=out, variant=variant, reverse=reverse)
    torch.cuda.synchronize()
    y = out.cpu().double()
    print(f"  max_rel={max_rel(y, expected):.3e} rel_fro={rel_fro(y, expected):.3e}", flush=True)
    if name == "single_step":
        assert max_rel(y, expected) <= 1e-4
    else:
        assert rel_fro(y, expected) < 0.012
