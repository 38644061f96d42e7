"""Recurrence parity where the signed decay ``adt`` is positive on some steps.

The reference weights the intra-chunk scores by ``2^min(cs_t - cs_u, 0)``
(``src/trifusion_l4/mamba_fused.py:144``): where ``adt > 0`` somewhere between
u and t inside a chunk, the weight is capped at 1. The inter-chunk term and the
state update carry no clamp (``:143, 150-152``). ``fused_mamba`` accepts any
sign of ``adt`` (``docs/api.md:73-74``), so every kernel is held to the oracle
on inputs where about a third of the steps grow instead of decay: all three
variants, forwards and ``reverse=True``, one workgroup per unit and the
chunk-parallel form, at ``max|y - y_ref| / max|y_ref| <= 1e-3``.
``tests/test_oracle_recurrence.py::test_chunked_clamps_positive_decay_within_chunks``
pins the oracle's clamp against an FP64 closed form; here the serial case
checks, on its own inputs, that dropping the clamp moves the FP64 closed form
by far more than the tolerance.

The positive steps are kept small (a fifth of the steps, a quarter of the
decay's size): where the state grows for long stretches, the reference's bf16
rounding points amplify rounding (with a third of the steps at half size over
3000 steps, the bf16-rounded oracle itself is 3.5e-3 of max|y| from the
unrounded FP64 form, and any two valid implementations drift apart by ~1e-3).
"""

import ctypes

import pytest
import torch

from oracle.recurrence import CHUNK, fused_mamba_attention_f64, fused_mamba_chunked, fused_mamba_reversed, max_rel
from trifusion_amd import _lib
from trifusion_amd.mamba_fused import build_args, fused_mamba, selected_variant
from trifusion_amd.synthetic import clip_inputs

pytestmark = pytest.mark.gpu

DEV = "cuda"
MAX_REL = 1e-3


def positive_decay_inputs(b, t, h, seed):
    """Clip operands with the sign of ``adt`` flipped (and quartered) on ~20% of steps."""
    args = list(clip_inputs(b, t, heads=h, seed=seed))
    g = torch.Generator().manual_seed(seed + 1000)
    adt = args[3]
    flip = torch.rand(adt.shape, generator=g) < 0.2
    args[3] = torch.where(flip, -0.25 * adt, adt)
    assert (args[3] > 0).any()
    return tuple(args)


def _workspace_bytes(dargs, out, variant):
    a = build_args(*dargs, out, None, variant)
    return _lib.load().tf_fused_mamba_workspace_size(ctypes.byref(a))


CASES = {
    # name: (B, T, H, chunk-parallel expected)
    "serial_b2_l400_h4": (2, 400, 4, False),
    "segmented_b1_l1500_h8": (1, 1500, 8, True),
}


@pytest.mark.parametrize("reverse", [False, True], ids=["forward", "reverse"])
@pytest.mark.parametrize("variant", ["generic", "mfma", "pipe"])
@pytest.mark.parametrize("case", sorted(CASES))
def test_positive_decay_steps_match_oracle(case, variant, reverse):
    b, t, h, segmented = CASES[case]
    args = positive_decay_inputs(b, t, h, seed=41)
    dargs = tuple(x.to(DEV) for x in args)
    try:
        selected_variant(*dargs, variant=variant)
    except ValueError:
        pytest.skip(f"{variant} kernel does not take this shape")
    out = torch.empty(dargs[2].shape, device=DEV, dtype=torch.float32)
    if segmented:
        if variant == "generic":
            pytest.skip("the generic kernel has no chunk-parallel form")
        assert _workspace_bytes(dargs, out, variant) > 0, "shape does not take the chunk-parallel path"
    print(f"case {case} variant={variant} reverse={reverse}", flush=True)
    with torch.inference_mode():
        fused_mamba(*dargs, out=out, variant=variant, reverse=reverse)
    torch.cuda.synchronize()
    y = out.cpu()
    ref = fused_mamba_reversed(*args) if reverse else fused_mamba_chunked(*args)
    assert torch.isfinite(y).all()
    err = max_rel(y, ref)
    print(f"  max_rel={err:.3e}", flush=True)
    assert err <= MAX_REL


def test_positive_decay_inputs_exercise_the_clamp():
    """On the serial case's inputs the FP64 closed form with the intra-chunk
    clamp and the one without differ by far more than the tolerance, so a
    kernel without the clamp fails the parity test above."""
    b, t, h, _ = CASES["serial_b2_l400_h4"]
    args = positive_decay_inputs(b, t, h, seed=41)
    clamped = fused_mamba_attention_f64(*args, clamp_chunk=CHUNK)
    unclamped = fused_mamba_attention_f64(*args)
    assert max_rel(unclamped, clamped) > 20 * MAX_REL
