"""The B/C RMSNorm fused into the recurrence (``q_norm=``/``k_norm=``).

The reference normalises B and C in the Mamba block before the recurrence
(``src/trifusion_l4/mamba.py:56-57``): ``x * rsqrt(mean(x^2) + eps) * w``
rounded to bf16 (``src/trifusion_l4/kernels/__init__.py:10-12``). The fused
form hands the kernels the raw columns and the weights. Each kernel variant is
held to the oracle run on rows the oracle's own ``rms_norm`` normalised, at
``max|y - y_ref| / max|y_ref| <= 1e-3``: one workgroup per unit and the
chunk-parallel form, forwards and reversed over valid prefixes, N = 16 .. 128.
The raw rows' RMS spans four decades, a few rows sit near ``eps``, and q and k
have different weights, so a skipped norm, swapped weights or a dropped eps
each fail by far more than the tolerance
(``tests/test_qk_norm_cpu.py`` shows it on the oracle). The Mamba block with
fused norms is also compared with the same block running the separate norm
launch.
"""

import ctypes

import pytest
import torch

from oracle.recurrence import fused_mamba_chunked, fused_mamba_reversed, max_rel
from test_qk_norm_cpu import EPS, MAX_REL, norm_inputs, normalised
from trifusion_amd import _lib
from trifusion_amd.mamba_fused import build_args, fused_mamba, selected_variant
from trifusion_amd.synthetic import clip_lengths

pytestmark = pytest.mark.gpu

DEV = "cuda"


CASES = {
    # name: (B, T, H, N, P, R, lengths low bound or None)
    "clip_b2_l300_h8": (2, 300, 8, 64, 64, None, None),
    "varlen_b3_l260_h4": (3, 260, 4, 64, 64, None, 70),
    "segmented_b1_l3000_h8": (1, 3000, 8, 64, 64, None, None),
    "n128_b2_l200_h4": (2, 200, 4, 128, 64, 32, None),
    "n32_b2_l150_h4": (2, 150, 4, 32, 32, 8, None),
    "n16_b2_l130_h4": (2, 130, 4, 16, 32, 4, None),
}


@pytest.mark.parametrize("reverse", [False, True], ids=["forward", "reverse"])
@pytest.mark.parametrize("variant", ["generic", "mfma", "pipe"])
@pytest.mark.parametrize("case", sorted(CASES))
def test_fused_norms_match_oracle(case, variant, reverse):
    b, t, h, n, p, r, low = CASES[case]
    args, wq, wk = norm_inputs(b, t, h, n, p, r)
    dargs = tuple(x.to(DEV) for x in args)
    lengths = None if low is None else clip_lengths(b, t, low, seed=9)
    dl = None if lengths is None else lengths.to(DEV)
    dwq, dwk = wq.to(DEV), wk.to(DEV)
    try:
        selected_variant(*dargs, variant=variant, lengths=dl, q_norm=dwq, k_norm=dwk)
    except ValueError:
        pytest.skip(f"{variant} kernel does not take this shape")
    print(f"case {case} variant={variant} reverse={reverse}", flush=True)
    out = torch.empty(dargs[2].shape, device=DEV, dtype=torch.float32)
    if case.startswith("segmented") and variant != "generic":
        a = build_args(*dargs, out, dl, variant, reverse, q_norm=dwq, k_norm=dwk)
        assert _lib.load().tf_fused_mamba_workspace_size(ctypes.byref(a)) > 0, "not the chunk-parallel path"
    with torch.inference_mode():
        fused_mamba(*dargs, out=out, lengths=dl, variant=variant, reverse=reverse, q_norm=dwq, k_norm=dwk, norm_eps=EPS)
    torch.cuda.synchronize()
    y = out.cpu()
    ref_args = normalised(args, wq, wk)
    ref = fused_mamba_reversed(*ref_args, lengths=lengths) if reverse else fused_mamba_chunked(*ref_args, lengths=lengths)
    assert torch.isfinite(y).all()
    err = max_rel(y, ref)
    print(f"  max_rel={err:.3e}", flush=True)
    assert err <= MAX_REL
    # the same kernel on rows normalised beforehand: the fused norm only
    # changes where an fp32 sum of squares rounds differently
    with torch.inference_mode():
        pre = fused_mamba(*tuple(x.to(DEV) for x in ref_args), out=torch.empty_like(out), lengths=dl,
                          variant=variant, reverse=reverse)
    torch.cuda.synchronize()
    assert max_rel(y, pre.cpu()) <= MAX_REL


def test_block_fused_norms_match_separate_norm_launch():
    """Mamba3Inference.mix with the norms fused (default) and with the
    separate rms_pair launch, on one projection."""
    from trifusion_amd.mamba import Mamba3Inference
    from trifusion_amd.model import ModelConfig

    torch.manual_seed(3)
    cfg = ModelConfig()
    block = Mamba3Inference(cfg).to(DEV).eval()
    with torch.no_grad():
        block.B_norm.weight.uniform_(0.5, 1.5)
        block.C_norm.weight.uniform_(0.5, 1.5)
    width = block.in_proj.out_features
    p = (torch.randn(4, 400, width, device=DEV) * 2).to(torch.bfloat16)
    lengths = torch.tensor([400, 311, 64, 250], device=DEV)
    print("case block fused vs separate norms", flush=True)
    with torch.inference_mode():
        assert block._fusable_norms()
        fused = block.mix(p, lengths).float()
        block.fuse_norms = False
        separate = block.mix(p, lengths).float()
    torch.cuda.synchronize()
    err = max_rel(fused.cpu(), separate.cpu())
    print(f"  max_rel={err:.3e}", flush=True)
    assert err <= MAX_REL
