"""Variable-length batch with the channels folded into the batch (MI355X).

B = 32 rows padded to L = 400: rows 2i and 2i+1 are clip i's channel slots,
clip lengths ~ U{50..400}, channels ~ U{1, 2}; a mono clip's second slot has
length 0 and is fully masked (``src/trifusion_l4/model.py:174`` masks the
recurrence output with the frame mask). H = 16, P = 64, N = 64, bf16 inputs.

Checked for both recurrence kernels, forwards and with ``reverse=True``
(the backward direction of the bidirectional block):
* valid rows against the oracle (``fused_mamba_chunked`` with lengths, or
  ``fused_mamba_reversed``) within ``max|dy| / max|y| <= 1e-3``;
* every row past a row's length, and every row of a length-0 slot, exactly 0.

Also lengths 0 and 1 next to full rows on a small batch, and the masked mean
over the folded batch against the oracle (a length-0 slot divides 0 by 0 there,
as ``decoder.py:60-62`` does: NaN in both).
"""

import pytest
import torch

from oracle.elementwise import masked_mean as masked_mean_ref
from oracle.recurrence import fused_mamba_chunked, fused_mamba_reversed, max_rel
from trifusion_amd.masking import masked_mean
from trifusion_amd.mamba_fused import fused_mamba, selected_variant
from trifusion_amd.synthetic import channel_fold_lengths, clip_inputs

pytestmark = pytest.mark.gpu

DEV = "cuda"
MAX_REL = 1e-3


def run(args, variant, lengths, reverse):
    dargs = tuple(a.to(DEV) for a in args)
    out = torch.full(dargs[2].shape, float("nan"), device=DEV, dtype=torch.float32)
    try:
        selected_variant(*dargs, variant=variant)
    except ValueError:
        pytest.skip(f"{variant} kernel does not take this shape")
    with torch.inference_mode():
        fused_mamba(*dargs, out=out, variant=variant, lengths=lengths.to(DEV), reverse=reverse)
    torch.cuda.synchronize()
    return out.cpu()


def check(y, ref, lengths):
    assert torch.isfinite(y).all()
    err = max_rel(y, ref)
    print(f"  max_rel={err:.3e}", flush=True)
    assert err <= MAX_REL
    for i, n in enumerate(lengths.tolist()):
        assert torch.all(y[i, n:] == 0), f"row {i} (length {n}) has nonzero padded outputs"


@pytest.mark.parametrize("reverse", [False, True])
@pytest.mark.parametrize("variant", ["generic", "mfma", "pipe"])
def test_channel_fold_batch(variant, reverse):
    lengths, channels = channel_fold_lengths(16, 400, 50, seed=12)
    assert (lengths == 0).any() and (channels == 2).any()
    args = clip_inputs(32, 400, seed=13)
    print(f"case channel_fold variant={variant} reverse={reverse} lengths={lengths.tolist()}", flush=True)
    y = run(args, variant, lengths, reverse)
    if reverse:
        ref = fused_mamba_reversed(*args, lengths=lengths)
    else:
        ref = fused_mamba_chunked(*args, lengths=lengths)
    check(y, ref, lengths)


@pytest.mark.parametrize("reverse", [False, True])
@pytest.mark.parametrize("variant", ["generic", "mfma", "pipe"])
def test_lengths_zero_and_one(variant, reverse):
    lengths = torch.tensor([0, 1, 130, 0, 1, 64, 65, 130])
    args = clip_inputs(8, 130, heads=4, head_dim=64, state=64, seed=14)
    print(f"case lengths_zero_one variant={variant} reverse={reverse}", flush=True)
    y = run(args, variant, lengths, reverse)
    ref = fused_mamba_reversed(*args, lengths=lengths) if reverse else fused_mamba_chunked(*args, lengths=lengths)
    check(y, ref, lengths)
    # a length-1 row is the single-step closed form; forwards and backwards agree
    other = run(args, variant, lengths, not reverse)
    assert torch.equal(y[1, :1], other[1, :1])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_masked_mean_channel_fold(dtype):
    lengths, _ = channel_fold_lengths(16, 400, 50, seed=12)
    g = torch.Generator().manual_seed(15)
    x = torch.randn(32, 400, 512, generator=g).to(dtype)
    print(f"case masked_mean_channel_fold dtype={dtype}", flush=True)
    y = masked_mean(x.to(DEV), lengths.to(DEV)).cpu()
    ref = masked_mean_ref(x, lengths)
    assert torch.isnan(y[lengths == 0]).all()
    torch.testing.assert_close(y, ref, rtol=1e-5, atol=1e-6, equal_nan=True)
