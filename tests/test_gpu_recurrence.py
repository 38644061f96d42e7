"""Parity of the HIP fused recurrence against the CPU oracle (MI355X).

Tolerances:
* fp32 outputs vs the chunked oracle with the reference's bf16 rounding points:
  ``max|y - y_ref| / max|y_ref| <= 1e-3`` (the recurrence tolerance);
* bf16 outputs (the reference's own output dtype) vs the oracle's bf16 output:
  rel-Frobenius < 0.006 and ``assert_close(atol=0.04, rtol=0.02)`` as in
  ``tests/test_recurrence.py:44-47`` of the reference;
* vs the FP64 loop: rel-Frobenius < 0.012 (``tests/test_recurrence.py:86``).
"""

import pytest
import torch

from oracle.recurrence import fused_mamba_chunked, fused_mamba_f64, max_rel, rel_fro
from trifusion_amd.mamba_fused import fused_mamba, selected_variant
from trifusion_amd.synthetic import clip_inputs, clip_lengths, reference_test_inputs

pytestmark = pytest.mark.gpu

DEV = "cuda"
VARIANTS = ["generic", "mfma", "pipe"]
MAX_REL = 1e-3


def to_dev(args):
    return tuple(a.to(DEV) for a in args)


def run(args, variant, out_dtype=torch.float32, lengths=None):
    dargs = to_dev(args)
    v = dargs[2]
    out = torch.empty(v.shape, device=DEV, dtype=out_dtype)
    with torch.inference_mode():
        y = fused_mamba(*dargs, out=out, variant=variant, lengths=None if lengths is None else lengths.to(DEV))
    torch.cuda.synchronize()
    assert y is out
    return y.cpu()


def needs(variant, args):
    dargs = to_dev(args)
    try:
        selected_variant(*dargs, variant=variant)
    except ValueError:
        pytest.skip(f"{variant} kernel does not take this shape")


REF_SHAPES = [(1, 1, 4), (2, 26, 4), (1, 63, 32), (1, 64, 32), (2, 65, 4), (1, 255, 32), (1, 1501, 32)]


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("batch,time,heads", REF_SHAPES)
def test_reference_shapes(variant, batch, time, heads):
    """The reference test's shapes and strided operands (N=128, P=64, R=32)."""
    args = reference_test_inputs(batch, time, heads)
    needs(variant, args)
    print(f"case variant={variant} B={batch} T={time} H={heads}", flush=True)
    ref = fused_mamba_chunked(*args)
    y = run(args, variant)
    assert torch.isfinite(y).all()
    print(f"  max_rel={max_rel(y, ref):.3e}", flush=True)
    assert max_rel(y, ref) <= MAX_REL
    yb = run(args, variant, out_dtype=torch.bfloat16)
    refb = ref.to(torch.bfloat16)
    assert rel_fro(yb, refb) < 0.006
    torch.testing.assert_close(yb.float(), refb.float(), atol=0.04, rtol=0.02)


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("case", ["clip", "varlen_reverse", "long"])
def test_bf16_output_is_rounded_fp32_output(variant, case):
    """The bf16 output path (its own stores) holds exactly the fp32 output
    rounded to nearest even, row by row, including rows past the lengths."""
    b, t, lens, rev = {"clip": (4, 400, None, False), "varlen_reverse": (3, 400, (400, 213, 0), True),
                       "long": (1, 3000, None, False)}[case]
    args = clip_inputs(b, t, heads=8, rotary=16, seed=23)
    needs(variant, args)
    dargs = to_dev(args)
    lengths = None if lens is None else torch.tensor(lens, dtype=torch.int64, device=DEV)
    print(f"case {case} variant={variant}", flush=True)
    with torch.inference_mode():
        y32 = fused_mamba(*dargs, out=torch.empty(dargs[2].shape, device=DEV), variant=variant, lengths=lengths,
                          reverse=rev)
        y16 = fused_mamba(*dargs, out=torch.empty(dargs[2].shape, device=DEV, dtype=torch.bfloat16), variant=variant,
                          lengths=lengths, reverse=rev)
    torch.cuda.synchronize()
    assert torch.equal(y16.cpu(), y32.cpu().to(torch.bfloat16))


@pytest.mark.parametrize("variant", VARIANTS)
def test_short_against_f64(variant):
    args = reference_test_inputs(1, 17, 4)
    needs(variant, args)
    y = run(args, variant, out_dtype=torch.bfloat16)
    assert rel_fro(y, fused_mamba_f64(*args)) < 0.012


CLIP_CASES = {
    # name: (B, T, H, P, N, R, Hq, dtype)
    "cpu_fp32_b2_l256_h4_p32_n16": (2, 256, 4, 32, 16, 4, 1, torch.float32),
    "clip_b16_l400_h16_p64_n64": (16, 400, 16, 64, 64, 16, 1, torch.bfloat16),
    "long_b1_l7200_h16_p64_n64": (1, 7200, 16, 64, 64, 16, 1, torch.bfloat16),
    "hq_equals_h": (2, 200, 8, 64, 64, 16, 8, torch.bfloat16),
    "n128_p64": (2, 150, 4, 64, 128, 32, 1, torch.bfloat16),
    "model_b16_l101_h32_p64_n128": (16, 101, 32, 64, 128, 32, 1, torch.bfloat16),
    "n32_p32": (3, 130, 4, 32, 32, 8, 2, torch.bfloat16),
    "n16_p32_bf16": (2, 100, 4, 32, 16, 4, 1, torch.bfloat16),
}


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("name", list(CLIP_CASES))
def test_clip_workloads(variant, name):
    b, t, h, p, n, r, hq, dtype = CLIP_CASES[name]
    args = clip_inputs(b, t, heads=h, head_dim=p, state=n, rotary=r, qk_heads=hq, dtype=dtype, seed=1)
    needs(variant, args)
    print(f"case variant={variant} {name}", flush=True)
    ref = fused_mamba_chunked(*args)
    y = run(args, variant)
    assert torch.isfinite(y).all()
    err = max_rel(y, ref)
    print(f"  max_rel={err:.3e} rel_fro={rel_fro(y, ref):.3e}", flush=True)
    assert err <= MAX_REL


@pytest.mark.parametrize("variant", VARIANTS)
def test_variable_length_batch(variant):
    """B=32 padded to L=400, lengths U{50..400}; padded rows must be exactly 0."""
    b, t = 32, 400
    args = clip_inputs(b, t, seed=3)
    needs(variant, args)
    lengths = clip_lengths(b, t, 50, seed=4)
    ref = fused_mamba_chunked(*args, lengths=lengths)
    y = run(args, variant, lengths=lengths)
    assert max_rel(y, ref) <= MAX_REL
    for i, n in enumerate(lengths.tolist()):
        assert torch.all(y[i, n:] == 0)
    # without lengths the valid rows are identical (causality)
    y_full = run(args, variant)
    for i, n in enumerate(lengths.tolist()):
        assert torch.equal(y_full[i, :n], y[i, :n])


@pytest.mark.parametrize("variant", ["pipe"])
def test_variable_length_batch_64_rows_with_ties(variant):
    """B=64 x 8 heads (512 units) with many equal lengths and zero lengths: the
    pipelined walk deals batch rows longest first; every unit must still be
    walked exactly once (oracle parity, padded rows exactly 0)."""
    b, t = 64, 200
    args = clip_inputs(b, t, heads=8, seed=13)
    needs(variant, args)
    base = [0, 1, 64, 65, 128, 200, 137, 63]
    lengths = torch.tensor([base[i % 8] for i in range(b)], dtype=torch.int64)
    print(f"case b64 ties variant={variant}", flush=True)
    ref = fused_mamba_chunked(*args, lengths=lengths)
    y = run(args, variant, lengths=lengths)
    assert max_rel(y, ref) <= MAX_REL
    for i, n in enumerate(lengths.tolist()):
        assert torch.all(y[i, n:] == 0)


@pytest.mark.parametrize("variant", VARIANTS)
def test_model_layout_strides(variant):
    """Operands as the Mamba block passes them: v/z/trap/ddt are column slices
    of one bf16 projection (trap a transposed view), angles a stride-0 expand
    over heads, adt/dt contiguous fp32 (reference src/trifusion_l4/mamba.py:40-83)."""
    g = torch.Generator().manual_seed(5)
    b, t, h, p, n, r = 2, 190, 16, 64, 64, 16
    width = 2 * h * p + 2 * n + 3 * h + r
    proj = (torch.randn(b, t, width, generator=g) * 0.5).to(torch.bfloat16)
    z = proj[..., : h * p].reshape(b, t, h, p)
    v = proj[..., h * p : 2 * h * p].reshape(b, t, h, p)
    k = proj[..., 2 * h * p : 2 * h * p + n].reshape(b, t, 1, n)
    q = proj[..., 2 * h * p + n : 2 * h * p + 2 * n].reshape(b, t, 1, n)
    base = 2 * h * p + 2 * n
    trap = proj[..., base + 2 * h : base + 3 * h].transpose(1, 2)
    angles = proj[..., base + 3 * h :].unsqueeze(2).expand(b, t, h, r)
    dt = torch.nn.functional.softplus(torch.randn(b, h, t, generator=g) - 2)
    adt = -dt * (torch.rand(b, h, t, generator=g) + 0.2)
    qb = 1 + 0.1 * torch.randn(h, n, generator=g)
    kb = 1 + 0.1 * torch.randn(h, n, generator=g)
    d = torch.ones(h)
    args = (q, k, v, adt, dt, trap, qb, kb, angles, d, z)
    needs(variant, args)
    ref = fused_mamba_chunked(*args)
    # device copies keep the strided layout: move the projection once, re-slice
    dproj = proj.to(DEV)
    dargs = (
        dproj[..., 2 * h * p + n : 2 * h * p + 2 * n].reshape(b, t, 1, n),
        dproj[..., 2 * h * p : 2 * h * p + n].reshape(b, t, 1, n),
        dproj[..., h * p : 2 * h * p].reshape(b, t, h, p),
        adt.to(DEV),
        dt.to(DEV),
        dproj[..., base + 2 * h : base + 3 * h].transpose(1, 2),
        qb.to(DEV),
        kb.to(DEV),
        dproj[..., base + 3 * h :].unsqueeze(2).expand(b, t, h, r),
        d.to(DEV),
        dproj[..., : h * p].reshape(b, t, h, p),
    )
    assert dargs[8].stride(2) == 0 and not dargs[2].is_contiguous()
    out = torch.empty((b, t, h, p), device=DEV, dtype=torch.float32)
    with torch.inference_mode():
        fused_mamba(*dargs, out=out, variant=variant)
    torch.cuda.synchronize()
    assert max_rel(out.cpu(), ref) <= MAX_REL


def test_default_output_matches_reference_contract():
    args = to_dev(clip_inputs(2, 70, heads=4, head_dim=64, state=64, seed=6))
    with torch.inference_mode():
        y = fused_mamba(*args)
    assert y.dtype == torch.bfloat16 and y.is_contiguous() and y.shape == args[2].shape


def test_unsupported_shapes_raise_value_error():
    args = list(to_dev(clip_inputs(1, 10, heads=2, head_dim=48, state=64, seed=1)))
    with pytest.raises(ValueError):
        fused_mamba(*args)
    args = list(to_dev(clip_inputs(1, 10, heads=2, head_dim=64, state=64, rotary=40, seed=1)))
    with pytest.raises(ValueError):
        fused_mamba(*args)


def test_empty_inputs():
    for b, t in ((0, 10), (2, 0)):
        args = to_dev(clip_inputs(b, t, heads=2, head_dim=64, state=64, seed=1))
        with torch.inference_mode():
            y = fused_mamba(*args)
        torch.cuda.synchronize()
        assert y.shape == args[2].shape


@pytest.mark.parametrize(
    "b,t,h,n,r,kernel",
    [
        (16, 400, 16, 64, 16, "pipe"),  # clip workload: pipelined walk
        (16, 101, 32, 128, 32, "mfma"),  # the model's bidirectional shape (N = 128)
        (1, 7200, 16, 64, 16, "pipe"),  # long clip: pipelined kernel, cut into time segments
        (2, 64, 16, 64, 16, "pipe"),
        (2, 256, 4, 16, 4, "mfma"),  # N = 16: the N = 32 kernel on zero-padded channels
    ],
)
def test_auto_selects_matrix_core_kernel(b, t, h, n, r, kernel):
    """The clip workload, the model's bidirectional shape and the long clip must
    take a matrix-core kernel (the generic one is ~70x slower), and the one
    meant for the shape."""
    args = to_dev(clip_inputs(b, t, heads=h, head_dim=64, state=n, rotary=r, seed=1))
    assert selected_variant(*args) == kernel
    assert selected_variant(*args, reverse=True) == kernel
