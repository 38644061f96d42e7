"""Backward direction and fused controls of the recurrence, and the kernels of
the bidirectional block (MI355X).

* ``reverse=True`` against the oracle's reversed form (every time-indexed
  operand's valid prefix reversed, the chunked oracle run, the output reversed
  back: the reference's ``reverse_valid(fused_mamba(reverse_valid(x)))``,
  ``src/trifusion_l4/model.py:174-179``), at the recurrence tolerance
  ``max|y - y_ref| / max|y_ref| <= 1e-3``, on ragged lengths, N = 16..128,
  Hq > 1, full-length rows, and on the chunk-parallel form;
* raw controls (``dt_bias=``) against the oracle's ``mamba_controls`` followed
  by the chunked oracle, and against the separate HIP controls kernel followed
  by the recurrence (the same per-step formula: agreement to 1e-6);
* ``reverse_valid`` bit-exact against the oracle on every copy width;
* ``mean_norm`` against the oracle within 1e-5 relative.
"""

import ctypes

import pytest
import torch

from oracle import elementwise as E
from oracle.recurrence import fused_mamba_chunked, fused_mamba_reversed, max_rel
from trifusion_amd import _lib
from trifusion_amd.kernels import reverse_valid
from trifusion_amd.kernels.buffers import mamba_controls
from trifusion_amd.kernels.native import mean_norm
from trifusion_amd.mamba_fused import build_args, fused_mamba, selected_variant
from trifusion_amd.synthetic import clip_inputs, clip_lengths

pytestmark = pytest.mark.gpu

DEV = "cuda"
MAX_REL = 1e-3
VARIANTS = ["generic", "mfma", "pipe"]


def to_dev(args):
    return tuple(a.to(DEV) for a in args)


def needs(variant, dargs, **kw):
    try:
        selected_variant(*dargs, variant=variant, **kw)
    except ValueError:
        pytest.skip(f"{variant} kernel does not take this shape")


def run(dargs, variant, lengths=None, **kw):
    out = torch.empty(dargs[2].shape, device=DEV, dtype=torch.float32)
    with torch.inference_mode():
        fused_mamba(*dargs, out=out, variant=variant, lengths=lengths, **kw)
    torch.cuda.synchronize()
    return out.cpu()


REVERSE_CASES = {
    # name: (B, T, H, P, N, R, Hq, lengths)
    "b3_l150_h4_p64_n64_ragged": (3, 150, 4, 64, 64, 16, 1, (150, 77, 1)),
    "b2_l200_h4_p32_n32_hq2": (2, 200, 4, 32, 32, 8, 2, (133, 64)),
    "b2_l130_h2_p64_n128": (2, 130, 2, 64, 128, 32, 1, (130, 65)),
    "b2_l100_h4_p32_n16": (2, 100, 4, 32, 16, 4, 1, (100, 37)),
    "b2_l90_h4_wide_rotary": (2, 90, 4, 64, 64, 24, 1, (90, 3)),
    "b2_l90_no_lengths": (2, 90, 4, 64, 64, 16, 1, None),
    "b16_l400_h16_varlen": (16, 400, 16, 64, 64, 16, 1, "random"),
    # the TriFusion block's shape: 512 units, more than one workgroup round
    "b16_l101_h32_p64_n128_varlen": (16, 101, 32, 64, 128, 32, 1, "random"),
}


def _lengths(spec, b, t):
    if spec is None:
        return None
    if spec == "random":
        return clip_lengths(b, t, 50, seed=21)
    return torch.tensor(spec, dtype=torch.int64)


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("name", list(REVERSE_CASES))
def test_reverse_matches_oracle(variant, name):
    b, t, h, p, n, r, hq, spec = REVERSE_CASES[name]
    args = clip_inputs(b, t, heads=h, head_dim=p, state=n, rotary=r, qk_heads=hq, seed=17)
    lengths = _lengths(spec, b, t)
    dargs = to_dev(args)
    needs(variant, dargs)
    print(f"case variant={variant} {name}", flush=True)
    ref = fused_mamba_reversed(*args, lengths=lengths)
    y = run(dargs, variant, None if lengths is None else lengths.to(DEV), reverse=True)
    assert torch.isfinite(y).all()
    err = max_rel(y, ref)
    print(f"  max_rel={err:.3e}", flush=True)
    assert err <= MAX_REL
    if lengths is not None:
        for i, m in enumerate(lengths.tolist()):
            assert not y[i, m:].any()


def test_reverse_mfma_matches_generic_kernel():
    """The two kernels are independent implementations of the reversed walk."""
    args = clip_inputs(3, 200, heads=4, head_dim=64, state=64, seed=18)
    lengths = torch.tensor([200, 131, 64], device=DEV)
    dargs = to_dev(args)
    a = run(dargs, "mfma", lengths, reverse=True)
    g = run(dargs, "generic", lengths, reverse=True)
    assert max_rel(a, g) <= MAX_REL


def _serial(dargs, out, lengths, **kw):
    a = build_args(*dargs, out, lengths, "mfma", **kw)
    lib = _lib.load()
    _lib.check(lib.tf_fused_mamba(ctypes.byref(a), _lib.stream_of(out)), "fused_mamba")
    torch.cuda.synchronize()
    return out.cpu()


@pytest.mark.parametrize("raw", [False, True])
def test_reverse_chunk_parallel_matches_oracle_and_serial(raw):
    """Long sequence over few units: the segmented form reversed (phase sums,
    summaries and outputs all read the reversed rows) equals the oracle and the
    serial walk."""
    b, t, h = 2, 1500, 4
    args = clip_inputs(b, t, heads=h, head_dim=64, state=64, seed=19)
    lengths = torch.tensor([1337, 700], dtype=torch.int64)
    dargs = to_dev(args)
    dl = lengths.to(DEV)
    kw = {"reverse": True}
    ref_args = args
    if raw:
        proj, dt_bias = _raw_projection(b, t, h, seed=20)
        adt_r, dt_r = E.mamba_controls(proj[..., h : 2 * h], proj[..., :h], dt_bias)
        ref_args = args[:3] + (adt_r, dt_r) + args[5:]
        dp = proj.to(DEV)
        dargs = dargs[:3] + (dp[..., h : 2 * h].transpose(1, 2), dp[..., :h].transpose(1, 2)) + dargs[5:]
        kw["dt_bias"] = dt_bias.to(DEV)
    out = torch.empty(dargs[2].shape, device=DEV, dtype=torch.float32)
    ws = _lib.load().tf_fused_mamba_workspace_size(ctypes.byref(build_args(*dargs, out, dl, "mfma", **kw)))
    assert ws > 0, "shape expected to take the chunk-parallel form"
    y = run(dargs, "mfma", dl, **kw)
    ser = _serial(dargs, torch.empty_like(out), dl, **kw)
    ref = fused_mamba_reversed(*ref_args, lengths=lengths)
    print(f"raw={raw} vs oracle {max_rel(y, ref):.3e} vs serial {max_rel(y, ser):.3e}", flush=True)
    assert max_rel(y, ref) <= MAX_REL
    assert max_rel(y, ser) <= MAX_REL
    for i, m in enumerate(lengths.tolist()):
        assert not y[i, m:].any()


def _raw_projection(b, t, h, seed, spikes=False):
    """In-projection columns [ddt | a | trap] as bf16 [B, T, 3H + 5] (five spare
    columns so the views are strided) and an fp32 dt_bias around the reference
    init of -4; a covers both signs of the decay control. ``spikes`` pushes a
    few ddt entries past the softplus threshold (dt = ddt + bias above 20)."""
    g = torch.Generator().manual_seed(seed)
    proj = torch.randn(b, t, 3 * h + 5, generator=g) * 1.5
    if spikes:
        proj[:, ::37, 0] = 30.0
    dt_bias = torch.randn(h, generator=g) - 4.0
    return proj.to(torch.bfloat16), dt_bias


RAW_CASES = {
    # name: (B, T, H, P, N, R, Hq, lengths)
    "b4_l400_h16_p64_n64": (4, 400, 16, 64, 64, 16, 1, None),
    "b3_l150_h4_p32_n32_ragged": (3, 150, 4, 32, 32, 8, 1, (150, 90, 5)),
    "b2_l130_h2_p64_n128": (2, 130, 2, 64, 128, 32, 1, None),
    "b2_l100_h4_p32_n16": (2, 100, 4, 32, 16, 4, 1, None),
    "b16_l101_h32_p64_n128": (16, 101, 32, 64, 128, 32, 1, None),
}


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("name", list(RAW_CASES))
@pytest.mark.parametrize("reverse", [False, True])
def test_raw_controls_match_oracle_and_separate_kernel(variant, name, reverse):
    _raw_case(variant, name, reverse, spikes=False)


@pytest.mark.parametrize("variant", VARIANTS)
def test_raw_controls_softplus_threshold(variant):
    """Steps with ddt + bias > 20 take dt = ddt + bias; their outputs dwarf the
    rest, so the separate-kernel agreement (1e-6) is the sharp check here."""
    _raw_case(variant, "b4_l400_h16_p64_n64", False, spikes=True)


def _raw_case(variant, name, reverse, spikes):
    b, t, h, p, n, r, hq, spec = RAW_CASES[name]
    args = clip_inputs(b, t, heads=h, head_dim=p, state=n, rotary=r, qk_heads=hq, seed=23)
    lengths = _lengths(spec, b, t)
    dl = None if lengths is None else lengths.to(DEV)
    proj, dt_bias = _raw_projection(b, t, h, seed=24, spikes=spikes)
    ddt, a, trap = proj[..., :h], proj[..., h : 2 * h], proj[..., 2 * h : 3 * h]
    dp = proj.to(DEV)
    dddt, da, dtrap = dp[..., :h], dp[..., h : 2 * h], dp[..., 2 * h : 3 * h]
    base = to_dev(args)
    raw_args = base[:3] + (da.transpose(1, 2), dddt.transpose(1, 2), dtrap.transpose(1, 2)) + base[6:]
    needs(variant, raw_args, dt_bias=dt_bias.to(DEV))
    print(f"case variant={variant} {name} reverse={reverse}", flush=True)
    y = run(raw_args, variant, dl, reverse=reverse, dt_bias=dt_bias.to(DEV), a_floor=1e-4)
    # oracle: the reference's call sequence, controls first (mamba.py:58-82)
    adt_r, dt_r = E.mamba_controls(a, ddt, dt_bias, 1e-4)
    ref_args = args[:3] + (adt_r, dt_r, trap.transpose(1, 2)) + args[6:]
    if reverse:
        ref = fused_mamba_reversed(*ref_args, lengths=lengths)
    else:
        ref = fused_mamba_chunked(*ref_args, lengths=lengths)
    err = max_rel(y, ref)
    # the separate HIP controls kernel, then the recurrence on its outputs
    adt_g, dt_g = mamba_controls(da, dddt, dt_bias.to(DEV), 1e-4)
    sep = run(base[:3] + (adt_g, dt_g, dtrap.transpose(1, 2)) + base[6:], variant, dl, reverse=reverse)
    print(f"  max_rel vs oracle {err:.3e}, vs separate controls {max_rel(y, sep):.3e} "
          f"(bitwise {torch.equal(y, sep)})", flush=True)
    assert err <= MAX_REL
    assert max_rel(y, sep) <= 1e-6


@pytest.mark.parametrize(
    "dtype,d",
    [(torch.float32, 512), (torch.bfloat16, 512), (torch.bfloat16, 6), (torch.float16, 3), (torch.float32, 5)],
)
def test_reverse_valid_kernel_is_exact(dtype, d):
    g = torch.Generator().manual_seed(d)
    x = torch.randn(6, 37, d, generator=g).to(dtype)
    lengths = torch.tensor([37, 20, 0, 1, 50, -2])
    y = reverse_valid(x.to(DEV), lengths.to(DEV)).cpu()
    assert torch.equal(y, E.reverse_valid(x, lengths))


@pytest.mark.parametrize("da,db,d", [(torch.float32, torch.float32, 512), (torch.bfloat16, torch.bfloat16, 512),
                                     (torch.float32, torch.bfloat16, 100), (torch.bfloat16, torch.float32, 1024)])
def test_mean_norm_kernel(da, db, d):
    g = torch.Generator().manual_seed(d + 1)
    a = torch.randn(33, d, generator=g).to(da)
    b = torch.randn(33, d, generator=g).to(db)
    w = torch.rand(d, generator=g) + 0.5
    y = mean_norm(a.to(DEV), b.to(DEV), w.to(DEV)).cpu()
    assert y.dtype == torch.float32
    assert max_rel(y, E.mean_norm(a, b, w)) <= 1e-5
