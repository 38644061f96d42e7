"""Parity of the HIP bandwidth kernels against the CPU oracle (MI355X)."""

import pytest
import torch

from oracle import elementwise as E
from trifusion_amd.kernels import RMSNorm, swiglu
from trifusion_amd.kernels.buffers import mamba_controls, mask_buffer
from trifusion_amd.kernels.native import add, add_rms, rms
from trifusion_amd.masking import masked_mean, time_mask

pytestmark = pytest.mark.gpu
DEV = "cuda"


def gen(seed):
    return torch.Generator().manual_seed(seed)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,d", [(6400, 512), (7, 64), (33, 1365), (5, 4096), (1, 1)])
def test_rmsnorm(dtype, rows, d):
    g = gen(rows + d)
    x = torch.randn(rows, d, generator=g).to(dtype)
    w = torch.rand(d, generator=g) + 0.5
    y = rms(x.to(DEV), w.to(DEV)).cpu()
    ref = E.rms_norm(x, w)
    assert y.dtype == dtype
    if dtype == torch.float32:
        torch.testing.assert_close(y, ref, rtol=1e-5, atol=1e-5)
    else:  # at most one bf16 ulp apart
        torch.testing.assert_close(y.float(), ref.float(), rtol=2 ** -7, atol=1e-6)


def test_rmsnorm_strided_rows_no_copy():
    g = gen(3)
    proj = torch.randn(4, 50, 300, generator=g).to(torch.bfloat16)
    x = proj[..., 100:164].reshape(4, 50, 1, 64)
    w = torch.rand(64, generator=g) + 0.5
    dx = proj.to(DEV)[..., 100:164].reshape(4, 50, 1, 64)
    assert not dx.is_contiguous()
    norm = RMSNorm(64).to(DEV)
    with torch.no_grad():
        norm.weight.copy_(w)
    y = norm(dx).cpu()
    torch.testing.assert_close(y.float(), E.rms_norm(x, w).float(), rtol=2 ** -7, atol=1e-6)


@pytest.mark.parametrize("bdtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("ydtype", [torch.float32, torch.bfloat16])
def test_add_rmsnorm(bdtype, ydtype):
    g = gen(4)
    a = torch.randn(16, 400, 512, generator=g)
    b = torch.randn(16, 400, 512, generator=g).to(bdtype)
    mask = E.time_mask(torch.randint(1, 401, (16,), generator=g), 400)
    w = torch.rand(512, generator=g) + 0.5
    s, y = add_rms(a.to(DEV), b.to(DEV), w.to(DEV), mask.to(DEV), out_dtype=ydtype)
    s_ref = E.add(a, b, mask)
    torch.testing.assert_close(s.cpu(), s_ref, rtol=0, atol=0)
    y_ref = E.rms_norm(s_ref, w).to(ydtype)
    tol = 1e-5 if ydtype == torch.float32 else 2 ** -7
    torch.testing.assert_close(y.cpu().float(), y_ref.float(), rtol=tol, atol=1e-5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(6400, 2730), (3, 8), (1, 2)])
def test_swiglu(dtype, shape):
    x = torch.randn(*shape, generator=gen(5)).to(dtype)
    y = swiglu(x.to(DEV)).cpu()
    ref = E.swiglu(x)
    tol = 1e-6 if dtype == torch.float32 else 2 ** -7
    torch.testing.assert_close(y.float(), ref.float(), rtol=tol, atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_mask_and_time_mask(dtype):
    g = gen(6)
    lengths = torch.tensor([400, 1, 0, 217])
    x = torch.randn(4, 400, 96, generator=g).to(dtype)
    m = time_mask(lengths.to(DEV), 400)
    assert torch.equal(m.cpu(), E.time_mask(lengths, 400))
    y = mask_buffer(x.to(DEV), m).cpu()
    assert torch.equal(y, E.mask_rows(x, E.time_mask(lengths, 400)))


@pytest.mark.parametrize("bf16", [False, True])
def test_add_masked(bf16):
    g = gen(7)
    a = torch.randn(8, 33, 512, generator=g)
    b = torch.randn(8, 33, 512, generator=g).to(torch.bfloat16)
    mask = torch.rand(8, 33, generator=g) > 0.3
    y = add(a.to(DEV), b.to(DEV), mask.to(DEV), bf16=bf16).cpu()
    assert torch.equal(y, E.add(a, b, mask, bf16=bf16))
    y = add(a.to(DEV), b.to(DEV)).cpu()
    assert torch.equal(y, E.add(a, b))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_mamba_controls(dtype):
    g = gen(8)
    b, t, h = 16, 400, 16
    proj = (torch.randn(b, t, 3 * h + 7, generator=g) * 3).to(dtype)
    proj[0, 0, :h] = 30.0  # softplus linear branch
    ddt, a = proj[..., :h], proj[..., h : 2 * h]
    bias = torch.full((h,), -4.0) + torch.randn(h, generator=g)
    dproj = proj.to(DEV)
    adt, dt = mamba_controls(dproj[..., h : 2 * h], dproj[..., :h], bias.to(DEV), 1e-4)
    adt_ref, dt_ref = E.mamba_controls(a, ddt, bias)
    assert adt.is_contiguous() and adt.shape == (b, h, t)
    torch.testing.assert_close(dt.cpu(), dt_ref, rtol=2e-6, atol=1e-7)
    torch.testing.assert_close(adt.cpu(), adt_ref, rtol=2e-6, atol=1e-7)


def test_control_step_softplus_range():
    """The step dt = softplus(ddt + bias), formed from the hardware exp2, log2
    and reciprocal with Kahan's log1p identity, over ddt + bias in [-100, 25]
    (plus points around e^v = 2^-24, where u = 1 + e^v rounds to 1, and
    around the linear threshold 20): within 8 float32 ulp of float64
    softplus where the result is a normal float, exactly v above 20, and 0
    (not NaN) from -104 down to -inf, where e^v is below the least subnormal; and the
    decay adt = min(-(relu(a) + 1/(1 - min(a, 0))), -floor) * dt within 8 ulp
    of its float64 value on the kernel's own dt."""
    v = torch.cat([torch.linspace(-100.0, 25.0, 8001),
                   torch.tensor([-17.5, -16.7, -16.6, -16.0, -1e-6, 0.0, 1e-6, 19.999, 20.0, 20.001]),
                   torch.tensor([-103.9, -104.0, -104.1, -150.0, -1e30, -float("inf")])])
    t = v.numel()
    a = torch.linspace(-3.0, 3.0, t)
    proj = torch.stack([v, a], dim=1).view(1, t, 2)  # columns ddt | a, head dim unit-strided
    dproj = proj.to(DEV)
    floor = 1e-4
    adt, dt = mamba_controls(dproj[..., 1:2], dproj[..., 0:1], torch.zeros(1, device=DEV), floor)
    dt = dt.cpu().view(-1).double()
    adt = adt.cpu().view(-1).double()
    vd = v.double()
    ref = torch.where(vd > 20, vd, torch.log1p(torch.exp(vd)))
    ulp = 2.0 ** -23
    normal = ref > torch.finfo(torch.float32).tiny
    rel = ((dt - ref).abs() / ref.clamp_min(1e-300))[normal]
    print(f"softplus: max error {rel.max().item() / ulp:.2f} ulp over {int(normal.sum())} normal results", flush=True)
    assert rel.max().item() <= 8 * ulp
    assert (dt[~normal] - ref[~normal]).abs().max().item() <= torch.finfo(torch.float32).tiny
    assert torch.equal(dt[vd > 20], vd[vd > 20])
    assert torch.isfinite(dt).all()
    assert torch.equal(dt[vd <= -104], torch.zeros_like(dt[vd <= -104]))
    ad = a.double()
    adt_ref = torch.minimum(-(ad.clamp_min(0) + 1.0 / (1.0 - ad.clamp_max(0))), torch.tensor(-floor, dtype=torch.float64)) * dt
    nz = adt_ref.abs() > torch.finfo(torch.float32).tiny
    rel_a = ((adt - adt_ref).abs() / adt_ref.abs().clamp_min(1e-300))[nz]
    print(f"decay: max error {rel_a.max().item() / ulp:.2f} ulp", flush=True)
    assert rel_a.max().item() <= 8 * ulp


MEAN_SHAPES = [
    # batch, time, d: the encoder pool (one split in fp32, two in bf16), a long
    # single clip (16 time splits), few frames (no split), d that is not a whole
    # number of 16-byte lanes (the per-column kernel)
    (16, 400, 512),
    (1, 3000, 96),
    (3, 50, 8),
    (4, 130, 6),
]


def mean64(x, lengths):
    """fp64 masked mean of the valid prefix (lengths >= 1)."""
    t = x.shape[1]
    mask = (torch.arange(t)[None, :] < lengths[:, None]).double()
    return (x.double() * mask[..., None]).sum(1) / lengths[:, None].double()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("b,t,d", MEAN_SHAPES)
def test_masked_mean(dtype, b, t, d):
    """Against the oracle (fp32) and an fp64 sum: a dropped or repeated frame
    moves a mean by |x| / length, at least 3e-4 here, far above the tolerance.
    Two calls are bitwise equal (the split sums are added in a fixed order)."""
    g = gen(9 + t)
    x = torch.randn(b, t, d, generator=g).to(dtype)
    lengths = torch.randint(1, t + 1, (b,), generator=g)
    lengths[0] = t
    print(f"case masked_mean b={b} t={t} d={d} dtype={dtype}", flush=True)
    dx, dl = x.to(DEV), lengths.to(DEV)
    y = masked_mean(dx, dl)
    assert torch.equal(y, masked_mean(dx, dl))
    y = y.cpu()
    torch.testing.assert_close(y, E.masked_mean(x, lengths), rtol=1e-5, atol=2e-6)
    assert (y.double() - mean64(x, lengths)).abs().max().item() <= 2e-6


def test_masked_mean_split_and_unsplit_agree():
    """A shape that splits time (bf16 encoder pool) computed with and without
    the workspace: both within fp32 rounding of the fp64 mean; zero and
    negative lengths give the oracle's non-finite or zero rows."""
    import ctypes

    from trifusion_amd import _lib

    lib = _lib.load()
    g = gen(11)
    b, t, d = 16, 400, 512
    x = torch.randn(b, t, d, generator=g).to(torch.bfloat16)
    lengths = torch.randint(1, t + 1, (b,), generator=g)
    lengths[1], lengths[2] = 0, -3
    code = _lib.dtype_code(x, "masked_mean")
    need = lib.tf_masked_mean_workspace_size(code, b, t, d)
    assert need == 2 * b * d * 4
    dx, dl = x.to(DEV), lengths.to(DEV)
    work = torch.empty(need // 4, device=DEV)
    outs = []
    for ws, nbytes in ((work.data_ptr(), need), (None, 0), (work.data_ptr(), need - 4)):
        y = torch.empty(b, d, device=DEV)
        status = lib.tf_masked_mean(dx.data_ptr(), code, dl.data_ptr(), y.data_ptr(), b, t, d, ws, nbytes,
                                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        assert status == 0
        torch.cuda.synchronize()
        outs.append(y.cpu())
    ref = E.masked_mean(x, lengths)
    valid = lengths > 0
    for y in outs:
        torch.testing.assert_close(y, ref, rtol=1e-5, atol=2e-6, equal_nan=True)
        assert (y[valid].double() - mean64(x[valid], lengths[valid])).abs().max().item() <= 2e-6
        assert torch.isnan(y[1]).all() and (y[2] == 0).all()
    # too small a workspace: the unsplit form, bit for bit (NaN rows included)
    torch.testing.assert_close(outs[1], outs[2], rtol=0, atol=0, equal_nan=True)
