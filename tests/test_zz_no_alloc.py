"""tf_fused_mamba_static (the entry point that allocates nothing) against
tf_fused_mamba with a caller workspace, through the C ABI (MI355X).

Two calls in a row on the library's static scratch, the second smaller, each
compared bit for bit with tf_fused_mamba on a torch-allocated workspace (both
run the same kernels with the same segment plan). Also a shape that needs no
scratch, and one whose scratch exceeds the static array, which must be
rejected with TF_ERR_WORKSPACE before anything is launched; and the entry
captured into a HIP graph, whose replays must equal the eager result.
"""

import ctypes

import pytest
import torch

from trifusion_amd import _lib
from trifusion_amd.mamba_fused import build_args
from trifusion_amd.synthetic import clip_inputs

pytestmark = pytest.mark.gpu

DEV = "cuda"
TF_ERR_WORKSPACE = 7


def call(entry, dargs, lengths=None, reverse=False, norms=None):
    lib = _lib.load()
    v = dargs[2]
    out = torch.full(v.shape, float("nan"), device=DEV, dtype=torch.float32)
    q_norm, k_norm = norms if norms is not None else (None, None)
    args = build_args(*dargs, out, lengths, "auto", reverse, None, 1e-4, q_norm, k_norm, 1e-5)
    workspace = None
    if entry == "tf_fused_mamba":
        need = lib.tf_fused_mamba_workspace_size(ctypes.byref(args))
        assert need >= 0
        if need:
            workspace = torch.empty(need, dtype=torch.uint8, device=DEV)
            args.workspace, args.workspace_bytes = workspace.data_ptr(), need
    rc = getattr(lib, entry)(ctypes.byref(args), _lib.stream_of(v))
    torch.cuda.synchronize()
    return rc, out


def test_static_scratch_matches_workspace_entry():
    lib = _lib.load()
    limit = lib.tf_fused_mamba_static_scratch_bytes()
    assert limit == 16 << 20
    cases = [
        ("long_b1_l7200_h16", clip_inputs(1, 7200, seed=21), None, False),
        ("smaller_b1_l3000_h8_reverse", clip_inputs(1, 3000, heads=8, seed=22), torch.tensor([2900]), True),
        ("serial_b4_l200_h16", clip_inputs(4, 200, seed=23), None, False),
    ]
    for name, args, lengths, reverse in cases:
        print(f"case {name}", flush=True)
        dargs = tuple(a.to(DEV) for a in args)
        dl = None if lengths is None else lengths.to(DEV)
        probe = build_args(*dargs, torch.empty(dargs[2].shape, device=DEV), dl, "auto", reverse, None, 1e-4)
        need = lib.tf_fused_mamba_workspace_size(ctypes.byref(probe))
        assert 0 <= need <= limit
        assert (need > 0) == (name != "serial_b4_l200_h16")
        rc_ref, ref = call("tf_fused_mamba", dargs, dl, reverse)
        rc, got = call("tf_fused_mamba_static", dargs, dl, reverse)
        assert rc_ref == 0 and rc == 0
        assert torch.isfinite(got).all()
        assert torch.equal(got, ref), f"{name}: max diff {(got - ref).abs().max().item():.3e}"


def test_static_entry_with_fused_norms():
    """The B/C norms fused into the recurrence (raw q/k rows and norm
    weights) through the static entry: the long clip's chunk-parallel
    kernels (summary pass and seeded walks both normalise the keys) equal
    tf_fused_mamba on a workspace bit for bit."""
    args = clip_inputs(1, 7200, seed=25)
    dargs = tuple(a.to(DEV) for a in args)
    g = torch.Generator().manual_seed(26)
    norms = tuple((0.5 + torch.rand(64, generator=g)).to(DEV) for _ in range(2))
    print("case fused norms long_b1_l7200_h16", flush=True)
    rc_ref, ref = call("tf_fused_mamba", dargs, norms=norms)
    rc, got = call("tf_fused_mamba_static", dargs, norms=norms)
    assert rc_ref == 0 and rc == 0
    assert torch.isfinite(got).all()
    assert torch.equal(got, ref)
    _, plain = call("tf_fused_mamba", dargs)
    assert not torch.equal(plain, ref), "the norm weights must change the result"


def test_static_entry_under_graph_capture():
    """tf_fused_mamba_static captured into a HIP graph (the callers it is for):
    after one eager call on the device (which looks up the scratch address),
    the capture launches the chunk-parallel kernels on the static scratch, and
    every replay, with eager work on the same buffers between replays, equals
    the eager tf_fused_mamba result bit for bit."""
    lib = _lib.load()
    args = clip_inputs(1, 7200, seed=24)
    dargs = tuple(a.to(DEV) for a in args)
    print("case graph long_b1_l7200_h16", flush=True)
    rc_ref, ref = call("tf_fused_mamba", dargs)
    rc, first = call("tf_fused_mamba_static", dargs)
    assert rc_ref == 0 and rc == 0 and torch.equal(first, ref)
    out = torch.full(dargs[2].shape, float("nan"), device=DEV, dtype=torch.float32)
    cargs = build_args(*dargs, out, None, "auto", False, None, 1e-4)
    codes = []
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            codes.append(lib.tf_fused_mamba_static(ctypes.byref(cargs), _lib.stream_of(out)))
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert codes == [0]
    for replay in range(3):
        out.fill_(float("nan"))
        # eager work between replays on the same device and buffers
        _, again = call("tf_fused_mamba_static", dargs)
        assert torch.equal(again, ref)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {replay}: max diff {(out - ref).abs().max().item():.3e}"


@pytest.mark.parametrize("variant,t,h", [("mfma", 16384, 128)])
def test_static_scratch_rejects_oversized_plans(variant, t, h):
    """Plans whose scratch exceeds the static area are refused before any
    launch: the chunked kernel's at B1 T16384 H128 (its phase sums grow with the
    chunk count). The pipelined kernel's plan has at most one record per CU
    (16 KB of state, 128 B of phase sums, 4 B of decay each) whatever the
    length, so it always fits."""
    lib = _lib.load()
    b, n, p, r = 1, 64, 64, 16
    print(f"case oversized variant={variant} t={t} h={h}", flush=True)
    bf = dict(device=DEV, dtype=torch.bfloat16)
    f32 = dict(device=DEV, dtype=torch.float32)
    q = torch.zeros(b, t, 1, n, **bf)
    k = torch.zeros(b, t, 1, n, **bf)
    v = torch.zeros(b, t, h, p, **bf)
    z = torch.zeros(b, t, h, p, **bf)
    ctl = [torch.zeros(b, h, t, **f32) for _ in range(3)]
    angles = torch.zeros(b, t, h, r, **f32)
    qb, kb, d = torch.zeros(h, n, **f32), torch.zeros(h, n, **f32), torch.ones(h, **f32)
    out = torch.full((b, t, h, p), -1.0, **bf)
    args = build_args(q, k, v, *ctl, qb, kb, angles, d, z, out, None, variant, False, None, 1e-4)
    assert lib.tf_fused_mamba_variant(ctypes.byref(args)) == {"pipe": 3, "mfma": 2}[variant]
    need = lib.tf_fused_mamba_workspace_size(ctypes.byref(args))
    assert need > lib.tf_fused_mamba_static_scratch_bytes()
    rc = lib.tf_fused_mamba_static(ctypes.byref(args), _lib.stream_of(v))
    torch.cuda.synchronize()
    assert rc == TF_ERR_WORKSPACE
    assert torch.all(out == -1.0), "a rejected call must launch nothing"
    with pytest.raises(ValueError, match="static area"):
        _lib.check(rc, "fused_mamba")
