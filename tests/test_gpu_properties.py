"""Exact properties of the HIP recurrence at the full workload sizes, where the
CPU oracle would take minutes per call: the clip workload B16 L400 H16 P64 N64
R16 Hq1 and the long clip B1 L7200, for each matrix-core kernel: the pipelined
walk ("pipe", one workgroup per unit) and the chunked kernel ("mfma": one
workgroup per unit at the clip size; at the long clip its chunk-parallel form:
phase sums, segment summaries, segment scan, outputs).
Every comparison is bitwise:

* causality: replacing every input at rows >= t* leaves the outputs at rows
  < t* unchanged (row t reads the halo step t + 1 only through kr_t, which
  reaches rows > t alone; mamba_fused.py:98-101,150-152);
* head permutation: permuting the heads together with their per-head
  parameters permutes the outputs;
* batch permutation: permuting the batch rows permutes the outputs;
* determinism: repeated calls, and a HIP graph replay, give the same bits.
"""

import pytest
import torch

from trifusion_amd.mamba_fused import fused_mamba, selected_variant
from trifusion_amd.synthetic import clip_inputs

pytestmark = pytest.mark.gpu

DEV = "cuda"
CLIP = dict(batch=16, time=400)
LONG = dict(batch=1, time=7200)


def inputs(batch, time, seed):
    return [a.to(DEV) for a in clip_inputs(batch, time, seed=seed)]


KERNELS = ["pipe", "mfma"]


def call(args, variant="auto"):
    with torch.inference_mode():
        y = fused_mamba(*args, variant=variant)
    torch.cuda.synchronize()
    return y


def replace_rows_from(args, fresh, t_star):
    """Rows >= t_star of every per-row input taken from ``fresh``."""
    q, k, v, adt, dt, trap, qb, kb, angles, d, z = [a.clone() for a in args]
    fq, fk, fv, fadt, fdt, ftrap, _, _, fang, _, fz = fresh
    for a, f in ((q, fq), (k, fk), (v, fv), (z, fz), (angles, fang)):  # [B, T, ...]
        a[:, t_star:] = f[:, t_star:]
    for a, f in ((adt, fadt), (dt, fdt), (trap, ftrap)):  # [B, H, T]
        a[..., t_star:] = f[..., t_star:]
    return [q, k, v, adt, dt, trap, qb, kb, angles, d, z]


@pytest.mark.parametrize("variant", KERNELS)
@pytest.mark.parametrize(
    "shape,t_star",
    [(CLIP, 1), (CLIP, 63), (CLIP, 64), (CLIP, 200), (CLIP, 399), (LONG, 3001), (LONG, 4096)],
)
def test_causality(shape, t_star, variant):
    print(f"case causality {shape} t*={t_star} variant={variant}", flush=True)
    args = inputs(shape["batch"], shape["time"], seed=11)
    assert selected_variant(*args, variant=variant) == variant
    fresh = inputs(shape["batch"], shape["time"], seed=12)
    y = call(args, variant)
    y2 = call(replace_rows_from(args, fresh, t_star), variant)
    assert torch.equal(y[:, :t_star], y2[:, :t_star])
    assert not torch.equal(y[:, t_star:], y2[:, t_star:])


@pytest.mark.parametrize("variant", KERNELS)
@pytest.mark.parametrize("shape", [CLIP, LONG])
def test_head_permutation(shape, variant):
    print(f"case head permutation {shape} variant={variant}", flush=True)
    args = inputs(shape["batch"], shape["time"], seed=13)
    q, k, v, adt, dt, trap, qb, kb, angles, d, z = args
    perm = torch.randperm(v.shape[2], generator=torch.Generator().manual_seed(0)).to(DEV)
    permuted = [q, k, v[:, :, perm], adt[:, perm], dt[:, perm], trap[:, perm], qb[perm], kb[perm],
                angles[:, :, perm], d[perm], z[:, :, perm]]
    permuted = [a.contiguous() for a in permuted]
    assert torch.equal(call(permuted, variant), call(args, variant)[:, :, perm])


@pytest.mark.parametrize("variant", KERNELS)
def test_batch_permutation(variant):
    print(f"case batch permutation variant={variant}", flush=True)
    args = inputs(CLIP["batch"], CLIP["time"], seed=14)
    perm = torch.randperm(CLIP["batch"], generator=torch.Generator().manual_seed(1)).to(DEV)
    permuted = [a if i in (6, 7, 9) else a[perm].contiguous() for i, a in enumerate(args)]
    assert torch.equal(call(permuted, variant), call(args, variant)[perm])


@pytest.mark.parametrize("variant", KERNELS)
@pytest.mark.parametrize("shape", [CLIP, LONG])
def test_repeat_and_graph_replay_are_bitwise(shape, variant):
    print(f"case determinism {shape} variant={variant}", flush=True)
    args = inputs(shape["batch"], shape["time"], seed=15)
    y0 = call(args, variant).clone()
    assert torch.equal(call(args, variant), y0)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    y_graph = torch.empty_like(y0)
    with torch.inference_mode():
        with torch.cuda.stream(stream):
            fused_mamba(*args, out=y_graph, variant=variant)  # warm-up on the capture stream
        stream.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            fused_mamba(*args, out=y_graph, variant=variant)
    torch.cuda.synchronize()
    for _ in range(3):
        y_graph.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y_graph, y0)
        assert torch.equal(call(args, variant), y0)
