"""The ``trifusion_amd::*`` operators: registration, Meta shapes, no CPU path.

Runs without a GPU: Meta tensors exercise shape/dtype propagation (what
``torch.compile``/``torch.export`` tracing sees), CPU tensors must fail loudly.
"""

import pytest
import torch

from trifusion_amd import fused_mamba
from trifusion_amd.kernels import rms, swiglu
from trifusion_amd.kernels.buffers import mamba_controls, mask_buffer
from trifusion_amd.kernels.native import add, add_rms
from trifusion_amd.masking import masked_mean, time_mask
from trifusion_amd.ops import OPERATORS, ops
from trifusion_amd.synthetic import clip_inputs

META = torch.device("meta")


def test_every_operator_is_registered():
    for name in OPERATORS:
        base, _, overload = name.partition(".")
        packet = getattr(ops, base)
        op = getattr(packet, overload or "default")
        assert op._schema.name == f"trifusion_amd::{base}"


def test_fused_mamba_meta_shapes():
    args = [a.to(META) for a in clip_inputs(2, 70, heads=4, head_dim=64, state=64, seed=0)]
    y = fused_mamba(*args)
    assert y.device == META and y.shape == args[2].shape and y.dtype == args[2].dtype
    out = torch.empty(args[2].shape, dtype=torch.float32, device=META)
    assert fused_mamba(*args, out=out) is out


def test_elementwise_meta_shapes():
    x = torch.empty(3, 5, 512, device=META)
    w = torch.empty(512, device=META)
    assert rms(x.to(torch.bfloat16), w).dtype == torch.bfloat16
    assert rms(x, w, out_dtype=torch.bfloat16).dtype == torch.bfloat16
    s, y = add_rms(x, x.to(torch.bfloat16), w)
    assert s.dtype == torch.float32 and y.dtype == torch.bfloat16 and y.shape == x.shape
    assert add(x, x.to(torch.bfloat16)).dtype == torch.float32
    assert add(x, x, bf16=True).dtype == torch.bfloat16
    g = torch.empty(7, 2730, dtype=torch.bfloat16, device=META)
    assert swiglu(g).shape == (7, 1365)
    m = torch.empty(3, 5, dtype=torch.bool, device=META)
    assert mask_buffer(x, m).shape == x.shape
    a = torch.empty(2, 9, 16, dtype=torch.bfloat16, device=META)
    adt, dt = mamba_controls(a, a, torch.empty(16, device=META), 1e-4)
    assert adt.shape == dt.shape == (2, 16, 9) and adt.dtype == torch.float32
    lengths = torch.empty(3, dtype=torch.int64, device=META)
    assert masked_mean(x, lengths).shape == (3, 512)
    assert time_mask(lengths, 11).shape == (3, 11) and time_mask(lengths, 11).dtype == torch.bool


def test_cpu_tensors_fail_loudly():
    args = clip_inputs(1, 8, heads=2, head_dim=64, state=64, seed=0)
    with pytest.raises(RuntimeError, match="no CPU path"):
        fused_mamba(*args)
    with pytest.raises(RuntimeError, match="no CPU path"):
        rms(torch.ones(2, 8), torch.ones(8))
    with pytest.raises(RuntimeError, match="no CPU path"):
        swiglu(torch.ones(2, 8))
