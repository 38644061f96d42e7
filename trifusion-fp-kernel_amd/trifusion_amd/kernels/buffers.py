"""Buffer kernels of the Mamba block (reference ``src/trifusion_l4/kernels/buffers.py``).

``mask_buffer`` replaces ``buffers.py:6-10`` (``_mask``, ``primitives.py:65-70``)
and ``mamba_controls`` replaces ``buffers.py:82-101`` (``_controls``,
``primitives.py:190-216``); ``depthwise_masked``, ``Pool4``, ``RotaryQKV`` and
``front_norm`` (``buffers.py:13-80``) live in ``kernels.block``.
"""

import torch

from .. import _lib
from ..ops import ops
from .block import Pool4, RotaryQKV, depthwise_masked, front_norm  # noqa: F401  (buffers.py:13-80)


def mask_buffer(x, mask):
    """Copy of ``x`` with rows whose ``mask`` entry is false set to zero
    (``trifusion_amd::mask_rows``)."""
    return ops.mask_rows(x, mask)


def launch_mask_rows(x, mask):
    lib = _lib.load()
    _lib.require_cuda(x, mask, what="mask_buffer")
    x = x.contiguous()
    y = torch.empty_like(x)
    d = x.shape[-1]
    rows = x.numel() // d if d else 0
    if mask.dtype != torch.bool or mask.numel() != rows:
        raise ValueError("mask_buffer: mask must be bool with one entry per row")
    mask = mask.contiguous()
    status = lib.tf_mask_rows(
        x.data_ptr(), y.data_ptr(), _lib.dtype_code(x, "mask_buffer"), mask.data_ptr(), rows, d, _lib.stream_of(x)
    )
    _lib.check(status, "mask_buffer")
    return y


def mamba_controls(a, dt, bias, floor):
    """``(adt, dt)`` as contiguous fp32 ``[B, H, T]`` from raw ``a``/``ddt`` ``[B, T, H]``.

    ``a`` and ``dt`` are column slices of one projection and share strides, the
    head dimension unit-strided (as at ``src/trifusion_l4/mamba.py:65``).
    Dispatches through ``trifusion_amd::mamba_controls``.
    """
    return ops.mamba_controls(a, dt, bias, float(floor))


def launch_mamba_controls(a, dt, bias, floor):
    lib = _lib.load()
    _lib.require_cuda(a, dt, bias, what="mamba_controls")
    b, t, h = a.shape
    if dt.shape != a.shape or dt.dtype != a.dtype:
        raise ValueError("mamba_controls: a and dt must have one shape and dtype")
    if a.stride(2) != 1 or dt.stride() != a.stride():
        a = a.contiguous()
        dt = dt.contiguous()
    bias = bias.float().contiguous()
    oa = torch.empty((b, h, t), device=a.device)
    od = torch.empty_like(oa)
    status = lib.tf_mamba_controls(
        a.data_ptr(),
        dt.data_ptr(),
        _lib.dtype_code(a, "mamba_controls"),
        a.stride(0),
        a.stride(1),
        bias.data_ptr(),
        oa.data_ptr(),
        od.data_ptr(),
        b,
        t,
        h,
        float(floor),
        _lib.stream_of(a),
    )
    _lib.check(status, "mamba_controls")
    return oa, od
