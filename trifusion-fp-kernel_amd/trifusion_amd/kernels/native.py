"""Row-norm and residual-add kernels (reference ``src/trifusion_l4/kernels/native.py``).

``rms`` replaces the MODE-0 ``_norm`` launch (``native.py:8-39,42-70``), ``add``
replaces ``_add`` (``:81-100``) and ``add_rms`` fuses an ``add`` with the
RMSNorm that follows it in the next block, writing both the residual sum and
its normalised copy in one pass. ``mean_norm`` replaces the MODE-2 ``_norm``
launch (``:77-78``): the RMSNorm of the mean of a bidirectional block's two
directions.
"""

import torch

from .. import _lib
from ..ops import ops
from .block import bands, evidence_norm, interpolate  # noqa: F401  (native.py:73-74,104-163)


def _row_view(x):
    """Return (tensor, row_stride) such that rows of length x.shape[-1] sit at a
    uniform element stride, copying only when no such stride exists."""
    d = x.shape[-1]
    if x.stride(-1) != 1 and d > 1:
        return x.contiguous(), d
    dims = [(s, st) for s, st in zip(x.shape[:-1], x.stride()[:-1]) if s != 1]
    if not dims:
        return x, d
    row = dims[-1][1]
    expected = row
    for s, st in reversed(dims):
        if st != expected:
            return x.contiguous(), d
        expected = st * s
    if row < d:
        return x.contiguous(), d
    return x, row


def rms(x, weight, eps=1e-5, out_dtype=None):
    """RMSNorm over the last dim with fp32 statistics; output dtype = x.dtype
    (``trifusion_amd::rms_norm``)."""
    return ops.rms_norm(x, weight, eps, out_dtype)


def launch_rms(x, weight, eps=1e-5, out_dtype=None):
    lib = _lib.load()
    _lib.require_cuda(x, weight, what="rms")
    if weight.dtype != torch.float32 or not weight.is_contiguous():
        weight = weight.float().contiguous()
    d = x.shape[-1]
    if weight.shape != (d,):
        raise ValueError(f"rms: weight must be [{d}]")
    xv, row_stride = _row_view(x)
    y = torch.empty(x.shape, device=x.device, dtype=out_dtype or x.dtype)
    rows = x.numel() // d if d else 0
    status = lib.tf_rmsnorm(
        xv.data_ptr(),
        _lib.dtype_code(xv, "rms"),
        row_stride,
        weight.data_ptr(),
        y.data_ptr(),
        _lib.dtype_code(y, "rms"),
        rows,
        d,
        float(eps),
        _lib.stream_of(x),
    )
    _lib.check(status, "rms")
    return y


def add(a, b, mask=None, bf16=False):
    """``a + b`` in fp32, zeroing rows whose mask is false; dtype as the reference
    (``trifusion_amd::add``)."""
    return ops.add(a, b, mask, bf16)


def launch_add(a, b, mask=None, bf16=False):
    lib = _lib.load()
    _lib.require_cuda(a, b, mask, what="add")
    a = a.contiguous()
    b = b.contiguous()
    if a.shape != b.shape:
        raise ValueError("add: shapes differ")
    dtype = torch.bfloat16 if bf16 else torch.promote_types(a.dtype, b.dtype)
    y = torch.empty(a.shape, device=a.device, dtype=dtype)
    d = a.shape[-1]
    rows = a.numel() // d if d else 0
    m = _mask_ptr(mask, rows)
    status = lib.tf_add(
        a.data_ptr(),
        _lib.dtype_code(a, "add"),
        b.data_ptr(),
        _lib.dtype_code(b, "add"),
        m,
        y.data_ptr(),
        _lib.dtype_code(y, "add"),
        rows,
        d,
        _lib.stream_of(a),
    )
    _lib.check(status, "add")
    return y


def add_rms(a, b, weight, mask=None, eps=1e-5, out_dtype=torch.bfloat16):
    """Fused ``s = add(a, b, mask)`` (fp32) and ``y = rms(s, weight)`` (``out_dtype``)
    (``trifusion_amd::add_rms_norm``)."""
    return ops.add_rms_norm(a, b, weight, mask, eps, out_dtype)


def launch_add_rms(a, b, weight, mask=None, eps=1e-5, out_dtype=torch.bfloat16):
    lib = _lib.load()
    _lib.require_cuda(a, b, mask, weight, what="add_rms")
    if a.dtype != torch.float32:
        raise TypeError("add_rms: the residual stream must be float32")
    a = a.contiguous()
    b = b.contiguous()
    d = a.shape[-1]
    rows = a.numel() // d if d else 0
    s = torch.empty(a.shape, device=a.device, dtype=torch.float32)
    y = torch.empty(a.shape, device=a.device, dtype=out_dtype)
    status = lib.tf_add_rmsnorm(
        a.data_ptr(),
        _lib.dtype_code(a, "add_rms"),
        b.data_ptr(),
        _lib.dtype_code(b, "add_rms"),
        _mask_ptr(mask, rows),
        weight.data_ptr(),
        s.data_ptr(),
        _lib.dtype_code(s, "add_rms"),
        y.data_ptr(),
        _lib.dtype_code(y, "add_rms"),
        rows,
        d,
        float(eps),
        _lib.stream_of(a),
    )
    _lib.check(status, "add_rms")
    return s, y


def mean_norm(a, b, weight, eps=1e-5):
    """``rms((a + b) / 2, weight)`` with fp32 math and an fp32 output
    (reference ``native.mean_norm``, ``src/trifusion_l4/kernels/native.py:77-78``;
    ``trifusion_amd::mean_rms_norm``)."""
    return ops.mean_rms_norm(a, b, weight, eps)


def launch_mean_rms(a, b, weight, eps=1e-5):
    lib = _lib.load()
    _lib.require_cuda(a, b, weight, what="mean_norm")
    if a.shape != b.shape:
        raise ValueError("mean_norm: shapes differ")
    if weight.dtype != torch.float32 or not weight.is_contiguous():
        weight = weight.float().contiguous()
    d = a.shape[-1]
    if weight.shape != (d,):
        raise ValueError(f"mean_norm: weight must be [{d}]")
    a = a.contiguous()
    b = b.contiguous()
    rows = a.numel() // d if d else 0
    y = torch.empty(a.shape, device=a.device, dtype=torch.float32)
    status = lib.tf_mean_rmsnorm(
        a.data_ptr(),
        _lib.dtype_code(a, "mean_norm"),
        b.data_ptr(),
        _lib.dtype_code(b, "mean_norm"),
        weight.data_ptr(),
        y.data_ptr(),
        rows,
        d,
        float(eps),
        _lib.stream_of(a),
    )
    _lib.check(status, "mean_norm")
    return y


def mask_rms(x, mask, weight, eps=1e-5, out_dtype=torch.bfloat16):
    """``s = x`` with rows whose mask is false set to 0 (fp32) and ``y = rms(s,
    weight)`` (``out_dtype``) in one pass (``trifusion_amd::mask_rms_norm``)."""
    return ops.mask_rms_norm(x, mask, weight, eps, out_dtype)


def launch_mask_rms(x, mask, weight, eps=1e-5, out_dtype=torch.bfloat16):
    lib = _lib.load()
    _lib.require_cuda(x, mask, weight, what="mask_rms")
    x = x.contiguous()
    d = x.shape[-1]
    if weight.shape != (d,) or weight.dtype != torch.float32:
        raise ValueError(f"mask_rms: weight must be float32 [{d}]")
    rows = x.numel() // d if d else 0
    s = torch.empty(x.shape, device=x.device, dtype=torch.float32)
    y = torch.empty(x.shape, device=x.device, dtype=out_dtype or torch.bfloat16)
    status = lib.tf_mask_rmsnorm(
        x.data_ptr(), _lib.dtype_code(x, "mask_rms"), _mask_ptr(mask, rows), weight.contiguous().data_ptr(),
        s.data_ptr(), y.data_ptr(), _lib.dtype_code(y, "mask_rms"), rows, d, float(eps), _lib.stream_of(x),
    )
    _lib.check(status, "mask_rms")
    return s, y


def rms_pair(x, w0, w1, eps=1e-5):
    """Two RMSNorms per row of ``x`` ``[..., 2d]``: the first ``d`` columns with
    ``w0``, the last ``d`` with ``w1``; returns contiguous ``[..., 2, d]`` in x's
    dtype (``trifusion_amd::rms_norm_pair``). Rows may sit at any stride."""
    return ops.rms_norm_pair(x, w0, w1, eps)


def launch_rms_pair(x, w0, w1, eps=1e-5):
    lib = _lib.load()
    _lib.require_cuda(x, w0, w1, what="rms_pair")
    two_d = x.shape[-1]
    if two_d % 2:
        raise ValueError("rms_pair: last dim must be even")
    d = two_d // 2
    for w in (w0, w1):
        if w.shape != (d,) or w.dtype != torch.float32 or not w.is_contiguous():
            raise ValueError(f"rms_pair: weights must be contiguous float32 [{d}]")
    xv, row_stride = _row_view(x)
    rows = x.numel() // two_d if two_d else 0
    y = torch.empty((*x.shape[:-1], 2, d), device=x.device, dtype=x.dtype)
    status = lib.tf_rmsnorm_pair(
        xv.data_ptr(), _lib.dtype_code(xv, "rms_pair"), row_stride, w0.data_ptr(), w1.data_ptr(), y.data_ptr(),
        _lib.dtype_code(y, "rms_pair"), rows, d, float(eps), _lib.stream_of(x),
    )
    _lib.check(status, "rms_pair")
    return y


def _mask_ptr(mask, rows):
    if mask is None:
        return None
    if mask.dtype != torch.bool or mask.numel() != rows or not mask.is_contiguous():
        raise ValueError("mask must be a contiguous bool tensor with one entry per row")
    return mask.data_ptr()
