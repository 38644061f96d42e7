"""Length masks and masked pooling (reference ``src/trifusion_l4/masking.py:6-11``,
``src/trifusion_l4/decoder.py:60-62``)."""

import torch

from . import _lib
from .ops import ops
from .kernels.buffers import mask_buffer


def time_mask(lengths, time):
    """``mask[b, t] = t < lengths[b]`` as a bool ``[B, T]`` device tensor
    (``trifusion_amd::time_mask``)."""
    return ops.time_mask(lengths, int(time))


def launch_time_mask(lengths, time):
    lib = _lib.load()
    _lib.require_cuda(lengths, what="time_mask")
    lengths = lengths.to(torch.int64).contiguous()
    mask = torch.empty((lengths.shape[0], time), device=lengths.device, dtype=torch.bool)
    status = lib.tf_time_mask(lengths.data_ptr(), mask.data_ptr(), lengths.shape[0], time, _lib.stream_of(lengths))
    _lib.check(status, "time_mask")
    return mask


def masked(x, mask):
    """Rows of ``x`` with a false mask set to zero (``masking.py:10-11``)."""
    return mask_buffer(x, mask)


def masked_mean(x, lengths):
    """``sum_{t < len} x[b, t] / len`` in fp32, ``x`` ``[B, T, D]`` -> ``[B, D]``
    (``trifusion_amd::masked_mean``)."""
    return ops.masked_mean(x, lengths)


def launch_masked_mean(x, lengths):
    lib = _lib.load()
    _lib.require_cuda(x, lengths, what="masked_mean")
    x = x.contiguous()
    lengths = lengths.to(torch.int64).contiguous()
    b, t, d = x.shape
    code = _lib.dtype_code(x, "masked_mean")
    y = torch.empty((b, d), device=x.device, dtype=torch.float32)
    need = lib.tf_masked_mean_workspace_size(code, b, t, d)
    if need < 0:
        _lib.check(-need, "masked_mean")
    work = torch.empty(need // 4, device=x.device, dtype=torch.float32) if need else None
    status = lib.tf_masked_mean(
        x.data_ptr(), code, lengths.data_ptr(), y.data_ptr(), b, t, d, work.data_ptr() if work is not None else None,
        need, _lib.stream_of(x),
    )
    _lib.check(status, "masked_mean")
    return y
