"""Inference kernels around the recurrence (reference ``src/trifusion_l4/kernels/__init__.py``).

``RMSNorm`` mirrors ``kernels/__init__.py:15-28``, ``swiglu`` mirrors
``:31-41`` and ``reverse_valid`` mirrors ``:44-55``; all launch gfx950 HIP
kernels through the C ABI.
"""

import torch
from torch import nn

from .. import _lib
from ..ops import ops
from .native import rms


class RMSNorm(nn.Module):
    def __init__(self, dim, eps=1e-5):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x):
        return rms(x, self.weight, self.eps)


def swiglu(x):
    """``silu(g) * u`` with ``g, u`` the halves of the last dim (fp32 math)
    (``trifusion_amd::swiglu``)."""
    return ops.swiglu(x)


def launch_swiglu(x):
    lib = _lib.load()
    _lib.require_cuda(x, what="swiglu")
    x = x.contiguous()
    if x.shape[-1] % 2:
        raise ValueError("swiglu: last dim must be even")
    d = x.shape[-1] // 2
    y = x.new_empty((*x.shape[:-1], d))
    rows = x.numel() // x.shape[-1] if x.shape[-1] else 0
    status = lib.tf_swiglu(x.data_ptr(), y.data_ptr(), _lib.dtype_code(x, "swiglu"), rows, d, _lib.stream_of(x))
    _lib.check(status, "swiglu")
    return y


def reverse_valid(x, lengths):
    """Reverse the valid prefix of each row of ``x`` ``[B, T, D]``:
    ``y[b, t] = x[b, lengths[b] - 1 - t]`` for ``t < lengths[b]``, else 0
    (``trifusion_amd::reverse_valid``)."""
    return ops.reverse_valid(x, lengths)


def launch_reverse_valid(x, lengths):
    lib = _lib.load()
    _lib.require_cuda(x, lengths, what="reverse_valid")
    if x.dim() != 3:
        raise ValueError(f"reverse_valid: x must be [B, T, D], got {tuple(x.shape)}")
    b, t, d = x.shape
    if tuple(lengths.shape) != (b,) or lengths.dtype != torch.int64:
        raise ValueError("reverse_valid: lengths must be an int64 tensor of shape [B]")
    x = x.contiguous()
    lengths = lengths.contiguous()
    y = torch.empty_like(x)
    if x.numel() == 0:
        return y
    status = lib.tf_reverse_valid(
        x.data_ptr(), y.data_ptr(), _lib.dtype_code(x, "reverse_valid"), lengths.data_ptr(), b, t, d,
        _lib.stream_of(x),
    )
    _lib.check(status, "reverse_valid")
    return y


from .block import gated_concat  # noqa: E402  (kernels/__init__.py:58-82)

__all__ = ["RMSNorm", "swiglu", "rms", "reverse_valid", "gated_concat"]
