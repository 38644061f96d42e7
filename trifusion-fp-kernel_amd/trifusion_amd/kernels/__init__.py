"""Inference kernels around the recurrence (reference ``src/trifusion_l4/kernels/__init__.py``).

``RMSNorm`` mirrors ``kernels/__init__.py:15-28`` and ``swiglu`` mirrors
``:31-41``; both launch gfx950 HIP kernels through the C ABI.
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


__all__ = ["RMSNorm", "swiglu", "rms"]
