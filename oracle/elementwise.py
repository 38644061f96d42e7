"""CPU restatements of the bandwidth-bound ops around the recurrence (oracle).

Test infrastructure only (see ``oracle/__init__.py``). Each function restates
one reference formula in fp32 PyTorch on the CPU.

Pinning (tests/test_oracle_elementwise.py): ``rms_norm`` against
``torch.nn.functional.rms_norm``; ``swiglu`` against ``F.silu(g) * u`` on an
independently split tensor; ``mamba_controls`` against ``F.softplus`` (same
threshold 20) and hand-evaluated special cases of the decay control;
``masked_mean`` against a Python loop over valid frames; ``mask_rows`` and
``add`` against explicit ``torch.where`` forms; ``reverse_valid`` against a
Python loop, ``torch.flip`` at full length and its own square (the masked
identity); ``mean_norm`` against ``F.rms_norm`` of the mean and the a == b case.
"""

import torch
import torch.nn.functional as F


def rms_norm(x, weight, eps=1e-5):
    """``y = x * rsqrt(mean(x^2) + eps) * w`` with fp32 statistics, output in x's dtype.

    Reference: ``src/trifusion_l4/kernels/__init__.py:10-12`` (``rms_reference``) and
    the MODE-0 row kernel ``src/trifusion_l4/kernels/native.py:8-39,42-70``.
    """
    xf = x.float()
    return (xf * torch.rsqrt(xf.square().mean(-1, keepdim=True) + eps) * weight.float()).to(x.dtype)


def swiglu(x):
    """``silu(g) * u`` over the two halves of the last dim, fp32 math.

    Reference: ``src/trifusion_l4/kernels/__init__.py:31-34``;
    ``src/trifusion_l4/kernels/primitives.py:25-37``.
    """
    gate, up = x.float().chunk(2, -1)
    return (F.silu(gate) * up).to(x.dtype)


def time_mask(lengths, time):
    """``mask[b, t] = t < lengths[b]`` (``src/trifusion_l4/masking.py:6-7``)."""
    return torch.arange(time, device=lengths.device)[None, :] < lengths[:, None]


def mask_rows(x, mask):
    """Zero rows whose mask is false (``masking.py:10-11``; ``primitives.py:65-70``)."""
    return x.masked_fill(~mask[..., None], 0)


def add(a, b, mask=None, bf16=False):
    """``a + b`` in fp32, rows with a false mask set to 0 (``native.py:81-100``)."""
    y = a.float() + b.float()
    if mask is not None:
        y = y.masked_fill(~mask.reshape(*y.shape[:-1], 1), 0)
    dtype = torch.bfloat16 if bf16 else torch.promote_types(a.dtype, b.dtype)
    return y.to(dtype)


def mamba_controls(a, ddt, dt_bias, floor=1e-4):
    """Discretisation controls of the Mamba-3 block.

    ``dt = softplus(ddt + dt_bias)`` (threshold 20) and
    ``adt = -max(relu(a) + 1/(1 - min(a, 0)), floor) * dt``, both returned as
    contiguous ``[B,H,T]`` fp32. Reference: ``src/trifusion_l4/mamba.py:58-63`` and
    ``src/trifusion_l4/kernels/primitives.py:190-216``.
    """
    af = a.float()
    v = ddt.float() + dt_bias.float()
    control = torch.clamp_max(-(af.clamp_min(0) + 1 / (1 - af.clamp_max(0))), -floor)
    dt = torch.where(v > 20, v, torch.log1p(torch.exp(v)))
    adt = control * dt
    return adt.transpose(1, 2).contiguous(), dt.transpose(1, 2).contiguous()


def masked_mean(x, lengths):
    """Masked mean over time, ``sum_t x*mask / length`` in fp32 (``decoder.py:60-62``)."""
    mask = time_mask(lengths, x.shape[1])
    return (x.float() * mask[..., None]).sum(1) / lengths[:, None]


def reverse_valid(x, lengths):
    """Reverse the valid prefix of each row of ``x`` ``[B, T, D]``:
    ``y[b, t] = x[b, L_b - 1 - t]`` for ``t < L_b``, else 0, with ``L_b`` the
    length clamped to ``[0, T]``.

    Reference: ``src/trifusion_l4/kernels/__init__.py:44-55`` (its gather form)
    and the ``_reverse`` kernel ``src/trifusion_l4/kernels/primitives.py:40-47``.
    """
    b, t, d = x.shape
    n = lengths.clamp(0, t)
    pos = torch.arange(t, device=x.device)[None, :]
    src = (n[:, None] - 1 - pos).clamp_min(0)
    y = torch.gather(x, 1, src[..., None].expand(b, t, d))
    return y.masked_fill((pos >= n[:, None])[..., None], 0)


def mean_norm(a, b, weight, eps=1e-5):
    """RMSNorm of the mean of two directions, fp32 math and output:
    ``s = (a + b) / 2``, ``y = s * rsqrt(mean(s^2) + eps) * w``.

    Reference: ``_norm`` MODE 2 ``src/trifusion_l4/kernels/native.py:8-39``
    (``x = (x + a) * 0.5``, fp32 output ``:46``) through ``mean_norm`` ``:77-78``.
    """
    s = (a.float() + b.float()) * 0.5
    return s * torch.rsqrt(s.square().mean(-1, keepdim=True) + eps) * weight.float()
