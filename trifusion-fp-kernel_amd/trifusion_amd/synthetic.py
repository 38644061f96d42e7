"""Seeded synthetic operands for ``fused_mamba`` and the encoder workloads.

Two families of distributions:

``reference_test_inputs``
    The reference test's operands (``tests/test_recurrence.py:15-31``):
    q, k ~ 0.2 N(0,1) bf16; v, z and angles are strided views of one
    0.2 N(0,1) bf16 projection buffer (angles a stride-0 expand over heads);
    dt ~ U(0.01, 0.11); adt = -dt * U(0.2, 2.2); trap ~ N(0,1);
    qb, kb = 1 + 0.1 N(0,1); d = 1.
``clip_inputs``
    The benchmark clip workloads: x=v, B=k, C=q ~ N(0,1) (bf16 by default);
    dt = softplus(N(0,1) - 2); A_h = -exp(U(0, ln 16)) per head, adt = A_h * dt;
    raw angles ~ U(-0.5, 0.5) per step, head and rotary channel; trap ~ N(0,1);
    qb, kb = 1 + 0.1 N(0,1); D = 1; z ~ N(0,1); Hq = 1 and R = N/4 by default.

Tensors are drawn on the CPU from a seeded ``torch.Generator`` and then moved to
``device``, so every device sees identical values.
"""

import math

import torch
import torch.nn.functional as F


def _gen(seed):
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def reference_test_inputs(batch, time, heads=4, state=128, head_dim=64, rotary=32, seed=None, device="cpu"):
    g = _gen(121 + time if seed is None else seed)
    q, k = [
        (torch.randn(batch, time, 1, state, generator=g) * 0.2).to(torch.bfloat16) for _ in range(2)
    ]
    raw = (torch.randn(batch, time, heads * head_dim * 2 + rotary, generator=g) * 0.2).to(torch.bfloat16)
    dt = torch.rand(batch, heads, time, generator=g) * 0.1 + 0.01
    adt = -dt * (torch.rand(dt.shape, generator=g) * 2 + 0.2)
    trap = torch.randn(dt.shape, generator=g)
    qb, kb = [torch.randn(heads, state, generator=g) * 0.1 + 1 for _ in range(2)]
    d = torch.ones(heads)
    q, k, raw, dt, adt, trap, qb, kb, d = (
        x.to(device) for x in (q, k, raw, dt, adt, trap, qb, kb, d)
    )
    v = raw[:, :, : heads * head_dim].reshape(batch, time, heads, head_dim)
    z = raw[:, :, heads * head_dim : heads * head_dim * 2].reshape_as(v)
    angles = raw[:, :, -rotary:].unsqueeze(2).expand(batch, time, heads, rotary)
    return q, k, v, adt, dt, trap, qb, kb, angles, d, z


def clip_inputs(
    batch,
    time,
    heads=16,
    head_dim=64,
    state=64,
    rotary=None,
    qk_heads=1,
    dtype=torch.bfloat16,
    ctrl_dtype=torch.float32,
    seed=1,
    device="cpu",
):
    rotary = state // 4 if rotary is None else rotary
    g = _gen(seed)
    q = torch.randn(batch, time, qk_heads, state, generator=g)
    k = torch.randn(batch, time, qk_heads, state, generator=g)
    v = torch.randn(batch, time, heads, head_dim, generator=g)
    z = torch.randn(batch, time, heads, head_dim, generator=g)
    dt = F.softplus(torch.randn(batch, heads, time, generator=g) - 2)
    a_head = -torch.exp(torch.rand(heads, generator=g) * math.log(16.0))
    adt = a_head[None, :, None] * dt
    angles = torch.rand(batch, time, heads, rotary, generator=g) - 0.5
    trap = torch.randn(batch, heads, time, generator=g)
    qb = 1 + 0.1 * torch.randn(heads, state, generator=g)
    kb = 1 + 0.1 * torch.randn(heads, state, generator=g)
    d = torch.ones(heads)
    q, k, v, z = (x.to(dtype) for x in (q, k, v, z))
    adt, dt, trap, angles = (x.to(ctrl_dtype) for x in (adt, dt, trap, angles))
    return tuple(x.to(device) for x in (q, k, v, adt, dt, trap, qb, kb, angles, d, z))


def clip_lengths(batch, time, low, seed=2, device="cpu"):
    """Valid lengths ~ U{low..time} per row (variable-length batches)."""
    g = _gen(seed)
    return torch.randint(low, time + 1, (batch,), generator=g).to(device)


def channel_fold_lengths(clips, time, low, seed=2, device="cpu"):
    """Valid lengths of a batch that folds each clip's channels into the batch:
    rows ``2i`` and ``2i + 1`` are clip ``i``'s two channel slots. Clip lengths
    ~ U{low..time} and channel counts ~ U{1, 2}; a mono clip's second slot has
    length 0 (fully masked, as the model masks it). Returns ``(lengths [2*clips],
    channels [clips])``."""
    g = _gen(seed)
    clip_len = torch.randint(low, time + 1, (clips,), generator=g)
    channels = torch.randint(1, 3, (clips,), generator=g)
    lengths = torch.stack((clip_len, torch.where(channels == 2, clip_len, torch.zeros_like(clip_len))), 1)
    return lengths.reshape(-1).to(device), channels.to(device)


def algorithmic_bytes(args, out_dtype=None, lengths=None):
    """Unique input bytes plus output bytes of one ``fused_mamba`` call.

    Stride-0 (broadcast) operands count once; with ``lengths`` the per-token
    operands count only valid tokens, plus the zero-fill of padded outputs.
    """
    q, k, v, adt, dt, trap, qb, kb, angles, d, z = args
    b, t, h, p = v.shape

    def unique(x):
        n = 1
        for size, stride in zip(x.shape, x.stride()):
            if stride != 0:
                n *= size
        return n * x.element_size()

    out_size = torch.empty((), dtype=out_dtype or v.dtype).element_size()
    total = sum(unique(x) for x in (q, k, v, adt, dt, trap, angles, z, qb, kb, d))
    total += b * t * h * p * out_size
    if lengths is not None:
        frac = float(lengths.double().clamp(0, t).sum()) / (b * t)
        per_token = total - sum(unique(x) for x in (qb, kb, d)) - b * t * h * p * out_size
        total = int(per_token * frac) + sum(unique(x) for x in (qb, kb, d)) + b * t * h * p * out_size
    return total
