"""CPU restatements of the TriFusion block and front-end kernels (oracle).

Test infrastructure only (see ``oracle/__init__.py``). Each function restates
the reference model's unfused PyTorch formulation, which its fused kernels
replace:

* ``depthwise_masked``: ``masked(merge_dw(v.transpose(1, 2)).transpose(1, 2))``
  (``src/trifusion_l4/model.py:188-190``), a grouped ``F.conv1d``;
* ``pool4`` and ``interpolate``: ``Grids.pool`` / ``Grids.interpolate``
  (``src/trifusion_l4/masking.py:59-80``) on grids built as ``Grids.make``
  builds them (``:29-57``);
* ``rotary_qkv``: the reference branch of ``GlobalAttention`` with ``rope``
  (``src/trifusion_l4/model.py:40-48,84-89``);
* ``front_norm``: the unfused CNN-stage norm ``silu(norm(clean(h)))``
  (``src/trifusion_l4/front.py:36-37``) with the RMSNorm output in the
  activation dtype;
* ``bands``: ``adaptive_avg_pool2d`` over frequency (``front.py:94-101``);
* ``evidence_norm``: ``masked(u_norm(x + value * 2 sigmoid(gate)))``
  (``src/trifusion_l4/model.py:166-167``);
* ``gated_concat``: the reference branch (``kernels/__init__.py:59-63``);
* ``evidence_down``: ``silu(e_down(cat(cn, an)))`` (``src/trifusion_l4/model.py:161``)
  under bf16 autocast: bf16 operands, fp32 sums, the linear's bf16 result, SiLU
  in fp32 rounded to bf16;
* ``front_stage``: a whole CNN stage (``front.py:19-43``) under bf16 autocast:
  ``F.conv2d`` on bf16-rounded operands with bf16 outputs, ``front_norm``, the
  1x1 skip, the bf16 residual sum and SiLU, rows past the length cleared;
* the block's fused runs under bf16 autocast (``model.py:140-200``), each the
  composition of the functions above and the elementwise oracle with the casts
  autocast makes: ``block_pre`` (mask, pre norm, 4:1 pool), ``glu_depthwise``,
  ``norm_silu``, ``pooled_attention`` (rotary, fp32 SDPA, head merge),
  ``merge_gate`` (mean norm, gate linear) and ``merge_conv`` (gated concat,
  depthwise merge, bf16 add);
* ``query_read``: the decoder's ``QueryRead`` attention (``decoder.py:24-30``,
  ``attention.py:8-18``): fp32 SDPA of the shared queries over a key prefix.

Pinning (tests/test_oracle_trifusion.py): each against an explicit loop or
closed form on small inputs.
"""

import torch
import torch.nn.functional as F

from .elementwise import mask_rows, mean_norm, rms_norm, time_mask


def depthwise_masked(x, weight, bias, lengths):
    """``[B, T, D]`` masked depthwise conv, same padding, fp32 math, x's dtype."""
    d, k = x.shape[-1], weight.shape[-1]
    y = F.conv1d(x.float().transpose(1, 2), weight.float().reshape(d, 1, k), bias.float(), padding=k // 2, groups=d)
    return mask_rows(y.transpose(1, 2), time_mask(lengths, x.shape[1])).to(x.dtype)


def grids(lengths, time):
    """``low_lengths``, ``left``, ``right``, ``alpha`` of the 4:1 attention grid
    (``masking.py:29-41``)."""
    low_lengths = (lengths + 3) // 4
    pos = torch.arange(time)[None, :].float() + 0.5
    pos = (pos * low_lengths[:, None] / lengths[:, None] - 0.5).clamp_min(0)
    pos = torch.minimum(pos, (low_lengths - 1)[:, None])
    left = pos.long()
    right = torch.minimum(left + 1, (low_lengths - 1)[:, None])
    return low_lengths, left, right, pos - left


def pool4(x, lengths):
    """Masked 4:1 time average; the last partial group divided by its valid count."""
    b, t, d = x.shape
    mask = time_mask(lengths, t)
    xp = F.pad(mask_rows(x, mask), (0, 0, 0, (-t) % 4))
    mp = F.pad(mask, (0, (-t) % 4)).view(b, -1, 4)
    y = xp.float().view(b, -1, 4, d).sum(2) / mp.sum(2).clamp_min(1)[..., None]
    return y.to(x.dtype)


def interpolate(low, left, right, alpha, lengths):
    """Linear interpolation of the pooled grid back to frames, masked rows 0."""
    shape = (*left.shape, low.shape[-1])
    a = low.gather(1, left[..., None].expand(shape))
    b = low.gather(1, right[..., None].expand(shape))
    y = a.float() + (b.float() - a.float()) * alpha[..., None]
    return mask_rows(y.to(low.dtype), time_mask(lengths, left.shape[1]))


def rotary_qkv(x, cos, sin, heads):
    """``[B, T, 3 H D]`` -> ``[3, B, H, T, D]``, q and k rotated by interleaved
    pairs with the [T, D/2] tables, v unchanged."""
    b, t, width = x.shape
    d = width // (3 * heads)
    qkv = x.view(b, t, 3, heads, d).permute(2, 0, 3, 1, 4)
    a, z = qkv.float().reshape(3, b, heads, t, d // 2, 2).unbind(-1)
    rot = torch.stack((a * cos - z * sin, a * sin + z * cos), -1).flatten(-2).to(x.dtype)
    return torch.stack((rot[0], rot[1], qkv[2]))


def front_norm(x, lengths, weight, eps=1e-5, silu=False):
    """``[B, C, T, F]`` -> ``[B, T, F, C]``: rows past the length cleared, RMSNorm
    over channels rounded to x's dtype, then SiLU when asked."""
    b, c, t, f = x.shape
    clean = x.masked_fill(~time_mask(lengths, t)[:, None, :, None], 0)
    h = clean.permute(0, 2, 3, 1).float()
    y = (h * torch.rsqrt(h.square().mean(-1, keepdim=True) + eps) * weight.float()).to(x.dtype)
    return F.silu(y.float()).to(x.dtype) if silu else y


def bands(x):
    """``[B, C, T, F]`` -> ``[B, T, 8, C]`` adaptive frequency average."""
    return F.adaptive_avg_pool2d(x.float(), (x.shape[2], 8)).to(x.dtype).permute(0, 2, 3, 1).contiguous()


def evidence_norm(x, value, gate, weight, mask, eps=1e-5):
    """fp32 ``rms(mask ? x + value * 2 sigmoid(gate) : 0) * weight``."""
    s = x.float() + value.float() * (2 * torch.sigmoid(gate.float()))
    y = s * torch.rsqrt(s.square().mean(-1, keepdim=True) + eps) * weight.float()
    return y if mask is None else mask_rows(y, mask)


def gated_concat(x, gate):
    """Each third of the last dim scaled by ``2 sigmoid`` of its gate column."""
    return (x.float().reshape(*x.shape[:-1], 3, -1) * (2 * gate.float().sigmoid())[..., None]).reshape_as(x).to(
        x.dtype
    )


def _bf(x):
    return x.to(torch.bfloat16).float()


def front_stage(x, lengths, conv1, conv2, skip, norm1, norm2, stride, eps=1e-5):
    """CNN stage ``[B, C, T, F] -> [B, T', F', C']`` (bf16), ``lengths`` the
    stage's output lengths; ``conv1``/``conv2``/``skip`` the ``Conv2d`` weights
    ``[cout, cin, k, k]``, ``norm1``/``norm2`` the RMSNorm weights."""
    def conv(v, w, s, pad):
        return _bf(F.conv2d(_bf(v), _bf(w), stride=s, padding=pad))

    h = conv(x, conv1, (stride, 2), 1)
    h = front_norm(h.to(torch.bfloat16), lengths, norm1, eps, silu=True).permute(0, 3, 1, 2)
    h = front_norm(conv(h, conv2, 1, 1).to(torch.bfloat16), lengths, norm2, eps).float()
    valid = time_mask(lengths, h.shape[1])[:, :, None, None]
    sk = conv(x, skip, (stride, 2), 0).permute(0, 2, 3, 1).masked_fill(~valid, 0)
    return F.silu(_bf(h + sk)).masked_fill(~valid, 0).to(torch.bfloat16)


BF16 = torch.bfloat16


def block_pre(x, lengths, weight, eps=1e-5):
    """``(mask(x), bf16(pre(x)), bf16(pool4(pre(x))))`` of the fp32 stream."""
    xm = mask_rows(x.float(), time_mask(lengths, x.shape[1]))
    h = rms_norm(xm, weight, eps)
    return xm, h.to(BF16), pool4(h, lengths).to(BF16)


def glu_depthwise(up, weight, bias, lengths):
    """``depthwise_masked(F.glu(up))`` on bf16 values."""
    return depthwise_masked(F.glu(up.float(), -1).to(BF16), weight.to(BF16), bias.to(BF16), lengths)


def norm_silu(x, weight, eps=1e-5):
    """``silu(rms_norm(x))`` of bf16 rows, each rounded to bf16."""
    return F.silu(rms_norm(x.to(BF16), weight, eps).float()).to(BF16)


def pooled_attention(qkv, cos, sin, low_lengths, heads):
    """Rotary q/k (bf16), fp32 masked SDPA, heads merged: ``[B, T, H D]`` bf16."""
    b, t, _ = qkv.shape
    q, k, v = rotary_qkv(qkv.to(BF16), cos, sin, heads).float().unbind(0)
    mask = time_mask(low_lengths, t)[:, None, None, :]
    y = F.scaled_dot_product_attention(q, k, v, attn_mask=mask)
    return y.transpose(1, 2).reshape(b, t, -1).to(BF16)


def evidence_down(cn, an, weight, bias):
    """``silu(e_down(cat(cn, an)))`` under autocast: ``bf16(silu(bf16(cat w^T + b)))``."""
    s = torch.cat((cn.to(BF16).float(), an.to(BF16).float()), -1)
    z = (s @ weight.to(BF16).float().t() + bias.to(BF16).float()).to(BF16)
    return F.silu(z.float()).to(BF16)


def merge_gate(cn, mf, mb, an, weight, gate_w, gate_b, eps=1e-5):
    """``mn = mean_norm(mf, mb)`` (fp32) and the gate linear of ``cat(cn, mn, an)``
    under autocast (bf16 operands, fp32 sums, bf16 result)."""
    mn = mean_norm(mf, mb, weight, eps)
    s = torch.cat((cn.float(), mn, an.float()), -1).to(BF16).float()
    g = s @ gate_w.to(BF16).float().t() + gate_b.to(BF16).float()
    return mn, g.to(BF16)


def merge_conv(cn, mn, an, g, weight, bias, lengths):
    """``bf16(v + depthwise_masked(bf16(v)))`` with ``v = gated_concat(cat(cn, mn, an), g)``
    in fp32."""
    v = gated_concat(torch.cat((cn.float(), mn.float(), an.float()), -1), g)
    conv = depthwise_masked(v.to(BF16), weight.to(BF16), bias.to(BF16), lengths).float()
    return (v + conv).to(BF16)


def query_read(q, kv, key_lengths, heads=8):
    """``q [Q, heads D]``, ``kv [B, T, 2 heads D]`` -> ``[B, Q, heads D]`` bf16: fp32
    SDPA with keys ``j < key_lengths[b]``."""
    b, t, width = kv.shape
    nq, qw = q.shape
    d = qw // heads
    k, v = kv.float().view(b, t, 2, heads, d).permute(2, 0, 3, 1, 4).unbind(0)
    qq = q.float().view(nq, heads, d).transpose(0, 1).unsqueeze(0).expand(b, -1, -1, -1)
    mask = time_mask(key_lengths, t)[:, None, None, :]
    y = F.scaled_dot_product_attention(qq, k, v, attn_mask=mask)
    return y.transpose(1, 2).reshape(b, nq, qw).to(BF16)
