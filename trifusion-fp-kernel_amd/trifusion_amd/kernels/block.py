"""Kernels of the TriFusion block and front end on gfx950.

The reference model's buffer and native kernels, each one C-ABI launch
(``csrc/trifusion_block.hip``) behind a ``trifusion_amd::*`` operator:

* ``depthwise_masked`` (``src/trifusion_l4/kernels/buffers.py:13-32``);
* ``Pool4.apply`` (``buffers.py:35-44``) and ``interpolate``
  (``src/trifusion_l4/kernels/native.py:119-133``), the 4:1 pooled attention
  grid and the way back to frames;
* ``RotaryQKV.apply`` (``buffers.py:46-56``);
* ``front_norm`` (``buffers.py:58-80``) and ``bands`` (``native.py:157-163``)
  of the CNN front end, and ``front_stage``: a whole CNN stage (``front.py:19-43``:
  both convolutions, norms, skip, residual and SiLU) in two fused kernels;
* ``evidence_norm`` (``native.py:73-74``) and ``gated_concat``
  (``src/trifusion_l4/kernels/__init__.py:58-82``) of the block's merge.

They are re-exported under the reference's module paths
(``kernels.buffers``, ``kernels.native``, ``kernels``).
"""

import ctypes

import torch

from .. import _lib
from ..ops import ops


def _autocast_dtype(x):
    if torch.is_autocast_enabled("cuda"):
        return torch.get_autocast_dtype("cuda")
    return x.dtype


def _strides(x):
    return (ctypes.c_int64 * 4)(*x.stride())


def _row_stride(t):
    """Common stride of the rows of ``t`` (last dim contiguous, leading dims
    collapsible to one row index), or None."""
    if t.dim() == 0 or t.stride(-1) != 1 and t.shape[-1] > 1:
        return None
    stride = t.stride(-2) if t.dim() > 1 else t.shape[-1]
    expect = stride
    for i in range(t.dim() - 2, -1, -1):
        if t.shape[i] > 1 and t.stride(i) != expect:
            return None
        expect *= t.shape[i]
    return stride


def depthwise_masked(x, layer, lengths):
    """Masked depthwise Conv1d over time (``layer``: ``Conv1d(D, D, K,
    padding=K//2, groups=D)``) on ``[B, T, D]``; rows past each length are 0.
    Computes in the autocast dtype like the reference (``trifusion_amd::depthwise_masked``)."""
    dtype = _autocast_dtype(x)
    return ops.depthwise_masked(x.to(dtype), layer.weight.to(dtype), layer.bias.to(dtype), lengths)


def launch_depthwise_masked(x, weight, bias, lengths):
    lib = _lib.load()
    _lib.require_cuda(x, weight, bias, lengths, what="depthwise_masked")
    b, t, d = x.shape
    k = weight.shape[-1]
    if weight.numel() != d * k or bias.shape != (d,) or weight.dtype != x.dtype or bias.dtype != x.dtype:
        raise ValueError("depthwise_masked: weight must be [D, 1, K] and bias [D], both of x's dtype")
    if k % 2 == 0:
        raise ValueError("depthwise_masked: odd kernel sizes only (same padding)")
    x = x.contiguous()
    y = torch.empty_like(x)
    status = lib.tf_depthwise_masked(
        x.data_ptr(), weight.contiguous().data_ptr(), bias.contiguous().data_ptr(),
        _lib.dtype_code(x, "depthwise_masked"), lengths.to(torch.int64).contiguous().data_ptr(), y.data_ptr(),
        b, t, d, k, _lib.stream_of(x),
    )
    _lib.check(status, "depthwise_masked")
    return y


class Pool4:
    @staticmethod
    def apply(x, lengths):
        """Masked 4:1 average over time, ``[B, T, D] -> [B, ceil(T/4), D]``
        (``trifusion_amd::pool4``)."""
        return ops.pool4(x, lengths)


def launch_pool4(x, lengths):
    lib = _lib.load()
    _lib.require_cuda(x, lengths, what="pool4")
    x = x.contiguous()
    b, t, d = x.shape
    y = x.new_empty((b, (t + 3) // 4, d))
    status = lib.tf_pool4(x.data_ptr(), _lib.dtype_code(x, "pool4"), lengths.to(torch.int64).contiguous().data_ptr(),
                          y.data_ptr(), b, t, d, _lib.stream_of(x))
    _lib.check(status, "pool4")
    return y


class RotaryQKV:
    @staticmethod
    def apply(x, cos, sin, heads):
        """``[B, T, 3 H D]`` projection -> rotated ``[3, B, H, T, D]`` (q and k
        rotated by interleaved pairs, v copied) (``trifusion_amd::rotary_qkv``)."""
        return ops.rotary_qkv(x, cos, sin, int(heads))


def launch_rotary_qkv(x, cos, sin, heads):
    lib = _lib.load()
    _lib.require_cuda(x, cos, sin, what="rotary_qkv")
    x = x.contiguous()
    b, t, width = x.shape
    d = width // (3 * heads)
    if 3 * heads * d != width or d % 2:
        raise ValueError("rotary_qkv: width must be 3 * heads * head_dim with an even head_dim")
    cos = cos.float().contiguous()
    sin = sin.float().contiguous()
    if cos.shape != (t, d // 2) or sin.shape != (t, d // 2):
        raise ValueError(f"rotary_qkv: cos/sin must be [{t}, {d // 2}]")
    y = x.new_empty((3, b, heads, t, d))
    status = lib.tf_rotary_qkv(x.data_ptr(), _lib.dtype_code(x, "rotary_qkv"), cos.data_ptr(), sin.data_ptr(),
                               y.data_ptr(), b, t, heads, d, _lib.stream_of(x))
    _lib.check(status, "rotary_qkv")
    return y


def front_norm(x, lengths, norm, silu=False):
    """Channel RMSNorm of a ``[B, C, T, F]`` map (rows ``t >= lengths`` zero,
    optional SiLU after the rounding), returned as the ``[B, C, T, F]`` view of
    a channels-last buffer (``trifusion_amd::front_norm``)."""
    return ops.front_norm(x, lengths, norm.weight, float(norm.eps), bool(silu)).permute(0, 3, 1, 2)


def launch_front_norm(x, lengths, weight, eps, silu):
    lib = _lib.load()
    _lib.require_cuda(x, lengths, weight, what="front_norm")
    b, c, t, f = x.shape
    y = x.new_empty((b, t, f, c))
    status = lib.tf_front_norm(
        x.data_ptr(), _lib.dtype_code(x, "front_norm"), _strides(x), weight.float().contiguous().data_ptr(),
        lengths.to(torch.int64).contiguous().data_ptr(), y.data_ptr(), b, c, t, f, float(eps), int(silu),
        _lib.stream_of(x),
    )
    _lib.check(status, "front_norm")
    return y


def pack_conv3x3(weight):
    """``Conv2d`` 3x3 weight ``[cout, cin, 3, 3]`` -> tap-major bf16 ``[9, cout, cin]``
    (tap = 3 dy + dx), the layout the front-stage kernels read."""
    cout, cin = weight.shape[:2]
    return weight.detach().permute(2, 3, 0, 1).reshape(9, cout, cin).to(torch.bfloat16).contiguous()


def _aligned16(t):
    """``t`` contiguous at a 16-byte aligned address (the kernels load 16 bytes at a time)."""
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _stage_input(x, what):
    """Stage input ``[B, C, T, F]`` as the kernels read it: fp32 ``[B, T, F]`` for
    one channel, else bf16 channels-last ``[B, T, F, C]``."""
    b, c, t, f = x.shape
    if c == 1:
        if x.dtype != torch.float32:
            raise TypeError(f"{what}: a one-channel stage input is the fp32 log spectrogram, got {x.dtype}")
        return x.reshape(b, t, f).contiguous()
    if x.dtype != torch.bfloat16:
        raise TypeError(f"{what}: stage input must be bf16, got {x.dtype}")
    return _aligned16(x.permute(0, 2, 3, 1))


def front_stage(stage, x, lengths):
    """One CNN stage of the front end (``front.py:19-43``) in two fused kernels:
    ``x [B, C, T, F]`` (fp32 with one channel, else bf16) -> bf16 ``[B, C', T', F']``
    view of a channels-last buffer. ``lengths`` are the stage's output lengths.
    ``stage`` provides ``stride``, ``packed()`` -> (conv1, conv2, skip) weights and
    the two norms (``trifusion_amd::front_conv1`` / ``front_conv2``)."""
    w1, w2, ws = stage.packed()
    n1, n2 = stage.norm1, stage.norm2
    h = ops.front_conv1(x, w1, n1.weight, lengths, int(stage.stride), float(n1.eps))
    y = ops.front_conv2(h, w2, n2.weight, x, ws, lengths, int(stage.stride), float(n2.eps))
    return y.permute(0, 3, 1, 2)


def _out_grid(x, stride):
    _, _, t, f = x.shape
    return (t - 1) // stride + 1, (f - 1) // 2 + 1


def launch_front_conv1(x, weight, norm_weight, lengths, stride, eps):
    lib = _lib.load()
    _lib.require_cuda(x, weight, norm_weight, lengths, what="front_conv1")
    b, cin, t, f = x.shape
    cout = weight.shape[1]
    if weight.shape != (9, cout, cin) or weight.dtype != torch.bfloat16 or norm_weight.shape != (cout,):
        raise ValueError("front_conv1: weight must be bf16 [9, cout, cin] and the norm weight [cout]")
    xs = _stage_input(x, "front_conv1")
    w = _aligned16(weight)
    to, fo = _out_grid(x, stride)
    y = torch.empty((b, to, fo, cout), device=x.device, dtype=torch.bfloat16)
    status = lib.tf_front_conv1(
        xs.data_ptr(), _lib.dtype_code(xs, "front_conv1"), w.data_ptr(), norm_weight.float().contiguous().data_ptr(),
        lengths.to(torch.int64).contiguous().data_ptr(), y.data_ptr(), b, t, f, cin, cout, int(stride), float(eps),
        _lib.stream_of(x),
    )
    _lib.check(status, "front_conv1")
    return y


def launch_front_conv2(h, weight, norm_weight, x, skip_weight, lengths, stride, eps):
    lib = _lib.load()
    _lib.require_cuda(h, weight, norm_weight, x, skip_weight, lengths, what="front_conv2")
    b, cin, t, f = x.shape
    to, fo = _out_grid(x, stride)
    cout = h.shape[-1]
    if h.shape != (b, to, fo, cout) or h.dtype != torch.bfloat16:
        raise ValueError(f"front_conv2: h must be bf16 [{b}, {to}, {fo}, cout], got {tuple(h.shape)} {h.dtype}")
    if weight.shape != (9, cout, cout) or weight.dtype != torch.bfloat16 or norm_weight.shape != (cout,):
        raise ValueError("front_conv2: weight must be bf16 [9, cout, cout] and the norm weight [cout]")
    if skip_weight.shape != (cout, cin) or skip_weight.dtype != torch.bfloat16:
        raise ValueError("front_conv2: skip weight must be bf16 [cout, cin]")
    xs = _stage_input(x, "front_conv2")
    hc, w, ws = _aligned16(h), _aligned16(weight), _aligned16(skip_weight)
    y = torch.empty_like(hc)
    status = lib.tf_front_conv2(
        hc.data_ptr(), w.data_ptr(), norm_weight.float().contiguous().data_ptr(), xs.data_ptr(),
        _lib.dtype_code(xs, "front_conv2"), ws.data_ptr(), lengths.to(torch.int64).contiguous().data_ptr(),
        y.data_ptr(), b, t, f, cin, cout, int(stride), float(eps), _lib.stream_of(x),
    )
    _lib.check(status, "front_conv2")
    return y


def interpolate(low, grids):
    """Pooled grid -> frames by the grid's left/right/alpha, rows past the
    lengths zero (``trifusion_amd::interpolate``)."""
    return ops.interpolate(low, grids.left, grids.right, grids.alpha, grids.lengths)


def launch_interpolate(low, left, right, alpha, lengths):
    lib = _lib.load()
    _lib.require_cuda(low, left, right, alpha, lengths, what="interpolate")
    low = low.contiguous()
    b, lt, d = low.shape
    t = left.shape[1]
    y = low.new_empty((b, t, d))
    status = lib.tf_interpolate(
        low.data_ptr(), _lib.dtype_code(low, "interpolate"), left.to(torch.int64).contiguous().data_ptr(),
        right.to(torch.int64).contiguous().data_ptr(), alpha.float().contiguous().data_ptr(),
        lengths.to(torch.int64).contiguous().data_ptr(), y.data_ptr(), b, t, lt, d, _lib.stream_of(low),
    )
    _lib.check(status, "interpolate")
    return y


def interpolate_rmsnorm_fits(low):
    """Rows ``tf_interpolate_rmsnorm`` takes: a width that is a multiple of 8 up to 4096."""
    d = low.shape[-1]
    return d % 8 == 0 and 8 <= d <= 4096


def interpolate_rmsnorm(low, grids, norm):
    """``norm(interpolate(low, grids))`` in one pass, the values the two
    launches give (``trifusion_amd::interpolate_rmsnorm``)."""
    return ops.interpolate_rmsnorm(low, grids.left, grids.right, grids.alpha, grids.lengths, norm.weight,
                                   float(norm.eps))


def launch_interpolate_rmsnorm(low, left, right, alpha, lengths, weight, eps):
    lib = _lib.load()
    _lib.require_cuda(low, left, right, alpha, lengths, weight, what="interpolate_rmsnorm")
    low = _aligned16(low)
    b, lt, d = low.shape
    t = left.shape[1]
    if weight.shape != (d,):
        raise ValueError(f"interpolate_rmsnorm: weight must be [{d}]")
    w = _aligned16(weight.float())
    y = low.new_empty((b, t, d))
    status = lib.tf_interpolate_rmsnorm(
        low.data_ptr(), _lib.dtype_code(low, "interpolate_rmsnorm"), left.to(torch.int64).contiguous().data_ptr(),
        right.to(torch.int64).contiguous().data_ptr(), alpha.float().contiguous().data_ptr(),
        lengths.to(torch.int64).contiguous().data_ptr(), w.data_ptr(), float(eps), y.data_ptr(), b, t, lt, d,
        _lib.stream_of(low),
    )
    _lib.check(status, "interpolate_rmsnorm")
    return y


def bands(x):
    """``[B, C, T, F]`` -> ``[B, T, 8, C]`` frequency-band means (``trifusion_amd::bands``)."""
    return ops.bands(x)


def launch_bands(x):
    lib = _lib.load()
    _lib.require_cuda(x, what="bands")
    b, c, t, f = x.shape
    y = x.new_empty((b, t, 8, c))
    status = lib.tf_bands(x.data_ptr(), _lib.dtype_code(x, "bands"), _strides(x), y.data_ptr(), b, c, t, f,
                          _lib.stream_of(x))
    _lib.check(status, "bands")
    return y


def evidence_norm(x, value, gate, weight, mask, eps=1e-5, bf16_out=False):
    """``rms(mask ? x + value * 2 sigmoid(gate) : 0) * weight`` in fp32, stored as
    fp32 or, with ``bf16_out``, rounded to bf16 for a consumer that would cast it
    (``trifusion_amd::evidence_norm``)."""
    return ops.evidence_norm(x, value, gate, weight, mask, float(eps), bool(bf16_out))


def launch_evidence_norm(x, value, gate, weight, mask, eps=1e-5, bf16_out=False):
    lib = _lib.load()
    _lib.require_cuda(x, value, gate, weight, mask, what="evidence_norm")
    x = x.float().contiguous()
    if value.dtype != gate.dtype:
        gate = gate.to(value.dtype)
    d = x.shape[-1]
    rows = x.numel() // d
    if value.shape != x.shape or gate.shape != x.shape:
        raise ValueError("evidence_norm: value and gate must match x")
    # value and gate may be column halves of one projection: rows a common stride apart
    stride = _row_stride(value)
    if stride is None or _row_stride(gate) != stride:
        value, gate = value.contiguous(), gate.contiguous()
        stride = d
    m = None
    if mask is not None:
        if mask.dtype != torch.bool or mask.numel() != rows:
            raise ValueError("evidence_norm: mask must be bool with one entry per row")
        m = mask.contiguous().data_ptr()
    y = torch.empty(x.shape, device=x.device, dtype=torch.bfloat16 if bf16_out else torch.float32)
    status = lib.tf_evidence_norm(x.data_ptr(), value.data_ptr(), gate.data_ptr(),
                                  _lib.dtype_code(value, "evidence_norm"), stride, m,
                                  weight.float().contiguous().data_ptr(),
                                  y.data_ptr(), _lib.dtype_code(y, "evidence_norm"), rows, d, float(eps),
                                  _lib.stream_of(x))
    _lib.check(status, "evidence_norm")
    return y


def gated_concat(x, gate):
    """``x [..., 3d]`` with each third scaled by ``2 sigmoid(gate[..., k])``
    (``trifusion_amd::gated_concat``)."""
    return ops.gated_concat(x, gate)


def launch_gated_concat(x, gate):
    lib = _lib.load()
    _lib.require_cuda(x, gate, what="gated_concat")
    x = x.contiguous()
    gate = gate.to(x.dtype).contiguous()
    if x.shape[-1] % 3 or gate.shape[-1] != 3 or gate.numel() * (x.shape[-1] // 3) != x.numel():
        raise ValueError("gated_concat: x [..., 3d] and gate [..., 3]")
    d = x.shape[-1] // 3
    y = torch.empty_like(x)
    status = lib.tf_gated_concat(x.data_ptr(), gate.data_ptr(), _lib.dtype_code(x, "gated_concat"), y.data_ptr(),
                                 gate.numel() // 3, d, _lib.stream_of(x))
    _lib.check(status, "gated_concat")
    return y


# ---- fused block kernels (csrc/block_fused.hip) ----


def _bf16(t, what, name):
    if t.dtype != torch.bfloat16:
        raise TypeError(f"{what}: {name} must be bf16, got {t.dtype}")
    return _aligned16(t)


def _lengths(lengths):
    return lengths.to(torch.int64).contiguous()


def block_pre(x, lengths, norm):
    """Start of a block: ``(mask(x) fp32, bf16(pre(x)), bf16(pool4(pre(x))))``
    (``trifusion_amd::block_pre``)."""
    return ops.block_pre(x, lengths, norm.weight, float(norm.eps))


def launch_block_pre(x, lengths, weight, eps):
    lib = _lib.load()
    _lib.require_cuda(x, lengths, weight, what="block_pre")
    if x.dtype != torch.float32 or x.dim() != 3:
        raise TypeError("block_pre: x must be fp32 [B, T, d]")
    b, t, d = x.shape
    xc, w = _aligned16(x), _aligned16(weight.float())
    xm = torch.empty_like(xc)
    h = torch.empty((b, t, d), device=x.device, dtype=torch.bfloat16)
    p = torch.empty((b, (t + 3) // 4, d), device=x.device, dtype=torch.bfloat16)
    status = lib.tf_block_pre(xc.data_ptr(), _lengths(lengths).data_ptr(), w.data_ptr(), float(eps), xm.data_ptr(),
                              h.data_ptr(), p.data_ptr(), b, t, d, _lib.stream_of(x))
    _lib.check(status, "block_pre")
    return xm, h, p


def block_pre_add_fits(x, addend):
    """``block_pre_add`` takes an fp32 residual and a bf16 addend of one shape."""
    return x.dtype == torch.float32 and addend.dtype == torch.bfloat16 and x.shape == addend.shape


def block_pre_add(x, addend, lengths, norm):
    """``block_pre(add(x, addend, mask))`` in one launch, the values of the two
    (``trifusion_amd::block_pre_add``)."""
    return ops.block_pre_add(x, addend, lengths, norm.weight, float(norm.eps))


def launch_block_pre_add(x, addend, lengths, weight, eps):
    lib = _lib.load()
    _lib.require_cuda(x, addend, lengths, weight, what="block_pre_add")
    if x.dtype != torch.float32 or x.dim() != 3 or not block_pre_add_fits(x, addend):
        raise TypeError("block_pre_add: x must be fp32 [B, T, d] and addend bf16 of the same shape")
    b, t, d = x.shape
    xc, ac, w = _aligned16(x), _aligned16(addend), _aligned16(weight.float())
    xm = torch.empty_like(xc)
    h = torch.empty((b, t, d), device=x.device, dtype=torch.bfloat16)
    p = torch.empty((b, (t + 3) // 4, d), device=x.device, dtype=torch.bfloat16)
    status = lib.tf_block_pre_add(xc.data_ptr(), ac.data_ptr(), _lengths(lengths).data_ptr(), w.data_ptr(),
                                  float(eps), xm.data_ptr(), h.data_ptr(), p.data_ptr(), b, t, d,
                                  _lib.stream_of(x))
    _lib.check(status, "block_pre_add")
    return xm, h, p


def norm_silu(x, norm):
    """``silu(norm(x))`` of bf16 rows, both rounded to bf16 (``trifusion_amd::norm_silu``)."""
    return ops.norm_silu(x, norm.weight, float(norm.eps))


def launch_norm_silu(x, weight, eps):
    lib = _lib.load()
    _lib.require_cuda(x, weight, what="norm_silu")
    xc, w = _bf16(x, "norm_silu", "x"), _aligned16(weight.float())
    d = x.shape[-1]
    y = torch.empty_like(xc)
    status = lib.tf_norm_silu(xc.data_ptr(), w.data_ptr(), y.data_ptr(), x.numel() // d, d, float(eps),
                              _lib.stream_of(x))
    _lib.check(status, "norm_silu")
    return y


def glu_depthwise(up, layer, lengths):
    """``depthwise_masked(F.glu(up), layer, lengths)`` in bf16 (``trifusion_amd::glu_depthwise``)."""
    return ops.glu_depthwise(up, layer.weight, layer.bias, lengths)


def launch_glu_depthwise(up, weight, bias, lengths):
    lib = _lib.load()
    _lib.require_cuda(up, weight, bias, lengths, what="glu_depthwise")
    uc = _bf16(up, "glu_depthwise", "up")
    b, t, d2 = uc.shape
    d, k = d2 // 2, weight.shape[-1]
    if weight.numel() != d * k or bias.shape != (d,):
        raise ValueError("glu_depthwise: weight must be [d, 1, k] and bias [d]")
    w = _aligned16(weight.to(torch.bfloat16))
    bb = _aligned16(bias.to(torch.bfloat16))
    y = torch.empty((b, t, d), device=up.device, dtype=torch.bfloat16)
    status = lib.tf_glu_depthwise(uc.data_ptr(), w.data_ptr(), bb.data_ptr(), _lengths(lengths).data_ptr(),
                                  y.data_ptr(), b, t, d, k, _lib.stream_of(up))
    _lib.check(status, "glu_depthwise")
    return y


def glu_norm_silu_fits(up, layer):
    """Shapes ``tf_glu_depthwise_norm_silu`` takes: d a multiple of 8 up to 1024, k 3 or 7."""
    d = up.shape[-1] // 2
    return d % 8 == 0 and 8 <= d <= 1024 and layer.weight.shape[-1] in (3, 7)


def glu_norm_silu(up, layer, lengths, norm):
    """``norm_silu(glu_depthwise(up, layer, lengths), norm)`` in one launch, the
    values of the two (``trifusion_amd::glu_norm_silu``)."""
    return ops.glu_norm_silu(up, layer.weight, layer.bias, lengths, norm.weight, float(norm.eps))


def launch_glu_norm_silu(up, weight, bias, lengths, norm_weight, eps):
    lib = _lib.load()
    _lib.require_cuda(up, weight, bias, lengths, norm_weight, what="glu_norm_silu")
    uc = _bf16(up, "glu_norm_silu", "up")
    b, t, d2 = uc.shape
    d, k = d2 // 2, weight.shape[-1]
    if weight.numel() != d * k or bias.shape != (d,) or norm_weight.shape != (d,):
        raise ValueError("glu_norm_silu: weight must be [d, 1, k], bias and norm weight [d]")
    w = _aligned16(weight.to(torch.bfloat16))
    bb = _aligned16(bias.to(torch.bfloat16))
    nw = _aligned16(norm_weight.float())
    y = torch.empty((b, t, d), device=up.device, dtype=torch.bfloat16)
    status = lib.tf_glu_depthwise_norm_silu(uc.data_ptr(), w.data_ptr(), bb.data_ptr(), _lengths(lengths).data_ptr(),
                                            nw.data_ptr(), float(eps), y.data_ptr(), b, t, d, k, _lib.stream_of(up))
    _lib.check(status, "glu_norm_silu")
    return y


def pooled_attention(qkv, grids, heads):
    """Rotary + masked attention on the pooled grid: ``qkv [B, T, 3 H D]`` bf16 ->
    ``[B, T, H D]`` bf16 (``trifusion_amd::pooled_attention``)."""
    return ops.pooled_attention(qkv, grids.rope_cos, grids.rope_sin, grids.low_lengths, int(heads))


def launch_pooled_attention(qkv, cos, sin, low_lengths, heads):
    lib = _lib.load()
    _lib.require_cuda(qkv, cos, sin, low_lengths, what="pooled_attention")
    qc = _bf16(qkv, "pooled_attention", "qkv")
    b, t, width = qc.shape
    hd = width // (3 * heads)
    if width != 3 * heads * hd or cos.shape != (t, hd // 2) or sin.shape != (t, hd // 2):
        raise ValueError("pooled_attention: qkv must be [B, T, 3 H D] with cos/sin [T, D/2]")
    y = torch.empty((b, t, heads * hd), device=qkv.device, dtype=torch.bfloat16)
    status = lib.tf_pooled_attention(qc.data_ptr(), cos.float().contiguous().data_ptr(),
                                     sin.float().contiguous().data_ptr(), _lengths(low_lengths).data_ptr(),
                                     y.data_ptr(), b, t, heads, hd, _lib.stream_of(qkv))
    _lib.check(status, "pooled_attention")
    return y


def merge_gate(cn, mf, mb, an, norm, gate):
    """``(mean_norm(mf, mb) fp32, gate(cat(cn, mn, an)) bf16 [.., 3])``
    (``trifusion_amd::merge_gate``)."""
    return ops.merge_gate(cn, mf, mb, an, norm.weight, float(norm.eps), gate.weight, gate.bias)


def launch_merge_gate(cn, mf, mb, an, norm_weight, eps, gate_weight, gate_bias):
    lib = _lib.load()
    _lib.require_cuda(cn, mf, mb, an, norm_weight, gate_weight, gate_bias, what="merge_gate")
    cc, fc, bc, ac = (_bf16(t, "merge_gate", n) for t, n in ((cn, "cn"), (mf, "mf"), (mb, "mb"), (an, "an")))
    d = cc.shape[-1]
    rows = cc.numel() // d
    if any(t.shape != cc.shape for t in (fc, bc, ac)) or gate_weight.shape != (3, 3 * d) or gate_bias.shape != (3,):
        raise ValueError("merge_gate: cn, mf, mb, an must match and the gate be Linear(3 d, 3)")
    gw = _aligned16(gate_weight.to(torch.bfloat16))
    gb = gate_bias.to(torch.bfloat16).contiguous()
    w = _aligned16(norm_weight.float())
    mn = torch.empty(cc.shape, device=cn.device, dtype=torch.float32)
    g = torch.empty((*cc.shape[:-1], 3), device=cn.device, dtype=torch.bfloat16)
    status = lib.tf_merge_gate(cc.data_ptr(), fc.data_ptr(), bc.data_ptr(), ac.data_ptr(), w.data_ptr(), float(eps),
                               gw.data_ptr(), gb.data_ptr(), mn.data_ptr(), g.data_ptr(), rows, d, _lib.stream_of(cn))
    _lib.check(status, "merge_gate")
    return mn, g


def evidence_down_fits(d, r):
    """Widths ``tf_evidence_down`` takes: ``d`` a multiple of 128, ``r`` one of 16, 32, 48, 64."""
    return d >= 128 and d % 128 == 0 and r in (16, 32, 48, 64)


def evidence_down(cn, an, layer):
    """``silu(layer(cat(cn, an)))`` for the block's ``e_down`` under autocast, with no
    concatenated copy (``trifusion_amd::evidence_down``)."""
    return ops.evidence_down(cn, an, layer.weight, layer.bias)


def launch_evidence_down(cn, an, weight, bias):
    lib = _lib.load()
    _lib.require_cuda(cn, an, weight, bias, what="evidence_down")
    cc, ac = _bf16(cn, "evidence_down", "cn"), _bf16(an, "evidence_down", "an")
    d = cc.shape[-1]
    r = weight.shape[0]
    if ac.shape != cc.shape or weight.shape != (r, 2 * d) or bias.shape != (r,):
        raise ValueError("evidence_down: cn and an must match and the layer be Linear(2 d, r)")
    if not evidence_down_fits(d, r):
        raise ValueError(f"evidence_down: needs d a multiple of 128 and r in (16, 32, 48, 64), got d={d}, r={r}")
    w = _aligned16(weight.to(torch.bfloat16))
    b = bias.to(torch.bfloat16).contiguous()
    z = torch.empty((*cc.shape[:-1], r), device=cn.device, dtype=torch.bfloat16)
    rows = cc.numel() // d
    status = lib.tf_evidence_down(cc.data_ptr(), ac.data_ptr(), w.data_ptr(), b.data_ptr(), z.data_ptr(), rows, d, r,
                                  _lib.stream_of(cn))
    _lib.check(status, "evidence_down")
    return z


def merge_conv(cn, mn, an, g, layer, lengths):
    """``add(v, depthwise_masked(v, layer), bf16=True)`` with ``v = gated_concat(cat(cn,
    mn, an), g)`` (``trifusion_amd::merge_conv``)."""
    return ops.merge_conv(cn, mn, an, g, layer.weight, layer.bias, lengths)


def launch_merge_conv(cn, mn, an, g, weight, bias, lengths):
    lib = _lib.load()
    _lib.require_cuda(cn, mn, an, g, weight, bias, lengths, what="merge_conv")
    cc, ac, gc = _bf16(cn, "merge_conv", "cn"), _bf16(an, "merge_conv", "an"), _bf16(g, "merge_conv", "g")
    if mn.dtype != torch.float32:
        raise TypeError("merge_conv: mn must be fp32")
    mc = _aligned16(mn)
    b, t, d = cc.shape
    k = weight.shape[-1]
    if mc.shape != cc.shape or ac.shape != cc.shape or gc.shape != (b, t, 3):
        raise ValueError("merge_conv: cn, mn, an must be [B, T, d] and g [B, T, 3]")
    if weight.numel() != 3 * d * k or bias.shape != (3 * d,):
        raise ValueError("merge_conv: weight must be [3 d, 1, k] and bias [3 d]")
    w = _aligned16(weight.to(torch.bfloat16))
    bb = _aligned16(bias.to(torch.bfloat16))
    y = torch.empty((b, t, 3 * d), device=cn.device, dtype=torch.bfloat16)
    status = lib.tf_merge_conv(cc.data_ptr(), mc.data_ptr(), ac.data_ptr(), gc.data_ptr(), w.data_ptr(),
                               bb.data_ptr(), _lengths(lengths).data_ptr(), y.data_ptr(), b, t, d, k,
                               _lib.stream_of(cn))
    _lib.check(status, "merge_conv")
    return y


def query_read(q, kv, key_lengths, heads=8):
    """Decoder query read: ``q [Q, heads D]`` (bf16, shared by the batch), ``kv
    [B, T, 2 heads D]`` -> ``[B, Q, heads D]`` bf16, fp32 softmax over keys
    ``j < key_lengths`` (``trifusion_amd::query_read``)."""
    return ops.query_read(q, kv, key_lengths, int(heads))


def launch_query_read(q, kv, key_lengths, heads):
    lib = _lib.load()
    _lib.require_cuda(q, kv, key_lengths, what="query_read")
    qc, kc = _bf16(q, "query_read", "q"), _bf16(kv, "query_read", "kv")
    b, t, width = kc.shape
    nq, qw = qc.shape
    d = qw // heads
    if width != 2 * qw or qw != heads * d:
        raise ValueError("query_read: kv must be [B, T, 2 heads D] and q [Q, heads D]")
    y = torch.empty((b, nq, qw), device=kv.device, dtype=torch.bfloat16)
    size = lib.tf_query_read_workspace_size(b, t, heads, nq, d)
    ws = torch.empty((max(size, 4),), device=kv.device, dtype=torch.uint8)
    status = lib.tf_query_read(qc.data_ptr(), kc.data_ptr(), _lengths(key_lengths).data_ptr(), y.data_ptr(),
                               ws.data_ptr(), ws.numel(), b, t, heads, nq, d, _lib.stream_of(kv))
    _lib.check(status, "query_read")
    return y


# ---- front-end preparations (csrc/front_prep.hip) ----


def mask_audio(audio, lengths, channels):
    """``[B, C, N]`` waveform -> fp32 ``[B C, N]`` with samples past each length and
    channels past each channel count cleared (``trifusion_amd::mask_audio``)."""
    return ops.mask_audio(audio, lengths, channels)


def launch_mask_audio(audio, lengths, channels):
    lib = _lib.load()
    _lib.require_cuda(audio, lengths, channels, what="mask_audio")
    x = audio.float().contiguous()
    b, c, n = x.shape
    y = torch.empty((b * c, n), device=x.device, dtype=torch.float32)
    status = lib.tf_mask_audio(x.data_ptr(), _lengths(lengths).data_ptr(), _lengths(channels).data_ptr(),
                               y.data_ptr(), b, c, n, _lib.stream_of(x))
    _lib.check(status, "mask_audio")
    return y


def log_power(spec, channels, sample_lengths, hop=160):
    """complex ``[B C, bins, frames]`` STFT -> fp32 ``[B, frames, bins]`` log power
    averaged over channels, frames past each clip's count 0 (``trifusion_amd::log_power``)."""
    return ops.log_power(spec, channels, sample_lengths, int(hop))


def launch_log_power(spec, channels, sample_lengths, hop):
    lib = _lib.load()
    _lib.require_cuda(spec, channels, sample_lengths, what="log_power")
    if spec.dtype != torch.complex64:
        raise TypeError("log_power: spectrum must be complex64")
    bc, bins, frames = spec.shape
    b = channels.shape[0]
    if bc % b:
        raise ValueError("log_power: spectrum rows must be batch x channels")
    y = torch.empty((b, frames, bins), device=spec.device, dtype=torch.float32)
    status = lib.tf_log_power(spec.data_ptr(), (ctypes.c_int64 * 3)(*spec.stride()), _lengths(channels).data_ptr(),
                              _lengths(sample_lengths).data_ptr(), y.data_ptr(), b, bc // b, bins, frames, hop,
                              _lib.stream_of(spec))
    _lib.check(status, "log_power")
    return y


def front_lengths(sample_lengths, hop=160, strides=(1, 2, 2)):
    """int64 ``[4, B]``: frames ``n // hop + 1`` and the counts after each CNN stage
    (``trifusion_amd::front_lengths``)."""
    return ops.front_lengths(sample_lengths, int(hop), [int(s) for s in strides])


def launch_front_lengths(sample_lengths, hop, strides):
    lib = _lib.load()
    _lib.require_cuda(sample_lengths, what="front_lengths")
    n = _lengths(sample_lengths)
    out = torch.empty((4, n.shape[0]), device=n.device, dtype=torch.int64)
    status = lib.tf_front_lengths(n.data_ptr(), out.data_ptr(), n.shape[0], hop, (ctypes.c_int64 * 3)(*strides),
                                  _lib.stream_of(n))
    _lib.check(status, "front_lengths")
    return out


def grids(lengths, time):
    """``(mask, low_lengths, low_mask, left, right, alpha)`` of the frame grid and its
    4:1 pooled grid (``trifusion_amd::grids``)."""
    return ops.grids(lengths, int(time))


def launch_grids(lengths, time):
    lib = _lib.load()
    _lib.require_cuda(lengths, what="grids")
    n = _lengths(lengths)
    b, dev = n.shape[0], n.device
    lt = (time + 3) // 4
    mask = torch.empty((b, time), device=dev, dtype=torch.bool)
    low = torch.empty((b,), device=dev, dtype=torch.int64)
    low_mask = torch.empty((b, lt), device=dev, dtype=torch.bool)
    left = torch.empty((b, time), device=dev, dtype=torch.int64)
    right = torch.empty((b, time), device=dev, dtype=torch.int64)
    alpha = torch.empty((b, time), device=dev, dtype=torch.float32)
    status = lib.tf_grids(n.data_ptr(), mask.data_ptr(), low.data_ptr(), low_mask.data_ptr(), left.data_ptr(),
                          right.data_ptr(), alpha.data_ptr(), b, time, _lib.stream_of(n))
    _lib.check(status, "grids")
    return mask, low, low_mask, left, right, alpha
