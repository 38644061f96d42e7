"""One-pass Mamba-3 SISO inference recurrence on MI355X (gfx950).

Drop-in for the reference's ``fused_mamba`` (``src/trifusion_l4/mamba_fused.py:155-191``):
same name, positional order and ``warps`` keyword, output allocated like
``torch.empty_like(v, memory_format=torch.contiguous_format)`` (``:161``), launch
on the current stream, forward only. Shapes are generalised from the
reference's fixed N=128, P=64, R=32 (``:159-160``) to N in {16, 32, 64, 128},
P in {32, 64} and any R <= N/2; other dims raise ``ValueError`` as the reference
does. Keyword-only extensions:

* ``out=``: write into a caller tensor (e.g. an fp32 one);
* ``lengths=``: per-row valid lengths; rows past the length are 0 and fully
  padded chunks are skipped;
* ``reverse=True``: run each row over its valid prefix in reverse and write the
  outputs back in place, the backward direction of the reference's
  bidirectional block (``reverse_valid(fused_mamba(reverse_valid(x)))``,
  ``src/trifusion_l4/model.py:174-179``) without the two reversed copies;
* ``dt_bias=`` (with ``a_floor=``): raw controls. ``adt`` and ``dt`` are then
  the raw ``a`` and ``ddt`` in-projection columns viewed as ``[B, H, T]``, and
  the recurrence computes ``mamba_controls`` (``src/trifusion_l4/kernels/
  buffers.py:82-101``) per step itself, so the ``[B, H, T]`` control tensors
  and their launch disappear;
* ``q_norm=``, ``k_norm=`` (with ``norm_eps=``): the Mamba block's C and B
  RMSNorm weights (``src/trifusion_l4/mamba.py:56-57``). ``q`` and ``k`` are
  then the raw in-projection columns, and each row is normalised as it is
  loaded, ``round(x * rsqrt(mean(x^2) + eps) * w)`` to q's dtype
  (``src/trifusion_l4/kernels/__init__.py:10-12``), so the normalised copies
  and the norm launch disappear.
"""

import ctypes

import torch

from . import _lib
from .ops import ops

SUPPORTED_STATE = (16, 32, 64, 128)
SUPPORTED_HEAD = (32, 64)


def _shape_error(message):
    return ValueError(f"fused_mamba: {message}")


def build_args(q, k, v, adt, dt, trap, qb, kb, angles, d, z, out, lengths=None, variant="auto", reverse=False,
               dt_bias=None, a_floor=1e-4, q_norm=None, k_norm=None, norm_eps=1e-5):
    """Validate the operands and pack them into a ``tf_mamba_args`` struct."""
    what = "fused_mamba"
    for name, t in (("q", q), ("k", k), ("v", v), ("z", z), ("angles", angles)):
        if t.dim() != 4:
            raise _shape_error(f"{name} must be 4-D, got {tuple(t.shape)}")
    for name, t in (("adt", adt), ("dt", dt), ("trap", trap)):
        if t.dim() != 3:
            raise _shape_error(f"{name} must be [B, H, T], got {tuple(t.shape)}")
    b, t, h, p = v.shape
    hq, n = q.shape[2], q.shape[3]
    r = angles.shape[-1]
    if n not in SUPPORTED_STATE or p not in SUPPORTED_HEAD or not 0 <= r <= n // 2:
        raise _shape_error(
            f"recurrence requires state in {SUPPORTED_STATE}, head in {SUPPORTED_HEAD} and "
            f"rotary <= state/2 (got state={n}, head={p}, rotary={r})"
        )
    if tuple(q.shape) != (b, t, hq, n) or tuple(k.shape) != (b, t, hq, n):
        raise _shape_error(f"q/k must be [B, T, Hq, N] = {(b, t, hq, n)}")
    if hq < 1 or h % hq:
        raise _shape_error(f"heads {h} must be divisible by q/k heads {hq}")
    if tuple(z.shape) != (b, t, h, p):
        raise _shape_error("z must match v")
    for name, ten in (("adt", adt), ("dt", dt), ("trap", trap)):
        if tuple(ten.shape) != (b, h, t):
            raise _shape_error(f"{name} must be [B, H, T] = {(b, h, t)}")
    if tuple(angles.shape[:3]) != (b, t, h):
        raise _shape_error("angles must be [B, T, H, R]")
    for name, ten, shape in (("qb", qb, (h, n)), ("kb", kb, (h, n)), ("d", d, (h,))):
        if tuple(ten.shape) != shape or ten.dtype != torch.float32 or not ten.is_contiguous():
            raise _shape_error(f"{name} must be a contiguous float32 tensor of shape {shape}")
    if tuple(out.shape) != (b, t, h, p):
        raise _shape_error("out must be [B, T, H, P]")
    if lengths is not None:
        if tuple(lengths.shape) != (b,) or lengths.dtype != torch.int64 or not lengths.is_contiguous():
            raise _shape_error("lengths must be a contiguous int64 tensor of shape [B]")
    if dt_bias is not None:
        if tuple(dt_bias.shape) != (h,) or dt_bias.dtype != torch.float32 or not dt_bias.is_contiguous():
            raise _shape_error(f"dt_bias must be a contiguous float32 tensor of shape {(h,)}")
        if adt.dtype != dt.dtype:
            raise TypeError("fused_mamba: raw controls a and ddt must share one dtype")
    if (q_norm is None) != (k_norm is None):
        raise _shape_error("q_norm and k_norm must be given together")
    for name, ten in (("q_norm", q_norm), ("k_norm", k_norm)):
        if ten is not None and (tuple(ten.shape) != (n,) or ten.dtype != torch.float32 or not ten.is_contiguous()):
            raise _shape_error(f"{name} must be a contiguous float32 tensor of shape {(n,)}")
    _lib.require_cuda(q, k, v, adt, dt, trap, qb, kb, angles, d, z, out, lengths, dt_bias, q_norm, k_norm, what=what)

    a = _lib.MambaArgs()
    for name, ten in (
        ("q", q),
        ("k", k),
        ("v", v),
        ("adt", adt),
        ("dt", dt),
        ("trap", trap),
        ("angles", angles),
        ("z", z),
        ("qb", qb),
        ("kb", kb),
        ("d", d),
        ("out", out),
    ):
        setattr(a, name, ten.data_ptr())
    a.lengths = lengths.data_ptr() if lengths is not None else None
    a.dt_bias = dt_bias.data_ptr() if dt_bias is not None else None
    a.a_floor = float(a_floor)
    a.reverse = 1 if reverse else 0
    a.q_norm = q_norm.data_ptr() if q_norm is not None else None
    a.k_norm = k_norm.data_ptr() if k_norm is not None else None
    a.norm_eps = float(norm_eps)
    for name, ten in (
        ("q", q),
        ("k", k),
        ("v", v),
        ("z", z),
        ("adt", adt),
        ("dt", dt),
        ("trap", trap),
        ("angles", angles),
        ("out", out),
    ):
        setattr(a, name + "_dtype", _lib.dtype_code(ten, what))
    for name, ten in (("q", q), ("k", k), ("v", v), ("z", z), ("angles", angles), ("out", out)):
        getattr(a, name + "_stride")[:] = ten.stride()
    for name, ten in (("adt", adt), ("dt", dt), ("trap", trap)):
        getattr(a, name + "_stride")[:] = ten.stride()
    a.batch, a.time, a.heads, a.qk_heads = b, t, h, hq
    a.state, a.head_dim, a.rotary = n, p, r
    try:
        a.variant = _lib.VARIANTS[variant]
    except KeyError:
        raise ValueError(f"fused_mamba: unknown variant {variant!r}") from None
    return a


def launch(q, k, v, adt, dt, trap, qb, kb, angles, d, z, out, lengths=None, variant="auto", reverse=False,
           dt_bias=None, a_floor=1e-4, q_norm=None, k_norm=None, norm_eps=1e-5):
    """Validate, then enqueue ``tf_fused_mamba`` on the current stream (the CUDA
    kernel of the ``trifusion_amd::fused_mamba`` operator); returns ``out``."""
    lib = _lib.load()
    args = build_args(q, k, v, adt, dt, trap, qb, kb, angles, d, z, out, lengths, variant, reverse, dt_bias, a_floor,
                      q_norm, k_norm, norm_eps)
    # Long sequences over few (batch, head) units run chunk-parallel on scratch
    # the library sizes; it comes from torch's caching allocator (the graph's
    # private pool under capture), the C side never allocates.
    need = lib.tf_fused_mamba_workspace_size(ctypes.byref(args))
    if need < 0:
        _lib.check(-need, "fused_mamba")
    workspace = None
    if need > 0:
        workspace = torch.empty(need, dtype=torch.uint8, device=v.device)
        args.workspace = workspace.data_ptr()
        args.workspace_bytes = need
    _lib.check(lib.tf_fused_mamba(ctypes.byref(args), _lib.stream_of(v)), "fused_mamba")
    return out


def fused_mamba(
    q,
    k,
    v,
    adt,
    dt,
    trap,
    qb,
    kb,
    angles,
    d,
    z,
    warps=8,
    *,
    out=None,
    lengths=None,
    variant="auto",
    reverse=False,
    dt_bias=None,
    a_floor=1e-4,
    q_norm=None,
    k_norm=None,
    norm_eps=1e-5,
):
    """Fused Mamba-3 recurrence forward; returns ``out`` ``[B, T, H, P]``.

    ``warps`` is accepted for signature compatibility; gfx950 launch shapes are
    chosen by the library. ``variant`` selects ``"auto"`` (an MFMA kernel
    where supported), ``"pipe"`` (pipelined walk, N = P = 64), ``"mfma"``
    (chunked scan) or ``"generic"``. ``reverse``, ``dt_bias``, ``a_floor``,
    ``q_norm``, ``k_norm`` and ``norm_eps`` are the extensions described in the
    module docstring.
    Dispatches through the ``trifusion_amd::fused_mamba`` operator
    (``fused_mamba.out`` with ``out=``).
    """
    del warps
    ext = (lengths, variant, bool(reverse), dt_bias, float(a_floor), q_norm, k_norm, float(norm_eps))
    if out is None:
        return ops.fused_mamba(q, k, v, adt, dt, trap, qb, kb, angles, d, z, *ext)
    return ops.fused_mamba.out(q, k, v, adt, dt, trap, qb, kb, angles, d, z, *ext, out=out)


def selected_variant(
    q, k, v, adt, dt, trap, qb, kb, angles, d, z, out=None, lengths=None, variant="auto", reverse=False, dt_bias=None,
    q_norm=None, k_norm=None,
):
    """Name of the kernel ``fused_mamba`` would launch for these operands."""
    lib = _lib.load()
    if out is None:
        out = torch.empty_like(v, memory_format=torch.contiguous_format)
    args = build_args(q, k, v, adt, dt, trap, qb, kb, angles, d, z, out, lengths, variant, reverse, dt_bias,
                      q_norm=q_norm, k_norm=k_norm)
    code = lib.tf_fused_mamba_variant(ctypes.byref(args))
    if code < 0:
        _lib.check(-code, "fused_mamba")
    return {1: "generic", 2: "mfma", 3: "pipe"}[code]
