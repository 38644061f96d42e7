"""CPU restatements of the fused Mamba-3 SISO inference recurrence (oracle).

Test infrastructure only: imported by ``tests/``, ``__graft_entry__.smoke()`` and
the CPU-baseline leg of ``bench.py``; never by the product package.

Three independent formulations of the same recurrence:

``fused_mamba_chunked``
    The reference kernel's arithmetic, restated chunk by chunk in fp32
    (reference ``src/trifusion_l4/mamba_fused.py:72-152``; the portable two-phase
    kernel ``src/trifusion_l4/mamba_portable.py:440-678`` has the same rounding
    points). Intermediate values are rounded to the operand dtypes exactly where
    the reference rounds them: ``qr`` to q's dtype and ``kr`` to k's dtype
    (``mamba_fused.py:127-132``), the carried state to q's dtype before the
    ``qr @ S^T`` product (``:143``), the decayed score to v's dtype (``:146``) and
    the decay-scaled v to k's dtype (``:151-152``). With fp32 operands every
    rounding is the identity.
``fused_mamba_f64``
    Unchunked FP64 step loop, generalising the reference's independent check
    ``tests/test_recurrence.py:50-86`` to any B, T, H, Hq, N, P and R.
``fused_mamba_reversed``
    The backward direction of the reference's bidirectional block: the
    chunked form over explicitly reversed valid prefixes
    (``src/trifusion_l4/model.py:174-179``).
``fused_mamba_attention_f64``
    Quadratic closed form ``y = silu(z) * ((L o (qr kr^T)) v + (D + delta) v)``
    with ``L[t,u] = exp(sum_{m=u+1..t} adt_m)`` for ``u < t``: no recurrence at
    all, so it pins the loop (and through it the chunked form).

Pinning (tests/test_oracle_recurrence.py): reversed == per-row truncate, flip,
chunked, flip back (exact), chunked(fp32) == f64 loop to 1e-5,
f64 loop == attention form to 1e-10, T=1 closed form, causal linear attention
special case, chunk-size independence, causality, phase against an FP64
cumulative sum, and planted mistakes that each check must catch.
"""

import math

import torch
import torch.nn.functional as F

# The reference multiplies adt by this rounded log2(e) before exp2
# (mamba_fused.py:139, mamba_portable.py:595).
LOG2E = 1.44269504089
TWO_PI = 6.283185307179586
CHUNK = 64


def _round(x, dtype):
    """Round an fp32 tensor to ``dtype`` and back (identity for fp32/fp64)."""
    if dtype in (torch.float32, torch.float64):
        return x
    return x.to(dtype).to(x.dtype)


def head_index(h, hq):
    """Head ``h`` reads q/k head ``h // (H // Hq)`` (mamba_fused.py:74)."""
    if h % hq:
        raise ValueError("H must be divisible by Hq")
    return torch.arange(h) // (h // hq)


def step_controls(dt, trap):
    """gamma_t = dt_t*sig_t, s_t = dt_{t+1}*(1-sig_{t+1}) + gamma_t.

    ``dt``/``trap`` are ``[B,H,T]``. Position ``t+1 >= T`` loads 0 for both dt and
    trap, so the shifted term vanishes there (mamba_fused.py:96-101).
    """
    sig = torch.sigmoid(trap)
    gamma = dt * sig
    dn = F.pad(dt[..., 1:], (0, 1))
    tn = torch.sigmoid(F.pad(trap[..., 1:], (0, 1)))
    return gamma, dn * (1 - tn) + gamma


def phase_chunked(angles, dt, pairs, chunk=CHUNK, accumulate=torch.float64):
    """Rotary phase ``(cumsum_t pi*tanh(theta)*dt) mod 2pi`` with a per-chunk carry.

    Follows the structure of ``src/trifusion_l4/angle.py:103-144`` and
    ``mamba_fused.py:102-111``: inside a chunk the phase is the inclusive cumsum
    plus the carried state, reduced with ``x - 2pi*floor(x/2pi)``; the carry adds
    the chunk sum and is reduced the same way. ``angles`` is ``[B,T,H,R]`` (raw,
    pre-tanh), ``dt`` is ``[B,H,T]``. Returns ``[B,T,H,pairs]`` fp32; pairs
    ``r >= R`` have phase 0 (no rotation).

    The arithmetic (tanh, products, sums, carry, reduction) is done in float64 and
    only the final phase is rounded to fp32. An fp32 carry accumulates ~1e-6 rad
    of rounding noise over long clips; after the bf16 rounding of the rotated
    q/k that noise alone moves outputs by up to ~6e-4 of max|y|, so the oracle
    keeps the phase exact to fp32 resolution and so do the HIP kernels.

    ``accumulate=torch.float32`` keeps every step in fp32 instead, as the
    reference's kernel does (``mamba_fused.py:105-109``: fp32 products, an fp32
    in-chunk cumsum plus the carried state, fp32 reductions; exact tanh and a
    sequential cumsum here, where the reference uses ``tanh_approx`` and a
    parallel scan). It measures how far the reference's own phase arithmetic
    sits from the exact phase; it is not the parity oracle.
    """
    b, t, h, r = angles.shape
    vals = (torch.tanh(angles.to(accumulate)) * math.pi) * dt.to(accumulate).transpose(1, 2)[..., None]
    out = torch.empty_like(vals)
    state = vals.new_zeros(b, h, r)
    two_pi = 2 * math.pi
    for c0 in range(0, t, chunk):
        blk = vals[:, c0 : c0 + chunk]
        ph = torch.cumsum(blk, 1) + state[:, None]
        out[:, c0 : c0 + chunk] = ph - two_pi * torch.floor(ph / two_pi)
        state = state + blk.sum(1)
        state = state - two_pi * torch.floor(state / two_pi)
    return F.pad(out.float(), (0, pairs - r))


def rotate_pairs(x, cos, sin):
    """Rotate interleaved pairs ``(x[2i], x[2i+1])`` by the pair's phase.

    ``rot(x)[2i] = x[2i] cos - x[2i+1] sin``, ``rot(x)[2i+1] = x[2i] sin +
    x[2i+1] cos`` (mamba_fused.py:125-132; tests/test_recurrence.py:59-62).
    """
    x0, x1 = x[..., 0::2], x[..., 1::2]
    return torch.stack((x0 * cos - x1 * sin, x0 * sin + x1 * cos), -1).flatten(-2)


def fused_mamba_chunked(
    q, k, v, adt, dt, trap, qb, kb, angles, d, z, chunk=CHUNK, out_dtype=None, lengths=None,
    phase_accumulate=torch.float64,
):
    """Chunked fp32 restatement of ``fused_mamba`` (mamba_fused.py:72-152).

    Shapes as in the reference entry point (``mamba_fused.py:155``; ``docs/api.md:61-74``):
    q, k ``[B,T,Hq,N]``; v, z ``[B,T,H,P]``; adt, dt, trap ``[B,H,T]``;
    qb, kb ``[H,N]``; angles ``[B,T,H,R]``; d ``[H]``. Returns ``[B,T,H,P]`` in fp32
    (or ``out_dtype``). ``lengths`` (optional ``[B]``) zeroes rows ``t >= lengths[b]``
    after the recurrence, the masking the model applies to the output
    (``src/trifusion_l4/model.py:174``); causality leaves valid rows unchanged.
    ``phase_accumulate`` selects the rotary phase arithmetic (``phase_chunked``).
    """
    bsz, t, hq, n = q.shape
    h, p = v.shape[2], v.shape[3]
    idx = head_index(h, hq)
    qf = q.float()[:, :, idx]
    kf = k.float()[:, :, idx]
    gamma, scale = step_controls(dt.float(), trap.float())
    phase = phase_chunked(angles, dt, n // 2, chunk, phase_accumulate)
    cos, sin = torch.cos(phase), torch.sin(phase)
    qt = qf + qb.float()[None, None]
    kt = kf + kb.float()[None, None]
    # skip term uses the unrotated, biased vectors (mamba_fused.py:124)
    qk = (qt * kt).sum(-1) * gamma.transpose(1, 2)
    qr = _round(rotate_pairs(qt, cos, sin), q.dtype)
    kr = _round(rotate_pairs(kt, cos, sin) * scale.transpose(1, 2)[..., None], k.dtype)
    # work in [B,H,T,*]
    qr = qr.permute(0, 2, 1, 3)
    kr = kr.permute(0, 2, 1, 3)
    vf = v.float().permute(0, 2, 1, 3)
    zf = z.float().permute(0, 2, 1, 3)
    qk = qk.permute(0, 2, 1)
    da_all = adt.float() * LOG2E
    skip = d.float()[None, :, None]
    state = qr.new_zeros(bsz, h, p, n)
    out = qr.new_empty(bsz, h, t, p)
    for c0 in range(0, t, chunk):
        sl = slice(c0, c0 + chunk)
        qc, kc, vc, zc = qr[:, :, sl], kr[:, :, sl], vf[:, :, sl], zf[:, :, sl]
        da = da_all[:, :, sl]
        cs = torch.cumsum(da, -1)
        total = da.sum(-1)
        acc = (qc @ _round(state, q.dtype).transpose(-1, -2)) * torch.exp2(cs)[..., None]
        score = (qc @ kc.transpose(-1, -2)) * torch.exp2(
            torch.clamp_max(cs[..., :, None] - cs[..., None, :], 0.0)
        )
        rows = qc.shape[2]
        strict = torch.ones(rows, rows, dtype=torch.bool).tril(-1)
        score = torch.where(strict, score, torch.zeros((), dtype=score.dtype))
        acc = acc + _round(score, v.dtype) @ vc
        acc = acc + (skip + qk[:, :, sl])[..., None] * vc
        acc = acc * (zc * torch.sigmoid(zc))
        out[:, :, sl] = acc
        scaled = _round(vc * torch.exp2(total[..., None] - cs)[..., None], k.dtype)
        state = state * torch.exp2(total)[..., None, None] + scaled.transpose(-1, -2) @ kc
    out = out.permute(0, 2, 1, 3)
    if lengths is not None:
        valid = torch.arange(t)[None, :] < lengths.cpu()[:, None]
        out = out * valid[:, :, None, None]
    return out if out_dtype is None else out.to(out_dtype)


def fused_mamba_reversed(q, k, v, adt, dt, trap, qb, kb, angles, d, z, lengths=None, out_dtype=None):
    """Backward direction of the reference's bidirectional block
    (``src/trifusion_l4/model.py:174-179``): every time-indexed operand has its
    valid prefix reversed (``reverse_valid``, ``kernels/__init__.py:44-55``), the
    recurrence runs, and its output is reversed back, so row ``t < L`` holds the
    output of step ``L-1-t`` and rows past ``L`` are 0. ``lengths`` ``None``
    reverses the whole sequence.
    """
    from .elementwise import reverse_valid

    bsz, t = v.shape[:2]
    n = torch.full((bsz,), t, dtype=torch.int64) if lengths is None else lengths.cpu().clamp(0, t)

    def rev_t(x):  # [B, T, ...]
        shape = x.shape
        return reverse_valid(x.reshape(shape[0], shape[1], -1), n).reshape(shape)

    def rev_ht(x):  # [B, H, T]
        return reverse_valid(x.transpose(1, 2), n).transpose(1, 2)

    y = fused_mamba_chunked(
        rev_t(q), rev_t(k), rev_t(v), rev_ht(adt), rev_ht(dt), rev_ht(trap), qb, kb, rev_t(angles), d, rev_t(z),
        lengths=n,
    )
    out = rev_t(y)
    return out if out_dtype is None else out.to(out_dtype)


def _rotated_f64(q, k, qb, kb, angles, dt, h):
    bsz, t, hq, n = q.shape
    r = angles.shape[-1]
    idx = head_index(h, hq)
    phase = (angles.double().tanh() * torch.pi * dt.double().transpose(1, 2)[..., None]).cumsum(1)
    phase = F.pad(phase, (0, n // 2 - r))
    qt = q.double()[:, :, idx] + qb.double()[None, None]
    kt = k.double()[:, :, idx] + kb.double()[None, None]
    cos, sin = phase.cos(), phase.sin()
    return qt, kt, rotate_pairs(qt, cos, sin), rotate_pairs(kt, cos, sin)


def fused_mamba_f64(q, k, v, adt, dt, trap, qb, kb, angles, d, z):
    """Unchunked FP64 loop; generalises ``tests/test_recurrence.py:50-86``.

    ``y_t = silu(z_t) * (exp(adt_t) * qr_t . S_{t-1} + (D + gamma_t q~_t . k~_t) v_t)``,
    ``S_t = exp(adt_t) S_{t-1} + s_t v_t (x) kr_t``. Phases are the un-reduced
    FP64 cumulative sum (cos/sin are 2pi-periodic, so no modulo is needed).
    """
    bsz, t, h, p = v.shape
    n = q.shape[-1]
    qt, kt, qr, kr = _rotated_f64(q, k, qb, kb, angles, dt, h)
    gamma, scale = step_controls(dt.double(), trap.double())
    state = torch.zeros(bsz, h, p, n, dtype=torch.float64)
    dd = d.double()[None]
    outputs = []
    for i in range(t):
        decay = adt[:, :, i].double().exp()
        vi = v[:, i].double()
        previous = torch.einsum("bhn,bhpn->bhp", qr[:, i], state) * decay[..., None]
        direct = (qt[:, i] * kt[:, i]).sum(-1) * gamma[:, :, i]
        outputs.append((previous + (dd + direct)[..., None] * vi) * F.silu(z[:, i].double()))
        state = (
            state * decay[..., None, None]
            + vi[..., None] * kr[:, i, :, None, :] * scale[:, :, i, None, None]
        )
    return torch.stack(outputs, 1)


def fused_mamba_attention_f64(q, k, v, adt, dt, trap, qb, kb, angles, d, z, clamp_chunk=None):
    """Quadratic (attention-form) FP64 closed form of the same recurrence.

    ``y = silu(z) * (sum_{u<t} exp(A_t - A_u) (qr_t . kr_u) s_u v_u + (D + delta_t) v_t)``
    with ``A = cumsum(adt)``. Unrolls the state recursion of
    ``tests/test_recurrence.py:64-84`` into an explicit lower-triangular kernel.

    ``clamp_chunk=C`` caps the weight at 1 for u and t in the same C-step
    chunk, ``exp(min(A_t - A_u, 0))``: the reference's intra-chunk score decay
    (``mamba_fused.py:144``). Pairs in different chunks meet through the carried
    state, which has no clamp (``:143, 150-152``). With ``adt <= 0`` the clamp
    changes nothing.
    """
    bsz, t, h, p = v.shape
    qt, kt, qr, kr = _rotated_f64(q, k, qb, kb, angles, dt, h)
    gamma, scale = step_controls(dt.double(), trap.double())
    a = adt.double().cumsum(-1)
    diff = a[..., :, None] - a[..., None, :]
    if clamp_chunk is not None:
        chunk_of = torch.arange(t) // clamp_chunk
        same = chunk_of[:, None] == chunk_of[None, :]
        diff = torch.where(same, diff.clamp_max(0.0), diff)
    strict = torch.ones(t, t, dtype=torch.bool).tril(-1)
    decay = diff.masked_fill(~strict, -torch.inf).exp()
    qr = qr.permute(0, 2, 1, 3)
    krs = kr.permute(0, 2, 1, 3) * scale[..., None]
    vv = v.double().permute(0, 2, 1, 3)
    scores = (qr @ krs.transpose(-1, -2)) * decay
    delta = (qt * kt).sum(-1).permute(0, 2, 1) * gamma
    y = scores @ vv + (d.double()[None, :, None] + delta)[..., None] * vv
    y = y * F.silu(z.double().permute(0, 2, 1, 3))
    return y.permute(0, 2, 1, 3)


def max_rel(actual, ref):
    """``max|a - r| / max|r|`` (the tolerance metric for recurrence outputs)."""
    a, r = actual.double(), ref.double()
    return float((a - r).abs().max() / r.abs().max().clamp_min(1e-30))


def rel_fro(actual, ref):
    """Relative Frobenius error (tests/test_recurrence.py:44-45,86)."""
    a, r = actual.double(), ref.double()
    return float((a - r).norm() / r.norm().clamp_min(1e-30))
