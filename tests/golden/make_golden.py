"""Writes ``recurrence_kat.npz``: known-answer cases of ``fused_mamba`` whose
expected outputs come from closed forms in float64 (numpy only; neither the
oracle nor the kernels are involved), so they pin both.

The reference ships no golden vectors for this path; these cases follow the
special cases its maths fixes (mamba_fused.py:72-152):

* ``single_step`` (T = 1): no history, so
  y = silu(z) * (D + dt * sigmoid(trap) * (q + qb).(k + kb)) * v.
* ``linear_attention`` (T = 96, across a 64-step chunk edge): no decay
  (adt = 0), no rotation (theta = 0) and trap = 30, whose fp32 sigmoid is
  exactly 1, so gamma_t = s_t = dt_t and
  y_t = silu(z_t) * (sum_{u<t} (q~_t . k~_u) dt_u v_u + (D + dt_t q~_t . k~_t) v_t),
  with q~ = q + qb, k~ = k + kb.

The remaining cases pin the trapezoid step s_u that scales key u
(mamba_fused.py:96-101), which the cases above cannot see: with trap = 30 the
next-step term dt_{u+1} (1 - sigmoid(trap_{u+1})) is exactly 0. Each uses
trap = +-40, whose sigmoid is 1 or 0 in float32 and float64 alike, no rotation
(theta = 0), and writes s_u from a table of the neighbours' sigmoids instead of
the formula, so a sigmoid written where 1 - sigmoid belongs, or step t read
where t + 1 belongs, changes the answer:

  sig_u  sig_{u+1} | s_u                 (u < T - 1)
    1       1      | dt_u
    1       0      | dt_u + dt_{u+1}
    0       1      | 0
    0       0      | dt_{u+1}
  and s_{T-1} = dt_{T-1} sig_{T-1} (the step past the sequence loads 0).

  y_t = silu(z_t) * (sum_{u<t} exp(sum_{m=u+1..t} adt_m) (q~_t . k~_u) s_u v_u
                     + (D + dt_t sig_t q~_t . k~_t) v_t).

* ``shift`` (T = 96): trap = -40 everywhere, no decay: s_u = dt_{u+1}, no skip
  term from the keys' own step.
* ``mixed_trap`` (T = 96): trap = +-40 at random, no decay: all four rows of
  the table occur.
* ``segmented`` (B = 1, H = 1, T = 300): mixed trap and a constant decay
  adt = -0.02. With a single (batch, head) unit the MFMA kernel cuts the
  sequence into segments (a boundary at t = 256), so the step at the end of a
  segment reads its halo from the next segment.
* ``mixed_trap_n64`` (T = 100, N = P = 64, R = 16): mixed trap and a constant
  decay adt = -0.05 at the state and head dims the pipelined kernel takes.

q, k, v and z are rounded to bf16 values (stored as float32), so bf16 kernels
read them exactly. Shapes use N = P = 32, R = 8, Hq = 1 (the generic and chunked
kernels), and N = P = 64, R = 16 for the last case (every kernel). Run from the repository root: ``python tests/golden/make_golden.py``.
"""

from pathlib import Path

import numpy as np

OUT = Path(__file__).with_name("recurrence_kat.npz")


def bf16_exact(x):
    """Round float32 values to the nearest bf16 (ties to even), kept as float32."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def silu(x):
    return x / (1.0 + np.exp(-x))


def inputs(rng, b, t, h, p, n, r):
    f = lambda *s: rng.standard_normal(s).astype(np.float32)
    q, k = bf16_exact(f(b, t, 1, n)), bf16_exact(f(b, t, 1, n))
    v, z = bf16_exact(f(b, t, h, p)), bf16_exact(f(b, t, h, p))
    dt = (0.5 + 0.5 * rng.random((b, h, t))).astype(np.float32)
    trap = f(b, h, t)
    qb = (0.1 * f(h, n)).astype(np.float32)
    kb = (0.1 * f(h, n)).astype(np.float32)
    d = np.full(h, 0.5, dtype=np.float32)
    angles = (rng.random((b, t, h, r)) - 0.5).astype(np.float32)
    adt = (-dt * (0.2 + rng.random((b, h, t)))).astype(np.float32)
    return dict(q=q, k=k, v=v, adt=adt, dt=dt, trap=trap, qb=qb, kb=kb, angles=angles, d=d, z=z)


def single_step(rng):
    c = inputs(rng, 2, 1, 2, 32, 32, 8)
    q = c["q"].astype(np.float64)[:, 0, 0]  # [B, N]
    k = c["k"].astype(np.float64)[:, 0, 0]
    qb, kb = c["qb"].astype(np.float64), c["kb"].astype(np.float64)  # [H, N]
    gamma = c["dt"][:, :, 0] / (1.0 + np.exp(-c["trap"][:, :, 0].astype(np.float64)))  # [B, H]
    dot = ((q[:, None] + qb[None]) * (k[:, None] + kb[None])).sum(-1)  # [B, H]
    coef = c["d"].astype(np.float64)[None] + gamma * dot
    y = silu(c["z"].astype(np.float64))[:, 0] * coef[..., None] * c["v"].astype(np.float64)[:, 0]
    c["expected"] = y[:, None]  # [B, 1, H, P]
    return c


def linear_attention(rng):
    c = inputs(rng, 1, 96, 2, 32, 32, 8)
    c["adt"][:] = 0.0
    c["angles"][:] = 0.0
    c["trap"][:] = 30.0
    q = c["q"].astype(np.float64)[:, :, 0]  # [B, T, N]
    k = c["k"].astype(np.float64)[:, :, 0]
    v = c["v"].astype(np.float64)  # [B, T, H, P]
    dt = c["dt"].astype(np.float64)  # [B, H, T]
    qt = q[:, :, None] + c["qb"].astype(np.float64)[None, None]  # [B, T, H, N]
    kt = k[:, :, None] + c["kb"].astype(np.float64)[None, None]
    scores = np.einsum("bthn,buhn->bhtu", qt, kt)  # [B, H, T, U]
    t = q.shape[1]
    strict = np.tril(np.ones((t, t)), -1)
    w = scores * strict[None, None] * dt[:, :, None, :]  # dt_u on the key side
    acc = np.einsum("bhtu,buhp->bthp", w, v)
    diag = np.einsum("bhtt->bht", scores) * dt  # dt_t q~_t . k~_t
    acc += (c["d"].astype(np.float64)[None, :, None] + diag).transpose(0, 2, 1)[..., None] * v
    c["expected"] = silu(c["z"].astype(np.float64)) * acc
    return c


def trapezoid_steps(dt, sig):
    """s_u by the table in the module docstring. ``dt``, ``sig``: [B, H, T]
    (sig in {0, 1})."""
    s = np.zeros_like(dt, dtype=np.float64)
    t = dt.shape[-1]
    for u in range(t):
        if u == t - 1:
            s[..., u] = dt[..., u] * sig[..., u]
            continue
        here, nxt = sig[..., u], sig[..., u + 1]
        table = {
            (1, 1): dt[..., u],
            (1, 0): dt[..., u] + dt[..., u + 1],
            (0, 1): np.zeros_like(dt[..., u]),
            (0, 0): dt[..., u + 1],
        }
        for (a, b), val in table.items():
            pick = (here == a) & (nxt == b)
            s[..., u] = np.where(pick, val, s[..., u])
    return s


def halo_case(rng, b, t, h, trap_sign, decay, n=32, r=8):
    """A trapezoid-step case (see the module docstring): ``trap_sign`` "neg"
    (all -40) or "mixed" (+-40 at random), ``decay`` a constant adt; state and
    head dim ``n``."""
    c = inputs(rng, b, t, h, n, n, r)
    decay = float(np.float32(decay))  # the float32 value the kernels read
    c["angles"][:] = 0.0
    c["adt"][:] = decay
    if trap_sign == "neg":
        sig = np.zeros((b, h, t))
    else:
        sig = (rng.random((b, h, t)) < 0.5).astype(np.float64)
    c["trap"] = np.where(sig == 1, 40.0, -40.0).astype(np.float32)
    dt = c["dt"].astype(np.float64)
    s = trapezoid_steps(dt, sig)
    q = c["q"].astype(np.float64)[:, :, 0]
    k = c["k"].astype(np.float64)[:, :, 0]
    qt = q[:, :, None] + c["qb"].astype(np.float64)[None, None]  # [B, T, H, N]
    kt = k[:, :, None] + c["kb"].astype(np.float64)[None, None]
    scores = np.einsum("bthn,buhn->bhtu", qt, kt)
    steps = np.arange(t)
    gap = (steps[:, None] - steps[None, :]).astype(np.float64)  # t - u
    weight = np.where(gap > 0, np.exp(decay * gap), 0.0)  # sum_{m=u+1..t} adt_m = decay (t - u)
    w = scores * weight[None, None] * s[:, :, None, :]
    acc = np.einsum("bhtu,buhp->bthp", w, c["v"].astype(np.float64))
    skip = np.einsum("bhtt->bht", scores) * dt * sig
    acc += (c["d"].astype(np.float64)[None, :, None] + skip).transpose(0, 2, 1)[..., None] * c["v"].astype(np.float64)
    c["expected"] = silu(c["z"].astype(np.float64)) * acc
    return c


def main():
    rng = np.random.default_rng(20240611)
    cases = {"single_step": single_step(rng), "linear_attention": linear_attention(rng)}
    cases["shift"] = halo_case(rng, 1, 96, 2, "neg", 0.0)
    cases["mixed_trap"] = halo_case(rng, 1, 96, 2, "mixed", 0.0)
    cases["segmented"] = halo_case(rng, 1, 300, 1, "mixed", -0.02)
    cases["mixed_trap_n64"] = halo_case(rng, 1, 100, 1, "mixed", -0.05, n=64, r=16)
    flat = {f"{name}/{key}": val for name, c in cases.items() for key, val in c.items()}
    np.savez_compressed(OUT, **flat)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
