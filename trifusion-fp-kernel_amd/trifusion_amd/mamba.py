"""Frozen Mamba-3 SISO block on the MI355X kernels.

Mirrors ``Mamba3Inference`` of the reference (``src/trifusion_l4/mamba.py:14-102``):
the same parameter names and in-projection layout ``z, x, B, C, dt, a, trap,
angles`` (``:26-30,43-55``), B/C RMSNorm over the state dim with one B/C head
(``:21,56-57``), the discretisation controls (``:58-65``), rotary angles shared by
all heads as a stride-0 view (``:66``) and the fused recurrence called on
strided column slices of the projection, no copies (``:70-82``). The norms and
recurrence are gfx950 HIP kernels; the two projections are torch GEMMs
(hipBLASLt).

By default the controls (``:58-65``) are computed inside the recurrence from
the raw ``a``/``ddt`` columns (``fuse_controls``; the same per-step formula as
the separate ``mamba_controls`` kernel, which ``fuse_controls = False``
restores), and so are the B/C norms (``:56-57``): the recurrence reads the raw
B/C columns and normalises each row as it loads it (``fuse_norms``; the same
rounding as the separate ``rms_pair`` launch, which ``fuse_norms = False``
restores). ``forward(u, lengths, reverse=True)`` is the backward direction of
the reference's bidirectional block, ``reverse_valid(backward_mamba(
reverse_valid(u)))`` (``src/trifusion_l4/model.py:174-179``): every step of the
block is per-row except the recurrence, which walks each valid prefix in
reverse, so no reversed copies are made.
"""

import torch
import torch.nn.functional as F
from torch import nn

from .kernels import RMSNorm
from .kernels.native import rms_pair
from .kernels.buffers import mamba_controls
from .mamba_fused import fused_mamba


def weight_key(t):
    """Identity of a weight's current contents for the derived-weight caches:
    its address, version counter, dtype and device. Inference tensors (a model
    loaded or cast under ``torch.inference_mode()``) have no version counter;
    they take -1, and a changed inference tensor is a new tensor at a new
    address."""
    return (t.data_ptr(), -1 if t.is_inference() else t._version, t.dtype, t.device)

# Output width the in-projection GEMM runs at: rows of zeros pad the weight to
# a multiple of this (2240 -> 2304 at dim 512); the extra columns of the
# projection are never read, the splits are views of its first 2240 columns.
PROJ_ALIGN = 128


class Mamba3Inference(nn.Module):
    def __init__(self, config):
        super().__init__()
        self.d_inner = config.dim * 2
        self.headdim = config.head_dim
        self.nheads = self.d_inner // self.headdim
        self.d_state = config.state_dim
        self.num_bc_heads = 1
        self.num_rope_angles = self.d_state // 4
        self.A_floor = 1e-4
        self.chunk_size = 64
        self.in_proj = nn.Linear(
            config.dim,
            2 * self.d_inner + 2 * self.d_state + 3 * self.nheads + self.num_rope_angles,
            bias=False,
        )
        self.out_proj = nn.Linear(self.d_inner, config.dim, bias=False)
        self.dt_bias = nn.Parameter(torch.full((self.nheads,), -4.0))
        self.B_bias = nn.Parameter(torch.ones(self.nheads, 1, self.d_state))
        self.C_bias = nn.Parameter(torch.ones_like(self.B_bias))
        self.D = nn.Parameter(torch.ones(self.nheads))
        self.B_norm = RMSNorm(self.d_state)
        self.C_norm = RMSNorm(self.d_state)
        # "pipe" (pipelined MFMA walk), "mfma" (chunked MFMA scan), "generic" (fp32-FMA kernel) or "auto"
        self.variant = "auto"
        self.fuse_controls = True
        self.fuse_norms = True
        self._padded = None
        self._padded_key = None

    def _padded_in_proj(self):
        """in_proj.weight with zero output rows up to a multiple of PROJ_ALIGN,
        rebuilt when the weight changes. The library GEMM runs an odd tile count
        (2240 = 17.5 x 128) markedly slower than the padded 2304."""
        w = self.in_proj.weight
        rows = w.shape[0]
        padded = -(-rows // PROJ_ALIGN) * PROJ_ALIGN
        if padded == rows:
            return w
        key = weight_key(w)
        if self._padded_key != key:
            with torch.no_grad():
                wp = w.new_zeros(padded, w.shape[1])
                wp[:rows] = w
            self._padded, self._padded_key = wp, key
        return self._padded

    def split(self, p):
        return p.split(
            [
                self.d_inner,
                self.d_inner,
                self.d_state,
                self.d_state,
                self.nheads,
                self.nheads,
                self.nheads,
                self.num_rope_angles,
            ],
            -1,
        )

    def forward(self, u, lengths=None, reverse=False):
        return self.out_proj(self.mix(self.project(u), lengths, reverse))

    def project(self, u):
        """The in-projection ``[B, T, width]`` (a view of the padded GEMM output)."""
        return F.linear(u, self._padded_in_proj())[..., : self.in_proj.out_features]

    def mix(self, p, lengths=None, reverse=False, out=None):
        """Norms, controls and the fused recurrence from the projection ``p``:
        ``[B, T, d_inner]`` before the out-projection (written into ``out``, a
        ``[B, T, H, P]`` buffer, when given)."""
        b, t, _ = p.shape
        z, v, k, q, ddt, a, trap, angles = self.split(p)
        norms = {}
        if self._fusable_norms():
            # raw B/C columns; the recurrence applies both norms as it loads a row
            q = q.reshape(b, t, 1, self.d_state)
            k = k.reshape(b, t, 1, self.d_state)
            norms = {"q_norm": self.C_norm.weight, "k_norm": self.B_norm.weight, "norm_eps": self.B_norm.eps}
        elif self.B_norm.eps == self.C_norm.eps:
            # B and C sit side by side in the projection: both norms, one launch
            n = self.d_state
            kq = p[..., 2 * self.d_inner : 2 * self.d_inner + 2 * n]
            y = rms_pair(kq, self.B_norm.weight, self.C_norm.weight, self.B_norm.eps)
            k, q = y[:, :, 0:1], y[:, :, 1:2]
        else:
            q = self.C_norm(q.reshape(b, t, 1, self.d_state))
            k = self.B_norm(k.reshape(b, t, 1, self.d_state))
        if self.fuse_controls and self.dt_bias.dtype == torch.float32:
            adt, dt = a.transpose(1, 2), ddt.transpose(1, 2)
            raw = {"dt_bias": self.dt_bias, "a_floor": self.A_floor}
        else:
            adt, dt = mamba_controls(a, ddt, self.dt_bias, self.A_floor)
            raw = {}
        angles = angles.unsqueeze(2).expand(b, t, self.nheads, self.num_rope_angles)
        y = fused_mamba(
            q,
            k,
            v.reshape(b, t, self.nheads, self.headdim),
            adt,
            dt,
            trap.transpose(1, 2),
            self.C_bias[:, 0],
            self.B_bias[:, 0],
            angles,
            self.D,
            z.reshape(b, t, self.nheads, self.headdim),
            lengths=lengths,
            variant=self.variant,
            reverse=reverse,
            out=out,
            **raw,
            **norms,
        )
        return y.reshape(b, t, self.d_inner)

    def _fusable_norms(self):
        weights = (self.B_norm.weight, self.C_norm.weight)
        return (
            self.fuse_norms
            and self.B_norm.eps == self.C_norm.eps
            and all(w.dtype == torch.float32 and w.is_contiguous() for w in weights)
        )
