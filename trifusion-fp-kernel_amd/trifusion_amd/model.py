"""Synthetic 8-block audio encoder built from the hot-path primitives.

The benchmark encoder for 4 s mono x 16 clips: a Conv1d stem (kernel 400,
stride 160, 1 -> 512 channels, padded so a 4 s clip gives 400 frames at a 10 ms
hop), ``depth`` blocks of

    RMSNorm -> Mamba-3 (in-proj 512 -> 2240, fused recurrence with SiLU(z) gate,
    out-proj 1024 -> 512) -> masked residual -> RMSNorm -> SwiGLU 512 -> 1365 ->
    512 -> masked residual

and a masked mean-pool over valid frames followed by a 512 -> 5 linear head.
With ``bidirectional=True`` each block also runs a backward Mamba-3 over each
clip's reversed valid prefix and feeds the RMSNorm of the two directions' mean
to the residual, the bidirectional mixing of the reference's TriFusion block
(``src/trifusion_l4/model.py:174-184``); the backward direction reverses
inside the recurrence (``reverse=True``) instead of through reversed copies.
``forward(audio, lengths, channels)`` returns ``{"logits": [B, 5]}``, the contract
``InferenceEngine`` relies on (reference ``src/trifusion_l4/runtime.py:82``,
``src/trifusion_l4/model.py:259-260``). The residual stream is fp32; each residual
add is fused with the RMSNorm that follows it (reference ``native.add`` +
``_norm``, ``src/trifusion_l4/kernels/native.py:8-39,81-100``). Rows past a clip's
length are zero after every residual (``src/trifusion_l4/model.py:143-147,199``).
"""

from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn

from .kernels import RMSNorm, swiglu
from .kernels.native import add, add_rms, mask_rms, mean_norm
from .mamba import Mamba3Inference, weight_key
from .masking import masked_mean
from .stem import frame_audio, frames_mask, small_linear


@dataclass
class ModelConfig:
    dim: int = 512
    depth: int = 8
    ffn_dim: int = 1365
    state_dim: int = 64
    head_dim: int = 64
    num_outputs: int = 5
    stem_kernel: int = 400
    stem_stride: int = 160
    stem_padding: int = 120
    norm_eps: float = 1e-5
    init_std: float = 0.02
    bidirectional: bool = False


FFN_ALIGN = 64  # FFN width the GEMMs and SwiGLU run at (each half zero-padded up to it)
STEM_ALIGN = 64  # stem GEMM depth: the frame width, zero columns past the kernel


class EncoderBlock(nn.Module):
    def __init__(self, c):
        super().__init__()
        self.pre = RMSNorm(c.dim, c.norm_eps)
        self.mamba = Mamba3Inference(c)
        if c.bidirectional:
            self.mamba_bwd = Mamba3Inference(c)
            self.mn = RMSNorm(c.dim, c.norm_eps)
        else:
            self.mamba_bwd = None
        self.ff_norm = RMSNorm(c.dim, c.norm_eps)
        self.gate_up = nn.Linear(c.dim, 2 * c.ffn_dim, bias=False)
        self.down = nn.Linear(c.ffn_dim, c.dim, bias=False)
        self._padded = None
        self._padded_key = None

    def _padded_ffn(self):
        """The FFN weights at a width the library GEMMs run well: each half of
        gate_up zero-padded to a multiple of FFN_ALIGN rows and stored K-major
        ([dim, 2 * width], used as ``h @ w``), and down with matching zero
        columns. An odd width (1365) leaves every GEMM tile and SwiGLU row
        misaligned; the padded rows give silu(0) * 0 = 0 and meet zero columns
        of down, so the result is the same up to the GEMMs' summation order.
        Rebuilt when either weight changes."""
        w1, w2 = self.gate_up.weight, self.down.weight
        key = (weight_key(w1), weight_key(w2))
        if self._padded_key != key:
            f, d = self.down.in_features, self.down.out_features
            fp = -(-f // FFN_ALIGN) * FFN_ALIGN
            with torch.no_grad():
                g1 = w1.new_zeros(2 * fp, d)
                g1[:f] = w1[:f]
                g1[fp : fp + f] = w1[f:]
                g2 = w2.new_zeros(d, fp)
                g2[:, :f] = w2
            self._padded, self._padded_key = (g1.t().contiguous(), g2), key
        return self._padded

    def ffn(self, h):
        g1t, g2 = self._padded_ffn()
        return F.linear(swiglu(h @ g1t), g2)


class Encoder(nn.Module):
    def __init__(self, config=None):
        super().__init__()
        self.config = c = config or ModelConfig()
        self.stem = nn.Conv1d(1, c.dim, c.stem_kernel, stride=c.stem_stride, padding=c.stem_padding, bias=False)
        self.blocks = nn.ModuleList([EncoderBlock(c) for _ in range(c.depth)])
        self.head = nn.Linear(c.dim, c.num_outputs)
        self._stem_w = None
        self._stem_key = None
        self.reset_parameters()

    def reset_parameters(self):
        for m in self.modules():
            if isinstance(m, (nn.Linear, nn.Conv1d)):
                nn.init.normal_(m.weight, std=self.config.init_std)
                if m.bias is not None:
                    nn.init.zeros_(m.bias)

    def set_variant(self, variant):
        """Select the recurrence kernel ("auto", "pipe", "mfma" or "generic") of every block."""
        for m in self.modules():
            if isinstance(m, Mamba3Inference):
                m.variant = variant

    def frames(self, lengths, time):
        """Valid frames per clip: floor(len / stride) for the padded stem, in [1, time]."""
        return (lengths // self.config.stem_stride).clamp(1, time)

    def _stem_weight(self):
        """The stem kernel as a [dim, width] GEMM weight, zero columns from
        stem_kernel up to a multiple of STEM_ALIGN (400 -> 448: the library GEMM
        runs K = 448 faster than K = 400); rebuilt when the weight changes."""
        cfg = self.config
        w = self.stem.weight
        key = weight_key(w)
        if self._stem_key != key:
            width = -(-cfg.stem_kernel // STEM_ALIGN) * STEM_ALIGN
            with torch.no_grad():
                wp = w.new_zeros(cfg.dim, width)
                wp[:, : cfg.stem_kernel] = w.reshape(cfg.dim, cfg.stem_kernel)
            self._stem_w, self._stem_key = wp, key
        return self._stem_w

    def stem_forward(self, audio, channels):
        """Channel mix and framing in one kernel (bf16 frames of the zero-padded
        channel mean, zero columns up to the padded weight's width), then the
        strided Conv1d stem as one GEMM."""
        cfg = self.config
        w = self._stem_weight()
        framed = frame_audio(audio.float(), channels.to(torch.int64), cfg.stem_kernel, cfg.stem_stride,
                             cfg.stem_padding, w.shape[1])
        return F.linear(framed.to(w.dtype), w)  # [B, T, dim]

    def encode(self, audio, lengths, channels):
        x = self.stem_forward(audio, channels)
        b, t, _ = x.shape
        frames, mask = frames_mask(lengths, self.config.stem_stride, t)
        blocks = self.blocks
        # masked fp32 residual and the first block's normalised input, one pass
        x, h = mask_rms(x, mask, blocks[0].pre.weight, blocks[0].pre.eps)
        for i, blk in enumerate(blocks):
            m = blk.mamba(h, frames)
            if blk.mamba_bwd is not None:
                # rows past each clip's length are 0 in both directions
                mb = blk.mamba_bwd(h, frames, reverse=True)
                m = mean_norm(m, mb, blk.mn.weight, blk.mn.eps)
            x, h = add_rms(x, m, blk.ff_norm.weight, mask, blk.ff_norm.eps)
            d = blk.ffn(h)
            if i + 1 < len(blocks):
                nxt = blocks[i + 1].pre
                x, h = add_rms(x, d, nxt.weight, mask, nxt.eps)
            else:
                x = add(x, d, mask)
        return x, frames

    def forward(self, audio, lengths, channels):
        x, frames = self.encode(audio, lengths, channels)
        pooled = masked_mean(x, frames)
        if self.head.weight.dtype == torch.bfloat16:
            logits = small_linear(pooled, self.head.weight, self.head.bias)
        else:
            logits = self.head(pooled.to(self.head.weight.dtype)).float()
        return {"logits": logits, "embedding": pooled}
