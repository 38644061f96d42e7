"""CPU forward of the synthetic 8-block encoder (oracle).

Test infrastructure only (see ``oracle/__init__.py``). Evaluates the same
parameters as ``trifusion_amd.model.Encoder`` with plain PyTorch CPU ops and the
recurrence oracle, rounding to bf16 where the GPU path holds bf16 values: GEMM
inputs and outputs under autocast (the reference runs its forward under
``torch.autocast("cuda", bfloat16)``, ``src/trifusion_l4/runtime.py:79-82``), the
B/C norms (output dtype = input dtype, ``src/trifusion_l4/kernels/native.py:46``),
SwiGLU and the recurrence output. The residual stream, norms' statistics and the
pooled embedding stay fp32. With ``cfg.bidirectional`` each block also runs the
backward direction the reference's way, on explicitly reversed valid prefixes
(``src/trifusion_l4/model.py:174-184``). Parity target: sigmoid probabilities
within 1e-2.
"""

import torch
import torch.nn.functional as F

from . import elementwise as E
from .recurrence import fused_mamba_chunked

BF16 = torch.bfloat16


def _bf(x):
    return x.to(BF16).float()


def _linear(x, w, b=None):
    """bf16 GEMM with fp32 accumulation and a bf16 result."""
    y = _bf(x) @ w.float().t()
    if b is not None:
        y = y + b.float()
    return _bf(y)


def channel_mean(audio, channels):
    """Mean over each clip's first ``channels[b]`` channels, fp32 ``[B, N]``."""
    c = audio.shape[1]
    chan = torch.arange(c)[None, :] < channels[:, None]
    return (audio * chan[..., None]).sum(1) / channels[:, None].to(audio.dtype)


def frame_audio(audio, channels, kernel, stride, pad, width=None):
    """bf16 frames ``[B, T, width]`` of the zero-padded channel mean: frame t
    holds samples ``t*stride - pad .. + kernel - 1``; columns past ``kernel``
    are 0. The stem Conv1d is ``frame_audio(...) @ w.T``."""
    mono = channel_mean(audio, channels)
    framed = F.pad(mono, (pad, pad)).unfold(1, kernel, stride)
    width = width or kernel
    return F.pad(framed, (0, width - kernel)).to(BF16)


def valid_frames(lengths, stride, time):
    """``clamp(floor(lengths / stride), 1, time)``: frames of a clip at the
    stem hop."""
    return torch.div(lengths, stride, rounding_mode="floor").clamp(1, time)


def small_linear(x, w, b=None):
    """The autocast bf16 linear layer on an fp32 input, fp32 result."""
    return _linear(x, w, None if b is None else b.to(BF16)).float()


def mamba_block(sd, prefix, cfg, h, frames):
    d_inner = 2 * cfg.dim
    heads = d_inner // cfg.head_dim
    n = cfg.state_dim
    r = n // 4
    b, t, _ = h.shape
    p = _linear(h, sd[prefix + "in_proj.weight"])
    z, v, k, q, ddt, a, trap, angles = p.split([d_inner, d_inner, n, n, heads, heads, heads, r], -1)
    q = E.rms_norm(q.reshape(b, t, 1, n).to(BF16), sd[prefix + "C_norm.weight"])
    k = E.rms_norm(k.reshape(b, t, 1, n).to(BF16), sd[prefix + "B_norm.weight"])
    adt, dt = E.mamba_controls(a.to(BF16), ddt.to(BF16), sd[prefix + "dt_bias"], 1e-4)
    y = fused_mamba_chunked(
        q,
        k,
        v.reshape(b, t, heads, cfg.head_dim).to(BF16),
        adt,
        dt,
        trap.transpose(1, 2).to(BF16),
        sd[prefix + "C_bias"][:, 0].float(),
        sd[prefix + "B_bias"][:, 0].float(),
        angles.unsqueeze(2).expand(b, t, heads, r).to(BF16),
        sd[prefix + "D"].float(),
        z.reshape(b, t, heads, cfg.head_dim).to(BF16),
        lengths=frames,
    )
    return _linear(_bf(y).reshape(b, t, d_inner), sd[prefix + "out_proj.weight"])


def encoder_forward(sd, cfg, audio, lengths, channels):
    """Logits [B, num_outputs] (fp32) of the encoder with state dict ``sd``."""
    sd = {k: v.detach().cpu() for k, v in sd.items()}
    audio, lengths, channels = audio.cpu(), lengths.cpu(), channels.cpu()
    framed = frame_audio(audio, channels, cfg.stem_kernel, cfg.stem_stride, cfg.stem_padding)
    x = _linear(framed.float(), sd["stem.weight"].reshape(cfg.dim, cfg.stem_kernel))
    t = x.shape[1]
    frames = valid_frames(lengths, cfg.stem_stride, t)
    mask = E.time_mask(frames, t)
    x = E.mask_rows(x.float(), mask)
    for i in range(cfg.depth):
        pre = f"blocks.{i}."
        h = _bf(E.rms_norm(x, sd[pre + "pre.weight"], cfg.norm_eps))
        m = mamba_block(sd, pre + "mamba.", cfg, h, frames)
        if getattr(cfg, "bidirectional", False):
            # the reference's backward direction on the reversed valid prefix
            # and the RMSNorm of the two directions' mean (model.py:174-184)
            hb = E.reverse_valid(h, frames)
            mb = E.reverse_valid(mamba_block(sd, pre + "mamba_bwd.", cfg, hb, frames), frames)
            m = E.mean_norm(m, mb, sd[pre + "mn.weight"], cfg.norm_eps)
        x = E.add(x, m, mask)
        h = _bf(E.rms_norm(x, sd[pre + "ff_norm.weight"], cfg.norm_eps))
        g = _linear(h, sd[pre + "gate_up.weight"])
        f = E.swiglu(g.to(BF16)).float()
        x = E.add(x, _linear(f, sd[pre + "down.weight"]), mask)
    pooled = E.masked_mean(x, frames)
    return small_linear(pooled, sd["head.weight"], sd["head.bias"])
