"""The TriFusion-FP model on the MI355X kernels.

The reference model's layout and forward (``src/trifusion_l4/model.py``,
``front.py``, ``decoder.py``, ``masking.py``, ``attention.py``) with the same
parameter names, so a checkpoint saved from either loads into the other:

* ``Frontend``: log power STFT (``torch.stft``, 512-point, hop 160, Hann 400),
  three CNN stages and 8 frequency bands (``tf_bands``) (``front.py:8-114``);
  under bf16 autocast each stage is two fused kernels (``tf_front_conv1``: 3x3
  conv, channel RMSNorm, SiLU; ``tf_front_conv2``: 3x3 conv, RMSNorm, 1x1 skip
  conv, residual, SiLU), otherwise Conv2d with ``tf_front_norm``;
* ``TriFusionBlock``: LocalCNN (GLU, masked depthwise conv ``tf_depthwise_masked``,
  RMSNorm), attention on the 4:1 pooled grid (``tf_pool4``, ``tf_rotary_qkv``,
  fp32 SDPA, ``tf_interpolate``), the evidence-gated norm (``tf_evidence_norm``),
  bidirectional Mamba-3 (the fused recurrence forward and with ``reverse=True``,
  its controls computed in the prologue) merged by ``tf_mean_rmsnorm``, the
  gated concatenation (``tf_gated_concat``) with a masked depthwise merge, and a
  SwiGLU FFN (``model.py:51-200``);
* ``Decoder``: learned queries read the deep and fine features with masked
  attention, global and memory features, top-k local evidence, and the five
  logits (``decoder.py:8-96``).

The forward runs under bf16 autocast, as the reference's engine runs it
(``runtime.py:79-82``). Dropout is identity at inference.
"""

import contextlib
import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn
from torch.nn.attention import SDPBackend, sdpa_kernel

from .kernels import RMSNorm, gated_concat, swiglu
from .kernels.block import (
    Pool4,
    RotaryQKV,
    bands,
    block_pre,
    block_pre_add,
    block_pre_add_fits,
    depthwise_masked,
    evidence_down,
    evidence_down_fits,
    evidence_norm,
    front_norm,
    front_stage,
    glu_depthwise,
    glu_norm_silu,
    glu_norm_silu_fits,
    interpolate,
    interpolate_rmsnorm,
    interpolate_rmsnorm_fits,
    merge_conv,
    merge_gate,
    norm_silu,
    pack_conv3x3,
    front_lengths,
    grids,
    log_power,
    mask_audio,
    pooled_attention,
    query_read,
)
from .kernels.buffers import mask_buffer
from .kernels.native import add, add_rms, mean_norm
from .mamba import Mamba3Inference, weight_key
from .masking import masked_mean, time_mask


@dataclass
class TriFusionConfig:
    """Model configuration; the fields and defaults of the reference's
    ``ModelConfig`` (``model.py:14-34``), training-only flags included so saved
    configurations load unchanged."""

    dim: int = 1024
    depth: int = 16
    ffn_dim: int = 2816
    heads: int = 16
    state_dim: int = 128
    evidence_rank: int = 64
    dropout: float = 0.1
    backend: str = "l4"
    checkpoint_blocks: bool = False
    checkpoint_frontend: bool = False
    channels_last: bool = False
    buffer_fusion: bool = True
    native_kernels: bool = True
    mamba_packed: bool = True
    paired_mamba: bool = False
    mamba_parallel_bwd: bool = True
    mamba_fast_launch: bool = True
    paired_mamba_grid_limit: int = 64


def _bf16_autocast():
    return torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16


class _MambaShape:
    """What ``Mamba3Inference`` reads from a config: 64-wide heads."""

    def __init__(self, c):
        self.dim, self.state_dim, self.head_dim = c.dim, c.state_dim, 64


def masked_attention(q, k, v, mask):
    """fp32 scaled-dot-product attention with a boolean key mask, result in q's
    dtype (``attention.py:8-18``)."""
    dtype = q.dtype
    with torch.autocast("cuda", enabled=False), sdpa_kernel([SDPBackend.EFFICIENT_ATTENTION, SDPBackend.MATH]):
        y = F.scaled_dot_product_attention(q.float(), k.float(), v.float(), attn_mask=mask, dropout_p=0.0)
    return y.to(dtype)


_ROPE = {}


def rope_tables(time, head_dim, device):
    """cos/sin ``[time, head_dim / 2]`` of the rotary phases t 10000^(-2i/D), kept per
    (time, head_dim, device): they depend on the shape only."""
    key = (time, head_dim, str(device))
    if key not in _ROPE:
        freq = 10000.0 ** (-torch.arange(0, head_dim, 2, device=device).float() / head_dim)
        phase = torch.arange(time, device=device).float()[:, None] * freq[None, :]
        _ROPE[key] = (phase.cos(), phase.sin())
    return _ROPE[key]


class Grids:
    """Frame grid, its 4:1 pooled grid and the interpolation back
    (``masking.py:14-57``): per clip the frame and pooled lengths and masks,
    the left/right pooled neighbours and weight of every frame, and the rotary
    tables of the pooled positions."""

    def __init__(self, lengths, time, head_dim):
        dev = lengths.device
        self.lengths = lengths
        low_t = (time + 3) // 4
        if lengths.is_cuda:
            self.mask, self.low_lengths, self.low_mask, self.left, self.right, self.alpha = grids(lengths, time)
        else:
            self.mask = time_mask(lengths, time)
            self.low_lengths = (lengths + 3) // 4
            self.low_mask = time_mask(self.low_lengths, low_t)
            centre = torch.arange(time, device=dev)[None, :].float() + 0.5
            pos = (centre * self.low_lengths[:, None] / lengths[:, None] - 0.5).clamp_min(0)
            pos = torch.minimum(pos, (self.low_lengths - 1)[:, None])
            self.left = pos.long()
            self.right = torch.minimum(self.left + 1, (self.low_lengths - 1)[:, None])
            self.alpha = pos - self.left
        self.rope_cos, self.rope_sin = rope_tables(low_t, head_dim, dev)

    def pool(self, x):
        return Pool4.apply(x.contiguous(), self.lengths)

    def interpolate(self, low):
        return interpolate(low, self)


class CNNStage(nn.Module):
    """Residual Conv2d stage: conv (time stride s, frequency stride 2) -> norm ->
    SiLU -> conv -> norm, plus a 1x1 strided skip (``front.py:8-43``)."""

    def __init__(self, cin, cout, stride):
        super().__init__()
        self.stride = stride
        self.conv1 = nn.Conv2d(cin, cout, 3, stride=(stride, 2), padding=1, bias=False)
        self.conv2 = nn.Conv2d(cout, cout, 3, padding=1, bias=False)
        self.skip = nn.Conv2d(cin, cout, 1, stride=(stride, 2), bias=False)
        self.norm1, self.norm2 = RMSNorm(cout), RMSNorm(cout)
        self._packed, self._packed_key = None, None

    def packed(self):
        """bf16 weights in the fused kernels' layout: conv1 and conv2 tap-major
        ``[9, cout, cin]``, the skip ``[cout, cin]``; rebuilt when a weight changes."""
        ws = (self.conv1.weight, self.conv2.weight, self.skip.weight)
        key = tuple(weight_key(w) for w in ws)
        if self._packed_key != key:
            with torch.no_grad():
                skip = ws[2].detach().flatten(1).to(torch.bfloat16).contiguous()
                self._packed = (pack_conv3x3(ws[0]), pack_conv3x3(ws[1]), skip)
            self._packed_key = key
        return self._packed

    def forward(self, x, lengths, out_lengths=None):
        """``lengths`` are the input's valid time steps; ``out_lengths``, when the
        caller has them, the output's (ceil(lengths / stride))."""
        lengths = (lengths + self.stride - 1) // self.stride if out_lengths is None else out_lengths
        if x.is_cuda and _bf16_autocast():
            return front_stage(self, x, lengths)
        h = front_norm(self.conv1(x), lengths, self.norm1, silu=True)
        h = front_norm(self.conv2(h), lengths, self.norm2)
        valid = time_mask(lengths, h.shape[2])[:, None, :, None]
        return F.silu(h + self.skip(x).masked_fill(~valid, 0)).masked_fill(~valid, 0)


class Frontend(nn.Module):
    """Log power spectrogram -> three CNN stages -> frequency bands
    (``front.py:46-114``)."""

    def __init__(self, channels_last=True):
        super().__init__()
        self.register_buffer("window", torch.hann_window(400, periodic=True), persistent=False)
        self.stages = nn.ModuleList([CNNStage(1, 32, 1), CNNStage(32, 64, 2), CNNStage(64, 128, 2)])
        self.channels_last = channels_last
        if channels_last:
            self.to(memory_format=torch.channels_last)

    def spectrogram(self, audio, sample_lengths, channels, frames=None):
        """Masked log power ``[B, 1, frames, 257]`` and the frame counts (``frames``
        when the caller has them)."""
        b, c, n = audio.shape
        if audio.is_cuda:
            # masking and the log-power post-processing as one launch each around rocFFT
            wave = mask_audio(audio, sample_lengths, channels)
            with torch.autocast("cuda", enabled=False):
                spec = torch.stft(wave, n_fft=512, hop_length=160, win_length=400, window=self.window.float(),
                                  center=True, pad_mode="constant", return_complex=True)
            if frames is None:
                frames = sample_lengths // 160 + 1
            return log_power(spec, channels, sample_lengths, 160).unsqueeze(1), frames
        with torch.autocast("cuda", enabled=False):
            keep = time_mask(sample_lengths, n)[:, None, :] & (torch.arange(c, device=audio.device)[None, :]
                                                               < channels[:, None])[..., None]
            wave = audio.float().masked_fill(~keep, 0)
            spec = torch.stft(wave.reshape(b * c, n), n_fft=512, hop_length=160, win_length=400,
                              window=self.window.float(), center=True, pad_mode="constant", return_complex=True)
            power = (spec.real.square() + spec.imag.square()).reshape(b, c, 257, -1).sum(1)
            power = power / channels[:, None, None]
            log = torch.log(1e-6 + power).transpose(1, 2).unsqueeze(1)
            lengths = sample_lengths // 160 + 1
            log = log.masked_fill(~time_mask(lengths, log.shape[2])[:, None, :, None], 0)
        return log, lengths

    def forward(self, audio, sample_lengths, channels):
        # on the GPU, the frame counts before and after every stage in one launch
        counts = front_lengths(sample_lengths, 160, [st.stride for st in self.stages]) if audio.is_cuda else None
        x, lengths = self.spectrogram(audio, sample_lengths, channels, None if counts is None else counts[0])
        if self.channels_last:
            x = x.contiguous(memory_format=torch.channels_last)
        fine = fine_lengths = None
        # outside bf16 autocast the stages run the library's convolutions, with
        # deterministic algorithms: some of the faster ones accumulate in a
        # run-dependent order, and repeated forwards (and graph replays against
        # eager calls) must give the same bits
        with torch.backends.cudnn.flags(enabled=torch.backends.cudnn.enabled, benchmark=False, deterministic=True,
                                        allow_tf32=False):
            for i, stage in enumerate(self.stages):
                if counts is None:
                    x = stage(x, lengths)
                    lengths = (lengths + stage.stride - 1) // stage.stride
                else:
                    x = stage(x, lengths, counts[i + 1])
                    lengths = counts[i + 1]
                if i == 1:
                    fine, fine_lengths = bands(x), lengths
        return bands(x).flatten(2), fine, lengths, fine_lengths


class LocalCNN(nn.Module):
    """GLU -> masked depthwise conv (7) -> RMSNorm -> SiLU -> linear (``model.py:51-75``)."""

    def __init__(self, c):
        super().__init__()
        self.up = nn.Linear(c.dim, 2 * c.dim, bias=False)
        self.dw = nn.Conv1d(c.dim, c.dim, 7, padding=3, groups=c.dim)
        self.norm = RMSNorm(c.dim)
        self.out = nn.Linear(c.dim, c.dim, bias=False)

    def forward(self, x, mask, lengths):
        h = depthwise_masked(F.glu(self.up(x), dim=-1), self.dw, lengths)
        return self.out(F.silu(self.norm(h)))


class GlobalAttention(nn.Module):
    """Rotary multi-head attention on the 4:1 pooled grid, interpolated back to
    frames (``model.py:78-98``)."""

    def __init__(self, c):
        super().__init__()
        self.heads, self.head_dim = c.heads, c.dim // c.heads
        self.qkv = nn.Linear(c.dim, 3 * c.dim, bias=False)
        self.out = nn.Linear(c.dim, c.dim, bias=False)

    def forward(self, x, grids):
        p = grids.pool(x)
        q, k, v = RotaryQKV.apply(self.qkv(p), grids.rope_cos, grids.rope_sin, self.heads).unbind(0)
        y = masked_attention(q, k, v, grids.low_mask[:, None, None, :])
        return grids.interpolate(self.out(y.transpose(1, 2).reshape(p.shape)))


class TriFusionBlock(nn.Module):
    """Local CNN, pooled attention and bidirectional Mamba-3 mixed by an
    evidence gate and a gated, depthwise-merged concatenation, then a SwiGLU
    FFN (``model.py:101-200``)."""

    def __init__(self, c):
        super().__init__()
        d, r = c.dim, c.evidence_rank
        self.pre = RMSNorm(d)
        self.local, self.attention = LocalCNN(c), GlobalAttention(c)
        self.cn, self.an, self.mn = RMSNorm(d), RMSNorm(d), RMSNorm(d)
        self.e_down = nn.Linear(2 * d, r)
        self.e_value, self.e_gate = nn.Linear(r, d), nn.Linear(r, d)
        self.u_norm = RMSNorm(d)
        shape = _MambaShape(c)
        self.forward_mamba, self.backward_mamba = Mamba3Inference(shape), Mamba3Inference(shape)
        self.gate = nn.Linear(3 * d, 3)
        self.merge_dw = nn.Conv1d(3 * d, 3 * d, 3, padding=1, groups=3 * d)
        self.merge = nn.Linear(3 * d, d, bias=False)
        self.ff_norm = RMSNorm(d)
        self.gate_up = nn.Linear(d, 2 * c.ffn_dim, bias=False)
        self.down = nn.Linear(c.ffn_dim, d, bias=False)
        self._fused_weights = {}
        self.branch_streams = True
        nn.init.zeros_(self.e_gate.weight)
        nn.init.zeros_(self.e_gate.bias)
        nn.init.normal_(self.e_value.weight, std=1e-3)
        nn.init.zeros_(self.e_value.bias)
        nn.init.zeros_(self.gate.weight)
        nn.init.zeros_(self.gate.bias)
        with torch.no_grad():
            self.merge.weight.mul_(1 / math.sqrt(2 * c.depth))
            self.down.weight.mul_(1 / math.sqrt(2 * c.depth))

    def fusable(self, x):
        """The fused forward applies: a CUDA fp32 residual stream under bf16
        autocast, widths the fused kernels take, the reference's kernel sizes."""
        d = x.shape[-1]
        return (x.is_cuda and x.dtype == torch.float32 and _bf16_autocast() and d % 8 == 0 and d <= 4096
                and self.attention.head_dim in (32, 64) and self.merge_dw.kernel_size[0] == 3
                and self.local.dw.kernel_size[0] in (3, 7))

    def forward(self, x, grids, defer=False):
        """``defer``: the fused forward may return its closing residual add
        unapplied, as ``(r, down)``, for the next block's start to apply
        (``forward`` accepts such a pair as ``x``)."""
        if isinstance(x, tuple):
            if self.fusable(x[0]):
                return self.forward_fused(x, grids, defer)
            x = add(x[0], x[1], grids.mask)
        if self.fusable(x):
            return self.forward_fused(x, grids, defer)
        mask, lengths = grids.mask, grids.lengths
        x = mask_buffer(x, mask)
        h = self.pre(x)
        cn = self.cn(self.local(h, mask, lengths))
        an = self.an(self.attention(h, grids))
        z = F.silu(self.e_down(torch.cat((cn, an), -1)))
        u = evidence_norm(x, self.e_value(z), self.e_gate(z), self.u_norm.weight, mask, self.u_norm.eps)
        # rows past each length come out of the recurrence as zeros in both directions
        mf = self.forward_mamba(u, lengths)
        mb = self.backward_mamba(u, lengths, reverse=True)
        mn = mean_norm(mf, mb, self.mn.weight, self.mn.eps)
        s = torch.cat((cn, mn, an), -1)
        v = gated_concat(s, self.gate(s))
        conv = depthwise_masked(v, self.merge_dw, lengths)
        bf16 = torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16
        r = x + self.merge(add(v, conv, bf16=bf16))
        f = swiglu(self.gate_up(self.ff_norm(r)))
        return add(r, self.down(f), mask), mf, mb

    def _joined(self, name, parts, build):
        """Weights of two layers that read the same input, joined for one GEMM;
        rebuilt when any part changes."""
        key = tuple(weight_key(t) for t in parts)
        hit = self._fused_weights.get(name)
        if hit is None or hit[0] != key:
            with torch.no_grad():
                hit = (key, build())
            self._fused_weights[name] = hit
        return hit[1]

    def _local_branch(self, h, lengths):
        """GLU, masked depthwise conv, norm, SiLU, out-projection and the cn
        norm: ``cn``."""
        local = self.local
        up = local.up(h)
        if glu_norm_silu_fits(up, local.dw):
            return self.cn(local.out(glu_norm_silu(up, local.dw, lengths, local.norm)))
        return self.cn(local.out(norm_silu(glu_depthwise(up, local.dw, lengths), local.norm)))

    def _attention_branch(self, p, grids):
        """Pooled attention, interpolated to frames and normalised: ``an``."""
        att = self.attention
        low = att.out(pooled_attention(att.qkv(p), grids, att.heads))
        if interpolate_rmsnorm_fits(low):
            return interpolate_rmsnorm(low, grids, self.an)
        return self.an(grids.interpolate(low))

    def forward_fused(self, x, grids, defer=False):
        """``forward`` with the elementwise runs between the GEMMs fused: the same
        tensors in the same dtypes as the autocast forward, the casts the GEMMs
        would make done by the producing kernels. Layers that read one input run
        as one GEMM: e_value with e_gate, and the in-projections of the two
        Mamba directions; the two out-projections run as one batched GEMM. ``x``
        may be the previous block's unapplied closing add ``(r, down)``, which
        the start kernel applies; with ``defer`` this block returns its own."""
        mask, lengths = grids.mask, grids.lengths
        if isinstance(x, tuple):
            b, t, d = x[0].shape
            x, h, p = block_pre_add(x[0], x[1], lengths, self.pre)
        else:
            b, t, d = x.shape
            x, h, p = block_pre(x, lengths, self.pre)
        # Under graph capture (and in the warm-ups before one, see eager_forks)
        # the attention branch, which reads only p, runs on the branch stream
        # while the local branch runs here, and rejoins before the evidence
        # path. Other eager calls stay on one stream: there the host cost of the
        # fork outweighs the overlap.
        if self.branch_streams and forking():
            side = branch_stream(x.device)
            main = torch.cuda.current_stream(x.device)
            side.wait_stream(main)
            try:
                with torch.cuda.stream(side):
                    an = self._attention_branch(p, grids)
                cn = self._local_branch(h, lengths)
            finally:
                # joined on every exit: an error inside a capture (out of
                # memory) must leave no stream forked off it
                main.wait_stream(side)
        else:
            an = self._attention_branch(p, grids)
            cn = self._local_branch(h, lengths)
        if evidence_down_fits(d, self.e_down.out_features):
            z = evidence_down(cn, an, self.e_down)
        else:
            z = F.silu(self.e_down(torch.cat((cn, an), -1)))
        ev, eg = self.e_value, self.e_gate
        wv = self._joined("evidence", (ev.weight, ev.bias, eg.weight, eg.bias),
                          lambda: (torch.cat((ev.weight, eg.weight)), torch.cat((ev.bias, eg.bias))))
        ve = F.linear(z, *wv)
        u = evidence_norm(x, ve[..., :d], ve[..., d:], self.u_norm.weight, mask, self.u_norm.eps, bf16_out=True)
        fw, bw = self.forward_mamba, self.backward_mamba
        pf, pb = fw._padded_in_proj(), bw._padded_in_proj()
        proj = F.linear(u, self._joined("in_proj", (pf, pb), lambda: torch.cat((pf, pb))))
        width, half = fw.in_proj.out_features, pf.shape[0]
        ys = torch.empty((2, b, t, fw.nheads, fw.headdim), device=x.device, dtype=torch.bfloat16)
        fw.mix(proj[..., :width], lengths, out=ys[0])
        bw.mix(proj[..., half : half + width], lengths, reverse=True, out=ys[1])
        wo = (fw.out_proj.weight, bw.out_proj.weight)
        wo = self._joined("out_proj", wo, lambda: torch.stack((wo[0].t(), wo[1].t())).contiguous())
        m = torch.bmm(ys.view(2, b * t, fw.d_inner), wo)
        mf, mb = m[0].view(b, t, d), m[1].view(b, t, d)
        mn, g = merge_gate(cn, mf, mb, an, self.mn, self.gate)
        merged = self.merge(merge_conv(cn, mn, an, g, self.merge_dw, lengths))
        r, f = add_rms(x, merged, self.ff_norm.weight, None, self.ff_norm.eps, torch.bfloat16)
        f = swiglu(self.gate_up(f))
        down = self.down(f)
        if defer and down.dtype == torch.bfloat16 and block_pre_add_fits(r, down):
            return (r, down), mf, mb
        return add(r, down, mask), mf, mb


_BRANCH_STREAMS = {}
_EAGER_FORKS = [0]


def forking():
    """Whether forward calls fork onto the branch streams: under graph capture,
    or inside ``eager_forks``."""
    return _EAGER_FORKS[0] > 0 or torch.cuda.is_current_stream_capturing()


@contextlib.contextmanager
def eager_forks():
    """Fork in eager calls too: the warm-ups before a capture run the captured
    schedule, so the branch streams have their library handles and workspaces
    before capture begins."""
    _EAGER_FORKS[0] += 1
    try:
        yield
    finally:
        _EAGER_FORKS[0] -= 1


def branch_stream(device, slot=0):
    """A second stream for work that forks off the caller's, one per (device,
    slot), at the default priority: slot 0 takes the fused block's attention
    branch, slot 1 the decoder's fine reads. Every fork waits for the caller's
    stream and is joined back before the forked results are used or its inputs
    dropped, so a tensor either side allocates is freed only after both have
    consumed it, and graph capture records the two as parallel paths."""
    index = torch.device(device).index
    key = (torch.cuda.current_device() if index is None else index, slot)
    if key not in _BRANCH_STREAMS:
        _BRANCH_STREAMS[key] = torch.cuda.Stream(device=key[0])
    return _BRANCH_STREAMS[key]


_SINPOS = {}


def sin_position(time, dim, device, dtype=torch.float32):
    """Interleaved sin/cos positions ``[time, dim]`` (``decoder.py:9-14``), formed
    in fp32 and cast to ``dtype``; kept per (time, dim, device, dtype), since they
    depend on the shape only (one table instead of eight launches per forward)."""
    key = (time, dim, str(device), dtype)
    if key not in _SINPOS:
        phase = torch.arange(time, device=device).float()[:, None] * (
            10000.0 ** (-torch.arange(0, dim, 2, device=device).float() / dim)
        )[None, :]
        _SINPOS[key] = torch.stack((phase.sin(), phase.cos()), -1).flatten(-2).to(dtype)
    return _SINPOS[key]


class QueryRead(nn.Module):
    """Ten learned 256-wide queries read a sequence with 8-head masked attention;
    returns the means of queries 0-3, 4-7 and 8-9 (``decoder.py:17-32``)."""

    def __init__(self, input_dim):
        super().__init__()
        self.kv = nn.Linear(input_dim, 512, bias=False)
        self.q = nn.Linear(256, 256, bias=False)
        self.out = nn.Linear(256, 256, bias=False)

    def forward(self, query, x, mask, key_lengths=None):
        """``mask`` marks the valid keys; ``key_lengths`` (valid keys form a prefix
        of that length) selects the fused query-read kernel under bf16 autocast."""
        b, t, _ = x.shape
        if key_lengths is not None and x.is_cuda and _bf16_autocast():
            h = self.out(query_read(self.q(query), self.kv(x), key_lengths, 8))
            return h[:, :4].mean(1), h[:, 4:8].mean(1), h[:, 8:].mean(1)
        k, v = self.kv(x).view(b, t, 2, 8, 32).permute(2, 0, 3, 1, 4).unbind(0)
        q = self.q(query).view(10, 8, 32).transpose(0, 1).unsqueeze(0).expand(b, -1, -1, -1)
        h = self.out(masked_attention(q, k, v, mask[:, None, None, :]).transpose(1, 2).reshape(b, 10, 256))
        return h[:, :4].mean(1), h[:, 4:8].mean(1), h[:, 8:].mean(1)


class Decoder(nn.Module):
    """Deep and fine query reads, global and memory features and top-25 local
    evidence into file, voice and music logits (``decoder.py:35-96``)."""

    def __init__(self, dim):
        super().__init__()
        self.query = nn.Parameter(torch.randn(10, 256) * 0.02)
        self.band = nn.Parameter(torch.randn(8, 64) * 0.02)
        self.deep_read, self.fine_read = QueryRead(dim), QueryRead(64)
        self.global_proj, self.memory_proj = nn.Linear(dim, 256), nn.Linear(2 * dim, 256)
        self.local_logits = nn.Linear(512, 2)
        self.local_features = nn.Linear(512, 256)
        self.voice_lat = nn.Sequential(nn.Linear(1280, 256), nn.SiLU())
        self.music_lat = nn.Sequential(nn.Linear(1280, 256), nn.SiLU())
        self.voice_head, self.music_head = nn.Linear(256, 2), nn.Linear(256, 2)
        self.file_head = nn.Sequential(nn.Linear(1536, 256), nn.SiLU(), nn.Linear(256, 1))

    def read_fine(self, fine, fine_lengths):
        """The reads that depend on the fine features alone: the fine mask, the
        fine query read, the local logits and the top-k evidence means."""
        b, tf, _, _ = fine.shape
        dev = fine.device
        fm = time_mask(fine_lengths, tf)
        fp = fine + sin_position(tf, 64, dev, fine.dtype)[None, :, None, :] + self.band.to(fine.dtype)[None, None]
        # the fine keys are (frame, band) pairs: valid exactly below 8 * fine_lengths
        fine_q = self.fine_read(self.query, fp.flatten(1, 2), fm[:, :, None].expand(b, tf, 8).reshape(b, -1),
                                8 * fine_lengths)
        flat = fine.flatten(2)
        local, features = self.local_logits(flat), self.local_features(flat)
        k = min(25, tf)
        idx = local.float().masked_fill(~fm[..., None], -torch.inf).transpose(1, 2).topk(k, -1).indices
        picked = features[:, None].expand(-1, 2, -1, -1).gather(2, idx[..., None].expand(-1, -1, -1, 256))
        valid_k = torch.arange(k, device=dev)[None, :] < fine_lengths.clamp_max(k)[:, None]
        top = (picked.float() * valid_k[:, None, :, None]).sum(2) / valid_k.sum(1)[:, None, None]
        return fm, fine_q, local.float(), top

    def forward(self, x, fine, grids, fine_lengths, mf, mb, fine_reads=None):
        """``fine_reads``: ``read_fine(fine, fine_lengths)`` when the caller has
        already formed it."""
        b = x.shape[0]
        dev = x.device
        fm, fine_q, local, top = fine_reads or self.read_fine(fine, fine_lengths)
        deep = self.deep_read(self.query, x, grids.mask, grids.lengths)
        if x.is_cuda:
            pooled = masked_mean(x.float(), grids.lengths)
        else:
            pooled = (x.float() * grids.mask[..., None]).sum(1) / grids.lengths[:, None]
        global_feature = self.global_proj(pooled)
        end = mf[torch.arange(b, device=dev), grids.lengths - 1]
        memory = self.memory_proj(torch.cat((end, mb[:, 0]), -1))
        voice = self.voice_lat(torch.cat((deep[0], fine_q[0], global_feature, top[:, 0], memory), -1))
        music = self.music_lat(torch.cat((deep[1], fine_q[1], global_feature, top[:, 1], memory), -1))
        v, m = self.voice_head(voice), self.music_head(music)
        f = self.file_head(torch.cat((deep[2], fine_q[2], global_feature, memory, voice, music), -1))
        logits = torch.cat((f, v[:, :1], m[:, :1], v[:, 1:], m[:, 1:]), -1).float()
        return {
            "logits": logits,
            "local_logits": local,
            "local_mask": fm,
            "features": x,
            "feature_mask": grids.mask,
            "embedding": global_feature.float(),
        }


class TriFusion(nn.Module):
    """Front end -> projection -> TriFusion blocks -> decoder (``model.py:203-260``)."""

    def __init__(self, config=None):
        super().__init__()
        self.config = c = config or TriFusionConfig()
        if c.dim % c.heads or c.dim % 32:
            raise ValueError("dim must divide attention heads and Mamba headdim")
        self.front = Frontend(c.channels_last)
        self.front_projection = nn.Identity() if c.dim == 1024 else nn.Linear(1024, c.dim, bias=False)
        self.blocks = nn.ModuleList([TriFusionBlock(c) for _ in range(c.depth)])
        self.decoder = Decoder(c.dim)
        self.memory_head = nn.Linear(c.dim, 2)
        self.fork_fine = True

    def set_variant(self, variant):
        """Select the recurrence kernel ("auto", "pipe", "mfma" or "generic") of every Mamba."""
        for m in self.modules():
            if isinstance(m, Mamba3Inference):
                m.variant = variant

    def encode(self, audio, lengths, channels):
        return self._blocks(*self.front(audio, lengths, channels))

    def _blocks(self, x, fine, main_lengths, fine_lengths):
        x = self.front_projection(x).float()
        grids = Grids(main_lengths, x.shape[1], self.config.dim // self.config.heads)
        mf = mb = None
        last = len(self.blocks) - 1
        for i, block in enumerate(self.blocks):
            # a block's closing residual add is applied by the next block's start
            x, mf, mb = block(x, grids, defer=i < last)
        return x, fine, grids, fine_lengths, mf, mb

    def forward(self, audio, lengths, channels):
        front = self.front(audio, lengths, channels)
        fine, fine_lengths = front[1], front[3]
        if not (self.fork_fine and fine.is_cuda and forking()):
            return self.decoder(*self._blocks(*front))
        # Under graph capture (and in the warm-ups before one) the fine reads,
        # which need only the front end's fine features, run on their own
        # stream beside the blocks.
        main, side = torch.cuda.current_stream(fine.device), branch_stream(fine.device, 1)
        side.wait_stream(main)
        try:
            with torch.cuda.stream(side):
                reads = self.decoder.read_fine(fine, fine_lengths)
            encoded = self._blocks(*front)
        finally:
            main.wait_stream(side)
        return self.decoder(*encoded, fine_reads=reads)


__all__ = ["TriFusion", "TriFusionConfig", "TriFusionBlock", "Frontend", "Decoder", "Grids"]
