"""CPU forward of the TriFusion-FP model (oracle).

Test infrastructure only (see ``oracle/__init__.py``). Evaluates a TriFusion
state dict with plain PyTorch CPU ops, the recurrence oracle and the
restatements in ``oracle/trifusion.py``, following the reference model's
forward (``src/trifusion_l4/model.py:140-260``, ``front.py:8-114``,
``decoder.py:8-96``, ``masking.py:14-80``). Values are rounded to bf16 where the
GPU forward under bf16 autocast holds bf16 (GEMM and convolution inputs and
outputs, norms of bf16 tensors, elementwise ops on bf16 tensors); the residual
stream, the evidence and mean norms, attention (fp32 SDPA) and the pooled
features stay fp32. The backward Mamba runs on explicitly reversed valid
prefixes, as the reference does. Parity target: sigmoid probabilities within
1e-2.
"""

import math
from types import SimpleNamespace

import torch
import torch.nn.functional as F

from . import elementwise as E
from . import trifusion as K
from .encoder import _bf, _linear, mamba_block

BF16 = torch.bfloat16


def _rms_bf(x, w, eps=1e-5):
    """RMSNorm of a bf16-valued tensor, bf16 result."""
    return E.rms_norm(x.to(BF16), w, eps).float()


def _attention(q, k, v, mask):
    return _bf(F.scaled_dot_product_attention(q.float(), k.float(), v.float(), attn_mask=mask))


def _stage(sd, pre, x, lengths, stride):
    lengths = (lengths + stride - 1) // stride
    y = K.front_stage(x, lengths, sd[pre + "conv1.weight"], sd[pre + "conv2.weight"], sd[pre + "skip.weight"],
                      sd[pre + "norm1.weight"], sd[pre + "norm2.weight"], stride)
    return y.float().permute(0, 3, 1, 2), lengths


def frontend(sd, audio, sample_lengths, channels):
    b, c, n = audio.shape
    keep = E.time_mask(sample_lengths, n)[:, None, :] & (torch.arange(c)[None, :] < channels[:, None])[..., None]
    wave = audio.float().masked_fill(~keep, 0)
    spec = torch.stft(wave.reshape(b * c, n), n_fft=512, hop_length=160, win_length=400,
                      window=torch.hann_window(400, periodic=True), center=True, pad_mode="constant",
                      return_complex=True)
    power = (spec.real.square() + spec.imag.square()).reshape(b, c, 257, -1).sum(1) / channels[:, None, None]
    x = torch.log(1e-6 + power).transpose(1, 2).unsqueeze(1)
    lengths = sample_lengths // 160 + 1
    x = x.masked_fill(~E.time_mask(lengths, x.shape[2])[:, None, :, None], 0)
    fine = fine_lengths = None
    for i, stride in enumerate((1, 2, 2)):
        x, lengths = _stage(sd, f"front.stages.{i}.", x, lengths, stride)
        if i == 1:
            fine, fine_lengths = K.bands(x.to(BF16)).float(), lengths
    return K.bands(x.to(BF16)).float().flatten(2), fine, lengths, fine_lengths


def block(sd, pre, cfg, x, lengths, grids):
    low_lengths, left, right, alpha, low_mask, cos, sin = grids
    mask = E.time_mask(lengths, x.shape[1])
    d = cfg.dim
    x = E.mask_rows(x, mask)
    h = E.rms_norm(x, sd[pre + "pre.weight"])
    # local CNN
    up = _linear(h, sd[pre + "local.up.weight"])
    g = _bf(F.glu(up, dim=-1))
    g = K.depthwise_masked(g.to(BF16), sd[pre + "local.dw.weight"].to(BF16), sd[pre + "local.dw.bias"].to(BF16),
                           lengths).float()
    loc = _linear(_bf(F.silu(_rms_bf(g, sd[pre + "local.norm.weight"]))), sd[pre + "local.out.weight"])
    cn = _rms_bf(loc, sd[pre + "cn.weight"])
    # pooled attention
    heads = cfg.heads
    p = K.pool4(h, lengths)
    qkv = _linear(p, sd[pre + "attention.qkv.weight"])
    q, k, v = K.rotary_qkv(qkv.to(BF16), cos, sin, heads).float().unbind(0)
    y = _attention(q, k, v, low_mask[:, None, None, :])
    y = _linear(y.transpose(1, 2).reshape(p.shape), sd[pre + "attention.out.weight"])
    an = _rms_bf(K.interpolate(y.to(BF16), left, right, alpha, lengths).float(), sd[pre + "an.weight"])
    # evidence-gated input of the recurrences
    z = _bf(F.silu(_linear(torch.cat((cn, an), -1), sd[pre + "e_down.weight"], sd[pre + "e_down.bias"].to(BF16))))
    value = _linear(z, sd[pre + "e_value.weight"], sd[pre + "e_value.bias"].to(BF16))
    gate = _linear(z, sd[pre + "e_gate.weight"], sd[pre + "e_gate.bias"].to(BF16))
    u = K.evidence_norm(x, value, gate, sd[pre + "u_norm.weight"], mask)
    mcfg = SimpleNamespace(dim=d, head_dim=64, state_dim=cfg.state_dim)
    mf = mamba_block(sd, pre + "forward_mamba.", mcfg, u, lengths)
    mb = E.reverse_valid(mamba_block(sd, pre + "backward_mamba.", mcfg, E.reverse_valid(u, lengths), lengths),
                         lengths)
    mn = E.mean_norm(mf, mb, sd[pre + "mn.weight"])
    s = torch.cat((cn, mn, an), -1)
    v = K.gated_concat(s, _linear(s, sd[pre + "gate.weight"], sd[pre + "gate.bias"].to(BF16)))
    conv = K.depthwise_masked(v.to(BF16), sd[pre + "merge_dw.weight"].to(BF16), sd[pre + "merge_dw.bias"].to(BF16),
                              lengths).float()
    r = x + _linear(_bf(v + conv), sd[pre + "merge.weight"])
    f = E.swiglu(_linear(E.rms_norm(r, sd[pre + "ff_norm.weight"]), sd[pre + "gate_up.weight"]).to(BF16)).float()
    out = E.mask_rows(r + _linear(f, sd[pre + "down.weight"]), mask)
    return out, mf, mb


def _query_read(sd, pre, query, x, mask):
    b, t, _ = x.shape
    k, v = _linear(x, sd[pre + "kv.weight"]).view(b, t, 2, 8, 32).permute(2, 0, 3, 1, 4).unbind(0)
    q = _linear(query, sd[pre + "q.weight"]).view(10, 8, 32).transpose(0, 1).unsqueeze(0).expand(b, -1, -1, -1)
    h = _attention(q, k, v, mask[:, None, None, :])
    h = _linear(h.transpose(1, 2).reshape(b, 10, 256), sd[pre + "out.weight"])
    return _bf(h[:, :4].mean(1)), _bf(h[:, 4:8].mean(1)), _bf(h[:, 8:].mean(1))


def _sin_position(time, dim):
    phase = torch.arange(time).float()[:, None] * (10000.0 ** (-torch.arange(0, dim, 2).float() / dim))[None, :]
    return torch.stack((phase.sin(), phase.cos()), -1).flatten(-2)


def decoder(sd, x, fine, lengths, fine_lengths, mf, mb):
    b, tf, _, _ = fine.shape
    fm = E.time_mask(fine_lengths, tf)
    mask = E.time_mask(lengths, x.shape[1])
    query = sd["decoder.query"]
    deep = _query_read(sd, "decoder.deep_read.", query, x, mask)
    fp = _bf(_bf(fine + _bf(_sin_position(tf, 64))[None, :, None, :]) + _bf(sd["decoder.band"])[None, None])
    fine_q = _query_read(sd, "decoder.fine_read.", query, fp.flatten(1, 2), fm[:, :, None].expand(b, tf, 8).reshape(b, -1))
    glob = _linear((x * mask[..., None]).sum(1) / lengths[:, None], sd["decoder.global_proj.weight"],
                   sd["decoder.global_proj.bias"].to(BF16))
    end = mf[torch.arange(b), lengths - 1]
    memory = _linear(torch.cat((end, mb[:, 0]), -1), sd["decoder.memory_proj.weight"],
                     sd["decoder.memory_proj.bias"].to(BF16))
    flat = fine.flatten(2)
    local = _linear(flat, sd["decoder.local_logits.weight"], sd["decoder.local_logits.bias"].to(BF16))
    features = _linear(flat, sd["decoder.local_features.weight"], sd["decoder.local_features.bias"].to(BF16))
    k = min(25, tf)
    idx = local.masked_fill(~fm[..., None], -math.inf).transpose(1, 2).topk(k, -1).indices
    picked = features[:, None].expand(-1, 2, -1, -1).gather(2, idx[..., None].expand(-1, -1, -1, 256))
    valid_k = torch.arange(k)[None, :] < fine_lengths.clamp_max(k)[:, None]
    top = (picked * valid_k[:, None, :, None]).sum(2) / valid_k.sum(1)[:, None, None]

    def lat(name, parts):
        return _bf(F.silu(_linear(torch.cat(parts, -1), sd[f"decoder.{name}.0.weight"],
                                  sd[f"decoder.{name}.0.bias"].to(BF16))))

    voice = lat("voice_lat", (deep[0], fine_q[0], glob, top[:, 0], memory))
    music = lat("music_lat", (deep[1], fine_q[1], glob, top[:, 1], memory))
    v = _linear(voice, sd["decoder.voice_head.weight"], sd["decoder.voice_head.bias"].to(BF16))
    m = _linear(music, sd["decoder.music_head.weight"], sd["decoder.music_head.bias"].to(BF16))
    hidden = lat("file_head", (deep[2], fine_q[2], glob, memory, voice, music))
    f = _linear(hidden, sd["decoder.file_head.2.weight"], sd["decoder.file_head.2.bias"].to(BF16))
    return torch.cat((f, v[:, :1], m[:, :1], v[:, 1:], m[:, 1:]), -1)


def trifusion_forward(sd, cfg, audio, lengths, channels):
    """Logits ``[B, 5]`` (fp32) of the TriFusion model with state dict ``sd``."""
    sd = {k: v.detach().cpu() for k, v in sd.items()}
    audio, lengths, channels = audio.cpu(), lengths.cpu(), channels.cpu()
    x, fine, main_lengths, fine_lengths = frontend(sd, audio, lengths, channels)
    if "front_projection.weight" in sd:
        x = _linear(x, sd["front_projection.weight"])
    x = x.float()
    t = x.shape[1]
    low_lengths, left, right, alpha = K.grids(main_lengths, t)
    low_t = (t + 3) // 4
    hd = cfg.dim // cfg.heads
    phase = torch.arange(low_t).float()[:, None] * (10000.0 ** (-torch.arange(0, hd, 2).float() / hd))[None, :]
    grids = (low_lengths, left, right, alpha, E.time_mask(low_lengths, low_t), phase.cos(), phase.sin())
    mf = mb = None
    for i in range(cfg.depth):
        x, mf, mb = block(sd, f"blocks.{i}.", cfg, x, main_lengths, grids)
    return decoder(sd, x, fine, main_lengths, fine_lengths, mf, mb).float()
