"""``trifusion_amd::*`` torch operators over the C-ABI library.

Every compute entry point of ``include/trifusion_amd.h`` is registered with
``torch.library`` in the ``trifusion_amd`` namespace:

* a CUDA kernel (ROCm devices dispatch through the CUDA key) that validates
  the operands and calls the C entry on the current stream;
* a Meta kernel giving output shapes and dtypes, so the operators trace under
  fake tensors (``torch.compile``, ``torch.export``) without a device;
* a CPU kernel that raises: there is no CPU path by design.

The public Python API (``fused_mamba``, ``kernels.rms``, ``kernels.swiglu``,
...) calls these operators, so eager calls, graph capture and tracing all go
through the same dispatcher entry. The reference launches its Triton kernels
directly from Python (``src/trifusion_l4/mamba_fused.py:162-190``); the
operator layer is the torch-native form of that launch.
"""

import torch

NAMESPACE = "trifusion_amd"

# keyword extensions of fused_mamba: valid lengths, kernel choice, reversed
# walk of the valid prefix, raw controls (dt_bias) and their decay floor, and
# the B/C RMSNorm weights applied to raw q/k rows (q_norm, k_norm, norm_eps)
_EXT = (
    "Tensor? lengths=None, str variant='auto', bool reverse=False, Tensor? dt_bias=None, float a_floor=0.0001, "
    "Tensor? q_norm=None, Tensor? k_norm=None, float norm_eps=1e-05"
)

_SCHEMAS = {
    "fused_mamba": "fused_mamba(Tensor q, Tensor k, Tensor v, Tensor adt, Tensor dt, Tensor trap, Tensor qb, "
    f"Tensor kb, Tensor angles, Tensor d, Tensor z, {_EXT}) -> Tensor",
    "fused_mamba.out": "fused_mamba.out(Tensor q, Tensor k, Tensor v, Tensor adt, Tensor dt, Tensor trap, "
    f"Tensor qb, Tensor kb, Tensor angles, Tensor d, Tensor z, {_EXT}, *, Tensor(a!) out) -> Tensor(a!)",
    "rms_norm": "rms_norm(Tensor x, Tensor weight, float eps=1e-05, ScalarType? out_dtype=None) -> Tensor",
    "add_rms_norm": "add_rms_norm(Tensor a, Tensor b, Tensor weight, Tensor? mask=None, float eps=1e-05, "
    "ScalarType? out_dtype=None) -> (Tensor, Tensor)",
    "add": "add(Tensor a, Tensor b, Tensor? mask=None, bool bf16=False) -> Tensor",
    "swiglu": "swiglu(Tensor x) -> Tensor",
    "mask_rows": "mask_rows(Tensor x, Tensor mask) -> Tensor",
    "mamba_controls": "mamba_controls(Tensor a, Tensor dt, Tensor bias, float floor) -> (Tensor, Tensor)",
    "masked_mean": "masked_mean(Tensor x, Tensor lengths) -> Tensor",
    "time_mask": "time_mask(Tensor lengths, int time) -> Tensor",
    "reverse_valid": "reverse_valid(Tensor x, Tensor lengths) -> Tensor",
    "mean_rms_norm": "mean_rms_norm(Tensor a, Tensor b, Tensor weight, float eps=1e-05) -> Tensor",
    "mask_rms_norm": "mask_rms_norm(Tensor x, Tensor mask, Tensor weight, float eps=1e-05, "
    "ScalarType? out_dtype=None) -> (Tensor, Tensor)",
    "rms_norm_pair": "rms_norm_pair(Tensor x, Tensor w0, Tensor w1, float eps=1e-05) -> Tensor",
    "frame_audio": "frame_audio(Tensor audio, Tensor channels, int kernel, int stride, int pad, int width) -> Tensor",
    "frames_mask": "frames_mask(Tensor lengths, int stride, int time) -> (Tensor, Tensor)",
    "small_linear": "small_linear(Tensor x, Tensor weight, Tensor? bias=None) -> Tensor",
    "depthwise_masked": "depthwise_masked(Tensor x, Tensor weight, Tensor bias, Tensor lengths) -> Tensor",
    "pool4": "pool4(Tensor x, Tensor lengths) -> Tensor",
    "rotary_qkv": "rotary_qkv(Tensor x, Tensor cos, Tensor sin, int heads) -> Tensor",
    "front_norm": "front_norm(Tensor x, Tensor lengths, Tensor weight, float eps, bool silu) -> Tensor",
    "interpolate": "interpolate(Tensor low, Tensor left, Tensor right, Tensor alpha, Tensor lengths) -> Tensor",
    "interpolate_rmsnorm": (
        "interpolate_rmsnorm(Tensor low, Tensor left, Tensor right, Tensor alpha, Tensor lengths, Tensor weight, "
        "float eps) -> Tensor"
    ),
    "bands": "bands(Tensor x) -> Tensor",
    "evidence_norm": (
        "evidence_norm(Tensor x, Tensor value, Tensor gate, Tensor weight, Tensor? mask, float eps, "
        "bool bf16_out=False) -> Tensor"
    ),
    "gated_concat": "gated_concat(Tensor x, Tensor gate) -> Tensor",
    "front_conv1": "front_conv1(Tensor x, Tensor weight, Tensor norm_weight, Tensor lengths, int stride, float eps) -> Tensor",
    "block_pre": "block_pre(Tensor x, Tensor lengths, Tensor weight, float eps) -> (Tensor, Tensor, Tensor)",
    "block_pre_add": (
        "block_pre_add(Tensor x, Tensor addend, Tensor lengths, Tensor weight, float eps) -> (Tensor, Tensor, Tensor)"
    ),
    "norm_silu": "norm_silu(Tensor x, Tensor weight, float eps) -> Tensor",
    "glu_depthwise": "glu_depthwise(Tensor up, Tensor weight, Tensor bias, Tensor lengths) -> Tensor",
    "pooled_attention": (
        "pooled_attention(Tensor qkv, Tensor cos, Tensor sin, Tensor low_lengths, int heads) -> Tensor"
    ),
    "merge_gate": (
        "merge_gate(Tensor cn, Tensor mf, Tensor mb, Tensor an, Tensor norm_weight, float eps, Tensor gate_weight, "
        "Tensor gate_bias) -> (Tensor, Tensor)"
    ),
    "evidence_down": "evidence_down(Tensor cn, Tensor an, Tensor weight, Tensor bias) -> Tensor",
    "glu_norm_silu": (
        "glu_norm_silu(Tensor up, Tensor weight, Tensor bias, Tensor lengths, Tensor norm_weight, float eps) -> Tensor"
    ),
    "merge_conv": (
        "merge_conv(Tensor cn, Tensor mn, Tensor an, Tensor g, Tensor weight, Tensor bias, Tensor lengths) -> Tensor"
    ),
    "query_read": "query_read(Tensor q, Tensor kv, Tensor key_lengths, int heads) -> Tensor",
    "mask_audio": "mask_audio(Tensor audio, Tensor lengths, Tensor channels) -> Tensor",
    "log_power": "log_power(Tensor spec, Tensor channels, Tensor sample_lengths, int hop) -> Tensor",
    "front_lengths": "front_lengths(Tensor sample_lengths, int hop, int[] strides) -> Tensor",
    "grids": "grids(Tensor lengths, int time) -> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)",
    "front_conv2": (
        "front_conv2(Tensor h, Tensor weight, Tensor norm_weight, Tensor x, Tensor skip_weight, Tensor lengths, "
        "int stride, float eps) -> Tensor"
    ),
}

OPERATORS = tuple(_SCHEMAS)


# ---- CUDA kernels: the ctypes launches (imported lazily: those modules call these operators) ----


def _cuda_fused_mamba(q, k, v, adt, dt, trap, qb, kb, angles, d, z, lengths=None, variant="auto", reverse=False,
                      dt_bias=None, a_floor=1e-4, q_norm=None, k_norm=None, norm_eps=1e-5):
    from .mamba_fused import launch

    out = torch.empty_like(v, memory_format=torch.contiguous_format)
    return launch(q, k, v, adt, dt, trap, qb, kb, angles, d, z, out, lengths, variant, reverse, dt_bias, a_floor,
                  q_norm, k_norm, norm_eps)


def _cuda_fused_mamba_out(q, k, v, adt, dt, trap, qb, kb, angles, d, z, lengths=None, variant="auto", reverse=False,
                          dt_bias=None, a_floor=1e-4, q_norm=None, k_norm=None, norm_eps=1e-5, *, out):
    from .mamba_fused import launch

    return launch(q, k, v, adt, dt, trap, qb, kb, angles, d, z, out, lengths, variant, reverse, dt_bias, a_floor,
                  q_norm, k_norm, norm_eps)


def _cuda_rms_norm(x, weight, eps=1e-5, out_dtype=None):
    from .kernels.native import launch_rms

    return launch_rms(x, weight, eps, out_dtype)


def _cuda_add_rms_norm(a, b, weight, mask=None, eps=1e-5, out_dtype=None):
    from .kernels.native import launch_add_rms

    return launch_add_rms(a, b, weight, mask, eps, out_dtype or torch.bfloat16)


def _cuda_add(a, b, mask=None, bf16=False):
    from .kernels.native import launch_add

    return launch_add(a, b, mask, bf16)


def _cuda_swiglu(x):
    from .kernels import launch_swiglu

    return launch_swiglu(x)


def _cuda_mask_rows(x, mask):
    from .kernels.buffers import launch_mask_rows

    return launch_mask_rows(x, mask)


def _cuda_mamba_controls(a, dt, bias, floor):
    from .kernels.buffers import launch_mamba_controls

    return launch_mamba_controls(a, dt, bias, floor)


def _cuda_masked_mean(x, lengths):
    from .masking import launch_masked_mean

    return launch_masked_mean(x, lengths)


def _cuda_time_mask(lengths, time):
    from .masking import launch_time_mask

    return launch_time_mask(lengths, time)


def _cuda_reverse_valid(x, lengths):
    from .kernels import launch_reverse_valid

    return launch_reverse_valid(x, lengths)


def _cuda_mean_rms_norm(a, b, weight, eps=1e-5):
    from .kernels.native import launch_mean_rms

    return launch_mean_rms(a, b, weight, eps)


def _cuda_mask_rms_norm(x, mask, weight, eps=1e-5, out_dtype=None):
    from .kernels.native import launch_mask_rms

    return launch_mask_rms(x, mask, weight, eps, out_dtype or torch.bfloat16)


def _cuda_rms_norm_pair(x, w0, w1, eps=1e-5):
    from .kernels.native import launch_rms_pair

    return launch_rms_pair(x, w0, w1, eps)


def _cuda_frame_audio(audio, channels, kernel, stride, pad, width):
    from .stem import launch_frame_audio

    return launch_frame_audio(audio, channels, kernel, stride, pad, width)


def _cuda_frames_mask(lengths, stride, time):
    from .stem import launch_frames_mask

    return launch_frames_mask(lengths, stride, time)


def _cuda_small_linear(x, weight, bias=None):
    from .stem import launch_small_linear

    return launch_small_linear(x, weight, bias)


def _block(name):
    def kernel(*args):
        from .kernels import block

        return getattr(block, "launch_" + name)(*args)

    return kernel


# ---- Meta kernels: output shapes and dtypes only ----


def _meta_fused_mamba(q, k, v, adt, dt, trap, qb, kb, angles, d, z, lengths=None, variant="auto", reverse=False,
                      dt_bias=None, a_floor=1e-4, q_norm=None, k_norm=None, norm_eps=1e-5):
    return torch.empty_like(v, memory_format=torch.contiguous_format)


def _meta_fused_mamba_out(q, k, v, adt, dt, trap, qb, kb, angles, d, z, lengths=None, variant="auto", reverse=False,
                          dt_bias=None, a_floor=1e-4, q_norm=None, k_norm=None, norm_eps=1e-5, *, out):
    return out


def _meta_rms_norm(x, weight, eps=1e-5, out_dtype=None):
    return x.new_empty(x.shape, dtype=out_dtype or x.dtype)


def _meta_add_rms_norm(a, b, weight, mask=None, eps=1e-5, out_dtype=None):
    return a.new_empty(a.shape, dtype=torch.float32), a.new_empty(a.shape, dtype=out_dtype or torch.bfloat16)


def _meta_add(a, b, mask=None, bf16=False):
    return a.new_empty(a.shape, dtype=torch.bfloat16 if bf16 else torch.promote_types(a.dtype, b.dtype))


def _meta_swiglu(x):
    return x.new_empty((*x.shape[:-1], x.shape[-1] // 2))


def _meta_mask_rows(x, mask):
    return torch.empty_like(x, memory_format=torch.contiguous_format)


def _meta_mamba_controls(a, dt, bias, floor):
    b, t, h = a.shape
    return a.new_empty((b, h, t), dtype=torch.float32), a.new_empty((b, h, t), dtype=torch.float32)


def _meta_masked_mean(x, lengths):
    return x.new_empty((x.shape[0], x.shape[2]), dtype=torch.float32)


def _meta_time_mask(lengths, time):
    return lengths.new_empty((lengths.shape[0], time), dtype=torch.bool)


def _meta_reverse_valid(x, lengths):
    return torch.empty_like(x, memory_format=torch.contiguous_format)


def _meta_mean_rms_norm(a, b, weight, eps=1e-5):
    return a.new_empty(a.shape, dtype=torch.float32)


def _meta_mask_rms_norm(x, mask, weight, eps=1e-5, out_dtype=None):
    return x.new_empty(x.shape, dtype=torch.float32), x.new_empty(x.shape, dtype=out_dtype or torch.bfloat16)


def _meta_rms_norm_pair(x, w0, w1, eps=1e-5):
    return x.new_empty((*x.shape[:-1], 2, x.shape[-1] // 2))


def _meta_frame_audio(audio, channels, kernel, stride, pad, width):
    b, _, n = audio.shape
    return audio.new_empty((b, (n + 2 * pad - kernel) // stride + 1, width), dtype=torch.bfloat16)


def _meta_frames_mask(lengths, stride, time):
    b = lengths.shape[0]
    return lengths.new_empty((b,), dtype=torch.int64), lengths.new_empty((b, time), dtype=torch.bool)


def _meta_small_linear(x, weight, bias=None):
    return x.new_empty((x.shape[0], weight.shape[0]), dtype=torch.float32)


def _meta_depthwise_masked(x, weight, bias, lengths):
    return torch.empty_like(x, memory_format=torch.contiguous_format)


def _meta_pool4(x, lengths):
    b, t, d = x.shape
    return x.new_empty((b, (t + 3) // 4, d))


def _meta_rotary_qkv(x, cos, sin, heads):
    b, t, width = x.shape
    return x.new_empty((3, b, heads, t, width // (3 * heads)))


def _meta_front_norm(x, lengths, weight, eps, silu):
    b, c, t, f = x.shape
    return x.new_empty((b, t, f, c))


def _meta_interpolate(low, left, right, alpha, lengths):
    return low.new_empty((low.shape[0], left.shape[1], low.shape[2]))


def _meta_interpolate_rmsnorm(low, left, right, alpha, lengths, weight, eps):
    return low.new_empty((low.shape[0], left.shape[1], low.shape[2]))


def _meta_bands(x):
    b, c, t, f = x.shape
    return x.new_empty((b, t, 8, c))


def _meta_evidence_norm(x, value, gate, weight, mask, eps, bf16_out=False):
    return x.new_empty(x.shape, dtype=torch.bfloat16 if bf16_out else torch.float32)


def _meta_block_pre(x, lengths, weight, eps):
    b, t, d = x.shape
    return (torch.empty_like(x, memory_format=torch.contiguous_format), x.new_empty((b, t, d), dtype=torch.bfloat16),
            x.new_empty((b, (t + 3) // 4, d), dtype=torch.bfloat16))


def _meta_block_pre_add(x, addend, lengths, weight, eps):
    return _meta_block_pre(x, lengths, weight, eps)


def _meta_norm_silu(x, weight, eps):
    return torch.empty_like(x, memory_format=torch.contiguous_format)


def _meta_glu_depthwise(up, weight, bias, lengths):
    return up.new_empty((*up.shape[:-1], up.shape[-1] // 2), dtype=torch.bfloat16)


def _meta_pooled_attention(qkv, cos, sin, low_lengths, heads):
    return qkv.new_empty((*qkv.shape[:-1], qkv.shape[-1] // 3), dtype=torch.bfloat16)


def _meta_merge_gate(cn, mf, mb, an, norm_weight, eps, gate_weight, gate_bias):
    return cn.new_empty(cn.shape, dtype=torch.float32), cn.new_empty((*cn.shape[:-1], 3), dtype=torch.bfloat16)


def _meta_glu_norm_silu(up, weight, bias, lengths, norm_weight, eps):
    return up.new_empty((*up.shape[:-1], up.shape[-1] // 2), dtype=torch.bfloat16)


def _meta_evidence_down(cn, an, weight, bias):
    return cn.new_empty((*cn.shape[:-1], weight.shape[0]), dtype=torch.bfloat16)


def _meta_merge_conv(cn, mn, an, g, weight, bias, lengths):
    return cn.new_empty((*cn.shape[:-1], 3 * cn.shape[-1]), dtype=torch.bfloat16)


def _meta_gated_concat(x, gate):
    return torch.empty_like(x, memory_format=torch.contiguous_format)


def _meta_front_conv1(x, weight, norm_weight, lengths, stride, eps):
    b, _, t, f = x.shape
    return x.new_empty((b, (t - 1) // stride + 1, (f - 1) // 2 + 1, weight.shape[1]), dtype=torch.bfloat16)


def _meta_front_conv2(h, weight, norm_weight, x, skip_weight, lengths, stride, eps):
    return torch.empty_like(h, memory_format=torch.contiguous_format)


def _meta_query_read(q, kv, key_lengths, heads):
    return kv.new_empty((kv.shape[0], q.shape[0], q.shape[1]), dtype=torch.bfloat16)


def _meta_mask_audio(audio, lengths, channels):
    b, c, n = audio.shape
    return audio.new_empty((b * c, n), dtype=torch.float32)


def _meta_log_power(spec, channels, sample_lengths, hop):
    return spec.new_empty((channels.shape[0], spec.shape[2], spec.shape[1]), dtype=torch.float32)


def _meta_front_lengths(sample_lengths, hop, strides):
    return sample_lengths.new_empty((4, sample_lengths.shape[0]), dtype=torch.int64)


def _meta_grids(lengths, time):
    b, lt = lengths.shape[0], (time + 3) // 4
    e = lengths.new_empty
    return (e((b, time), dtype=torch.bool), e((b,), dtype=torch.int64), e((b, lt), dtype=torch.bool),
            e((b, time), dtype=torch.int64), e((b, time), dtype=torch.int64), e((b, time), dtype=torch.float32))


# ---- CPU kernels: loud failure, no fallback ----


def _no_cpu(name):
    def kernel(*args, **kwargs):
        raise RuntimeError(
            f"{NAMESPACE}::{name} runs only on a ROCm GPU (gfx950); there is no CPU path. "
            "Move the operands to a cuda device."
        )

    return kernel


_KERNELS = {
    "fused_mamba": (_cuda_fused_mamba, _meta_fused_mamba),
    "fused_mamba.out": (_cuda_fused_mamba_out, _meta_fused_mamba_out),
    "rms_norm": (_cuda_rms_norm, _meta_rms_norm),
    "add_rms_norm": (_cuda_add_rms_norm, _meta_add_rms_norm),
    "add": (_cuda_add, _meta_add),
    "swiglu": (_cuda_swiglu, _meta_swiglu),
    "mask_rows": (_cuda_mask_rows, _meta_mask_rows),
    "mamba_controls": (_cuda_mamba_controls, _meta_mamba_controls),
    "masked_mean": (_cuda_masked_mean, _meta_masked_mean),
    "time_mask": (_cuda_time_mask, _meta_time_mask),
    "reverse_valid": (_cuda_reverse_valid, _meta_reverse_valid),
    "mean_rms_norm": (_cuda_mean_rms_norm, _meta_mean_rms_norm),
    "mask_rms_norm": (_cuda_mask_rms_norm, _meta_mask_rms_norm),
    "rms_norm_pair": (_cuda_rms_norm_pair, _meta_rms_norm_pair),
    "frame_audio": (_cuda_frame_audio, _meta_frame_audio),
    "frames_mask": (_cuda_frames_mask, _meta_frames_mask),
    "small_linear": (_cuda_small_linear, _meta_small_linear),
    **{
        name: (_block(name), globals()["_meta_" + name])
        for name in ("depthwise_masked", "pool4", "rotary_qkv", "front_norm", "interpolate", "interpolate_rmsnorm",
                     "bands", "evidence_norm", "gated_concat", "front_conv1", "front_conv2", "block_pre",
                     "block_pre_add", "norm_silu", "glu_depthwise", "glu_norm_silu", "pooled_attention", "merge_gate",
                     "evidence_down", "merge_conv", "query_read", "mask_audio", "log_power", "front_lengths", "grids")
    },
}

_LIBRARY = torch.library.Library(NAMESPACE, "DEF")
for _name, _schema in _SCHEMAS.items():
    _LIBRARY.define(_schema)
    _cuda, _meta = _KERNELS[_name]
    _LIBRARY.impl(_name, _cuda, "CUDA")
    _LIBRARY.impl(_name, _meta, "Meta")
    _LIBRARY.impl(_name, _no_cpu(_name), "CPU")

ops = getattr(torch.ops, NAMESPACE)
