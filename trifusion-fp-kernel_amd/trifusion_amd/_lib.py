"""ctypes binding of the C ABI in ``include/trifusion_amd.h``.

The library is loaded lazily, after ``torch`` (whose bundled HIP runtime then
satisfies the library's ``libamdhip64.so.7`` dependency, so kernels and torch
share one runtime, one device context and one set of streams). There is no CPU
fallback: if the library is missing every entry point raises ``RuntimeError``.
"""

import ctypes
import threading

import torch

from .build import LIB_PATH

c_i32 = ctypes.c_int32
c_i64 = ctypes.c_int64
c_ptr = ctypes.c_void_p
c_f32 = ctypes.c_float

TF_FLOAT32, TF_BFLOAT16, TF_FLOAT16 = 0, 1, 2
DTYPE_CODES = {torch.float32: TF_FLOAT32, torch.bfloat16: TF_BFLOAT16, torch.float16: TF_FLOAT16}

STATUS = {
    1: "a required pointer is NULL",
    2: "unsupported or inconsistent dimensions",
    3: "unsupported dtype",
    4: "unsupported layout (strides)",
    5: "requested kernel variant cannot run these arguments",
    6: "the HIP runtime rejected the kernel launch",
    7: "needs more scratch than the library's static area holds",
}

VARIANTS = {"auto": 0, "generic": 1, "mfma": 2, "pipe": 3}


class MambaArgs(ctypes.Structure):
    """Mirror of ``struct tf_mamba_args``."""

    _fields_ = [
        *[(name, c_ptr) for name in ("q", "k", "v", "adt", "dt", "trap", "angles", "z")],
        *[(name, c_ptr) for name in ("qb", "kb", "d")],
        ("out", c_ptr),
        ("lengths", c_ptr),
        *[
            (name, c_i32)
            for name in (
                "q_dtype",
                "k_dtype",
                "v_dtype",
                "z_dtype",
                "adt_dtype",
                "dt_dtype",
                "trap_dtype",
                "angles_dtype",
                "out_dtype",
                "variant",
            )
        ],
        *[(name, c_i64 * 4) for name in ("q_stride", "k_stride", "v_stride", "z_stride")],
        *[(name, c_i64 * 4) for name in ("angles_stride", "out_stride")],
        *[(name, c_i64 * 3) for name in ("adt_stride", "dt_stride", "trap_stride")],
        *[
            (name, c_i64)
            for name in ("batch", "time", "heads", "qk_heads", "state", "head_dim", "rotary")
        ],
        ("workspace", c_ptr),
        ("workspace_bytes", c_i64),
        ("dt_bias", c_ptr),
        ("a_floor", c_f32),
        ("reverse", c_i32),
        ("q_norm", c_ptr),
        ("k_norm", c_ptr),
        ("norm_eps", c_f32),
    ]


# name -> (argtypes, restype)
_SIGNATURES = {
    "tf_fused_mamba": ([ctypes.POINTER(MambaArgs), c_ptr], c_i32),
    "tf_fused_mamba_variant": ([ctypes.POINTER(MambaArgs)], c_i32),
    "tf_fused_mamba_workspace_size": ([ctypes.POINTER(MambaArgs)], c_i64),
    "tf_fused_mamba_static": ([ctypes.POINTER(MambaArgs), c_ptr], c_i32),
    "tf_fused_mamba_static_scratch_bytes": ([], c_i64),
    "tf_rmsnorm": ([c_ptr, c_i32, c_i64, c_ptr, c_ptr, c_i32, c_i64, c_i64, c_f32, c_ptr], c_i32),
    "tf_add_rmsnorm": (
        [c_ptr, c_i32, c_ptr, c_i32, c_ptr, c_ptr, c_ptr, c_i32, c_ptr, c_i32, c_i64, c_i64, c_f32, c_ptr],
        c_i32,
    ),
    "tf_swiglu": ([c_ptr, c_ptr, c_i32, c_i64, c_i64, c_ptr], c_i32),
    "tf_mask_rows": ([c_ptr, c_ptr, c_i32, c_ptr, c_i64, c_i64, c_ptr], c_i32),
    "tf_add": ([c_ptr, c_i32, c_ptr, c_i32, c_ptr, c_ptr, c_i32, c_i64, c_i64, c_ptr], c_i32),
    "tf_mamba_controls": (
        [c_ptr, c_ptr, c_i32, c_i64, c_i64, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_f32, c_ptr],
        c_i32,
    ),
    "tf_masked_mean": ([c_ptr, c_i32, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_ptr, c_i64, c_ptr], c_i32),
    "tf_masked_mean_workspace_size": ([c_i32, c_i64, c_i64, c_i64], c_i64),
    "tf_time_mask": ([c_ptr, c_ptr, c_i64, c_i64, c_ptr], c_i32),
    "tf_reverse_valid": ([c_ptr, c_ptr, c_i32, c_ptr, c_i64, c_i64, c_i64, c_ptr], c_i32),
    "tf_mean_rmsnorm": ([c_ptr, c_i32, c_ptr, c_i32, c_ptr, c_ptr, c_i64, c_i64, c_f32, c_ptr], c_i32),
    "tf_mask_rmsnorm": ([c_ptr, c_i32, c_ptr, c_ptr, c_ptr, c_ptr, c_i32, c_i64, c_i64, c_f32, c_ptr], c_i32),
    "tf_rmsnorm_pair": ([c_ptr, c_i32, c_i64, c_ptr, c_ptr, c_ptr, c_i32, c_i64, c_i64, c_f32, c_ptr], c_i32),
    "tf_frame_audio": ([c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_ptr], c_i32),
    "tf_frames_mask": ([c_ptr, c_i64, c_ptr, c_ptr, c_i64, c_i64, c_ptr], c_i32),
    "tf_small_linear": ([c_ptr, c_ptr, c_ptr, c_i32, c_ptr, c_i64, c_i64, c_i64, c_ptr], c_i32),
    "tf_depthwise_masked": ([c_ptr, c_ptr, c_ptr, c_i32, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_i64, c_ptr], c_i32),
    "tf_pool4": ([c_ptr, c_i32, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_ptr], c_i32),
    "tf_rotary_qkv": ([c_ptr, c_i32, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_i64, c_ptr], c_i32),
    "tf_front_norm": (
        [c_ptr, c_i32, ctypes.POINTER(c_i64), c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_i64, c_f32, c_i32, c_ptr],
        c_i32,
    ),
    "tf_interpolate": ([c_ptr, c_i32, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_i64, c_ptr], c_i32),
    "tf_bands": ([c_ptr, c_i32, ctypes.POINTER(c_i64), c_ptr, c_i64, c_i64, c_i64, c_i64, c_ptr], c_i32),
    "tf_evidence_norm": (
        [c_ptr, c_ptr, c_ptr, c_i32, c_i64, c_ptr, c_ptr, c_ptr, c_i32, c_i64, c_i64, c_f32, c_ptr],
        c_i32,
    ),
    "tf_gated_concat": ([c_ptr, c_ptr, c_i32, c_ptr, c_i64, c_i64, c_ptr], c_i32),
    "tf_front_conv1": (
        [c_ptr, c_i32, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_f32, c_ptr],
        c_i32,
    ),
    "tf_front_conv2": (
        [c_ptr, c_ptr, c_ptr, c_ptr, c_i32, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_f32,
         c_ptr],
        c_i32,
    ),
    "tf_block_pre": ([c_ptr, c_ptr, c_ptr, c_f32, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_ptr], c_i32),
    "tf_norm_silu": ([c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_f32, c_ptr], c_i32),
    "tf_glu_depthwise": ([c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_i64, c_ptr], c_i32),
    "tf_pooled_attention": ([c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_i64, c_ptr], c_i32),
    "tf_merge_gate": (
        [c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_f32, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_ptr],
        c_i32,
    ),
    "tf_block_pre_add": (
        [c_ptr, c_ptr, c_ptr, c_ptr, c_f32, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_ptr],
        c_i32,
    ),
    "tf_glu_depthwise_norm_silu": (
        [c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_f32, c_ptr, c_i64, c_i64, c_i64, c_i64, c_ptr],
        c_i32,
    ),
    "tf_interpolate_rmsnorm": (
        [c_ptr, c_i32, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_f32, c_ptr, c_i64, c_i64, c_i64, c_i64, c_ptr],
        c_i32,
    ),
    "tf_evidence_down": ([c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_ptr], c_i32),
    "tf_merge_conv": (
        [c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_i64, c_ptr],
        c_i32,
    ),
    "tf_query_read_workspace_size": ([c_i64, c_i64, c_i64, c_i64, c_i64], c_i64),
    "tf_query_read": ([c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_ptr], c_i32),
    "tf_mask_audio": ([c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_ptr], c_i32),
    "tf_log_power": (
        [c_ptr, ctypes.POINTER(c_i64), c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_i64, c_i64, c_ptr],
        c_i32,
    ),
    "tf_front_lengths": ([c_ptr, c_ptr, c_i64, c_i64, ctypes.POINTER(c_i64), c_ptr], c_i32),
    "tf_grids": ([c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_ptr], c_i32),
    "tf_version": ([], ctypes.c_char_p),
}

EXPORTED = tuple(_SIGNATURES)

_lock = threading.Lock()
_lib = None


def load():
    """Load (once) and return the ctypes handle of ``libtrifusion_amd.so``."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"trifusion_amd native library not built ({LIB_PATH}); run "
                    "`python -c 'import __graft_entry__ as g; g.build()'` from the repository root"
                )
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (argtypes, restype) in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = argtypes
                fn.restype = restype
            _lib = lib
    return _lib


def check(status, what):
    if status == 0:
        return
    message = STATUS.get(status, f"status {status}")
    if status in (2, 4, 5, 7):
        raise ValueError(f"{what}: {message}")
    if status == 3:
        raise TypeError(f"{what}: {message}")
    raise RuntimeError(f"{what}: {message}")


def dtype_code(t, what):
    try:
        return DTYPE_CODES[t.dtype]
    except KeyError:
        raise TypeError(f"{what}: unsupported dtype {t.dtype}") from None


def stream_of(t):
    """Handle of the current torch stream on ``t``'s device (graph-capture safe)."""
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def require_cuda(*tensors, what):
    device = None
    for t in tensors:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{what}: expected tensors")
        if t.device.type != "cuda":
            raise ValueError(f"{what}: tensors must be on a ROCm (cuda) device, got {t.device}")
        if device is None:
            device = t.device
        elif t.device != device:
            raise ValueError(f"{what}: tensors must be on one device ({device} vs {t.device})")
    return device
