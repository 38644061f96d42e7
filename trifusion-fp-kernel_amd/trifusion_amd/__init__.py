"""TriFusion-FP fused inference hot path for AMD Instinct MI355X (gfx950).

Public API mirrors the reference package ``trifusion_l4`` (``src/trifusion_l4/__init__.py:10-35``):
``configure_runtime``, ``load_student``, ``InferenceEngine`` and ``fused_mamba``
are resolved lazily, so importing the package needs neither torch nor the
native library.
"""

from importlib import import_module

__version__ = "0.1.0"
__all__ = ["__version__", "configure_runtime", "load_student", "InferenceEngine", "fused_mamba"]

_EXPORTS = {
    "configure_runtime": (".runtime", "configure_runtime"),
    "load_student": (".runtime", "load_student"),
    "InferenceEngine": (".runtime", "InferenceEngine"),
    "fused_mamba": (".mamba_fused", "fused_mamba"),
}


def __getattr__(name):
    if name not in _EXPORTS:
        raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
    module_name, attribute = _EXPORTS[name]
    try:
        value = getattr(import_module(module_name, __name__), attribute)
    except ModuleNotFoundError as error:
        if error.name in {"torch", "numpy"}:
            raise ModuleNotFoundError(
                "The MI355X runtime requires PyTorch built for ROCm.", name=error.name
            ) from error
        raise
    globals()[name] = value
    return value


def __dir__():
    return sorted(set(globals()) | set(__all__))
