"""CPU oracle for the fused Mamba-3 inference path (test infrastructure only).

This package restates, in plain PyTorch on the CPU, the arithmetic of the
reference's GPU path so that the HIP kernels can be checked against it. It is
the checker, never the thing measured or shipped: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` import
it. The product package (``trifusion_amd``) never imports it and has no CPU
fallback.

Modules
-------
recurrence
    ``phase_chunked`` / ``fused_mamba_chunked`` (fp32, chunked, with the
    reference's bf16 rounding points) and ``fused_mamba_f64`` (unchunked FP64
    loop) plus ``fused_mamba_attention_f64`` (quadratic closed form).
elementwise
    RMSNorm, SwiGLU, row masking, masked residual add, Mamba controls and
    masked mean-pooling.
encoder
    Eager forward of the synthetic 8-block Conv1d/Mamba encoder, evaluated
    on the same parameters as the HIP model.

Pinning status (what each function is checked against) is listed in each
module header.
"""
