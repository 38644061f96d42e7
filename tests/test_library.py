"""The C-ABI library loads and exports every entry point the header declares
(no compute calls: runs without a GPU)."""

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "trifusion_amd.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^(?:int|int64_t|const char \*)\s*(tf_\w+)\s*\(", text, re.M)))


def test_header_declares_entry_points():
    names = declared_functions()
    assert "tf_fused_mamba" in names and "tf_rmsnorm" in names and len(names) >= 10


def test_library_exports_every_declared_symbol():
    import torch  # noqa: F401  (the library binds to torch's HIP runtime)

    from trifusion_amd import _lib

    if not _lib.LIB_PATH.exists():
        pytest.fail(f"native library missing: {_lib.LIB_PATH} (run __graft_entry__.build())")
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert set(declared_functions()) == set(_lib.EXPORTED)


def test_struct_layout_matches_header():
    from trifusion_amd._lib import MambaArgs

    # 13 pointers, 10 int32, 33 int64 strides, 7 int64 dims, workspace pointer + bytes,
    # dt_bias pointer, a_floor float, reverse int32, two norm-weight pointers,
    # norm_eps float and the tail padding to 8 bytes
    assert ctypes.sizeof(MambaArgs) == 13 * 8 + 10 * 4 + 33 * 8 + 7 * 8 + 8 + 8 + 8 + 4 + 4 + 8 + 8 + 4 + 4
    text = HEADER.read_text()
    body = text[text.index("typedef struct tf_mamba_args") : text.index("} tf_mamba_args;")]
    names_in_header = re.findall(r"\*?(\w+)(?:\[\d\])?[,;]", body)
    names_in_struct = [f[0] for f in MambaArgs._fields_]
    assert names_in_header == names_in_struct


def _host_args(batch, time, heads, state=64, head_dim=64, rotary=16):
    """tf_mamba_args with contiguous strides and aligned placeholder addresses:
    the workspace query is host logic and never dereferences them."""
    from trifusion_amd._lib import MambaArgs

    a = MambaArgs()
    for name in ("q", "k", "v", "adt", "dt", "trap", "angles", "z", "qb", "kb", "d", "out"):
        setattr(a, name, 1 << 20)
    a.q_dtype = a.k_dtype = a.v_dtype = a.z_dtype = a.out_dtype = 1  # bf16
    a.adt_dtype = a.dt_dtype = a.trap_dtype = a.angles_dtype = 0  # fp32

    def contiguous(shape):
        st, acc = [], 1
        for s in reversed(shape):
            st.append(acc)
            acc *= s
        return list(reversed(st))

    a.q_stride[:] = a.k_stride[:] = contiguous((batch, time, 1, state))
    a.v_stride[:] = a.z_stride[:] = a.out_stride[:] = contiguous((batch, time, heads, head_dim))
    a.angles_stride[:] = contiguous((batch, time, heads, rotary))
    a.adt_stride[:] = a.dt_stride[:] = a.trap_stride[:] = contiguous((batch, heads, time))
    a.batch, a.time, a.heads, a.qk_heads = batch, time, heads, 1
    a.state, a.head_dim, a.rotary = state, head_dim, rotary
    return a


def test_workspace_size_query():
    import torch  # noqa: F401

    from trifusion_amd import _lib

    lib = _lib.load()
    size = lambda a: lib.tf_fused_mamba_workspace_size(ctypes.byref(a))  # noqa: E731
    # long clip over 16 units: chunk-parallel, 15 segments of 8 chunks; 256-byte
    # aligned blocks. The pipelined kernel (auto): per segment a 16 KB state,
    # 128 B of fixed-point phase sums and a 4 B decay. The chunked kernel: per
    # segment a 16 KB state and a 4 B decay, per chunk 512 B of fp64 phase sums.
    recs, chunks = 16 * 15, 16 * 113
    up = lambda x: (x + 255) // 256 * 256  # noqa: E731
    assert size(_host_args(1, 7200, 16)) == up(recs * 16384) + up(recs * 128) + up(recs * 4)
    forced = _host_args(1, 7200, 16)
    forced.variant = 2
    assert size(forced) == up(recs * 16384) + up(chunks * 512) + up(recs * 4)
    assert size(_host_args(16, 400, 16)) == 0  # 256 units: one workgroup each
    assert size(_host_args(1, 64, 16)) == 0  # one chunk: nothing to split
    # N = 16 (bf16): the chunked kernel at N = 32 on zero-padded channels, per
    # segment a 4 KB state record
    assert size(_host_args(1, 7200, 16, state=16, head_dim=32, rotary=4)) == (
        up(recs * 4096) + up(chunks * 512) + up(recs * 4)
    )
    fp32 = _host_args(1, 7200, 16, state=16, head_dim=32, rotary=4)
    fp32.q_dtype = fp32.k_dtype = fp32.v_dtype = fp32.z_dtype = fp32.out_dtype = 0
    assert size(fp32) == 0  # fp32 operands: the generic kernel, one workgroup per unit
    bad = _host_args(1, 100, 16)
    bad.heads = 0
    assert size(bad) < 0


def test_fused_norm_weights_come_as_a_pair():
    """The B/C norm weights are both given or both NULL; one alone is
    TF_ERR_NULL from the host checks, before any kernel is chosen."""
    from trifusion_amd import _lib

    lib = _lib.load()
    a = _host_args(16, 400, 16)
    assert lib.tf_fused_mamba_variant(ctypes.byref(a)) == 3
    a.q_norm, a.norm_eps = 1 << 20, 1e-5
    assert lib.tf_fused_mamba_variant(ctypes.byref(a)) == -1
    a.k_norm = 1 << 20
    assert lib.tf_fused_mamba_variant(ctypes.byref(a)) == 3
    a.q_norm = None
    assert lib.tf_fused_mamba_variant(ctypes.byref(a)) == -1


def test_version_string():
    import torch  # noqa: F401

    from trifusion_amd import _lib

    lib = _lib.load()
    assert lib.tf_version().startswith(b"trifusion_amd")


def test_lazy_public_api():
    import trifusion_amd

    assert set(trifusion_amd.__all__) >= {"configure_runtime", "load_student", "InferenceEngine", "fused_mamba"}
    with pytest.raises(AttributeError):
        trifusion_amd.not_an_export  # noqa: B018
