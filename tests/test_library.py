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
    return sorted(set(re.findall(r"^(?:int|const char \*)\s*(tf_\w+)\s*\(", text, re.M)))


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

    # 13 pointers, 10 int32, 33 int64 strides, 7 int64 dims
    assert ctypes.sizeof(MambaArgs) == 13 * 8 + 10 * 4 + 33 * 8 + 7 * 8
    text = HEADER.read_text()
    body = text[text.index("typedef struct tf_mamba_args") : text.index("} tf_mamba_args;")]
    names_in_header = re.findall(r"\*?(\w+)(?:\[\d\])?[,;]", body)
    names_in_struct = [f[0] for f in MambaArgs._fields_]
    assert names_in_header == names_in_struct


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
