"""The C-ABI library loads and exports exactly what include/tokserve_hip.h declares.

No kernel is launched: only host-side entry points and argument validation
(which returns before any HIP call) run here.
"""

import ctypes
import re
from pathlib import Path

import pytest

from tokserve_amd.kernels import _lib

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "tokserve_hip.h"


def declared_functions() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"\b(tks_[a-z0-9_]+)\s*\(", text))


def test_header_declares_the_binding_signatures() -> None:
    assert declared_functions() == set(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol() -> None:
    library = ctypes.CDLL(str(_lib.library_path()))
    for name in declared_functions():
        assert hasattr(library, name), name


def test_abi_version_and_status_strings() -> None:
    library = _lib.load()
    assert library.tks_abi_version() == _lib.ABI_VERSION
    assert library.tks_status_string(_lib.TKS_OK) == b"ok"
    assert library.tks_status_string(_lib.TKS_ERR_INDEX) == b"layer_index is out of range"
    assert library.tks_status_string(-99) == b"unknown status"


def test_status_codes_map_to_reference_exception_types() -> None:
    with pytest.raises(ValueError):
        _lib.check(_lib.TKS_ERR_VALUE, "op")
    with pytest.raises(TypeError):
        _lib.check(_lib.TKS_ERR_TYPE, "op")
    with pytest.raises(IndexError):
        _lib.check(_lib.TKS_ERR_INDEX, "op")
    with pytest.raises(ValueError):
        _lib.check(_lib.TKS_ERR_WORKSPACE, "op")
    with pytest.raises(_lib.HipKernelError):
        _lib.check(_lib.TKS_ERR_LAUNCH, "op")


def test_argument_validation_happens_before_any_launch() -> None:
    library = _lib.load()
    # Unsupported dtype code.
    assert library.tks_kv_append(
        None, 0, 0, None, 0, 0, 1, None, None, 1, 1, 1, 16, 8, 0, None, 7, None
    ) == _lib.TKS_ERR_TYPE
    # Layer index out of range.
    assert library.tks_kv_append(
        None, 0, 0, None, 0, 0, 1, None, None, 2, 4, 1, 16, 8, 2, None, 0, None
    ) == _lib.TKS_ERR_INDEX
    # Zero tokens is a successful no-op.
    assert library.tks_kv_append(
        None, 0, 0, None, 0, 0, 0, None, None, 2, 4, 1, 16, 8, 1, None, 0, None
    ) == _lib.TKS_OK
    # Query heads not divisible by KV heads.
    assert library.tks_paged_attention_decode(
        None, 0, 0, None, None, 1, 4, 3, 16, 64, 0, None, 4, None, None, 1, 8, 16, 1.0, 0,
        None, 0, 0, None, 0, 2, None
    ) == _lib.TKS_ERR_VALUE
    # RMSNorm: bf16 weight with fp32 output breaks torch promotion.
    assert library.tks_rms_norm(
        None, 0, None, 0, None, 0, None, None, 0, 1, 8, 1e-6, 2, 2, 0, None
    ) == _lib.TKS_ERR_TYPE
    # RoPE: odd head_dim.
    assert library.tks_rope(
        None, None, 0, 0, 0, 0, 0, 0, 1, None, None, 0, 0, 0, 0, 0, 0, 1, 1, 1, 7,
        None, None, None, 8, 0, None
    ) == _lib.TKS_ERR_VALUE


def test_decode_workspace_sizes() -> None:
    library = _lib.load()
    # A single split needs no workspace.
    assert library.tks_paged_attention_decode_workspace_bytes(4, 32, 8, 128, 16, 256, 32) == 0
    # Split partials: rows * heads * splits * (2 + Dh) floats with m and l padded to 64
    # (nothing else: splits are merged by a second launch).
    size = library.tks_paged_attention_decode_workspace_bytes(2, 4, 1, 64, 16, 1024, 16)
    splits = 4
    n = 2 * 4 * splits
    assert size == (2 * ((n + 63) // 64 * 64) + n * 64) * 4
    assert library.tks_paged_attention_decode_workspace_bytes(-1, 4, 1, 64, 16, 1024, 16) == -1
