"""ctypes binding of libtokserve_hip.so (the C ABI declared in include/tokserve_hip.h).

The shared library is loaded lazily on the first kernel call, so importing the
package never touches HIP (the pattern of tokserve/kernels/vector.py:36-38).
There is no fallback: when the library is missing or a call fails, the error
surfaces as an exception carrying the C status.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

LIBRARY_NAME = "libtokserve_hip.so"
ABI_VERSION = 12

TKS_OK = 0
TKS_ERR_VALUE = -1
TKS_ERR_TYPE = -2
TKS_ERR_INDEX = -3
TKS_ERR_WORKSPACE = -4
TKS_ERR_LAUNCH = -5

DTYPE_CODES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

_c_void_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float

# Exported symbol -> (restype, argtypes). Must match include/tokserve_hip.h.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "tks_abi_version": (_i32, []),
    "tks_status_string": (ctypes.c_char_p, [_i32]),
    "tks_last_hip_error": (ctypes.c_char_p, []),
    "tks_kv_append": (
        _i32,
        [_c_void_p, _i64, _i64, _c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p,
         _i32, _i64, _i32, _i32, _i32, _i32, _c_void_p, _i32, _c_void_p],
    ),
    "tks_paged_gather": (
        _i32,
        [_c_void_p, _c_void_p, _i32, _i64, _i32, _i32, _i32, _i32, _c_void_p, _i32,
         _c_void_p, _c_void_p, _i32, _i32, _c_void_p, _c_void_p, _i64, _i64, _i32,
         _c_void_p],
    ),
    "tks_paged_attention_decode_workspace_bytes": (
        _i64, [_i32, _i32, _i32, _i32, _i32, _i32, _i32],
    ),
    "tks_paged_attention_decode": (
        _i32,
        [_c_void_p, _i64, _i64, _c_void_p, _c_void_p, _i32, _i64, _i32, _i32, _i32, _i32,
         _c_void_p, _i32, _c_void_p, _c_void_p, _i32, _i32, _i32, _f32, _i32, _c_void_p,
         _i64, _i64,
         _c_void_p, _i64, _i32, _c_void_p],
    ),
    "tks_rope_append_paged_decode": (
        _i32,
        [_c_void_p, _i64, _i64, _c_void_p, _i64, _i64, _c_void_p, _i64, _i64,
         _c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p,
         _c_void_p, _c_void_p, _i32, _i64, _i32, _i32, _i32, _i32,
         _c_void_p, _i32, _c_void_p, _c_void_p, _i32, _i32, _i32, _f32, _i32,
         _c_void_p, _i64, _i64, _c_void_p, _i64, _i32, _c_void_p],
    ),
    "tks_rope_append_paged_decode_fp8": (
        _i32,
        [_c_void_p, _i64, _i64, _c_void_p, _i64, _i64, _c_void_p, _i64, _i64,
         _c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p,
         _c_void_p, _c_void_p, _i32, _i64, _i32, _i32, _i32, _i32,
         _c_void_p, _i32, _c_void_p, _c_void_p, _i32, _i32, _i32, _f32, _i32,
         _c_void_p, _i64, _i64, _c_void_p, _i64, _f32, _f32, _i32, _c_void_p],
    ),
    "tks_paged_attention_decode_noalloc_max_workspace_bytes": (_i64, []),
    "tks_paged_attention_decode_noalloc": (
        _i32,
        [_c_void_p, _i64, _i64, _c_void_p, _c_void_p, _i32, _i64, _i32, _i32, _i32, _i32,
         _c_void_p, _i32, _c_void_p, _c_void_p, _i32, _i32, _i32, _f32, _i32, _c_void_p,
         _i64, _i64, _i32, _c_void_p],
    ),
    "tks_paged_attention_prefill": (
        _i32,
        [_c_void_p, _i64, _i64, _c_void_p, _c_void_p, _i32, _i64, _i32, _i32, _i32, _i32,
         _c_void_p, _i32, _c_void_p, _c_void_p, _c_void_p, _i32, _i64, _i32, _i32, _i32, _f32,
         _c_void_p, _i64, _i64, _i32, _c_void_p],
    ),
    "tks_rms_norm": (
        _i32,
        [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _i64, _c_void_p, _c_void_p, _i64,
         _i64, _i32, _f32, _i32, _i32, _i32, _c_void_p],
    ),
    "tks_rope": (
        _i32,
        [_c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i64, _i64, _i32,
         _c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i64, _i64, _i32,
         _i32, _i64, _i32, _c_void_p, _c_void_p, _c_void_p, _i64, _i32, _c_void_p],
    ),
    "tks_argmax": (_i32, [_c_void_p, _i64, _i64, _i64, _c_void_p, _i32, _c_void_p]),
    "tks_rope_kv_append": (
        _i32,
        [_c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i32,
         _c_void_p, _c_void_p, _i64, _i64, _i64, _i64,
         _c_void_p, _i64, _i64, _i32, _i64, _i32, _c_void_p, _c_void_p, _c_void_p, _i64,
         _c_void_p, _c_void_p, _i32, _i64, _i32, _i32, _c_void_p, _i32, _c_void_p],
    ),
    "tks_rope_kv_append_fp8": (
        _i32,
        [_c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i32,
         _c_void_p, _c_void_p, _i64, _i64, _i64, _i64,
         _c_void_p, _i64, _i64, _i32, _i64, _i32, _c_void_p, _c_void_p, _c_void_p, _i64,
         _c_void_p, _c_void_p, _i32, _i64, _i32, _i32, _c_void_p, _f32, _f32, _i32,
         _c_void_p],
    ),
    "tks_vector_add": (_i32, [_c_void_p, _c_void_p, _c_void_p, _i64, _i32, _c_void_p]),
    "tks_silu_mul": (_i32, [_c_void_p, _i64, _i64, _i64, _c_void_p, _i64, _i32, _c_void_p]),
    "tks_kv_append_fp8": (
        _i32,
        [_c_void_p, _i64, _i64, _c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p,
         _i32, _i64, _i32, _i32, _i32, _i32, _c_void_p, _f32, _f32, _i32, _c_void_p],
    ),
    "tks_paged_gather_fp8": (
        _i32,
        [_c_void_p, _c_void_p, _i32, _i64, _i32, _i32, _i32, _i32, _c_void_p, _i32,
         _c_void_p, _c_void_p, _i32, _i32, _c_void_p, _c_void_p, _i64, _i64, _f32, _f32,
         _i32, _c_void_p],
    ),
    "tks_paged_attention_decode_fp8": (
        _i32,
        [_c_void_p, _i64, _i64, _c_void_p, _c_void_p, _i32, _i64, _i32, _i32, _i32, _i32,
         _c_void_p, _i32, _c_void_p, _c_void_p, _i32, _i32, _i32, _f32, _i32, _c_void_p,
         _i64, _i64,
         _c_void_p, _i64, _f32, _f32, _i32, _c_void_p],
    ),
    "tks_paged_attention_prefill_fp8_workspace_bytes": (
        _i64, [_i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32],
    ),
    "tks_paged_attention_prefill_fp8": (
        _i32,
        [_c_void_p, _i64, _i64, _c_void_p, _c_void_p, _i32, _i64, _i32, _i32, _i32, _i32,
         _c_void_p, _i32, _c_void_p, _c_void_p, _c_void_p, _i32, _i64, _i32, _i32, _i32, _f32,
         _c_void_p, _i64, _i64, _c_void_p, _i64, _f32, _f32, _i32, _c_void_p],
    ),
    # fp8 pools with one scale per pool row: the scale arrays follow the pools.
    "tks_kv_append_fp8_rows": (
        _i32,
        [_c_void_p, _i64, _i64, _c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p,
         _c_void_p, _c_void_p, _i32, _i64, _i32, _i32, _i32, _i32, _c_void_p, _i32, _c_void_p],
    ),
    "tks_paged_gather_fp8_rows": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _i32, _i64, _i32, _i32, _i32, _i32,
         _c_void_p, _i32, _c_void_p, _c_void_p, _i32, _i32, _c_void_p, _c_void_p, _i64, _i64,
         _i32, _c_void_p],
    ),
    "tks_paged_attention_decode_fp8_rows": (
        _i32,
        [_c_void_p, _i64, _i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i32, _i64, _i32,
         _i32, _i32, _i32, _c_void_p, _i32, _c_void_p, _c_void_p, _i32, _i32, _i32, _f32, _i32,
         _c_void_p, _i64, _i64, _c_void_p, _i64, _i32, _c_void_p],
    ),
    "tks_paged_attention_prefill_fp8_rows": (
        _i32,
        [_c_void_p, _i64, _i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i32, _i64, _i32,
         _i32, _i32, _i32, _c_void_p, _i32, _c_void_p, _c_void_p, _c_void_p, _i32, _i64, _i32,
         _i32, _i32, _f32, _c_void_p, _i64, _i64, _c_void_p, _i64, _i32, _c_void_p],
    ),
    "tks_rope_kv_append_fp8_rows": (
        _i32,
        [_c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i32,
         _c_void_p, _c_void_p, _i64, _i64, _i64, _i64,
         _c_void_p, _i64, _i64, _i32, _i64, _i32, _c_void_p, _c_void_p, _c_void_p, _i64,
         _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i32, _i64, _i32, _i32, _c_void_p, _i32,
         _c_void_p],
    ),
    "tks_rope_append_paged_decode_fp8_rows": (
        _i32,
        [_c_void_p, _i64, _i64, _c_void_p, _i64, _i64, _c_void_p, _i64, _i64,
         _c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p,
         _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i32, _i64, _i32, _i32, _i32, _i32,
         _c_void_p, _i32, _c_void_p, _c_void_p, _i32, _i32, _i32, _f32, _i32,
         _c_void_p, _i64, _i64, _c_void_p, _i64, _i32, _c_void_p],
    ),
}

_lib: ctypes.CDLL | None = None


class HipKernelError(RuntimeError):
    """A kernel launch reported a HIP error."""


def library_path() -> Path:
    """Return where the built shared library is expected (overridable by env)."""

    override = os.environ.get("TOKSERVE_HIP_LIBRARY")
    if override:
        return Path(override)
    return Path(__file__).resolve().parent.parent / LIBRARY_NAME


def load() -> ctypes.CDLL:
    """Load the shared library once and bind every exported symbol."""

    global _lib
    if _lib is not None:
        return _lib
    path = library_path()
    if not path.is_file():
        raise RuntimeError(
            f"{LIBRARY_NAME} is not built at {path}; run "
            "`python -c 'import __graft_entry__ as g; g.build()'` "
            "or `make -C tokserve_amd/csrc`"
        )
    library = ctypes.CDLL(str(path))
    for name, (restype, argtypes) in SIGNATURES.items():
        function = getattr(library, name)
        function.restype = restype
        function.argtypes = argtypes
    version = library.tks_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"{LIBRARY_NAME} ABI {version} does not match binding {ABI_VERSION}")
    _lib = library
    return library


def check(status: int, operation: str) -> None:
    """Translate a C status into the reference's exception types."""

    if status == TKS_OK:
        return
    library = load()
    text = library.tks_status_string(status).decode()
    message = f"{operation}: {text}"
    if status == TKS_ERR_TYPE:
        raise TypeError(message)
    if status == TKS_ERR_INDEX:
        raise IndexError(message)
    if status in (TKS_ERR_VALUE, TKS_ERR_WORKSPACE):
        raise ValueError(message)
    if status == TKS_ERR_LAUNCH:
        raise HipKernelError(f"{message} ({library.tks_last_hip_error().decode()})")
    raise RuntimeError(f"{operation}: unknown status {status}")


def dtype_code(dtype: torch.dtype) -> int:
    """Return the ABI code of a supported floating dtype."""

    try:
        return DTYPE_CODES[dtype]
    except KeyError as error:
        raise TypeError(f"unsupported dtype {dtype}") from error


def ptr(tensor: torch.Tensor | None) -> int | None:
    """Device address of a tensor's first element (None for a missing tensor)."""

    if tensor is None:
        return None
    return tensor.data_ptr()


def stream_of(tensor: torch.Tensor) -> int:
    """The current torch stream (a hipStream_t) of the tensor's device."""

    return torch.cuda.current_stream(tensor.device).cuda_stream
