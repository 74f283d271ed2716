"""Load the gfx950 C-ABI library (``libvllm_rlt_hip.so``) once and bind it.

The library sits in ``vllm_rlt/_lib`` next to this package (built in-tree by
``make -C vllm-rlt_amd``). It is loaded with :mod:`ctypes`; every entry point
returns 0 on success, otherwise :func:`check` raises ``RuntimeError`` with the
library's own message. A missing or unloadable library raises ``ImportError``
(file absent) or ``OSError`` (loader failure), the two errors the attention
backend factory treats as "backend unavailable" (reference:
vllm_rlt/attention/backend.py:148-152 and vllm_rlt/kernels/_extension.py:7-23).
There is no fallback implementation.
"""

from __future__ import annotations

import ctypes
import os
from functools import cache

LIBRARY_NAME = "libvllm_rlt_hip.so"
LIBRARY_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "_lib",
                            LIBRARY_NAME)
ABI_VERSION = 5

VRH_DTYPE_F32, VRH_DTYPE_F16, VRH_DTYPE_BF16 = 0, 1, 2

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_INT = ctypes.c_int
_SZ = ctypes.c_size_t

# Signatures of include/vllm_rlt_hip.h (argument order must match the header).
SIGNATURES: dict[str, tuple[object, list]] = {
    "vrh_abi_version": (_INT, []),
    "vrh_last_error": (ctypes.c_char_p, []),
    "vrh_kv_append": (
        _INT,
        [_INT, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P,
         _P, _P, _I64, _I32, _I32, _I32, _I64, _I32, _P],
    ),
    "vrh_paged_decode_workspace_bytes": (_SZ, [_I64, _I32, _I32]),
    "vrh_paged_decode": (
        _INT,
        [_INT, _P, _P, _P, _P, _P, _P, _I64, _I32, _I32, _I32, _I32, _I32, _I64, _I64, _I64, _I64,
         _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _P, _SZ, _P],
    ),
    "vrh_paged_decode_noalloc_max_bytes": (_SZ, []),
    "vrh_paged_decode_noalloc": (
        _INT,
        [_INT, _P, _P, _P, _P, _P, _P, _I64, _I32, _I32, _I32, _I32, _I32, _I64, _I64, _I64, _I64,
         _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _P],
    ),
    "vrh_paged_prefill": (
        _INT,
        [_INT, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I32, _I32, _I32, _I32, _I32, _I32, _I64,
         _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P, _SZ, _P],
    ),
    "vrh_paged_prefill_workspace_bytes": (_SZ, [_I64, _I32, _I32, _I32]),
    "vrh_kv_gather": (_INT, [_P, _P, _P, _P, _P, _I64, _I32, _I64, _I64, _I64, _P]),
    "vrh_kv_finalize": (
        _INT, [_P, _P, _P, _P, _I64, _I32, _I32, _I32, _I32, _I64, _I64, _I64, _I64, _P]
    ),
    "vrh_kv_finalize_token": (
        _INT, [_P, _P, _I64, _P, _I32, _I32, _P, _I32, _I64, _I64, _I64, _I64, _P]
    ),
    "vrh_kv_copy_blocks": (_INT, [_P, _P, _I64, _I64, _P, _P, _I64, _P]),
    "vrh_expand_kv_addresses": (_INT, [_P, _P, _P, _P, _P, _I64, _I32, _I32, _P]),
    "vrh_routing_metadata": (
        _INT, [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I32, _I32, _I32, _I32, _P]
    ),
    "vrh_routing_slots": (_INT, [_P, _P, _I64, _I64, _P]),
    "vrh_kv_blocks_to_host": (_INT, [_P, _P, _I64, _I64, _P, _P, _P, _I64, _P]),
    "vrh_kv_blocks_from_host": (_INT, [_P, _P, _I64, _I64, _P, _P, _P, _I64, _P]),
    "vrh_gather_rows": (_INT, [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P]),
    "vrh_scatter_rows": (_INT, [_P, _P, _P, _I64, _I64, _I64, _I64, _P]),
    "vrh_gather_segments": (_INT, [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P]),
    "vrh_scatter_segments": (_INT, [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P]),
    "vrh_silu_and_mul": (_INT, [_INT, _P, _P, _P, _I64, _P]),
}


class _Library:
    def __init__(self, handle: ctypes.CDLL):
        self.handle = handle
        for name, (restype, argtypes) in SIGNATURES.items():
            function = getattr(handle, name)
            function.restype = restype
            function.argtypes = argtypes
            setattr(self, name, function)

    def check(self, code: int, what: str) -> None:
        if code != 0:
            message = self.vrh_last_error().decode(errors="replace")
            raise RuntimeError(f"{what} failed (code {code}): {message}")


@cache
def library() -> _Library:
    """Return the bound library; ImportError if it was never built."""
    if not os.path.exists(LIBRARY_PATH):
        raise ImportError(
            f"{LIBRARY_NAME} is not built (expected at {LIBRARY_PATH}); "
            "run `make -C vllm-rlt_amd` or __graft_entry__.build()"
        )
    lib = _Library(ctypes.CDLL(LIBRARY_PATH))
    version = lib.vrh_abi_version()
    if version != ABI_VERSION:
        raise OSError(f"{LIBRARY_NAME} ABI version {version}, expected {ABI_VERSION}")
    return lib
