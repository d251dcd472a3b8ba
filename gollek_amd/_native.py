"""ctypes binding of libgollek_hip.so (include/gollek_hip.h).

This is what a Java FFM binding does with Linker.downcallHandle: resolve each
exported symbol and declare its C signature.  Loading fails loudly when the
library has not been built; there is no fallback implementation.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libgollek_hip.so"

OK = 0
ERR_NULL = -1
ERR_ARG = -2
ERR_UNSUPPORTED = -3
ERR_DEVICE = -4
ERR_NOMEM = -5

Q4_0 = 2
Q8_0 = 8
Q4_K = 12
Q5_K = 13
Q6_K = 14

_c = ctypes
_P = _c.c_void_p
_I32 = _c.c_int32
_I64 = _c.c_int64
_SZ = _c.c_size_t
_CHARP = _c.c_char_p

# name -> (restype, argtypes); the exports declared in include/gollek_hip.h.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "gollek_hip_version": (_I32, []),
    "gollek_hip_init": (_I32, [_I32, _CHARP, _SZ]),
    "gollek_hip_last_error": (_CHARP, []),
    "gollek_hip_last_status": (_I32, []),
    "gollek_hip_weight_upload": (_P, [_I32, _P, _I64, _I64, _I64, _CHARP, _SZ]),
    "gollek_hip_weight_wrap_device": (_P, [_I32, _P, _I64, _I64, _I64, _CHARP, _SZ]),
    "gollek_hip_weight_free": (None, [_P]),
    "gollek_hip_weight_prepare": (_I32, [_P, _CHARP, _SZ]),
    "gollek_hip_weight_unprepare": (_I32, [_P, _CHARP, _SZ]),
    "gollek_hip_weight_compact": (_I32, [_P, _CHARP, _SZ]),
    "gollek_hip_weight_info": (_I32, [_P, _P, _P, _P, _P]),
    "gollek_hip_dequantize_rows": (_I32, [_P, _I64, _I64, _P, _I64, _CHARP, _SZ]),
    "gollek_hip_dot_row": (_I32, [_P, _I64, _P, _I64, _P, _CHARP, _SZ]),
    "gollek_hip_matvec_rows": (_I32, [_P, _P, _I64, _P, _I64, _I64, _CHARP, _SZ]),
    "gollek_hip_dequantize_rows_device": (_I32, [_P, _I64, _I64, _P, _P, _CHARP, _SZ]),
    "gollek_hip_matvec_device": (_I32, [_P, _P, _P, _I64, _P, _CHARP, _SZ]),
    "gollek_hip_gemm_bf16": (_I32, [_P, _P, _I64, _I64, _P, _I64, _CHARP, _SZ]),
    "gollek_hip_gemm_bf16_device": (_I32, [_P, _P, _I64, _P, _P, _CHARP, _SZ]),
    "gollek_hip_gemm_bf16_device_noalloc": (_I32, [_P, _P, _I64, _P, _P, _CHARP, _SZ]),
    "gollek_hip_moe_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64, _I64]),
    "gollek_hip_moe_grouped": (_I32, [_P, _P, _P, _I64, _P, _I64, _P, _P, _I64, _P, _I64,
                                      _CHARP, _SZ]),
    "gollek_hip_moe_grouped_device": (_I32, [_P, _P, _P, _I64, _P, _P, _P, _I64, _I64, _P, _P,
                                             _I64, _P, _CHARP, _SZ]),
    "gollek_hip_moe_select_topk": (_I32, [_P, _I64, _I64, _I64, _I32, _P, _P, _CHARP, _SZ]),
    "gollek_hip_moe_select_topk_device": (_I32, [_P, _I64, _I64, _I64, _I32, _P, _P, _P, _CHARP,
                                                 _SZ]),
    "gollek_hip_moe_block": (_I32, [_P, _P, _P, _I64, _P, _I64, _P, _I64, _I32, _P, _I64, _CHARP,
                                    _SZ]),
    "gollek_hip_moe_block_device": (_I32, [_P, _P, _P, _I64, _P, _P, _I64, _I64, _I32, _P, _P, _P,
                                           _P, _I64, _P, _CHARP, _SZ]),
    "gollek_hip_moe_shared_expert": (_I32, [_P, _P, _P, _P, _P, _I64, _P, _I64, _CHARP, _SZ]),
    "gollek_hip_moe_shared_workspace_bytes": (_I64, [_I64, _I64, _I64]),
    "gollek_hip_moe_shared_expert_device": (_I32, [_P, _P, _P, _P, _P, _I64, _P, _P, _I64, _P, _CHARP,
                                                   _SZ]),
    "gollek_hip_gguf_open": (_P, [_CHARP, _CHARP, _SZ]),
    "gollek_hip_gguf_close": (None, [_P]),
    "gollek_hip_gguf_info": (_I32, [_P, _P, _P, _P, _P, _P, _P]),
    "gollek_hip_gguf_tensor": (_I32, [_P, _I64, _CHARP, _SZ, _P, _P, _P, _P, _P]),
    "gollek_hip_gguf_find": (_I64, [_P, _CHARP]),
    "gollek_hip_gguf_upload": (_P, [_P, _I64, _CHARP, _SZ]),
}

# Test-only export (gollek_amd/csrc/gollek_hip_testing.h; not part of the
# drop-in ABI): forces a GEMV / MoE kernel family onto shapes another one
# is picked for, so the parity tests reach every family.
TESTING_SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "gollek_hip_testing_set_option": (_I32, [_CHARP, _I64, _CHARP, _SZ]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load the library and declare every signature; raises if absent."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = Path(os.environ.get("GOLLEK_HIP_LIBRARY", str(LIB_PATH)))
        if not path.exists():
            raise RuntimeError(
                f"{path} is not built; build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'`")
        lib = ctypes.CDLL(str(path))
        for name, (restype, argtypes) in {**SIGNATURES, **TESTING_SIGNATURES}.items():
            fn = getattr(lib, name, None)
            if fn is None:
                continue  # symbol tests report missing exports explicitly
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
        return lib


class ErrBuf:
    """Caller-owned error buffer, as the Java side allocates in an Arena."""

    def __init__(self, size: int = 512):
        self.buf = ctypes.create_string_buffer(size)
        self.size = size

    @property
    def text(self) -> str:
        return self.buf.value.decode("utf-8", "replace")
