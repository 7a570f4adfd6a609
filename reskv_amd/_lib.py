"""ctypes binding of the C ABI in ``include/reskv_hip.h`` (``libreskv_hip.so``).

There is no fallback: if the library is missing or fails to load, every
operation raises.  Build it with ``python -m reskv_amd.build``.
"""

import ctypes
import threading
from pathlib import Path

_HERE = Path(__file__).resolve().parent
LIB_PATH = _HERE / "libreskv_hip.so"

_vp, _i, _i64, _f = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float

# reskv_abi_version() of the library these signatures describe
ABI_VERSION = 7


class CTensor(ctypes.Structure):
    """Mirror of ``reskv_ctensor``."""

    _fields_ = [
        ("centroids", _vp),
        ("ids", _vp),
        ("payload", _vp),
        ("meta", _vp),
        ("scale", _vp),
        ("nc", _i),
        ("format", _i),
        ("width", _i),
        ("bits", _i),
        ("t_stride", _i),
        ("c_stride", _i),
    ]


FMT_BITMAP, FMT_TILED, FMT_STRUCT16, FMT_STRUCT_INT4, FMT_QUANT = range(5)

# name -> (restype, argtypes); the exported surface of include/reskv_hip.h
SIGNATURES = {
    "reskv_last_error": (ctypes.c_char_p, []),
    "reskv_abi_version": (_i, []),
    "reskv_compress_fp16": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp]),
    "reskv_compress_bitmap": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "reskv_compress_fp16_kv": (_i, [_vp] * 10 + [_i] * 7 + [_vp]),
    "reskv_linspace_rows": (_i, [_i, _i, _vp]),
    "reskv_compress_bitmap_kv": (_i, [_vp] * 10 + [_i] * 6 + [_vp]),
    "reskv_compress_quantized": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp]),
    "reskv_compress_structured_int4": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "reskv_kmeans_workspace_bytes": (_i64, [_i, _i, _i]),
    "reskv_kmeans": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp, _i64, _vp]),
    "reskv_kmeans_assign": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _vp, _i64, _vp]),
    "reskv_kmeans_kv": (_i, [_vp] * 8 + [_i, _i, _i, _i, _vp, _i64, _vp]),
    "reskv_decode_workspace_bytes": (_i64, [_i, _i, _i, _i, _i]),
    "reskv_decode_splits": (_i, [ctypes.POINTER(CTensor), ctypes.POINTER(CTensor), _i, _i, _i, _i, _i, _i]),
    "reskv_decode": (_i, [_vp, ctypes.POINTER(CTensor), ctypes.POINTER(CTensor), _vp, _i, _i, _i, _i, _i, _i,
                          _f, _i, _vp, _vp, _vp, _vp, _i64, _vp]),
    "reskv_decode_rope": (_i, [_vp, ctypes.POINTER(CTensor), ctypes.POINTER(CTensor), _vp, _vp, _i, _i, _i, _i,
                               _i, _i, _f, _i, _vp, _vp, _vp, _vp, _i64, _vp]),
    "reskv_decode_recent": (_i, [_vp, ctypes.POINTER(CTensor), ctypes.POINTER(CTensor), _vp, _vp, _i, _i, _i, _i,
                                 _i, _i, _f, _i, _vp, _vp, _vp, _i, _i, _vp, _vp, _i64, _vp]),
    "reskv_decode_recent_noalloc": (_i, [_vp, ctypes.POINTER(CTensor), ctypes.POINTER(CTensor), _vp, _vp, _i, _i,
                                         _i, _i, _i, _i, _f, _i, _vp, _vp, _vp, _i, _i, _vp, _vp]),
    "reskv_rope_table": (_i, [_vp, _i, _vp, _vp]),
    "reskv_merge_recent_scores": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp]),
    "reskv_merge_recent_qk": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _f, _vp, _vp]),
    "reskv_decode_dense": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _f, _i, _vp, _vp, _vp, _vp, _i64,
                                _vp]),
    # include/reskv_llama.h: fused steps of the end-to-end decode harness
    "reskv_llama_rmsnorm": (_i, [_vp, _vp, _vp, _i, _i, _f, _vp]),
    "reskv_llama_silu_mul": (_i, [_vp, _vp, _i, _i, _vp]),
    "reskv_llama_qkv_rope": (_i, [_vp] * 4 + [_i, _i, _i] + [_vp] * 9 + [_i64, _i64, _i64, _vp]),
}

_lock = threading.Lock()
_lib = None


def lib():
    """The loaded library (raises RuntimeError if it is not built or not loadable)."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not LIB_PATH.exists():
                    raise RuntimeError(
                        f"{LIB_PATH.name} is not built; run `python -m reskv_amd.build` (hipcc, gfx950)"
                    )
                handle = ctypes.CDLL(str(LIB_PATH))
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.restype = res
                    fn.argtypes = args
                found = handle.reskv_abi_version()
                if found != ABI_VERSION:
                    raise RuntimeError(f"{LIB_PATH.name} has ABI version {found}, this binding needs "
                                       f"{ABI_VERSION}; rebuild with `python -m reskv_amd.build`")
                _lib = handle
    return _lib


def check(status: int, what: str):
    if status != 0:
        msg = lib().reskv_last_error().decode(errors="replace")
        raise RuntimeError(f"{what}: {msg}")
