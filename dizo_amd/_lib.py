"""ctypes binding of the C ABI declared in include/dizo_amd.h.

The shared library is built in-tree (``dizo_amd/libdizo_amd.so``). There is no
fallback: if the library is missing or fails to load, every entry point raises.
"""
from __future__ import annotations

import ctypes as C
import os
import threading

from .build import LIB_PATH

DZ_DTYPE_F32 = 0
DZ_DTYPE_F16 = 1
DZ_DTYPE_BF16 = 2

DZ_PROJ_SUMSQ = 0
DZ_PROJ_APPLY = 1
DZ_PROJ_REVERSE = 2
DZ_PROJ_REVERSE_SUMSQ = 3
DZ_PROJ_APPLY_F32ALPHA = 4

DZ_STREAM_PARAM = 0
DZ_STREAM_GAMMA = 1
DZ_STREAM_INIT = 2

TAB_ENTRIES = 32768


class DzError(RuntimeError):
    """A libdizo_amd call returned an error code."""


_p = C.c_void_p
_u64 = C.c_uint64
_i64 = C.c_int64
_i32 = C.c_int32
_u32 = C.c_uint32
_f32 = C.c_float

# name -> (restype, argtypes); mirrors include/dizo_amd.h.
SIGNATURES = {
    "dz_version": (_i32, []),
    "dz_last_error": (C.c_char_p, []),
    "dz_normal_table": (_i32, [_i32, _p, _i64]),
    "dz_philox_host": (_i32, [_u64, _u32, _u64, C.POINTER(_u32)]),
    "dz_table_create": (_i32, [_p, _p, _p, _p, _i32, _i32, _i32, C.POINTER(_p)]),
    "dz_table_destroy": (_i32, [_p]),
    "dz_table_matches": (_i32, [_p, _p, _i32]),
    "dz_table_z_offset": (_i32, [_p, _i32, C.POINTER(_u64)]),
    "dz_table_time_next": (_i32, [_p, _p, _p]),
    "dz_table_set_prefetch_min_tiles": (_i32, [_p, _u32]),
    "dz_perturb": (_i32, [_p, _u64, _f32, _f32, _p, _p]),
    "dz_update": (_i32, [_p, _u64, _f32, _f32, _p, _p, _p, _p]),
    "dz_restore_update": (_i32, [_p, _u64, _f32, _f32, _f32, _p, _p, _p, _p]),
    "dz_restore_update_perturb": (_i32, [_p, _u64, _u64, _f32, _f32, _f32, _p, _p, _p, _p, _p]),
    "dz_normals": (_i32, [_u64, _u32, _u64, _i64, _i32, _p, _p]),
    "dz_export_z": (_i32, [_p, _u64, _i32, _p, _p]),
    "dz_philox": (_i32, [_u64, _u32, _u64, _i64, _p, _p]),
    "dz_group_sumsq": (_i32, [_p, _p, _p, _p, _p]),
    "dz_init": (_i32, [_i32]),
    "dz_group_sumsq_static": (_i32, [_p, _p, _p, _i32, _i32, _p, _p, _p, _p]),
    "dz_project": (_i32, [_p, _p, _i32, _p, _p, _p, _p]),
    "dz_group_dot": (_i32, [_p, _p, _p, _p, _p]),
}

_lock = threading.Lock()
_lib = None


def lib_path() -> str:
    """The library to load: dizo_amd/libdizo_amd.so, or $DIZO_AMD_LIB if set
    (a variant built elsewhere, e.g. with other compile-time tile sizes)."""
    return os.environ.get("DIZO_AMD_LIB") or LIB_PATH


def load() -> C.CDLL:
    """Loads the library once; raises DzError if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            path = lib_path()
            if not os.path.exists(path):
                raise DzError(
                    f"{path} is not built; run `python -m dizo_amd.build` "
                    "(or __graft_entry__.build()) first")
            L = C.CDLL(path)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(L, name)
                fn.restype = res
                fn.argtypes = args
            _lib = L
    return _lib


def call(name: str, *args) -> int:
    """Calls an entry point and raises DzError on a negative return code."""
    L = load()
    rc = getattr(L, name)(*args)
    if rc < 0:
        msg = L.dz_last_error().decode(errors="replace")
        raise DzError(f"{name} failed ({rc}): {msg}")
    return rc


def u64_array(values):
    arr = (_u64 * len(values))(*[int(v) for v in values])
    return arr


def i64_array(values):
    return (_i64 * len(values))(*[int(v) for v in values])
