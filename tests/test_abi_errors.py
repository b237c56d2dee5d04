"""The C ABI's host-side checks without a GPU: every entry point called with
invalid arguments returns a negative code and a message (never aborts or
throws across the ABI), and the host-only entry points (version, quantile
tables, host Philox) return results. Under the host-sanitizer build
(python -m dizo_amd.build_sanitized) this runs the validation, table and
plan code paths with AddressSanitizer and UndefinedBehaviorSanitizer."""
import ctypes as C

import numpy as np
import pytest

from dizo_amd import _lib as L
from oracle import rng


@pytest.fixture(scope="module")
def lib():
    return L.load()


def _err(lib, rc, *words):
    assert rc < 0, rc
    msg = lib.dz_last_error().decode()
    assert msg, "no message"
    for w in words:
        assert w in msg, (w, msg)


def test_host_entry_points(lib):
    assert lib.dz_version() == 30000
    for dt, ctype in ((L.DZ_DTYPE_F32, C.c_uint32), (L.DZ_DTYPE_F16, C.c_uint16), (L.DZ_DTYPE_BF16, C.c_uint16)):
        buf = (ctype * L.TAB_ENTRIES)()
        assert lib.dz_normal_table(dt, C.cast(buf, C.c_void_p), L.TAB_ENTRIES) == 0
        name = {L.DZ_DTYPE_F32: "f32", L.DZ_DTYPE_F16: "f16", L.DZ_DTYPE_BF16: "bf16"}[dt]
        np.testing.assert_array_equal(np.frombuffer(buf, dtype=ctype), rng.quantile_table(name))
    out = (C.c_uint32 * 4)()
    for seed, stream, q in ((0, 0, 0), (2**64 - 1, 2, 2**64 - 1), (123, 1, 2**32)):
        assert lib.dz_philox_host(seed, stream, q, out) == 0
        assert list(out) == rng.philox_groups(seed, stream, [q])[0].tolist()


def test_invalid_arguments_return_errors(lib):
    """NULL tables and outputs, counts and dtypes out of range: an error code
    and a message (entry points that look up the current device first may
    report the missing GPU instead)."""
    p = C.c_void_p
    tab = p()
    one = (C.c_uint64 * 1)(4096)
    n1 = (C.c_int64 * 1)(8)
    _err(lib, lib.dz_normal_table(9, None, L.TAB_ENTRIES), "dtype")
    _err(lib, lib.dz_normal_table(L.DZ_DTYPE_F16, None, L.TAB_ENTRIES), "NULL")
    _err(lib, lib.dz_philox_host(1, 0, 0, None), "NULL")
    _err(lib, lib.dz_table_create(None, None, None, None, 1, L.DZ_DTYPE_F16, 0, C.byref(tab)), "NULL")
    _err(lib, lib.dz_table_create(one, None, n1, None, 0, L.DZ_DTYPE_F16, 0, C.byref(tab)), "count")
    _err(lib, lib.dz_table_create(one, None, n1, None, 1, 7, 0, C.byref(tab)), "dtype")
    _err(lib, lib.dz_table_create(one, None, n1, None, 1, L.DZ_DTYPE_F16, 0, None), "NULL")
    assert lib.dz_table_destroy(None) == 0
    _err(lib, lib.dz_perturb(None, 1, 1.0, 1e-3, None, None))
    _err(lib, lib.dz_update(None, 1, 0.5, 1e-6, None, None, None, None))
    _err(lib, lib.dz_restore_update(None, 1, 1e-3, 0.5, 1e-6, None, None, None, None))
    _err(lib, lib.dz_restore_update_perturb(None, 1, 2, 1e-3, 0.5, 1e-6, None, None, None, None, None))
    _err(lib, lib.dz_table_matches(None, None, 0))
    _err(lib, lib.dz_table_z_offset(None, 0, None))
    _err(lib, lib.dz_table_time_next(None, None, None))
    _err(lib, lib.dz_table_set_prefetch_min_tiles(None, 0))
    _err(lib, lib.dz_export_z(None, 1, 0, None, None))
    _err(lib, lib.dz_group_sumsq(None, None, None, None, None))
    _err(lib, lib.dz_project(None, None, L.DZ_PROJ_APPLY, None, None, None, None))
    _err(lib, lib.dz_group_dot(None, None, None, None, None))
    _err(lib, lib.dz_normals(1, 0, 0, 10, L.DZ_DTYPE_F16, None, None))
    _err(lib, lib.dz_philox(1, 0, 0, 10, None, None))
    # the allocation-free entry point: argument checks before any device work
    big = 4097
    ptrs = (C.c_uint64 * big)(*([4096] * big))
    numels = (C.c_int64 * big)(*([8] * big))
    _err(lib, lib.dz_group_sumsq_static(None, None, None, 1, L.DZ_DTYPE_F16, None, None, None, None), "NULL")
    _err(lib, lib.dz_group_sumsq_static(ptrs, ptrs, numels, 0, L.DZ_DTYPE_F16, None, None, None, None),
         "group count")
    _err(lib, lib.dz_group_sumsq_static(ptrs, ptrs, numels, big, L.DZ_DTYPE_F16, None, None, None, None),
         "group count")
    _err(lib, lib.dz_group_sumsq_static(ptrs, ptrs, numels, 3, 5, None, None, None, None), "dtype")
    neg = (C.c_int64 * 2)(8, -1)
    rc = lib.dz_group_sumsq_static(ptrs, ptrs, neg, 2, L.DZ_DTYPE_F16, None, None, None, None)
    assert rc < 0


def test_device_entry_points_without_a_gpu(lib):
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    _err(lib, lib.dz_init(0))
    ptrs = (C.c_uint64 * 1)(4096)
    numels = (C.c_int64 * 1)(32768 * 262144 + 1)
    _err(lib, lib.dz_group_sumsq_static(ptrs, ptrs, numels, 1, L.DZ_DTYPE_F16, None, None, None, None))
    tab = C.c_void_p()
    n1 = (C.c_int64 * 1)(8)
    _err(lib, lib.dz_table_create(ptrs, None, n1, None, 1, L.DZ_DTYPE_F16, 0, C.byref(tab)))
