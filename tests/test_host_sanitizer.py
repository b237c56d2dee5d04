"""The host-sanitizer build (dizo_amd.build_sanitized): the C ABI's host code
compiled with AddressSanitizer and UndefinedBehaviorSanitizer (device code as
in the product build) runs the host-side ABI tests cleanly. CPU only."""
import os
import shutil

import pytest

from dizo_amd import build as B
from dizo_amd import build_sanitized as S


def test_sanitized_host_code_runs_the_abi_tests_clean():
    try:
        B.hipcc()
        S.asan_runtime()
    except RuntimeError as e:
        pytest.skip(str(e))
    if shutil.which("gcc") is None:
        pytest.skip("no gcc")
    lib = S.build()
    assert os.path.exists(lib)
    rc = S.run_tests(["tests/test_abi.py", "tests/test_c_consumer.py", "tests/test_abi_errors.py",
                      "tests/test_oracle_rng.py"], lib=lib)
    assert rc == 0, f"sanitized run exited {rc} (86: AddressSanitizer, 87: UndefinedBehaviorSanitizer)"
