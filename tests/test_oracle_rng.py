"""Pins the oracle's Philox and quantile table, and checks the library's
host-side copies of both against it (no GPU needed)."""
import json
import math
import os

import numpy as np
import pytest
import torch

from oracle import rng
from oracle.arith import BF16, F16, F32, to_f32

DT_TORCH = {F32: torch.float32, F16: torch.float16, BF16: torch.bfloat16}


@pytest.fixture(scope="module")
def kat(golden_dir):
    with open(os.path.join(golden_dir, "philox_kat.json")) as f:
        return json.load(f)


def test_random123_kat_vectors(kat):
    for ctr, key, expected in kat["random123"]:
        assert rng.philox_scalar(ctr, key) == expected
        got = rng.philox4x32(*[np.array([c], dtype=np.uint64) for c in ctr], key[0], key[1])[0]
        assert got.tolist() == expected


def test_torch_engine_kat(kat):
    for e in kat["torch_engine"]:
        got = rng.philox_groups(e["seed"], e["stream"], np.array([e["q"]], dtype=np.uint64), rounds=10)[0]
        assert got.tolist() == e["block"], e


def test_torch_engine_kat_seven_rounds(kat):
    # the z generator (Philox4x32-7) against torch's engine run with 7 rounds
    assert rng.ROUNDS == 7
    for e in kat["torch_engine_r7"]:
        got = rng.philox_groups(e["seed"], e["stream"], np.array([e["q"]], dtype=np.uint64))[0]
        assert got.tolist() == e["block"], e


def _more_rounds(block, key, done: int, extra: int):
    """`extra` further Philox rounds applied to the output of `done` rounds
    (the key bumped `done` times first)."""
    k0 = (key[0] + done * rng.W0) & rng.MASK32
    k1 = (key[1] + done * rng.W1) & rng.MASK32
    return rng.philox_scalar(block, [k0, k1], rounds=extra) if extra else list(block)


def test_seven_rounds_are_a_prefix_of_ten(kat):
    # Rounds 8-10 applied to the 7-round output reproduce the Random123 10-round
    # vectors. A round is a bijection of the counter for a fixed key, so a wrong
    # 7-round block cannot continue into the right 10-round one.
    for ctr, key, expected in kat["random123"]:
        b7 = rng.philox_scalar(ctr, key, rounds=7)
        assert _more_rounds(b7, key, 7, 3) == expected
        assert b7 != expected


def test_fewer_rounds_differ(kat):
    # A dropped round must not pass the KAT (guards the round count).
    assert rng.philox_scalar([0, 0, 0, 0], [0, 0], rounds=9) != [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]
    e = kat["torch_engine_r7"][0]
    for r in (6, 8):
        got = rng.philox_groups(e["seed"], e["stream"], np.array([e["q"]], dtype=np.uint64), rounds=r)[0]
        assert got.tolist() != e["block"]


def test_library_host_philox_matches_oracle(kat):
    from dizo_amd import table as T
    for e in kat["torch_engine_r7"]:
        assert T.philox_host(e["seed"], e["stream"], e["q"]) == e["block"]
    r = np.random.default_rng(0)
    for _ in range(200):
        seed = int(r.integers(0, 2**63)) * 2 + int(r.integers(0, 2))
        q = int(r.integers(0, 2**63))
        stream = int(r.integers(0, 3))
        want = rng.philox_groups(seed, stream, np.array([q], dtype=np.uint64))[0].tolist()
        assert T.philox_host(seed, stream, q) == want


@pytest.mark.parametrize("dt", [F16, BF16, F32])
def test_library_quantile_table_matches_oracle(dt):
    from dizo_amd import table as T
    prod = T.normal_table(DT_TORCH[dt])
    view = torch.int32 if dt == F32 else torch.int16
    pb = prod.view(view).numpy().view(np.uint32 if dt == F32 else np.uint16)
    np.testing.assert_array_equal(pb, rng.quantile_table(dt))


def test_quantile_table_fp16_fp32_cross_check():
    # numpy's own double->half / double->float conversions agree with the
    # exact-rational rounding used by the oracle.
    from scipy.special import ndtri
    x = ndtri(0.5 + (np.arange(32768) + 0.5) / 65536.0)
    np.testing.assert_array_equal(x.astype(np.float16).view(np.uint16), rng.quantile_table(F16))
    np.testing.assert_array_equal(x.astype(np.float32).view(np.uint32), rng.quantile_table(F32))


@pytest.mark.parametrize("dt", [F16, BF16, F32])
def test_quantile_table_shape(dt):
    q = to_f32(rng.quantile_table(dt), dt).astype(np.float64)
    assert np.all(q > 0)
    assert np.all(np.diff(q) >= 0)  # monotone (ties only from rounding in bf16/f16)
    # first / last entries: Phi^-1(1/2 + 1/2^17) and Phi^-1(1 - 1/2^17)
    assert q[0] == pytest.approx(math.sqrt(2 * math.pi) / 2**17, rel=1e-2)
    assert q[-1] == pytest.approx(4.3250, abs=0.02)
    # Discrete distribution +-Q with equal mass: variance = mean(Q^2) just below 1
    # (mass beyond |z| = 4.33 is missing).
    var = float(np.mean(q * q))
    assert 0.997 < var < 1.0005, var
    kurt = float(np.mean(q**4)) / var**2
    assert 2.95 < kurt < 3.0


def test_z_bits_statistics():
    n = 1 << 20
    z = to_f32(rng.z_bits(1234, 0, np.arange(n, dtype=np.uint64), F32), F32).astype(np.float64)
    assert abs(z.mean()) < 5 / math.sqrt(n)
    assert abs(z.var() - 1.0) < 0.01
    # distinct seeds and streams give uncorrelated sequences
    z2 = to_f32(rng.z_bits(1235, 0, np.arange(n, dtype=np.uint64), F32), F32).astype(np.float64)
    z3 = to_f32(rng.z_bits(1234, 1, np.arange(n, dtype=np.uint64), F32), F32).astype(np.float64)
    assert abs(np.corrcoef(z, z2)[0, 1]) < 5 / math.sqrt(n)
    assert abs(np.corrcoef(z, z3)[0, 1]) < 5 / math.sqrt(n)
    # Kolmogorov-Smirnov against N(0,1) (the 2^-16 quantisation is far below the KS bound)
    from scipy.stats import kstest
    assert kstest(z[:200000], "norm").pvalue > 1e-4


def test_z_dtype_consistency():
    # z_T = RNE_T of one common real quantile, so fp16/bf16 z equal the fp32 z
    # rounded to T, except where rounding twice (double -> fp32 -> T) lands on
    # the other side of a T midpoint: then they differ by one unit in the last place.
    from oracle.arith import from_f32
    e = np.arange(1 << 16, dtype=np.uint64)
    z32 = to_f32(rng.z_bits(7, 0, e, F32), F32)
    for dt in (F16, BF16):
        zt = rng.z_bits(7, 0, e, dt).astype(np.int64)
        via32 = from_f32(z32, dt).astype(np.int64)
        diff = np.abs(via32 - zt)
        assert diff.max() <= 1
        assert np.count_nonzero(diff) < len(e) * 1e-3


def test_layout_z_offsets():
    assert rng.layout_z_offsets([5, 8, 1, 0, 9]) == [0, 8, 16, 24, 24]
