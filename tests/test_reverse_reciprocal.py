"""The bf16 reverse pass's quotient (csrc/dz_kernels.hip, recip_div): the
reference divides R_bf16(theta - theta0) by alpha in fp32 and rounds to bf16
(trainer.py:447-451); the kernel multiplies by inv = fp32(1 / alpha) and
falls back to the division where inv is not finite or the product is a
nonzero value below the smallest normal fp32 number. Checked here over every
pair of bf16 values (2^32 pairs, inf and NaN dividends included), against
the oracle's IEEE division (oracle.arith.reverse's quotient)."""
import multiprocessing as mp

import numpy as np
import pytest

from oracle import arith as A

MIN_NORMAL = np.float32(2.0 ** -126)


def _kernel_rule(d: np.ndarray, a: np.float32) -> np.ndarray:
    """The kernel's quotient, restated: bf16 bits of R_bf16(d / a)."""
    with np.errstate(all="ignore"):
        inv = np.float32(np.float32(1.0) / a)
        q = (d * inv).astype(np.float32)
        fast = np.isfinite(inv) & ~((q != 0) & (np.abs(q) < MIN_NORMAL))
        div = (d / a).astype(np.float32)
    return A.from_f32(np.where(fast, q, div), A.BF16)


def _chunk(lo_hi):
    lo, hi = lo_hi
    f = A.to_f32(np.arange(65536, dtype=np.uint32).astype(np.uint16), A.BF16).astype(np.float32)
    bad, fast = [], 0
    for ai in range(lo, hi):
        a = f[ai]
        if a == 0 or not np.isfinite(a):
            continue  # alpha = gamma / (norm + 1e-8) is finite and nonzero; the kernel divides for these anyway
        with np.errstate(all="ignore"):
            want = A.from_f32((f / a).astype(np.float32), A.BF16)
        got = _kernel_rule(f, a)
        nan = np.isnan(A.to_f32(got, A.BF16)) & np.isnan(A.to_f32(want, A.BF16))
        m = (got != want) & ~nan
        if m.any():
            bad.append((ai, int(np.nonzero(m)[0][0])))
    return bad


def test_reciprocal_quotient_rounds_like_division_for_every_bf16_pair():
    chunks = [(i, i + 4096) for i in range(0, 65536, 4096)]
    with mp.get_context("fork").Pool(8) as pool:
        bad = [b for r in pool.map(_chunk, chunks) for b in r]
    assert not bad, f"{len(bad)} alphas with a mismatch, e.g. (alpha bits, dividend bits) {bad[:4]}"


def test_rule_needs_the_fallback():
    """Without the fallback the product misrounds: alphas below 2^-128 (inf
    reciprocal) and quotients in the fp32 subnormal range."""
    f = A.to_f32(np.arange(65536, dtype=np.uint32).astype(np.uint16), A.BF16).astype(np.float32)
    a = f[0x0001]  # the smallest bf16 subnormal: 1 / a overflows
    with np.errstate(all="ignore"):
        plain = A.from_f32((f * np.float32(np.float32(1.0) / a)).astype(np.float32), A.BF16)
        want = A.from_f32((f / a).astype(np.float32), A.BF16)
    fin = np.isfinite(f) & (f != 0)
    assert (plain[fin] != want[fin]).any()
    assert np.array_equal(_kernel_rule(f[fin], a), want[fin])
