"""Philox4x32-R and the z definition, restated in numpy (test oracle only).

Philox4x32-R follows Salmon, Moraes, Dror and Shaw, "Parallel Random
Numbers: As Easy as 1, 2, 3" (SC'11). One round maps counter (c0, c1, c2, c3)
under key (k0, k1) to
  (mulhi(M1, c2) ^ c1 ^ k0, mullo(M1, c2), mulhi(M0, c0) ^ c3 ^ k1, mullo(M0, c0))
with M0 = 0xD2511F53, M1 = 0xCD9E8D57; the key is bumped by the Weyl
constants 0x9E3779B9, 0xBB67AE85 between rounds. The paper's default is
R = 10; z uses R = ROUNDS = 7, the fewest rounds the paper found
Crush-resistant for Philox4x32 (the library's dz_common.h defines the same).

The z that replaces torch.normal (trainer.py:1441, 1607) is defined as
  q = e >> 3, j = e & 7, w = Philox4x32-7(counter = (stream, q lo, 0, q hi), key = seed)
  h = 16-bit field j of w (word j >> 1, half j & 1)
  z = (-1)^(h >> 15) * Q_T[h & 0x7fff],  Q_T[i] = RNE_T(Phi^-1(1/2 + (i + 1/2) / 65536)).
"""
from __future__ import annotations

import math
from fractions import Fraction
from functools import lru_cache

import numpy as np

from .arith import BF16, F16, F32

ROUNDS = 7  # rounds of the Philox that defines z
M0, M1 = 0xD2511F53, 0xCD9E8D57
W0, W1 = 0x9E3779B9, 0xBB67AE85
MASK32 = 0xFFFFFFFF


def philox4x32(c0, c1, c2, c3, k0: int, k1: int, rounds: int = 10):
    """Vectorised Philox4x32-R over numpy arrays of counters; returns (n, 4) uint32."""
    c0 = np.asarray(c0, dtype=np.uint64)
    c1 = np.asarray(c1, dtype=np.uint64)
    c2 = np.asarray(c2, dtype=np.uint64)
    c3 = np.asarray(c3, dtype=np.uint64)
    c0, c1, c2, c3 = np.broadcast_arrays(c0, c1, c2, c3)
    m32 = np.uint64(MASK32)
    s32 = np.uint64(32)
    for _ in range(rounds):
        p0 = np.uint64(M0) * c0
        p1 = np.uint64(M1) * c2
        n0 = (p1 >> s32) ^ c1 ^ np.uint64(k0)
        n1 = p1 & m32
        n2 = (p0 >> s32) ^ c3 ^ np.uint64(k1)
        n3 = p0 & m32
        c0, c1, c2, c3 = n0, n1, n2, n3
        k0 = (k0 + W0) & MASK32
        k1 = (k1 + W1) & MASK32
    return np.stack([c0, c1, c2, c3], axis=-1).astype(np.uint32)


def philox_scalar(ctr, key, rounds: int = 10):
    """Pure-python Philox4x32-R of one block (for tiny cross-checks)."""
    c = [int(x) & MASK32 for x in ctr]
    k0, k1 = int(key[0]) & MASK32, int(key[1]) & MASK32
    for _ in range(rounds):
        p0 = M0 * c[0]
        p1 = M1 * c[2]
        c = [((p1 >> 32) ^ c[1] ^ k0) & MASK32, p1 & MASK32, ((p0 >> 32) ^ c[3] ^ k1) & MASK32, p0 & MASK32]
        k0 = (k0 + W0) & MASK32
        k1 = (k1 + W1) & MASK32
    return c


def philox_groups(seed: int, stream: int, q, rounds: int = ROUNDS) -> np.ndarray:
    """Blocks for counters q (uint64 array) under key = seed: (n, 4) uint32
    (the z generator's Philox4x32-7 unless `rounds` says otherwise). Counter
    words: (stream, q lo, 0, q hi)."""
    q = np.asarray(q, dtype=np.uint64)
    return philox4x32(np.uint64(stream), q & np.uint64(MASK32), np.uint64(0), q >> np.uint64(32),
                      seed & MASK32, (seed >> 32) & MASK32, rounds)


# --------------------------------------------------------- quantile table ---

FORMAT = {F32: (24, -126), F16: (11, -14), BF16: (8, -126)}


def round_exact(x: float, p: int, emin: int) -> Fraction:
    """Exact round-to-nearest-even of a positive double to (p bits, emin)."""
    fx = Fraction(x)
    _, e2 = math.frexp(x)
    E = max(e2 - 1, emin)
    quantum = Fraction(2) ** (E - (p - 1))
    return round(fx / quantum) * quantum  # Fraction.__round__ ties to even


def _bits_of(v: Fraction, dt: str) -> int:
    if dt == F32:
        return int(np.float32(float(v)).view(np.uint32))
    if dt == BF16:
        return int(np.float32(float(v)).view(np.uint32)) >> 16
    return int(np.float16(float(v)).view(np.uint16))  # v is exactly representable


@lru_cache(maxsize=None)
def quantile_table(dt: str) -> np.ndarray:
    """Q_T bit patterns, built from scipy.special.ndtri with exact rounding."""
    from scipy.special import ndtri

    r = (np.arange(32768, dtype=np.float64) + 0.5) / 65536.0
    x = ndtri(0.5 + r)
    p, emin = FORMAT[dt]
    bits = [_bits_of(round_exact(float(v), p, emin), dt) for v in x]
    return np.asarray(bits, dtype=np.uint32 if dt == F32 else np.uint16)


def z_bits(seed: int, stream: int, e, dt: str) -> np.ndarray:
    """z(seed, stream, e) for global element indices e, as T bit patterns."""
    e = np.asarray(e, dtype=np.uint64)
    w = philox_groups(seed, stream, e >> np.uint64(3))
    j = (e & np.uint64(7)).astype(np.int64)
    word = w[np.arange(len(e)), j >> 1].astype(np.uint32)
    h = (word >> (16 * (j & 1)).astype(np.uint32)) & np.uint32(0xFFFF)
    tab = quantile_table(dt)
    mag = tab[(h & np.uint32(0x7FFF)).astype(np.int64)].astype(np.uint32)
    sign = (h >> np.uint32(15)) << np.uint32(31 if dt == F32 else 15)
    out = mag | sign
    return out.astype(np.uint32 if dt == F32 else np.uint16)


def layout_z_offsets(numels) -> list[int]:
    """Global z offsets of tensors laid end to end, each rounded up to 8 elements."""
    offs, z = [], 0
    for n in numels:
        offs.append(z)
        z += (int(n) + 7) // 8 * 8
    return offs


def tensor_z_bits(seed: int, z_offset: int, numel: int, dt: str, stream: int = 0) -> np.ndarray:
    return z_bits(seed, stream, np.arange(numel, dtype=np.uint64) + np.uint64(z_offset), dt)
