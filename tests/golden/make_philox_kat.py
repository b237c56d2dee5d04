"""Writes tests/golden/philox_kat.json: Philox4x32-10 and Philox4x32-7 known answers.

Two independent sources:
  * the Random123 known-answer vectors for philox4x32-10 (Salmon et al.,
    SC'11 distribution, kat_vectors), typed in below;
  * PyTorch's header-only engine ``at::Philox4_32`` (ATen/core/PhiloxRNGEngine.h,
    BSD source shipped with the installed torch), compiled with g++ and run
    for a set of (seed, subsequence, offset) triples, with its default 10
    rounds and with 7 (the engine takes the round count as an argument; 7 is
    the z generator's). That engine keys Philox with the seed and uses the
    counter words (offset lo, offset hi, subsequence lo, subsequence hi), so
    its first output block equals the z generator's block for key = seed,
    counter = (stream, q lo, 0, q hi) when offset = stream + 2^32 q lo and
    subsequence = 2^32 q hi.

Run: python tests/golden/make_philox_kat.py
"""
from __future__ import annotations

import json
import os
import subprocess
import tempfile

import torch

HERE = os.path.dirname(os.path.abspath(__file__))

RANDOM123_KAT = [
    # counter (4 x u32), key (2 x u32), expected output (4 x u32)
    [[0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]],
    [[0xFFFFFFFF] * 4, [0xFFFFFFFF, 0xFFFFFFFF], [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]],
    [[0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
     [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]],
]

CASES = [  # (seed, stream, q)
    (0, 0, 0), (1, 0, 0), (26, 0, 1), (123456789, 0, 7), (999999999, 1, 12345),
    (2**32 + 3, 2, 2**32 + 11), (2**64 - 1, 0, 2**64 - 1), (42, 1, 2**40), (7, 0, 3_000_000_000),
]

PROG = r"""
#include <ATen/core/PhiloxRNGEngine.h>
#include <cstdio>
#include <cstdlib>
int main(int argc, char** argv) {
  int rounds = atoi(argv[1]);
  for (int i = 2; i + 2 < argc; i += 3) {
    unsigned long long seed = strtoull(argv[i], 0, 10), sub = strtoull(argv[i+1], 0, 10),
                       off = strtoull(argv[i+2], 0, 10);
    at::Philox4_32 eng(seed, sub, off);
    unsigned a = eng(rounds), b = eng(rounds), c = eng(rounds), d = eng(rounds);
    printf("%u %u %u %u\n", a, b, c, d);
  }
  return 0;
}
"""


def engine_args(seed: int, stream: int, q: int):
    """(seed, subsequence, offset) of at::Philox4_32 whose counter is the z
    generator's (stream, q lo, 0, q hi)."""
    return seed, (q >> 32) << 32, stream + ((q & 0xFFFFFFFF) << 32)


def torch_engine_blocks(cases, rounds: int = 10):
    inc = os.path.join(os.path.dirname(torch.__file__), "include")
    with tempfile.TemporaryDirectory() as td:
        src = os.path.join(td, "kat.cpp")
        exe = os.path.join(td, "kat")
        with open(src, "w") as f:
            f.write(PROG)
        subprocess.run(["g++", "-O1", "-std=c++17", f"-I{inc}", src, "-o", exe], check=True)
        args = [str(x) for c in cases for x in engine_args(*c)]
        out = subprocess.run([exe, str(rounds), *args], check=True, capture_output=True, text=True).stdout
    return [[int(x) for x in line.split()] for line in out.strip().splitlines()]


def main():
    blocks = torch_engine_blocks(CASES)
    blocks7 = torch_engine_blocks(CASES, rounds=7)
    data = {
        "random123": RANDOM123_KAT,
        "torch_engine": [{"seed": s, "stream": st, "q": q, "block": b}
                         for (s, st, q), b in zip(CASES, blocks)],
        "torch_engine_r7": [{"seed": s, "stream": st, "q": q, "block": b}
                            for (s, st, q), b in zip(CASES, blocks7)],
        "source": "tests/golden/make_philox_kat.py",
    }
    with open(os.path.join(HERE, "philox_kat.json"), "w") as f:
        json.dump(data, f, indent=1)
    print(f"wrote {len(blocks)} + {len(blocks7)} torch-engine blocks (10 and 7 rounds)")


if __name__ == "__main__":
    main()
