"""MI355X-native DiZO / MeZO zeroth-order step.

The hot path (seeded perturbation, restore, update, DiZO layer-wise
projection) runs as hand-written HIP kernels for gfx950 behind the C ABI in
include/dizo_amd.h; this package is the Python host side that mirrors the
reference trainer's interface (trainer.py, luozoupi/DiZO).
"""
from ._lib import DzError  # noqa: F401

__version__ = "0.1.0"
