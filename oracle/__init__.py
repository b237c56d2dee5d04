"""CPU oracle for the DiZO zeroth-order step hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or the timed
CPU baseline). The product (``dizo_amd``) never imports it: its path is the
HIP library, and it raises when that library is missing.

Modules
  arith     numpy restatement of the reference's per-element arithmetic
            (trainer.py:1442, 1608, 1587, 428-464, 545-614, 1100-1102) with the
            PyTorch rounding recipe: one fp32 op, then RNE to the dtype.
  rng       Philox4x32-R (Salmon et al., SC'11; z uses R = 7) and the z definition
            z(seed, stream, e) = sign * Q_T[15-bit index], with Q_T built from
            scipy.special.ndtri and exact rational rounding.
  ref_torch the reference's own expressions (trainer.py:1429-1444, 1597-1608,
            1587, 405-465, 564-614) written with torch ops and injectable z /
            gamma noise / norm; runs on the CPU here and on the ROCm device on
            the GPU box, to pin ``arith`` against torch's real arithmetic and
            the kernels against the reference fed the same z. On the CPU it is
            also the timed CPU baseline (bench.py).
  loss      float64 brute-force restatement of the option-masked
            classification loss (trainer.py:1446-1522).

How each part is pinned (tests/):
  * Philox: Random123 known-answer vectors and PyTorch's own header-only
    at::Philox4_32 engine (fixture tests/golden/philox_kat.json, made by
    tests/golden/make_philox_kat.py); a dropped round fails.
  * Q_T: exact-rational rounding of ndtri, cross-checked against numpy's own
    float16/float32 conversions of the same values, against the library's
    independently computed table (Newton on erf/erfc), and by monotonicity,
    symmetry and moments.
  * arith: bit-exact against ref_torch on the CPU (torch's real kernels), on
    edge values (subnormals, +-0, odd sizes), and against closed forms (scale
    0 / lr 0 leave theta unchanged except -0 -> +0, alpha = 1 etc.); the
    device divide-by-scalar rule against torch on the ROCm device.
  * LR schedule: the learning rates printed in the reference's own training
    logs (fixture tests/golden/reference_log.json).
  * loss: closed forms (uniform logits give log 2, a certain candidate gives
    log(1 + 1/7) over 7 tokens, pad targets are dropped) and the reference's
    own masking loop.
No function here is left without such a check.
"""
