"""CPU oracle for the DiZO zeroth-order step hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or the timed
CPU baseline). The product (``dizo_amd``) never imports it: its path is the
HIP library and it raises when that library is missing.

Modules
  arith     numpy restatement of the reference's per-element arithmetic
            (trainer.py:1442, 1608, 1587, 428-464, 545-614, 1100-1102) with the
            PyTorch rounding recipe: one fp32 op, then RNE to the dtype.
  rng       Philox4x32-10 (Salmon et al., SC'11) and the z definition
            z(seed, stream, e) = sign * Q_T[15-bit index], with Q_T built from
            scipy.special.ndtri and exact rational rounding.
  ref_torch the reference's own expressions (trainer.py) written with torch
            ops and injectable z; runs on CPU here and on the ROCm device on
            the GPU box to pin ``arith`` against torch's real arithmetic.
  loss      float64 brute-force verbalizer loss (trainer.py:1446-1522).

Pinning (what makes this oracle trustworthy, see tests/):
  * Philox: Random123 known-answer vectors and PyTorch's own header-only
    ``at::Philox4_32`` engine (fixture tests/golden/philox_kat.json).
  * Q_T: exact-rational rounding of ndtri, cross-checked against numpy's
    float16/float32 conversions, monotonicity and symmetry, and moments.
  * arith: bit-exact against ref_torch on CPU (torch's real kernels), on
    edge values (subnormals, +-0, odd sizes), and against closed forms
    (scale 0 / lr 0 leave theta unchanged except -0 -> +0, alpha = 1 etc).
  * LR schedule: the learning rates printed in the reference's own training
    log (output-DiZO-SST2.log), fixture tests/golden/reference_log_lr.json.
"""
