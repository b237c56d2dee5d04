"""numpy restatement of the ZO / DiZO per-element arithmetic (test oracle only).

Values of a dtype T are carried as their bit patterns (uint16 for fp16/bf16,
uint32 for fp32). PyTorch evaluates every elementwise op as one IEEE fp32
operation on fp32-widened operands ("opmath") followed by a round-to-nearest-
even conversion to T; python scalars enter as fp32. ``rt`` is that rounding.
"""
from __future__ import annotations

import numpy as np

F32, F16, BF16 = "f32", "f16", "bf16"
DTYPES = (F32, F16, BF16)
BITS_DTYPE = {F32: np.uint32, F16: np.uint16, BF16: np.uint16}


def to_f32(bits, dt: str) -> np.ndarray:
    b = np.asarray(bits)
    if dt == F32:
        return b.astype(np.uint32).view(np.float32)
    if dt == F16:
        return b.astype(np.uint16).view(np.float16).astype(np.float32)
    if dt == BF16:
        return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)
    raise ValueError(dt)


def from_f32(x, dt: str) -> np.ndarray:
    """Round fp32 values to T (RNE) and return T's bit patterns."""
    x = np.asarray(x, dtype=np.float32)
    if dt == F32:
        return x.view(np.uint32).copy()
    if dt == F16:
        with np.errstate(over="ignore"):  # overflow rounds to +-inf, as in torch
            return x.astype(np.float16).view(np.uint16)
    if dt == BF16:
        u = x.view(np.uint32).astype(np.uint64)
        r = ((u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16))
        r = (r & np.uint64(0xFFFF)).astype(np.uint16)
        return np.where(np.isnan(x), np.uint16(0x7FC0), r)
    raise ValueError(dt)


def rt(x, dt: str) -> np.ndarray:
    """R_T: round an fp32 result to T and widen back to fp32."""
    if dt == F32:
        return np.asarray(x, dtype=np.float32)
    return to_f32(from_f32(x, dt), dt)


def f32(v) -> np.float32:
    """A python scalar as PyTorch's opmath sees it (static_cast<float>)."""
    return np.float32(v)


# ---------------------------------------------------------------- ZO step ---

def perturb(theta_bits, z_bits, scale, eps, dt: str) -> np.ndarray:
    """trainer.py:1442  param.data + scaling_factor * z * eps."""
    th = to_f32(theta_bits, dt)
    z = to_f32(z_bits, dt)
    a = rt(f32(scale) * z, dt)
    b = rt(a * f32(eps), dt)
    return from_f32(th + b, dt)


def update(theta_bits, z_bits, grad, lr, dt: str) -> np.ndarray:
    """trainer.py:1608  param.data - lr * (projected_grad * z)."""
    th = to_f32(theta_bits, dt)
    z = to_f32(z_bits, dt)
    c = rt(f32(grad) * z, dt)
    d = rt(f32(lr) * c, dt)
    return from_f32(th - d, dt)


def restore_update(theta_bits, z_bits, eps, grad, lr, dt: str) -> np.ndarray:
    """trainer.py:1593 (perturb with scaling_factor=+1) followed by trainer.py:1608."""
    return update(perturb(theta_bits, z_bits, 1, eps, dt), z_bits, grad, lr, dt)


def scalar_div_device(x_bits, divisor: float, dt: str):
    """T tensor / python scalar on the GPU (trainer.py:1587 and :607).

    torch's device true-divide by a CPU scalar multiplies by a reciprocal
    instead of dividing; the reciprocal is formed from the double-precision
    scalar and rounded once to fp32, then R_T(x * inv). Pinned on the ROCm
    device by tests/test_gpu_zo.py::test_projected_grad_device_rule (for
    divisor 0.002 the rule x * fp32(1/0.002f) = x * 499.99997 differs from
    torch in about 1% of fp16 inputs; this one matches bit for bit).
    """
    inv = np.float32(1.0 / float(divisor))
    return from_f32(to_f32(x_bits, dt) * inv, dt)


def scalar_div_cpu(x_bits, divisor: float, dt: str):
    """T tensor / python scalar on the CPU: a true fp32 division, one rounding to T."""
    return from_f32(to_f32(x_bits, dt) / np.float32(divisor), dt)


SCALAR_DIV = {"device": scalar_div_device, "cpu": scalar_div_cpu}


def projected_grad(loss1_bits, loss2_bits, eps: float, dt: str, rule: str = "device") -> float:
    """trainer.py:1587  ((loss1 - loss2) / (2 * zo_eps)).item()."""
    d = from_f32(to_f32(loss1_bits, dt) - to_f32(loss2_bits, dt), dt)
    return float(np.ravel(to_f32(SCALAR_DIV[rule](d, 2 * eps, dt), dt))[0])


def zo_lr(base_lr: float, step: int, max_steps: int) -> float:
    """Learning rate applied by the update of 0-indexed global step `step`.

    trainer.py:1100-1102: LambdaLR with lambda = 1 - global_step / (2 max_steps),
    evaluated at construction (global_step 0) and after each update
    (trainer.py:1617, before global_step += 1).
    """
    k = max(step - 1, 0)
    return base_lr * (1 - k / (2 * max_steps))


# ------------------------------------------------------------- projection ---

def diff(theta_bits, theta0_bits, dt: str) -> np.ndarray:
    return rt(to_f32(theta_bits, dt) - to_f32(theta0_bits, dt), dt)


def group_sumsq(theta_bits, theta0_bits, dt: str) -> float:
    """Exact-as-float64 sum of squares of R(theta - theta0)."""
    d = diff(theta_bits, theta0_bits, dt).astype(np.float64)
    return float(np.dot(d.ravel(), d.ravel()))


def norm_from_sumsq(sumsq: float, dt: str):
    """torch.norm's finish: fp32 sqrt of the fp32 accumulator, cast to T (bits)."""
    return from_f32(np.sqrt(np.float32(sumsq)), dt)


def alpha(gamma_bits, norm_bits, dt: str):
    """trainer.py:464  constraint / (norms + 1e-8)."""
    n1 = rt(to_f32(norm_bits, dt) + f32(1e-8), dt)
    return from_f32(to_f32(gamma_bits, dt) / n1, dt)


def apply(theta_bits, theta0_bits, alpha_bits, dt: str) -> np.ndarray:
    """trainer.py:428-436  (new - anchor) * alpha + anchor."""
    d = diff(theta_bits, theta0_bits, dt)
    v = rt(d * to_f32(alpha_bits, dt), dt)
    return from_f32(v + to_f32(theta0_bits, dt), dt)


def reverse(theta_bits, theta0_bits, alpha_bits, dt: str) -> np.ndarray:
    """trainer.py:447-451  (new - anchor) / alpha + anchor."""
    d = diff(theta_bits, theta0_bits, dt)
    v = rt(d / to_f32(alpha_bits, dt), dt)
    return from_f32(v + to_f32(theta0_bits, dt), dt)


# ------------------------------------------------------- gamma SPSA (ZO) ----
# trainer.py:545-614 with tau = 0.2, zo_eps = 0.1, step_size = 2, vectorised
# over groups (each op is elementwise, so per-group results are unchanged).

TAU, GAMMA_EPS, STEP_SIZE = 0.2, 0.1, 2


def clip_z(z_bits, ts_bits, dt: str):
    """trainer.py:555  torch.clip(z, (-tau/zo_eps)*ts, (tau/zo_eps)*ts)."""
    ts = to_f32(ts_bits, dt)
    lo = rt(f32(-TAU / GAMMA_EPS) * ts, dt)
    hi = rt(f32(TAU / GAMMA_EPS) * ts, dt)
    z = to_f32(z_bits, dt)
    return from_f32(np.minimum(np.maximum(z, lo), hi), dt)


def perturb_gamma(gamma_bits, zc_bits, delta: int, dt: str):
    """trainer.py:560  gamma + delta * z * zo_eps."""
    a = rt(f32(delta) * to_f32(zc_bits, dt), dt)
    b = rt(a * f32(GAMMA_EPS), dt)
    return from_f32(to_f32(gamma_bits, dt) + b, dt)


def gamma_step(gamma_bits, ts_bits, zc_bits, loss1_bits, loss2_bits, dt: str, rule: str = "device"):
    """trainer.py:607-612: grad = (L1-L2)/(2 zo_eps); clip(gamma - 2 ts grad z, 0.8 ts, 1.2 ts)."""
    d = from_f32(to_f32(loss1_bits, dt) - to_f32(loss2_bits, dt), dt)
    g = to_f32(SCALAR_DIV[rule](d, 2 * GAMMA_EPS, dt), dt)
    ts = to_f32(ts_bits, dt)
    t1 = rt(f32(STEP_SIZE) * ts, dt)
    t2 = rt(t1 * g, dt)
    t3 = rt(t2 * to_f32(zc_bits, dt), dt)
    new = rt(to_f32(gamma_bits, dt) - t3, dt)
    lo = rt(f32(1 - TAU) * ts, dt)
    hi = rt(f32(1 + TAU) * ts, dt)
    return from_f32(np.minimum(np.maximum(new, lo), hi), dt)
