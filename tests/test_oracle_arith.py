"""Pins oracle.arith against torch's real CPU kernels evaluating the
reference's own expressions (oracle.ref_torch), and against closed forms."""
import numpy as np
import pytest
import torch

from oracle import arith as A
from oracle import ref_torch as R
from oracle import rng
from oracle.arith import BF16, F16, F32, from_f32, to_f32

from tests._util import DT_TORCH, assert_bits_equal, random_theta, to_bits, to_torch

DTS = [F32, F16, BF16]


def _z(n, dt, seed=11):
    return rng.tensor_z_bits(seed, 0, n, dt)


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("scale", [1, -2, 0.5, 3])
def test_perturb_matches_torch(dt, scale):
    n = 20011
    th = random_theta(n, dt, 1)
    z = _z(n, dt)
    eps = 1e-3
    p = to_torch(th, dt)
    R.zo_perturb_parameters([p], [to_torch(z, dt)], scale, eps)
    assert_bits_equal(A.perturb(th, z, scale, eps, dt), to_bits(p), dt, "perturb")


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("grad,lr", [(0.25, 1e-6), (-3.75, 9.93875e-07), (123.0, 1e-3), (0.0, 1e-6)])
def test_update_matches_torch(dt, grad, lr):
    n = 20011
    th = random_theta(n, dt, 2)
    z = _z(n, dt, 12)
    p = to_torch(th, dt)
    R.zo_update([p], [to_torch(z, dt)], grad, lr)
    assert_bits_equal(A.update(th, z, grad, lr, dt), to_bits(p), dt, "update")


@pytest.mark.parametrize("dt", DTS)
def test_step_sequence_matches_torch(dt):
    """+1, -2, +1 (trainer.py:1580-1593) then update, with general (non-table) z too."""
    n = 4099
    th = random_theta(n, dt, 3)
    r = np.random.default_rng(5)
    z = from_f32(r.standard_normal(n).astype(np.float32), dt)
    z[:4] = from_f32(np.array([0.0, -0.0, 1e-30, -7e-8], np.float32), dt)
    eps, g, lr = 1e-3, -1.5, 1e-6
    p = to_torch(th, dt)
    zt = to_torch(z, dt)
    want = th
    for s in (1, -2, 1):
        R.zo_perturb_parameters([p], [zt], s, eps)
        want = A.perturb(want, z, s, eps, dt)
        assert_bits_equal(want, to_bits(p), dt, f"perturb s={s}")
    R.zo_update([p], [zt], g, lr)
    assert_bits_equal(A.update(want, z, g, lr, dt), to_bits(p), dt, "update")
    # the fused restore+update equals restore then update
    fused = A.restore_update(A.perturb(A.perturb(th, z, 1, eps, dt), z, -2, eps, dt), z, eps, g, lr, dt)
    assert_bits_equal(fused, to_bits(p), dt, "restore_update")


@pytest.mark.parametrize("dt", [F16, BF16])
def test_restore_is_not_identity(dt):
    # theta + eps z - 2 eps z + eps z != theta in 16-bit types: the drift is real
    # and must be reproduced, not repaired.
    n = 50000
    th = random_theta(n, dt, 4, with_edges=False)
    z = _z(n, dt, 99)
    back = A.perturb(A.perturb(A.perturb(th, z, 1, 1e-3, dt), z, -2, 1e-3, dt), z, 1, 1e-3, dt)
    assert np.count_nonzero(back != th) > 0


@pytest.mark.parametrize("dt", DTS)
def test_closed_forms(dt):
    th = random_theta(5000, dt, 6)
    z = _z(5000, dt)
    th_f = to_f32(th, dt)
    nz = th_f != 0
    # scale 0: the added term is a signed zero, so nonzero theta is unchanged
    # and zero theta stays zero (sign per IEEE: -0 + +0 = +0).
    out = A.perturb(th, z, 0, 1e-3, dt)
    assert np.array_equal(out[nz], th[nz])
    assert np.all(to_f32(out[~nz], dt) == 0)
    # lr 0: likewise for the update
    out2 = A.update(th, z, 1.0, 0.0, dt)
    assert np.array_equal(out2[nz], th[nz])
    assert np.all(to_f32(out2[~nz], dt) == 0)
    # eps = 1 and theta = 0 recovers z exactly
    zeros = from_f32(np.zeros(5000, np.float32), dt)
    assert np.array_equal(A.perturb(zeros, z, 1, 1.0, dt), z)
    # scale -2 doubles exactly: theta=0, eps=1 gives -2z
    assert np.array_equal(A.perturb(zeros, z, -2, 1.0, dt), from_f32(-2 * to_f32(z, dt), dt))


def test_bf16_rounding_matches_torch():
    r = np.random.default_rng(0)
    x = np.concatenate([r.standard_normal(100000).astype(np.float32) * 10.0 ** r.integers(-40, 38, 100000),
                        np.array([np.inf, -np.inf, np.nan, 0.0, -0.0, 3.3895314e38, 1e-39], np.float32)])
    x = x.astype(np.float32)
    want = to_bits(torch.from_numpy(x).to(torch.bfloat16))
    assert_bits_equal(from_f32(x, BF16), want, BF16, "bf16 rounding")
    want16 = to_bits(torch.from_numpy(x).to(torch.float16))
    assert_bits_equal(from_f32(x, F16), want16, F16, "fp16 rounding")


@pytest.mark.parametrize("dt", DTS)
def test_projected_grad_and_scalar_div(dt):
    # CPU torch divides truly; the device rule multiplies by the reciprocal of
    # the double scalar rounded to fp32. Check the device rule against its
    # definition and its closeness to the CPU rule (at most one ulp apart).
    r = np.random.default_rng(1)
    l1 = from_f32((r.random(2000) * 2).astype(np.float32), dt)
    l2 = from_f32((r.random(2000) * 2).astype(np.float32), dt)
    d = from_f32(to_f32(l1, dt) - to_f32(l2, dt), dt)
    dev = A.scalar_div_device(d, 0.002, dt).astype(np.int64)
    cpu = to_bits(to_torch(d, dt) / 0.002).astype(np.int64)
    assert np.abs(dev - cpu).max() <= 1
    want = to_f32(from_f32(to_f32(d, dt) * np.float32(500.0), dt), dt)
    assert A.projected_grad(l1[:1], l2[:1], 1e-3, dt) == float(want[0])
    # the CPU rule is torch's CPU division, bit for bit
    assert_bits_equal(A.scalar_div_cpu(d, 0.002, dt), cpu.astype(np.uint64), dt, "cpu div")
    for k in range(20):
        want_cpu = R.projected_grad(to_torch(l1[k:k + 1], dt), to_torch(l2[k:k + 1], dt), 1e-3)
        assert A.projected_grad(l1[k:k + 1], l2[k:k + 1], 1e-3, dt, rule="cpu") == want_cpu


@pytest.mark.parametrize("dt", DTS)
def test_projection_matches_torch(dt):
    r = np.random.default_rng(7)
    shapes = [(64, 64), (33, 17), (5,)]
    ths, t0s, gams = [], [], []
    for i, s in enumerate(shapes):
        n = int(np.prod(s))
        t0 = random_theta(n, dt, 10 + i, with_edges=False)
        th = from_f32(to_f32(t0, dt) + (r.standard_normal(n) * 1e-3).astype(np.float32), dt)
        ths.append(th)
        t0s.append(t0)
        gams.append(from_f32(np.array([0.9 * np.sqrt(A.group_sumsq(th, t0, dt))], np.float32), dt))
    news = [to_torch(x, dt).reshape(s) for x, s in zip(ths, shapes)]
    anchors = [to_torch(x, dt).reshape(s) for x, s in zip(t0s, shapes)]
    cons = [to_torch(g, dt) for g in gams]
    alphas = R.apply_constraints(news, anchors, cons)
    for i in range(len(shapes)):
        nt = to_bits(torch.norm(to_torch(ths[i], dt) - to_torch(t0s[i], dt)).reshape(1))
        no = A.norm_from_sumsq(A.group_sumsq(ths[i], t0s[i], dt), dt)
        assert abs(int(nt[0]) - int(no)) <= 1, (dt, i, nt, no)
        a = A.alpha(gams[i], nt, dt)
        assert_bits_equal(a, to_bits(alphas[i]), dt, "alpha")
        applied = A.apply(ths[i], t0s[i], a, dt)
        assert_bits_equal(applied, to_bits(news[i]).ravel(), dt, "apply")
    R.reverse_constraints(news, anchors, alphas)
    for i in range(len(shapes)):
        a = to_bits(alphas[i])
        back = A.reverse(A.apply(ths[i], t0s[i], a, dt), t0s[i], a, dt)
        assert_bits_equal(back, to_bits(news[i]).ravel(), dt, "reverse")


@pytest.mark.parametrize("dt", [F16, BF16, F32])
def test_norm_closed_forms(dt):
    t0 = from_f32(np.zeros(1000, np.float32), dt)
    th = from_f32(np.full(1000, 0.5, np.float32), dt)
    # ||0.5 * ones(1000)|| = 0.5 * sqrt(1000)
    n = to_f32(A.norm_from_sumsq(A.group_sumsq(th, t0, dt), dt), dt)
    assert n == to_f32(from_f32(np.float32(0.5 * np.sqrt(1000.0)), dt), dt)
    # alpha = 0 projects onto theta0 exactly; alpha = 1 gives R(R(theta - theta0) + theta0)
    zero = from_f32(np.zeros(1, np.float32), dt)
    assert np.array_equal(A.apply(th, t0, zero, dt), t0)
    one = from_f32(np.ones(1, np.float32), dt)
    r = np.random.default_rng(0)
    t0b = random_theta(1000, dt, 3, with_edges=False)
    thb = random_theta(1000, dt, 4, with_edges=False)
    want = from_f32(A.diff(thb, t0b, dt) + to_f32(t0b, dt), dt)
    assert np.array_equal(A.apply(thb, t0b, one, dt), want)


@pytest.mark.parametrize("dt", [F16, BF16, F32])
def test_gamma_iteration_matches_torch(dt):
    """One ZO gamma iteration (trainer.py:564-614) with supplied noise and losses."""
    r = np.random.default_rng(3)
    G, n = 4, 300
    t0s = [random_theta(n, dt, 20 + g, with_edges=False) for g in range(G)]
    ths = [from_f32(to_f32(t, dt) + (r.standard_normal(n) * 2e-3).astype(np.float32), dt) for t in t0s]
    zg = from_f32(r.standard_normal(G).astype(np.float32) * 3, dt)
    losses = from_f32(np.array([0.7031, 0.6875], np.float32), dt)
    news = [to_torch(x, dt) for x in ths]
    anchors = [to_torch(x, dt) for x in t0s]
    gammas = [torch.zeros(1) for _ in range(G)]
    ts_t, _, _ = R.dizo_zo_iteration(news, anchors, gammas, True, [to_torch(zg[g:g + 1], dt) for g in range(G)],
                                     lambda k: to_torch(losses[k:k + 1], dt).reshape(()))
    # oracle, vectorised over groups. Norms: the float64 oracle agrees with
    # torch.norm to one unit in the last place; the chain below takes torch's
    # norm of each intermediate theta so that everything else is pinned bitwise.
    def tnorm(th, t0):
        return to_bits(torch.norm(to_torch(th, dt) - to_torch(t0, dt)).reshape(1))[0]

    ts = np.array([A.norm_from_sumsq(A.group_sumsq(ths[g], t0s[g], dt), dt) for g in range(G)])
    for g in range(G):
        assert abs(int(ts[g]) - int(to_bits(ts_t[g].reshape(1))[0])) <= 1
    ts = np.array([tnorm(ths[g], t0s[g]) for g in range(G)])
    zc = A.clip_z(zg, ts, dt)
    gam = A.perturb_gamma(ts, zc, 1, dt)
    th1 = [A.reverse(A.apply(ths[g], t0s[g], A.alpha(gam[g:g + 1], ts[g:g + 1], dt), dt), t0s[g],
                     A.alpha(gam[g:g + 1], ts[g:g + 1], dt), dt) for g in range(G)]
    n2 = np.array([tnorm(th1[g], t0s[g]) for g in range(G)])
    gam = A.perturb_gamma(gam, zc, -2, dt)
    th2 = [A.reverse(A.apply(th1[g], t0s[g], A.alpha(gam[g:g + 1], n2[g:g + 1], dt), dt), t0s[g],
                     A.alpha(gam[g:g + 1], n2[g:g + 1], dt), dt) for g in range(G)]
    gam = A.perturb_gamma(gam, zc, 1, dt)
    gam = A.gamma_step(gam, ts, zc, losses[0:1], losses[1:2], dt, rule="cpu")
    for g in range(G):
        assert_bits_equal(gam[g:g + 1], to_bits(gammas[g].reshape(1)), dt, f"gamma {g}")
        assert_bits_equal(th2[g], to_bits(news[g]), dt, f"theta {g}")


def _tie_cases(dt, n_want=64, seed=5):
    """(value, fp32 scalar) pairs whose fp32 product lies exactly halfway between
    two neighbours in dt while the exact product does not: rounding the exact
    product once and rounding the fp32 product (to even) can differ."""
    g = np.random.default_rng(seed)
    out = []
    while len(out) < n_want:
        v = torch.tensor(g.standard_normal(1 << 16) * 40, dtype=torch.float32).to(dt)
        s = float(np.float32(g.uniform(1e-7, 2e-6)))
        exact = v.double() * s
        p32 = exact.float()
        lo = p32.to(dt)
        away = torch.where(p32 > lo.float(), torch.tensor(np.inf), torch.tensor(-np.inf)).to(dt)
        nxt = torch.nextafter(lo, away)
        mid = (lo.double() + nxt.double()) / 2
        hit = (p32.double() == mid) & (exact != p32.double()) & (lo != nxt) & torch.isfinite(nxt.float())
        for i in hit.nonzero().flatten().tolist()[:8]:
            out.append((float(v[i]), s))
    return out


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_recipe_reference_equals_torch_cpu_on_ties(dt):
    """oracle.ref_torch's recipe form (exact float64 products rounded to fp32,
    then to dt) gives torch's CPU kernels bit for bit on products whose fp32
    value is an exact tie in dt, where a single rounding of the exact product
    would differ; among them the update seen at OPT-2.7B scale, lr 9.15e-07
    times -33.90625 (a tie at -520.5 fp16 subnormal units)."""
    cases = _tie_cases(dt)
    if dt == torch.float16:
        cases.append((-33.90625, float(np.float32(9.15e-07))))
    c = torch.tensor([v for v, _ in cases], dtype=torch.float32).to(dt)
    for i, (v, s) in enumerate(cases):
        x = c[i:i + 1].clone()
        want = s * x                                     # torch's CPU kernel
        got = R._rt(x.double() * R._f32(s), dt)          # recipe
        assert torch.equal(want.view(torch.int16), got.view(torch.int16)), (v, s, float(want), float(got))


@pytest.mark.parametrize("dt", [torch.float32, torch.float16, torch.bfloat16])
def test_recipe_step_equals_torch_cpu(dt):
    """The recipe forms of the perturbation and the update equal the reference's
    expressions on torch's CPU kernels (random weights and z, several scales)."""
    g = torch.Generator().manual_seed(3)
    p = (torch.randn(50000, generator=g) * 0.02).to(dt)
    z = torch.randn(50000, generator=g).to(dt)
    for s, eps, gr, lr in ((1, 1e-3, 0.75, 1e-6), (-2, 1e-3, -51.03125, 9.15e-07), (1, 3e-4, 2.5, 1e-3)):
        a, b = [p.clone()], [p.clone()]
        R.zo_perturb_parameters(a, [z], s, eps)
        R.zo_perturb_parameters_recipe(b, [z], s, eps)
        assert torch.equal(a[0].view(BITS[dt]), b[0].view(BITS[dt]))
        R.zo_update(a, [z], gr, lr)
        R.zo_update_recipe(b, [z], gr, lr)
        assert torch.equal(a[0].view(BITS[dt]), b[0].view(BITS[dt]))


BITS = {torch.float32: torch.int32, torch.float16: torch.int16, torch.bfloat16: torch.int16}
