"""GPU parity of the DiZO projection kernels (group norms, apply, reverse)."""
import numpy as np
import pytest
import torch

from oracle import arith as A
from oracle import ref_torch as R
from oracle.arith import BF16, F16, F32, from_f32, to_f32

from tests._util import DT_TORCH, assert_bits_equal, random_theta, to_bits, to_torch

pytestmark = pytest.mark.gpu

DTS = [F16, BF16, F32]
# around the projection chunk (32768 elements) and its multiples, tiny, ragged and many-chunk groups
SIZES = [32768, 32767, 32769, 5, 64 * 64 * 5 + 3, 300000, 65536 + 8, 8191]


def _groups(dt, seed, sizes=SIZES, rel=1e-2):
    dev = torch.device("cuda", 0)
    r = np.random.default_rng(seed)
    th_h, t0_h = [], []
    for i, n in enumerate(sizes):
        t0 = random_theta(n, dt, seed + i, with_edges=False)
        th = from_f32(to_f32(t0, dt) + (r.standard_normal(n) * 0.02 * rel).astype(np.float32), dt)
        th_h.append(th)
        t0_h.append(t0)
    ths = [to_torch(x, dt, dev) for x in th_h]
    t0s = [to_torch(x, dt, dev) for x in t0_h]
    return ths, t0s, th_h, t0_h


@pytest.mark.parametrize("dt", DTS)
def test_group_norms(dt):
    from dizo_amd.table import ProjTable
    ths, t0s, th_h, t0_h = _groups(dt, 1)
    tab = ProjTable(ths, t0s)
    G = len(ths)
    dev = ths[0].device
    sumsq = torch.empty(G, dtype=torch.float64, device=dev)
    nf = torch.empty(G, dtype=torch.float32, device=dev)
    nt = torch.empty(G, dtype=DT_TORCH[dt], device=dev)
    tab.group_sumsq(sumsq, nf, nt)
    for g in range(G):
        want = A.group_sumsq(th_h[g], t0_h[g], dt)
        assert float(sumsq[g]) == pytest.approx(want, rel=1e-12)
        n_or = A.norm_from_sumsq(want, dt)
        assert abs(int(to_bits(nt[g:g + 1])[0]) - int(n_or)) <= 1
        # and within one ulp of torch.norm on the device (what the reference computes)
        tn = to_bits(torch.norm(ths[g] - t0s[g]).reshape(1))[0]
        assert abs(int(to_bits(nt[g:g + 1])[0]) - int(tn)) <= 1
    tab.close()


@pytest.mark.parametrize("dt", DTS)
def test_apply_reverse_match_oracle(dt):
    from dizo_amd._lib import DZ_PROJ_APPLY, DZ_PROJ_REVERSE, DZ_PROJ_REVERSE_SUMSQ
    from dizo_amd.table import ProjTable
    ths, t0s, th_h, t0_h = _groups(dt, 5)
    tab = ProjTable(ths, t0s)
    G = len(ths)
    dev = ths[0].device
    alphas = from_f32(np.linspace(0.85, 1.1, G).astype(np.float32), dt)
    alpha_t = to_torch(alphas, dt, dev)
    tab.project(alpha_t, DZ_PROJ_APPLY)
    app = [A.apply(th_h[g], t0_h[g], alphas[g:g + 1], dt) for g in range(G)]
    for g in range(G):
        assert_bits_equal(to_bits(ths[g]), app[g], dt, f"apply group {g}")
    sumsq = torch.empty(G, dtype=torch.float64, device=dev)
    nt = torch.empty(G, dtype=DT_TORCH[dt], device=dev)
    tab.project(alpha_t, DZ_PROJ_REVERSE_SUMSQ, sumsq=sumsq, norm_T=nt)
    rev = [A.reverse(app[g], t0_h[g], alphas[g:g + 1], dt) for g in range(G)]
    for g in range(G):
        assert_bits_equal(to_bits(ths[g]), rev[g], dt, f"reverse group {g}")
        want = A.group_sumsq(rev[g], t0_h[g], dt)
        assert float(sumsq[g]) == pytest.approx(want, rel=1e-12)
    # the fused norms equal a standalone norm pass over the same theta
    s2 = torch.empty(G, dtype=torch.float64, device=dev)
    tab.group_sumsq(s2)
    assert torch.equal(sumsq, s2)
    tab.project(alpha_t, DZ_PROJ_REVERSE)
    rev2 = [A.reverse(rev[g], t0_h[g], alphas[g:g + 1], dt) for g in range(G)]
    for g in range(G):
        assert_bits_equal(to_bits(ths[g]), rev2[g], dt, f"reverse2 group {g}")
    tab.close()


@pytest.mark.parametrize("dt", DTS)
def test_apply_reverse_match_torch_on_device(dt):
    """apply_constraints / reverse_constraints of the reference run by ROCm torch."""
    from dizo_amd._lib import DZ_PROJ_APPLY, DZ_PROJ_REVERSE
    from dizo_amd.table import ProjTable
    ths, t0s, th_h, t0_h = _groups(dt, 9, sizes=[32768, 4099, 70000])
    ref = [t.clone() for t in ths]
    G = len(ths)
    gammas = [0.9 * torch.norm(ths[g] - t0s[g]) for g in range(G)]
    alphas = R.apply_constraints(ref, t0s, gammas)
    alpha_t = torch.stack([a.reshape(()) for a in alphas]).contiguous()
    tab = ProjTable(ths, t0s)
    tab.project(alpha_t, DZ_PROJ_APPLY)
    for g in range(G):
        assert_bits_equal(to_bits(ths[g]), to_bits(ref[g]), dt, f"apply group {g}")
    R.reverse_constraints(ref, t0s, alphas)
    tab.project(alpha_t, DZ_PROJ_REVERSE)
    for g in range(G):
        assert_bits_equal(to_bits(ths[g]), to_bits(ref[g]), dt, f"reverse group {g}")
    tab.close()


def test_empty_and_rejects():
    from dizo_amd._lib import DZ_PROJ_APPLY, DzError
    from dizo_amd.table import ProjTable
    dev = torch.device("cuda", 0)
    a = [torch.zeros(0, device=dev), torch.ones(10, device=dev)]
    b = [torch.zeros(0, device=dev), torch.zeros(10, device=dev)]
    tab = ProjTable(a, b)
    s = torch.empty(2, dtype=torch.float64, device=dev)
    tab.group_sumsq(s)
    assert s.tolist() == [0.0, 10.0]
    with pytest.raises(DzError):
        tab.project(torch.ones(3, device=dev), DZ_PROJ_APPLY)  # wrong alpha length
    with pytest.raises(DzError):
        ProjTable(a, [torch.zeros(0, device=dev), torch.zeros(11, device=dev)])
    tab.close()
    # a written tensor may not overlap another tensor or any anchor; anchors may be shared
    base = torch.zeros(40, device=dev)
    anchor = torch.zeros(10, device=dev)
    with pytest.raises(DzError, match="overlaps"):
        ProjTable([base[:10], base[5:15]], [anchor, anchor])
    with pytest.raises(DzError, match="overlaps"):
        ProjTable([base[:10], base[10:20]], [anchor, base[15:25]])
    with pytest.raises(DzError, match="overlaps"):
        ProjTable([base[:10]], [base[:10]])
    ProjTable([base[:10], base[10:20]], [anchor, anchor]).close()


@pytest.mark.parametrize("dt", DTS)
def test_apply_f32_alpha_matches_torch(dt):
    """APPLY_F32ALPHA: the reference's apply with an fp32 gamma (first-order path):
    (theta - theta0) * alpha + theta0 with alpha float32 of shape (1,), copied into T."""
    from dizo_amd._lib import DZ_PROJ_APPLY_F32ALPHA
    from dizo_amd.table import ProjTable
    ths, t0s, _, _ = _groups(dt, 13, sizes=[32768, 4099, 70000, 7, 32769])
    ref = [t.clone() for t in ths]
    G = len(ths)
    alphas = torch.tensor(np.linspace(0.5, 1.3, G), dtype=torch.float32, device=ths[0].device)
    tab = ProjTable(ths, t0s)
    tab.project(alphas, DZ_PROJ_APPLY_F32ALPHA)
    for g in range(G):
        want = ((ref[g] - t0s[g]) * alphas[g:g + 1] + t0s[g]).to(DT_TORCH[dt])
        assert_bits_equal(to_bits(ths[g]), to_bits(want), dt, f"apply_f32 group {g}")
    tab.close()


@pytest.mark.parametrize("dt", DTS)
def test_group_dot_matches_fp64(dt):
    """group_dot: sum fp32(other) * fp32(R(theta - theta0)) per group, fp64 accumulation,
    against the same sum formed in float64 by torch (up to summation order)."""
    from dizo_amd.table import ProjTable
    ths, t0s, _, _ = _groups(dt, 21, sizes=[32768, 32767, 300000, 5, 0, 8191])
    gen = torch.Generator(device="cuda").manual_seed(5)
    others = [torch.randn(t.numel(), device=t.device, generator=gen).to(DT_TORCH[dt]) for t in ths]
    G = len(ths)
    dot = torch.empty(G, dtype=torch.float64, device=ths[0].device)
    dotf = torch.empty(G, dtype=torch.float32, device=ths[0].device)
    tab = ProjTable(ths, t0s)
    tab.group_dot(others, dot, dotf)
    for g in range(G):
        delta = (ths[g] - t0s[g]).double()
        want = float((others[g].double() * delta).sum())
        assert float(dot[g]) == pytest.approx(want, rel=1e-12, abs=1e-300)
        assert float(dotf[g]) == np.float32(float(dot[g]))
    tab.close()


def test_group_dot_more_groups_than_one_launch_takes():
    """200 groups (more than the 128 one dot launch takes): every group's sum
    against float64 torch, including empty groups at a batch boundary."""
    from dizo_amd.table import ProjTable
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(6)
    sizes = [(1000 + 37 * i) if i not in (127, 128) else 0 for i in range(200)]
    ths = [(torch.randn(n, device=dev, generator=gen) * 0.02).half() for n in sizes]
    t0s = [(t.float() - 1e-3).half() for t in ths]
    others = [torch.randn(n, device=dev, generator=gen).half() for n in sizes]
    dot = torch.empty(200, dtype=torch.float64, device=dev)
    tab = ProjTable(ths, t0s)
    tab.group_dot(others, dot)
    for g in range(200):
        want = float((others[g].double() * (ths[g] - t0s[g]).double()).sum())
        assert float(dot[g]) == pytest.approx(want, rel=1e-12, abs=1e-300), g
    tab.close()


@pytest.mark.parametrize("dt", [F16, F32])
def test_more_groups_than_the_lds_alpha_table(dt):
    """More groups (4100) than a projection workgroup keeps alphas for in LDS
    (4096): each chunk then reads its group's alpha from memory. Apply, reverse
    and the group norms against the oracle, on views of one buffer."""
    from dizo_amd._lib import DZ_PROJ_APPLY, DZ_PROJ_REVERSE_SUMSQ
    from dizo_amd.table import ProjTable
    G, n = 4100, 37
    dev = torch.device("cuda", 0)
    r = np.random.default_rng(3)
    t0_all = random_theta(G * n, dt, 7, with_edges=False)
    th_all = from_f32(to_f32(t0_all, dt) + (r.standard_normal(G * n) * 2e-4).astype(np.float32), dt)
    th_buf, t0_buf = to_torch(th_all, dt, dev), to_torch(t0_all, dt, dev)
    ths = [th_buf[g * n:(g + 1) * n] for g in range(G)]
    t0s = [t0_buf[g * n:(g + 1) * n] for g in range(G)]
    alphas = from_f32(np.linspace(0.6, 1.2, G).astype(np.float32), dt)
    tab = ProjTable(ths, t0s)
    tab.project(to_torch(alphas, dt, dev), DZ_PROJ_APPLY)
    got = to_bits(th_buf)
    want = np.concatenate([A.apply(th_all[g * n:(g + 1) * n], t0_all[g * n:(g + 1) * n], alphas[g:g + 1], dt)
                           for g in range(G)])
    assert_bits_equal(got, want, dt, "apply")
    sumsq = torch.empty(G, dtype=torch.float64, device=dev)
    tab.project(to_torch(alphas, dt, dev), DZ_PROJ_REVERSE_SUMSQ, sumsq=sumsq)
    rev = [A.reverse(want[g * n:(g + 1) * n], t0_all[g * n:(g + 1) * n], alphas[g:g + 1], dt) for g in range(G)]
    assert_bits_equal(to_bits(th_buf), np.concatenate(rev), dt, "reverse")
    s = sumsq.cpu().numpy()
    for g in range(0, G, 97):
        assert s[g] == pytest.approx(A.group_sumsq(rev[g], t0_all[g * n:(g + 1) * n], dt), rel=1e-12), g
    tab.close()


def _edge_alphas(dt):
    """Alphas across the range: subnormal ones (for bf16, 1 / alpha overflows
    below 2^-128), the smallest normal, tiny, typical, huge and negative
    values, and random ratios near 1."""
    r = np.random.default_rng(17)
    vals = [2.0 ** -126, 2.0 ** -100, 2.0 ** -64, 1e-8, 1e-3, 0.5, 0.9, 1.0, 1.1, 2.0, 3.0, 7.0, 1e3, 2.0 ** 60,
            -0.75, -3.0] + list(r.uniform(0.5, 2.0, 16))
    bits = [int(b) for b in from_f32(np.array(vals, dtype=np.float32), dt)]
    if dt == BF16:
        bits += [0x0001, 0x0040, 0x007f, 0x0080, 0x7f7f]  # subnormals, min normal, max
    else:
        bits += [0x0001, 0x0200, 0x03ff, 0x0400, 0x7bff]
    out = []
    for b in bits:
        v = float(to_f32(np.array([b], dtype=A.BITS_DTYPE[dt]), dt)[0])
        if v != 0 and np.isfinite(v) and b not in out:
            out.append(b)
    return np.array(out, dtype=A.BITS_DTYPE[dt])


@pytest.mark.parametrize("dt", [BF16, F16])
def test_reverse_every_dividend_matches_oracle(dt):
    """reverse and reverse+norm with theta0 = 0 and theta running through all
    65536 16-bit patterns (inf, NaN, subnormals and zeros included), so the
    quotient R_T(R_T(theta - theta0) / alpha) meets every dividend, for ~40
    alphas from subnormal to huge: bit for bit against the oracle's IEEE
    division (the bf16 kernel divides by multiplying with fp32(1 / alpha),
    falling back to the division where that could round differently)."""
    from dizo_amd._lib import DZ_PROJ_REVERSE, DZ_PROJ_REVERSE_SUMSQ
    from dizo_amd.table import ProjTable
    dev = torch.device("cuda", 0)
    alphas = _edge_alphas(dt)
    G = len(alphas)
    every = np.arange(65536, dtype=np.uint32).astype(A.BITS_DTYPE[dt])
    zeros = np.zeros(65536, dtype=A.BITS_DTYPE[dt])
    ths = [to_torch(every, dt, dev) for _ in range(G)]
    t0s = [to_torch(zeros, dt, dev) for _ in range(G)]
    tab = ProjTable(ths, t0s)
    alpha_t = to_torch(alphas, dt, dev)
    for mode, what in ((DZ_PROJ_REVERSE, "reverse"), (DZ_PROJ_REVERSE_SUMSQ, "reverse+norm")):
        for t in ths:
            t.copy_(to_torch(every, dt, dev))
        if mode == DZ_PROJ_REVERSE_SUMSQ:
            sumsq = torch.empty(G, dtype=torch.float64, device=dev)
            tab.project(alpha_t, mode, sumsq=sumsq)
        else:
            tab.project(alpha_t, mode)
        for g in range(G):
            want = A.reverse(every, zeros, alphas[g:g + 1], dt)
            assert_bits_equal(to_bits(ths[g]), want, dt, f"{what}, alpha bits {hex(int(alphas[g]))}")
    tab.close()
