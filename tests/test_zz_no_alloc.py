"""The allocation-free norm pass (dz_group_sumsq_static) against the table-based
one (dz_group_sumsq), through the C ABI: sums of squares, fp32 norms and norms
in the model dtype bit for bit, on two calls in a row whose second input is
smaller (the static scratch keeps the first call's contents), with more than
64 groups (two plan launches), empty, odd-sized and misaligned tensors."""
import numpy as np
import pytest
import torch

from dizo_amd import _lib as L
from dizo_amd.table import ProjTable, dtype_code

pytestmark = pytest.mark.gpu


def _groups(sizes, dt, seed, misaligned=()):
    gen = torch.Generator().manual_seed(seed)
    th, t0 = [], []
    for i, n in enumerate(sizes):
        extra = 1 if i in misaligned else 0
        a = (torch.randn(n + extra, generator=gen) * 0.02).to(dt).cuda()
        b = (a.float() + 1e-3 * torch.randn(n + extra, generator=gen).cuda()).to(dt)
        th.append(a[extra:])
        t0.append(b[extra:])
    return th, t0


def _static(th, t0, dt):
    n = len(th)
    ptrs = L.u64_array([t.data_ptr() for t in th])
    anchors = L.u64_array([t.data_ptr() for t in t0])
    numels = L.i64_array([t.numel() for t in th])
    sumsq = torch.full((n,), -1.0, dtype=torch.float64, device="cuda")
    nf = torch.full((n,), -1.0, dtype=torch.float32, device="cuda")
    nt = torch.full((n,), -1.0, dtype=dt, device="cuda")
    L.call("dz_group_sumsq_static", ptrs, anchors, numels, n, dtype_code(dt), sumsq.data_ptr(), nf.data_ptr(),
           nt.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return sumsq, nf, nt


def _table(th, t0, dt):
    n = len(th)
    tab = ProjTable(th, t0)
    sumsq = torch.empty(n, dtype=torch.float64, device="cuda")
    nf = torch.empty(n, dtype=torch.float32, device="cuda")
    nt = torch.empty(n, dtype=dt, device="cuda")
    tab.group_sumsq(sumsq=sumsq, norm_f32=nf, norm_T=nt)
    torch.cuda.synchronize()
    tab.close()
    return sumsq, nf, nt


def _bits(t):
    return t.view({8: torch.int64, 4: torch.int32, 2: torch.int16}[t.element_size()]).cpu()


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32])
def test_static_norms_equal_table_norms_two_calls(dt):
    rng = np.random.default_rng(11)
    big = [int(x) for x in rng.integers(1, 200_000, size=70)]
    big[3], big[10], big[40] = 0, 32768, 32768 * 5 + 1
    small = [70_001, 1, 65_536]
    for sizes, seed, mis in ((big, 1, (7, 65)), (small, 2, (0,))):
        th, t0 = _groups(sizes, dt, seed, misaligned=mis)
        got = _static(th, t0, dt)
        want = _table(th, t0, dt)
        for g, w, what in zip(got, want, ("sumsq", "norm_f32", "norm_T")):
            assert torch.equal(_bits(g), _bits(w)), f"{what} differs for {len(sizes)} groups"
        assert float(got[0][3 if len(sizes) > 3 else 0]) >= 0.0


def test_static_rejects_more_than_the_scratch_holds():
    dt = torch.float16
    th, t0 = _groups([8], dt, 3)
    ptrs = L.u64_array([th[0].data_ptr()] * 4097)
    anchors = L.u64_array([t0[0].data_ptr()] * 4097)
    numels = L.i64_array([8] * 4097)
    with pytest.raises(L.DzError, match="group count"):
        L.call("dz_group_sumsq_static", ptrs, anchors, numels, 4097, dtype_code(dt), None, None, None, None)
    # 262,145 chunks: one 32,768-element chunk too many (a 16 GiB allocation is not needed to ask)
    t = torch.empty(8, dtype=dt, device="cuda")
    numels = L.i64_array([32768 * 262144 + 1])
    with pytest.raises(L.DzError, match="fit the static scratch"):
        L.call("dz_group_sumsq_static", L.u64_array([t.data_ptr()]), L.u64_array([t.data_ptr()]), numels, 1,
               dtype_code(dt), None, None, None, None)
