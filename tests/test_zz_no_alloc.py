"""The allocation-free norm pass (dz_group_sumsq_static) against the table-based
one (dz_group_sumsq), through the C ABI: sums of squares, fp32 norms and norms
in the model dtype bit for bit, on two calls in a row whose second input is
smaller (the static scratch keeps the first call's contents), with more than
64 groups (two plan launches), empty, odd-sized and misaligned tensors. In a
fresh process whose first library calls are dz_init and then the entry point,
free device memory is unchanged across the calls; inside a captured graph the
call records, and every replay gives the eager result."""
import json
import os
import subprocess
import sys
import textwrap

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
    # 262,145 chunks: one chunk too many (32,768 elements of a 16-bit type, 8,192 of fp32; no
    # allocation of that size is needed to ask)
    for dt2, chunk in ((torch.float16, 32768), (torch.bfloat16, 32768), (torch.float32, 8192)):
        t = torch.empty(8, dtype=dt2, device="cuda")
        numels = L.i64_array([chunk * 262144 + 1])
        with pytest.raises(L.DzError, match="fit the static scratch"):
            L.call("dz_group_sumsq_static", L.u64_array([t.data_ptr()]), L.u64_array([t.data_ptr()]), numels, 1,
                   dtype_code(dt2), None, None, None, None)


_FRESH = textwrap.dedent("""
    import json, sys
    sys.path.insert(0, sys.argv[1])
    import torch
    from dizo_amd import _lib as L
    from dizo_amd.table import dtype_code
    dt = torch.float16
    gen = torch.Generator().manual_seed(9)
    sizes = [70001, 1, 65536, 32768 * 3]
    th = [(torch.randn(n, generator=gen) * 0.02).to(dt).cuda() for n in sizes]
    t0 = [(t.float() + 1e-3).to(dt) for t in th]
    n = len(th)
    sumsq = torch.zeros(n, dtype=torch.float64, device="cuda")
    nf = torch.zeros(n, dtype=torch.float32, device="cuda")
    nt = torch.zeros(n, dtype=dt, device="cuda")
    args = (L.u64_array([t.data_ptr() for t in th]), L.u64_array([t.data_ptr() for t in t0]),
            L.i64_array([t.numel() for t in th]), n, dtype_code(dt), sumsq.data_ptr(), nf.data_ptr(),
            nt.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    L.call("dz_init", torch.cuda.current_device())
    torch.cuda.synchronize()
    free = [torch.cuda.mem_get_info()[0]]
    for _ in range(2):
        L.call("dz_group_sumsq_static", *args)
        torch.cuda.synchronize()
        free.append(torch.cuda.mem_get_info()[0])
    # the difference rounds to the parameter type (as param - anchor does); its square is exact in fp64
    ref = [float(((a - b).double() ** 2).sum()) for a, b in zip(th, t0)]
    print(json.dumps({"free": free, "sumsq": sumsq.tolist(), "ref": ref}))
""")


def test_first_call_after_init_allocates_nothing():
    """A fresh process: its first library calls are dz_init and two calls of
    the entry point; free device memory (hipMemGetInfo) is the same before and
    after them, and the sums are the float64 sums of the rounded differences
    (to fp64 rounding)."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    out = subprocess.run([sys.executable, "-c", _FRESH, root], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr[-2000:]
    res = json.loads([ln for ln in out.stdout.splitlines() if ln.startswith("{")][-1])
    print("free device memory before and after the calls:", res["free"], flush=True)
    assert res["free"][1] == res["free"][0] and res["free"][2] == res["free"][0], res["free"]
    for got, want in zip(res["sumsq"], res["ref"]):
        assert abs(got - want) <= 1e-12 * max(want, 1e-300), (got, want)


def test_static_call_in_a_captured_graph():
    """The entry point recorded in a hipGraph (torch.cuda.graph) after dz_init:
    the capture succeeds, and each of several replays, with eager launches on
    the inputs and synchronisations between them, gives the eager call's
    outputs bit for bit."""
    dt = torch.bfloat16
    th, t0 = _groups([50_000, 7, 32768 * 2, 1000], dt, 12, misaligned=(1,))
    L.call("dz_init", torch.cuda.current_device())
    want = _static(th, t0, dt)
    n = len(th)
    ptrs = L.u64_array([t.data_ptr() for t in th])
    anchors = L.u64_array([t.data_ptr() for t in t0])
    numels = L.i64_array([t.numel() for t in th])
    sumsq = torch.zeros(n, dtype=torch.float64, device="cuda")
    nf = torch.zeros(n, dtype=torch.float32, device="cuda")
    nt = torch.zeros(n, dtype=dt, device="cuda")
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        L.call("dz_group_sumsq_static", ptrs, anchors, numels, n, dtype_code(dt), sumsq.data_ptr(),
               nf.data_ptr(), nt.data_ptr(), torch.cuda.current_stream().cuda_stream)
    for r in range(3):
        for o in (sumsq, nf, nt):
            o.fill_(-7.0)  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for got, w, what in zip((sumsq, nf, nt), want, ("sumsq", "norm_f32", "norm_T")):
            assert torch.equal(_bits(got), _bits(w)), f"replay {r}: {what}"
    del g
