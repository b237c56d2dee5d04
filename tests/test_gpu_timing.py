"""Kernel-stamped timing events (dz_table_time_next, KernelTimer spans with
tables): the events bracket the library's kernels, and asking for them changes
nothing in what the kernels compute."""
import pytest
import torch

from dizo_amd import _lib as L
from dizo_amd.table import ProjTable, ZOTable
from dizo_amd.timing import KernelTimer

pytestmark = pytest.mark.gpu


def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.contiguous().view({2: torch.int16, 4: torch.int32}[t.element_size()])


def _tensors(dtype, sizes, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return [torch.randn(n, generator=g, device="cuda", dtype=torch.float32).to(dtype) for n in sizes]


def _created_events():
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    e1.record()
    return e0, e1


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_kernel_events_bracket_the_kernel_and_change_nothing(dtype):
    sizes = [1 << 23, 4097, 3, 1 << 20]
    plain = _tensors(dtype, sizes, 1)
    timed = [t.clone() for t in plain]
    tp, tt = ZOTable(plain), ZOTable(timed)
    for tab in (tp, tt):
        tab.perturb(11, 1.0, 1e-3)
    torch.cuda.synchronize()
    kernel_ms, host_ms = [], []
    for rep in range(3):
        tp.restore_update_perturb(11 + rep, 12 + rep, 1e-3, 0.75, 1e-2)
        torch.cuda.synchronize()
        e0, e1 = _created_events()
        h0, h1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        tt.time_next(e0, e1)
        h0.record()
        tt.restore_update_perturb(11 + rep, 12 + rep, 1e-3, 0.75, 1e-2)
        h1.record()
        torch.cuda.synchronize()
        kernel_ms.append(e0.elapsed_time(e1))
        host_ms.append(h0.elapsed_time(h1))
    for a, b in zip(plain, timed):
        assert torch.equal(_bits(a), _bits(b))
    print(f"{dtype}: kernel events {kernel_ms} ms, host-bracketed {host_ms} ms")
    for k, h in zip(kernel_ms, host_ms):
        assert 0 < k <= h * 1.02 + 2e-3
    tp.close()
    tt.close()


def test_kernel_events_on_projection_calls():
    dtype = torch.float16
    sizes = [1 << 21, 5000, 1 << 16]
    th = _tensors(dtype, sizes, 2)
    t0 = [(t.float() + 1e-2).to(dtype) for t in th]
    th_b = [t.clone() for t in th]
    pa, pb = ProjTable(th, t0), ProjTable(th_b, t0)
    G = len(sizes)
    alpha = torch.full((G,), 0.875, dtype=dtype, device="cuda")
    others = _tensors(dtype, sizes, 3)
    outs = {}
    for name, tab in (("plain", pa), ("timed", pb)):
        res = []
        calls = [
            lambda n: tab.group_sumsq(norm_T=n),
            lambda n: tab.project(alpha, L.DZ_PROJ_APPLY),
            lambda n: tab.project(alpha, L.DZ_PROJ_REVERSE_SUMSQ, norm_T=n),
            lambda n: tab.group_dot(others, dot=n),
        ]
        for call in calls:
            n = torch.zeros(G, dtype=torch.float64 if call is calls[3] else dtype, device="cuda")
            if name == "timed":
                e0, e1 = _created_events()
                tab.time_next(e0, e1)
                call(n)
                torch.cuda.synchronize()
                assert e0.elapsed_time(e1) > 0
            else:
                call(n)
            res.append(n.clone())
        torch.cuda.synchronize()
        outs[name] = res
    for a, b in zip(outs["plain"], outs["timed"]):
        assert torch.equal(a, b)
    for a, b in zip(th, th_b):
        assert torch.equal(_bits(a), _bits(b))
    pa.close()
    pb.close()


def test_timer_span_over_two_tables():
    """A span over two tables takes its start from the first table's kernel
    and its end from the last table's; the interval covers both launches."""
    a = _tensors(torch.float16, [1 << 22], 4)
    b = _tensors(torch.float32, [1 << 21], 5)
    ta, tb = ZOTable(a), ZOTable(b)
    timer = KernelTimer()
    for _ in range(2):
        with timer.span("both", 1, [ta, tb]):
            ta.perturb(7, 1.0, 1e-3)
            tb.perturb(7, 1.0, 1e-3)
        torch.cuda.synchronize()
        with timer.span("first", 1, [ta]):
            ta.perturb(7, 1.0, 1e-3)
        torch.cuda.synchronize()
    s = timer.summary()
    assert s["both"]["mean_ms"] > s["first"]["mean_ms"] > 0
    ta.close()
    tb.close()


def test_time_next_rejects_events_that_do_not_exist_yet():
    t = ZOTable(_tensors(torch.float16, [1024], 6))
    e = torch.cuda.Event(enable_timing=True)
    with pytest.raises(L.DzError):
        t.time_next(e, None)
    t.close()


def test_calls_with_nothing_to_launch_record_their_events():
    """A table of empty tensors launches no kernel; the requested events are
    then recorded on the stream at the call (elapsed time about zero, after
    a slow kernel queued before it)."""
    z = ZOTable([torch.empty(0, dtype=torch.float16, device="cuda")])
    e = torch.empty(0, dtype=torch.float16, device="cuda")
    p = ProjTable([e], [e.clone()])
    alpha = torch.ones(1, dtype=torch.float16, device="cuda")
    big = torch.randn(1 << 26, device="cuda")
    for call, tab in ((lambda: z.perturb(3, 1.0, 1e-3), z), (lambda: p.project(alpha, L.DZ_PROJ_APPLY), p)):
        torch.cuda.synchronize()
        e0, e1 = _created_events()
        torch.cuda.synchronize()
        tab.time_next(e0, e1)
        before = torch.cuda.Event(enable_timing=True)
        before.record()
        big.mul_(1.0)  # device work queued before the call
        call()
        torch.cuda.synchronize()
        assert before.elapsed_time(e0) > 0  # recorded at the call, after the queued work
        assert 0 <= e0.elapsed_time(e1) < 0.05
    z.close()
    p.close()
