"""cwlb_spmm_mean_f32_noalloc against cwlb_spmm_mean_f32.

The allocation-free entry point (no context, status word in the library's
own device array) must give the context entry point's result on the same
inputs, to the parity tolerance, call after call: two calls in a row, the
second on a smaller problem, then error reporting and the schedule
arguments.  Everything goes through the C ABI.
"""
import numpy as np
import pytest

import oracle
from conftest import SKEWED_COSTS, UNIT_COSTS
from cwlb_amd import capi, synth, workloads

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-5, 1e-6


def _dev(torch, a):
    a = np.ascontiguousarray(a)
    if a.size == 0:
        a = np.zeros(1, a.dtype)
    return torch.from_numpy(a).cuda()


def _inputs(torch, cfg, seed, K, S, costs):
    g = workloads.small(cfg, seed=seed)
    p = workloads.prepare(g, costs, S)
    H = synth.features(g.n, K, seed)
    d = [_dev(torch, x) for x in (p.row_ptr, p.col_idx, p.val, p.origin)]
    d_t = _dev(torch, np.ascontiguousarray(p.tasks, np.int32).reshape(-1))
    return g, p, H, d, _dev(torch, H), d_t


def _both(gpu_ctx, torch, g, p, d, d_H, d_t, K, flags=0, m=0, sl=0):
    """(no-alloc result, context result) of one problem."""
    stream = torch.cuda.current_stream().cuda_stream
    C_na = torch.full((g.n, K), float("nan"), dtype=torch.float32, device="cuda")
    capi.spmm_noalloc(stream, d[0], d[1], d[2], d[3], g.n, g.nnz, d_H, g.n, K, d_t,
                      len(p.tasks), C_na, flags=flags, tasks_per_wave=m, feature_slices=sl)
    C_ctx = torch.full((g.n, K), float("nan"), dtype=torch.float32, device="cuda")
    gpu_ctx.set_schedule(m, sl)
    try:
        gpu_ctx.spmm(d[0], d[1], d[2], d[3], g.n, g.nnz, d_H, g.n, K, d_t, len(p.tasks), C_ctx,
                     flags=flags, large_k=K > 1024)
    finally:
        gpu_ctx.set_schedule(0, 0)
    return C_na.cpu().numpy(), C_ctx.cpu().numpy()


def test_noalloc_matches_context_entry_twice(gpu_ctx):
    """A larger problem, then a smaller one, on the same device array."""
    import torch
    for cfg, seed, K, S in ((4, 31, 128, 9), (1, 5, 32, 6)):
        g, p, H, d, d_H, d_t = _inputs(torch, cfg, seed, K, S, SKEWED_COSTS)
        got, want = _both(gpu_ctx, torch, g, p, d, d_H, d_t, K)
        np.testing.assert_allclose(got, want, rtol=RTOL, atol=ATOL)
        ref = oracle.spmm_mean_f32(p.row_ptr, p.col_idx, p.val, p.origin, H, p.tasks)
        np.testing.assert_allclose(got, ref, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("flags,m,sl", [(0, 8, 2), (capi.ZERO_OUTPUT, 0, 0),
                                        (capi.PER_TASK, 0, 0), (0, 64, 4),
                                        (capi.KEEP_EMPTY_ROWS, 8, 2)])
def test_noalloc_flags_and_schedule(gpu_ctx, flags, m, sl):
    import torch
    g, p, H, d, d_H, d_t = _inputs(torch, 4, 12, 64, 5, UNIT_COSTS)
    got, want = _both(gpu_ctx, torch, g, p, d, d_H, d_t, 64, flags=flags, m=m, sl=sl)
    np.testing.assert_allclose(got, want, rtol=RTOL, atol=ATOL)


def test_noalloc_large_k_and_errors(gpu_ctx):
    """K above the work-group limit, a bad column index reported (and
    cleared by the next good call), and argument errors."""
    import torch
    g, p, H, d, d_H, d_t = _inputs(torch, 1, 9, 1100, 5, UNIT_COSTS)
    got, want = _both(gpu_ctx, torch, g, p, d, d_H, d_t, 1100)
    np.testing.assert_allclose(got, want, rtol=RTOL, atol=ATOL)
    stream = torch.cuda.current_stream().cuda_stream
    C = torch.zeros((g.n, 1100), dtype=torch.float32, device="cuda")
    ci = p.col_idx.copy()
    ci[len(ci) // 2] = g.n + 3
    bad = _dev(torch, ci)
    with pytest.raises(capi.CwlbError) as e:
        capi.spmm_noalloc(stream, d[0], bad, d[2], d[3], g.n, g.nnz, d_H, g.n, 1100, d_t,
                          len(p.tasks), C)
    assert e.value.status == capi.INVALID_ARG
    capi.spmm_noalloc(stream, d[0], d[1], d[2], d[3], g.n, g.nnz, d_H, g.n, 1100, d_t,
                      len(p.tasks), C)
    np.testing.assert_allclose(C.cpu().numpy(), want, rtol=RTOL, atol=ATOL)
    for kw in ({"tasks_per_wave": -1}, {"tasks_per_wave": (1 << 20) + 1}, {"feature_slices": 3}):
        with pytest.raises(capi.CwlbError) as e:
            capi.spmm_noalloc(stream, d[0], d[1], d[2], d[3], g.n, g.nnz, d_H, g.n, 1100, d_t,
                              len(p.tasks), C, **kw)
        assert e.value.status == capi.INVALID_ARG


def test_noalloc_captured_into_a_graph(gpu_ctx):
    """The allocation-free call captured into a HIP graph and replayed, with
    eager work between the replays, gives the context entry's result on
    every replay."""
    import torch
    g, p, H, d, d_H, d_t = _inputs(torch, 4, 33, 64, 7, SKEWED_COSTS)
    _, want = _both(gpu_ctx, torch, g, p, d, d_H, d_t, 64)
    C = torch.zeros((g.n, 64), dtype=torch.float32, device="cuda")
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            capi.spmm_noalloc(side.cuda_stream, d[0], d[1], d[2], d[3], g.n, g.nnz, d_H, g.n,
                              64, d_t, len(p.tasks), C, synchronize=False)
    torch.cuda.synchronize()
    for i in range(3):
        C.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        np.testing.assert_allclose(C.cpu().numpy(), want, rtol=RTOL, atol=ATOL)
        _ = (d_H * 2.0).sum().item()  # eager work between replays


def test_noalloc_synchronize_refused_under_capture(gpu_ctx):
    """Under graph capture, a call that asks to synchronise (read the status
    word back and wait) is refused with CWLB_INVALID_ARG before anything is
    enqueued: the capture stays valid, and the call captured after it with
    synchronize=False replays to the context entry's result."""
    import torch
    g, p, H, d, d_H, d_t = _inputs(torch, 4, 35, 64, 7, SKEWED_COSTS)
    _, want = _both(gpu_ctx, torch, g, p, d, d_H, d_t, 64)
    C = torch.zeros((g.n, 64), dtype=torch.float32, device="cuda")
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    status = None
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            try:
                capi.spmm_noalloc(side.cuda_stream, d[0], d[1], d[2], d[3], g.n, g.nnz, d_H,
                                  g.n, 64, d_t, len(p.tasks), C, synchronize=True)
            except capi.CwlbError as e:
                status, msg = e.status, str(e)
            capi.spmm_noalloc(side.cuda_stream, d[0], d[1], d[2], d[3], g.n, g.nnz, d_H, g.n,
                              64, d_t, len(p.tasks), C, synchronize=False)
    assert status == capi.INVALID_ARG and "graph capture" in msg
    torch.cuda.synchronize()
    for _ in range(2):
        C.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        np.testing.assert_allclose(C.cpu().numpy(), want, rtol=RTOL, atol=ATOL)
