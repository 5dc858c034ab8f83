"""Reductions (and, in the last test, the long-row softmax, a split-K GEMM
and the MLP step) captured into a HIP graph and replayed.

A flat reduction's writers tag their partials with a per-call tag that a
graph replays unchanged, so a call made under stream capture has its reader
clear every slot it consumed; the no-allocation entry point (meant for such
callers) always does.  Each replay here runs on new input data, with eager
reductions of other shapes on the same stream between the replays, and must
give the bits an eager call gives on that data.  The captured launches
record kernels only: the regions they use exist before capture starts (an
eager call first), so no allocation or memset is captured."""
import ctypes

import numpy as np
import pytest

from cortexmind_amd._lib import call
from cortexmind_amd.data import SplitMix64
from cortexmind_amd.device import DeviceArray, Stream

pytestmark = pytest.mark.gpu

CAPTURE_RELAXED = 2


def hip_rt():
    h = ctypes.CDLL("libamdhip64.so.7")
    for name, args in {
        "hipStreamBeginCapture": [ctypes.c_void_p, ctypes.c_int],
        "hipStreamEndCapture": [ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)],
        "hipGraphInstantiate": [ctypes.POINTER(ctypes.c_void_p), ctypes.c_void_p, ctypes.c_void_p,
                                ctypes.c_char_p, ctypes.c_size_t],
        "hipGraphLaunch": [ctypes.c_void_p, ctypes.c_void_p],
        "hipGraphExecDestroy": [ctypes.c_void_p],
        "hipGraphDestroy": [ctypes.c_void_p],
    }.items():
        getattr(h, name).argtypes = args
        getattr(h, name).restype = ctypes.c_int
    return h


def capture(h, stream, fn):
    assert h.hipStreamBeginCapture(stream.handle, CAPTURE_RELAXED) == 0
    fn()
    graph = ctypes.c_void_p()
    assert h.hipStreamEndCapture(stream.handle, ctypes.byref(graph)) == 0
    exe = ctypes.c_void_p()
    assert h.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
    return graph, exe


@pytest.mark.parametrize("entry,sizes", [
    ("cxm_reduce_sum_flat_f32", (1 << 24,)),
    ("cxm_reduce_mean_flat_f32", (1000003,)),
    ("cxm_reduce_max_flat_f32", (1 << 22,)),
    ("cxm_reduce_sum_noalloc_f32", (1, 1 << 24, 1)),
    ("cxm_reduce_sum_noalloc_f32", (3, 500000, 1)),
    ("cxm_reduce_sum_f32", (1, 4096, 4096)),
    ("cxm_reduce_max_f32", (2, 3000, 512)),
])
def test_replays_match_eager(hip, entry, sizes):
    h = hip_rt()
    s = Stream()
    n = int(np.prod(sizes))
    n_out = 1 if len(sizes) == 1 else sizes[0] * sizes[2]
    dx = DeviceArray((n,), np.float32)
    dz = DeviceArray((n_out,), np.float32)
    other_x = DeviceArray((1 << 20,), np.float32)
    other_z = DeviceArray((256,), np.float32)
    g = SplitMix64(0x6A + n)
    other_x.upload(g.uniform((1 << 20,), -1.0, 1.0))

    def run():
        call(entry, dx.ptr, dz.ptr, *sizes, s.handle)

    dx.upload(g.uniform((n,), -1.0, 1.0))
    run()  # the regions exist before capture
    s.sync()
    graph, exe = capture(h, s, run)
    try:
        for rep in range(4):
            x = g.uniform((n,), -1.0, 1.0)
            dx.upload(x)
            run()  # eager reference on this data
            want = dz.numpy(s).copy()
            dz.fill_bytes(0xFF, s)
            assert h.hipGraphLaunch(exe, s.handle) == 0
            got = dz.numpy(s)
            assert got.tobytes() == want.tobytes(), (entry, rep)
            # eager reductions of other shapes on the same stream between replays
            call("cxm_reduce_sum_flat_f32", other_x.ptr, other_z.ptr, (1 << 20) - 5 * rep, s.handle)
            call("cxm_reduce_sum_noalloc_f32", other_x.ptr, other_z.ptr, 1, (1 << 19) + rep, 1, s.handle)
            call("cxm_reduce_max_f32", other_x.ptr, other_z.ptr, 16, 1 << 16, 1, s.handle)
            call("cxm_reduce_sum_f32", other_x.ptr, other_z.ptr, 1, 4096 - 16 * rep, 256, s.handle)
            s.sync()
    finally:
        h.hipGraphExecDestroy(exe)
        h.hipGraphDestroy(graph)
        s.close()


def _wait_limit(polls):
    old = ctypes.c_uint(0)
    call("cxm_exchange_wait_limit", polls, ctypes.byref(old))
    return old.value


@pytest.mark.parametrize("entry,sizes", [
    ("cxm_reduce_sum_flat_f32", (1 << 24,)),
    ("cxm_reduce_sum_noalloc_f32", (1, 1 << 24, 1)),
])
def test_replays_after_missed_slots(hip, entry, sizes):
    """Captured with a wait limit of 0, the reader gives up on every slot
    not yet written when it looks and recomputes that partial; the late
    writer's slot must not survive into the next replay, which reuses the
    captured tag (it would be taken for that replay's partial).  Every
    replay, on new data, gives the bits of an eager call."""
    h = hip_rt()
    s = Stream()
    n = int(np.prod(sizes))
    dx = DeviceArray((n,), np.float32)
    dz = DeviceArray((1,), np.float32)
    g = SplitMix64(0x6B + n)

    def run():
        call(entry, dx.ptr, dz.ptr, *sizes, s.handle)

    dx.upload(g.uniform((n,), -1.0, 1.0))
    run()
    s.sync()
    old = _wait_limit(0)
    try:
        graph, exe = capture(h, s, run)
    finally:
        _wait_limit(old)
    try:
        # eager results first: an eager call between replays would overwrite
        # every slot with its own tag and hide a stale one
        xs = [g.uniform((n,), -1.0, 1.0) for _ in range(6)]
        wants = []
        for x in xs:
            dx.upload(x)
            run()  # default wait limit
            wants.append(dz.numpy(s).copy())
        for rep, x in enumerate(xs):
            dx.upload(x)
            dz.fill_bytes(0xFF, s)
            assert h.hipGraphLaunch(exe, s.handle) == 0
            got = dz.numpy(s)
            assert got.tobytes() == wants[rep].tobytes(), (entry, rep, got, wants[rep])
            s.sync()
    finally:
        h.hipGraphExecDestroy(exe)
        h.hipGraphDestroy(graph)
        s.close()


def test_capture_softmax_gemm_mlp_step(hip):
    """The long-row softmax (its row exchange keeps a device-side epoch),
    a split-K weight-gradient GEMM (ticket counters) and the full C5 MLP step
    (fused head, split-K SGD epilogues) captured into one graph and replayed
    on new inputs: every replay gives the eager bits."""
    from cortexmind_amd.data import c5_mlp
    from cortexmind_amd import engine

    h = hip_rt()
    s = Stream()
    g = SplitMix64(0x6C)
    R, C = 64, 131072
    sx, sy, sg, sdx = (DeviceArray((R * C,), np.float32) for _ in range(4))
    M, K, N = 1024, 4096, 1024
    ga, gb, gc = DeviceArray((K * M,), np.float32), DeviceArray((K * N,), np.float32), DeviceArray((M * N,), np.float32)
    x, labels, params0 = c5_mlp()
    net = engine.Mlp3(x.shape[0], 784, 1024, 1024, 10)
    dx_m, dlab, dloss = DeviceArray.from_numpy(x), DeviceArray.from_numpy(labels), DeviceArray((1,), np.float32)
    dp = {k: DeviceArray.from_numpy(v) for k, v in params0.items()}

    def run():
        call("cxm_softmax_fwd_f32", sx.ptr, sy.ptr, R, C, 0, s.handle)
        call("cxm_softmax_bwd_f32", sy.ptr, sg.ptr, sdx.ptr, R, C, 0, s.handle)
        call("cxm_gemm_f32", ga.ptr, gb.ptr, gc.ptr, M, K, N, 1, 0, None, 0, None, s.handle)
        net.step(dx_m, dlab, dp, 0.01, dloss, s)

    def new_inputs():
        sx.upload(g.uniform((R * C,), -4.0, 4.0))
        sg.upload(g.uniform((R * C,), -1.0, 1.0))
        ga.upload(g.uniform((K * M,), -1.0, 1.0))
        gb.upload(g.uniform((K * N,), -1.0, 1.0))
        dx_m.upload(g.uniform(x.shape, -1.0, 1.0))
        for k, v in params0.items():
            dp[k].upload(v)

    def outputs():
        outs = [sy.numpy(s), sdx.numpy(s), gc.numpy(s), dloss.numpy(s)]
        return outs + [dp[k].numpy(s) for k in sorted(dp)]

    new_inputs()
    run()  # the workspaces exist before capture
    s.sync()
    graph, exe = capture(h, s, run)
    try:
        for rep in range(3):
            new_inputs()
            assert h.hipGraphLaunch(exe, s.handle) == 0
            got = outputs()
            for k, v in params0.items():  # same start for the eager step
                dp[k].upload(v)
            run()
            want = outputs()
            for i, (a, b) in enumerate(zip(got, want)):
                assert a.tobytes() == b.tobytes(), (rep, i)
            s.sync()
    finally:
        h.hipGraphExecDestroy(exe)
        h.hipGraphDestroy(graph)
        net.close()
        s.close()
