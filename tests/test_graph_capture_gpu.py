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


def _query(stream, which):
    base, nbytes, pinned = ctypes.c_void_p(), ctypes.c_size_t(), ctypes.c_int()
    call("cxm_workspace_query", stream.handle, which, ctypes.byref(base), ctypes.byref(nbytes), ctypes.byref(pinned))
    return base.value, nbytes.value, pinned.value


def _allocated(h, ptr):
    """hipPointerGetAttributes succeeds on a live device allocation only."""
    attrs = (ctypes.c_char * 256)()
    h.hipPointerGetAttributes.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    h.hipPointerGetAttributes.restype = ctypes.c_int
    return h.hipPointerGetAttributes(attrs, ctypes.c_void_p(ptr)) == 0


def test_capture_without_scratch_is_refused(hip):
    """Under capture, a call that needs scratch its stream does not have
    yet returns CXM_E_CAPTURE before allocating, filling, waiting for or
    launching anything, and capture ends cleanly with an empty graph."""
    from cortexmind_amd._lib import E_CAPTURE, lib

    h = hip_rt()
    s = Stream()
    L = lib()
    # x holds the largest input read here: the [4096, 4096] column sum and
    # the 2^24-element flat sum (the [64, 131072] softmax reads the first half)
    x = DeviceArray((1 << 24,), np.float32)
    y = DeviceArray((64 * 131072,), np.float32)
    z = DeviceArray((4096,), np.float32)
    assert x.size >= max(1 << 24, 4096 * 4096, 64 * 131072)
    try:
        assert h.hipStreamBeginCapture(s.handle, CAPTURE_RELAXED) == 0
        st = [
            L.cxm_reduce_sum_flat_f32(x.ptr, z.ptr, 1 << 24, s.handle),          # tagged slots
            L.cxm_reduce_sum_f32(x.ptr, z.ptr, 1, 4096, 4096, s.handle),        # workspace (column ticket)
            L.cxm_softmax_fwd_f32(x.ptr, y.ptr, 64, 131072, 0, s.handle),       # exchange region
        ]
        graph = ctypes.c_void_p()
        assert h.hipStreamEndCapture(s.handle, ctypes.byref(graph)) == 0
        n = ctypes.c_size_t(99)
        h.hipGraphGetNodes.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(ctypes.c_size_t)]
        h.hipGraphGetNodes.restype = ctypes.c_int
        assert h.hipGraphGetNodes(graph, None, ctypes.byref(n)) == 0
        h.hipGraphDestroy(graph)
        assert st == [E_CAPTURE] * 3, st
        assert n.value == 0
        for which in (0, 1, 2):
            assert _query(s, which)[0] is None  # nothing was allocated for this stream
        # the same calls made eagerly afterwards work
        call("cxm_reduce_sum_f32", x.ptr, z.ptr, 1, 4096, 4096, s.handle)
        s.sync()
        assert _query(s, 0)[0] is not None
    finally:
        s.close()


def test_captured_workspace_survives_growth(hip):
    """A region handed to a captured launch is pinned: a later eager call
    that needs a larger workspace on the same stream gets a new region and
    the old one stays allocated, so the graph still replays correctly."""
    h = hip_rt()
    s = Stream()
    g = SplitMix64(0x6D)
    x = DeviceArray((4096 * 4096,), np.float32)
    z = DeviceArray((4096,), np.float32)
    M, K, N = 1024, 4096, 1024  # split-K A^T B: 64 tiles x 4 splits of 128x128 partials (16 MiB)
    ga, gb, gc = DeviceArray((K * M,), np.float32), DeviceArray((K * N,), np.float32), DeviceArray((M * N,), np.float32)
    ga.upload(g.uniform((K * M,), -1.0, 1.0))
    gb.upload(g.uniform((K * N,), -1.0, 1.0))

    def red():
        call("cxm_reduce_sum_f32", x.ptr, z.ptr, 1, 4096, 4096, s.handle)

    x.upload(g.uniform((4096 * 4096,), -1.0, 1.0))
    red()  # sizes the workspace (the default 8 MiB of partials)
    s.sync()
    base0, bytes0, pinned0 = _query(s, 0)
    assert pinned0 == 0
    graph, exe = capture(h, s, red)
    try:
        base1, bytes1, pinned1 = _query(s, 0)
        assert (base1, bytes1, pinned1) == (base0, bytes0, 1)
        call("cxm_gemm_f32", ga.ptr, gb.ptr, gc.ptr, M, K, N, 1, 0, None, 0, None, s.handle)  # grows it
        s.sync()
        base2, bytes2, pinned2 = _query(s, 0)
        assert base2 != base0 and bytes2 > bytes0 and pinned2 == 0
        assert _allocated(h, base0), "the pinned region was freed while a graph holds it"
        for rep in range(3):
            x.upload(g.uniform((4096 * 4096,), -1.0, 1.0))
            red()
            want = z.numpy(s).copy()
            z.fill_bytes(0xFF, s)
            assert h.hipGraphLaunch(exe, s.handle) == 0
            assert z.numpy(s).tobytes() == want.tobytes(), rep
    finally:
        h.hipGraphExecDestroy(exe)
        h.hipGraphDestroy(graph)
        s.close()


def test_tags_differ_across_streams(hip):
    """Flat-reduction tags come from one process-wide counter: two streams'
    calls interleaved never reuse a tag, and a region freed with one stream
    and taken by another holds no slot that matches (checked through the
    results: each stream's sums equal the eager bits on fresh data)."""
    g = SplitMix64(0x6E)
    n = 1 << 22
    xs = [DeviceArray((n,), np.float32) for _ in range(2)]
    zs = [DeviceArray((1,), np.float32) for _ in range(2)]
    ref = DeviceArray((1,), np.float32)
    for rep in range(4):
        streams = [Stream(), Stream()]
        data = [g.uniform((n,), -1.0, 1.0) for _ in range(2)]
        for i in range(2):
            xs[i].upload(data[i])
        for i in range(2):
            call("cxm_reduce_sum_flat_f32", xs[i].ptr, zs[i].ptr, n - rep, streams[i].handle)
        for i in range(2):
            streams[i].sync()
            call("cxm_reduce_sum_noalloc_f32", xs[i].ptr, ref.ptr, 1, n - rep, 1, None)
            assert zs[i].numpy(streams[i]).tobytes() == ref.numpy().tobytes(), (rep, i)
        for st in streams:
            st.close()
