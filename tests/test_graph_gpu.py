"""Parity of the autograd graph (include/cortex_hip_graph.hpp) with the CPU
oracle and the float64 fixtures, through the test-only C entry points of
tests/cpp/graph_shim.cpp (libgraph_shim.so over libcxm_hip.so).

The reference declares meta::GradientFlow::backward and GradientLink
(source/CortexMind/framework/Graph/flow.hpp:15-24, Graph/link.cpp:11-13)
without any concrete flow; the graph's flows are checked here against the
oracle's compositions of the reference primitives, not against the fused
HIP kernels they share code with:
  * the MLP trained through matmul / add_bias / relu / softmax_cross_entropy /
    backward / sgd against orc_mlp_step (reduced batch and the full C5
    config) and against the float64 torch fixture;
  * act(X * scale + b) at the C3 size, fused and as mul_row -> add_bias ->
    activation, against orc_affine_act_fwd / orc_affine_act_bwd: dX bit-exact,
    dscale and dbias within 1e-5 of the sums of their terms' magnitudes;
  * softmax and log-softmax at the C1 and C4 sizes against orc_softmax_fwd /
    orc_softmax_bwd, with the softmax test module's bars;
  * sum and mean over an axis: dX is dZ broadcast (/ dim), bit-exact;
  * the loss gradient seeded with a value other than 1, and a tensor whose
    gradient has two contributions.
"""
import ctypes
import os

import numpy as np
import pytest

from cortexmind_amd.data import SplitMix64, c1_softmax, c3_affine, c4_long_softmax, c5_mlp

from gpu_util import bits_equal, ulp_dist

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
SHIM = os.path.join(HERE, "cpp", "libgraph_shim.so")
FIX = np.load(os.path.join(HERE, "golden", "fixtures_f64.npz"))
ACT_NONE, ACT_RELU, ACT_SIGMOID, ACT_TANH = 0, 1, 2, 3

_F = ctypes.POINTER(ctypes.c_float)
_I = ctypes.POINTER(ctypes.c_int32)
_SZ = ctypes.c_size_t


@pytest.fixture(scope="module")
def shim(hip):
    lib = ctypes.CDLL(SHIM)
    sigs = {
        "gs_mlp_steps": [_F, _I] + [_F] * 6 + [_SZ] * 5 + [ctypes.c_float, ctypes.c_int, _F],
        "gs_affine": [_F, _F, _F, _F, _SZ, _SZ, ctypes.c_int, ctypes.c_int, _F, _F, _F, _F],
        "gs_softmax": [_F, _F, _SZ, _SZ, ctypes.c_int, _F, _F],
        "gs_reduce": [_F, _F, _SZ, _SZ, _SZ, ctypes.c_int, _F, _F],
        "gs_xent": [_F, _I, _SZ, _SZ, ctypes.c_float, _F, _F],
        "gs_two_paths": [_F, _F, _SZ, ctypes.c_float, ctypes.c_float, _F, _F],
    }
    for name, args in sigs.items():
        getattr(lib, name).argtypes = args
        getattr(lib, name).restype = ctypes.c_int
    return lib


def f(a):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_F)


def i32(a):
    assert a.dtype == np.int32 and a.flags.c_contiguous
    return a.ctypes.data_as(_I)


# ------------------------------------------------------------------ MLP

def graph_mlp(shim, x, labels, params, lr, steps):
    p = {k: v.copy() for k, v in params.items()}
    losses = np.zeros(steps, np.float32)
    b, d0 = x.shape
    d1, d2, d3 = p["w1"].shape[1], p["w2"].shape[1], p["w3"].shape[1]
    assert shim.gs_mlp_steps(f(np.ascontiguousarray(x)), i32(np.ascontiguousarray(labels, np.int32)), f(p["w1"]),
                             f(p["b1"]), f(p["w2"]), f(p["b2"]), f(p["w3"]), f(p["b3"]), b, d0, d1, d2, d3, lr, steps,
                             f(losses)) == 0
    return [float(v) for v in losses], p


def check_mlp_vs_oracle(orc, x, labels, params, steps, losses, final):
    ref = {k: v.copy() for k, v in params.items()}
    ref_losses = [orc.mlp_step(x, labels, ref, 0.01) for _ in range(steps)]
    for got, want in zip(losses, ref_losses):
        assert abs(got - want) <= 1e-5 * abs(want), (losses, ref_losses)
    # each layer's weight and bias within 1e-4 of that layer's weight scale
    for k in ref:
        w = "w" + k[1]
        scale = max(np.abs(params[w]).max(), np.abs(ref[w]).max())
        assert np.max(np.abs(final[k] - ref[k])) <= 1e-4 * scale, k


def test_graph_mlp_vs_oracle_reduced_batch(shim, orc):
    x, labels, params = c5_mlp(batch=256)
    losses, final = graph_mlp(shim, x, labels, params, 0.01, 3)
    check_mlp_vs_oracle(orc, x, labels, params, 3, losses, final)


def test_graph_mlp_full_size_vs_oracle(shim, orc):
    """The C5 config (batch 4096, 10 steps) trained through the graph."""
    x, labels, params = c5_mlp()
    losses, final = graph_mlp(shim, x, labels, params, 0.01, 10)
    check_mlp_vs_oracle(orc, x, labels, params, 10, losses, final)
    assert losses[-1] < losses[0]


def test_graph_mlp_float64_fixture(shim):
    """Two steps of a 49 -> 32 -> 32 -> 10 MLP against float64 torch."""
    x, labels = FIX["mlp_x"].astype(np.float32), FIX["mlp_labels"].astype(np.int32)
    params = {k: FIX[f"mlp_init_{k}"].astype(np.float32) for k in ["w1", "b1", "w2", "b2", "w3", "b3"]}
    losses, final = graph_mlp(shim, x, labels, params, 0.01, 2)
    for got, want in zip(losses, FIX["mlp_losses"]):
        assert abs(got - want) <= 1e-5 * abs(want)
    for k in params:
        want = FIX[f"mlp_final_{k}"]
        assert np.max(np.abs(final[k] - want)) <= 1e-5 * (np.abs(want).max() + 1e-3), k


# ------------------------------------------------------- affine + act

def graph_affine(shim, x, s, b, dy, act, fused):
    m, n = x.shape
    y, dx = np.empty_like(x), np.empty_like(x)
    ds, db = np.empty(n, np.float32), np.empty(n, np.float32)
    assert shim.gs_affine(f(x), f(s), f(b), f(dy), m, n, act, fused, f(y), f(dx), f(ds), f(db)) == 0
    return y, dx, ds, db


def f64_act(t, act):
    t = t.astype(np.float64)
    return {ACT_SIGMOID: lambda v: 1.0 / (1.0 + np.exp(-v)), ACT_TANH: np.tanh}[act](t)


def check_affine(orc, x, s, b, g, act, y, dx, ds, db):
    if act in (ACT_NONE, ACT_RELU):
        assert bits_equal(y, orc.affine_act_fwd(x, s, b, act))
    else:
        t = ((x * s[None, :]).astype(np.float32) + b[None, :]).astype(np.float32)
        assert int(ulp_dist(y, f64_act(t, act)).max()) <= 2
    rdx, rds, rdb = orc.affine_act_bwd(x, s, y, g, act)
    assert bits_equal(dx, rdx)
    dz_abs = np.abs(g.astype(np.float64))  # |act'| <= 1
    assert np.all(np.abs(ds.astype(np.float64) - rds) <= 1e-5 * (np.abs(x) * dz_abs).sum(axis=0) + 1e-30)
    assert np.all(np.abs(db.astype(np.float64) - rdb) <= 1e-5 * dz_abs.sum(axis=0) + 1e-30)


@pytest.fixture(scope="module")
def c3():
    return c3_affine()


@pytest.mark.parametrize("act", [ACT_RELU, ACT_SIGMOID, ACT_TANH])
def test_graph_affine_c3_fused(shim, orc, c3, act):
    x, s, b, g = c3
    check_affine(orc, x, s, b, g, act, *graph_affine(shim, x, s, b, g, act, 1))


@pytest.mark.parametrize("act", [ACT_RELU, ACT_SIGMOID, ACT_TANH])
def test_graph_affine_c3_composed(shim, orc, c3, act):
    """mul_row -> add_bias -> activation: three flows, the same bits as the
    one fused flow for Y and dX."""
    x, s, b, g = c3
    got = graph_affine(shim, x, s, b, g, act, 0)
    check_affine(orc, x, s, b, g, act, *got)
    fused = graph_affine(shim, x, s, b, g, act, 1)
    assert bits_equal(got[0], fused[0]) and bits_equal(got[1], fused[1])


@pytest.mark.parametrize("m,n", [(7, 264), (33, 1025), (1, 4)])
def test_graph_affine_shapes(shim, orc, m, n):
    r = SplitMix64(m * 1009 + n)
    x, g = r.normal((m, n)), r.normal((m, n))
    s, b = r.uniform((n,), 0.5, 1.5), r.normal((n,), 0.0, 0.1)
    for act in (ACT_NONE, ACT_TANH):
        check_affine(orc, x, s, b, g, act, *graph_affine(shim, x, s, b, g, act, 0))


# ----------------------------------------------------------- softmax

def graph_softmax(shim, x, dy, log):
    r, c = x.shape
    y, dx = np.empty_like(x), np.empty_like(x)
    assert shim.gs_softmax(f(x), f(dy), r, c, int(log), f(y), f(dx)) == 0
    return y, dx


def check_softmax(orc, x, dy, log, y, dx):
    ref = orc.softmax_fwd(x, log)
    x64, ref64 = x.astype(np.float64), ref.astype(np.float64)
    fin = np.isfinite(ref64)
    if log:
        m = np.max(np.where(np.isfinite(x64), x64, -np.inf), axis=1, keepdims=True)
        with np.errstate(invalid="ignore"):
            ls = np.abs(np.where(fin, ref64 - (x64 - m), 0.0)).max(axis=1, keepdims=True)
        tol = 1e-5 * (np.abs(np.where(np.isfinite(x64), x64 - m, 0.0)) + ls + 1.0)
        assert np.array_equal(np.isneginf(y), np.isneginf(ref))
    else:
        tol = 1e-5 * np.abs(ref64) + 1e-40
        assert np.all(y[ref == 0] == 0)
    with np.errstate(invalid="ignore"):
        err = np.abs(y.astype(np.float64) - ref64)
    assert np.all(err[fin] <= tol[fin])
    # backward from the graph's own forward output, as the flow runs it
    yb = y.copy()
    rdx = orc.softmax_bwd(yb, dy, log)
    y64, g64 = yb.astype(np.float64), dy.astype(np.float64)
    if log:
        tol = 1e-5 * (np.abs(g64) + np.exp(y64) * np.abs(g64).sum(axis=1, keepdims=True))
    else:
        tol = 1e-5 * np.abs(y64) * (np.abs(g64) + np.abs(g64 * y64).sum(axis=1, keepdims=True))
    assert np.all(np.abs(dx.astype(np.float64) - rdx.astype(np.float64)) <= tol + 1e-38)


@pytest.mark.parametrize("log", [False, True])
def test_graph_softmax_c4(shim, orc, log):
    """C4 [64, 131072] with 10% -inf per row, forward and backward."""
    x, dy = c4_long_softmax()
    check_softmax(orc, x, dy, log, *graph_softmax(shim, x, dy, log))


@pytest.mark.parametrize("log", [False, True])
def test_graph_softmax_c1(shim, orc, log):
    x = c1_softmax()
    dy = SplitMix64(0xC1D).normal(x.shape)
    check_softmax(orc, x, dy, log, *graph_softmax(shim, x, dy, log))


# --------------------------------------------------------- reductions

@pytest.mark.parametrize("sizes", [(4096, 4096, 1), (1, 4096, 4096), (3, 50, 7), (1, 1 << 20, 1), (5, 33, 1)])
@pytest.mark.parametrize("mean", [0, 1])
def test_graph_sum_mean(shim, orc, sizes, mean):
    o, d, i = sizes
    r = SplitMix64(o * 31 + d * 7 + i + mean)
    x, dz = r.uniform(sizes, -1.0, 1.0), r.normal((o, i))
    z, dx = np.empty((o, i), np.float32), np.empty_like(x)
    assert shim.gs_reduce(f(x), f(dz), o, d, i, mean, f(z), f(dx)) == 0
    ref = orc.reduce_axis("mean" if mean else "sum", x, o, d, i).reshape(o, i)
    tol = 1e-5 * np.abs(x.astype(np.float64)).sum(axis=1) / (d if mean else 1)
    assert np.all(np.abs(z.astype(np.float64) - ref) <= tol + 1e-30)
    want = dz / np.float32(d) if mean else dz
    assert bits_equal(dx, np.broadcast_to(want[:, None, :], (o, d, i)))


# ------------------------------------------------------ seeds, paths

def test_graph_xent_seed(shim, orc):
    """backward(loss, seed) scales the loss's dlogits by the seed read on the
    device (one rounding): bit for bit dlogits(seed 1) * seed.  Seed 1 (the
    default of backward(loss)) against the oracle with test_xent's bar."""
    b, c = 4096, 10
    r = SplitMix64(0x5EED)
    logits = r.normal((b, c), 0.0, 3.0)
    labels = (r.next_u64(b) % np.uint64(c)).astype(np.int32)

    def run(seed):
        loss, dl = np.zeros(1, np.float32), np.empty_like(logits)
        assert shim.gs_xent(f(logits), i32(labels), b, c, seed, f(loss), f(dl)) == 0
        return float(loss[0]), dl

    loss1, dl1 = run(1.0)
    rloss, rdl = orc.softmax_xent(logits, labels)
    assert abs(loss1 - rloss) <= 1e-5 * abs(rloss)
    assert np.all(np.abs(dl1 - rdl) <= 1e-5 * (np.abs(rdl) + 1.0 / b))
    for seed in (2.5, -0.125, 3.0e-3):
        loss_s, dls = run(seed)
        assert loss_s == loss1
        assert bits_equal(dls, dl1 * np.float32(seed)), seed


def test_graph_two_paths_accumulate(shim):
    n = 100003
    r = SplitMix64(0x2A)
    x, dy = r.normal((n,)), r.normal((n,))
    a, c = np.float32(1.5), np.float32(-0.75)
    y, dx = np.empty_like(x), np.empty_like(x)
    assert shim.gs_two_paths(f(x), f(dy), n, a, c, f(y), f(dx)) == 0
    assert bits_equal(y, (x * a) + (x * c))
    # the first contribution is written, the second added in: dy*a + dy*c
    assert bits_equal(dx, (dy * a) + (dy * c))
