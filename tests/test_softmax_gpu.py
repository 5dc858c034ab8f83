"""Parity of the gfx950 row softmax / log-softmax (forward and backward) and
softmax cross-entropy with the CPU oracle, which composes them from the
reference primitives (reduce::max, Broadcast::col::sub/div, reduce::sum).

Bars: |dy| <= 1e-5 relative to the magnitudes each result is formed from:
  softmax fwd     |gpu - ref| <= 1e-5 * |ref| (+1e-40 for denormal outputs)
  log-softmax fwd |gpu - ref| <= 1e-5 * (|x - max| + |log s| + 1): the
                  1e-5 relative bar on s becomes 1e-5 absolute on log s
  softmax bwd     |gpu - ref| <= 1e-5 * |y| * (|dy| + sum|dy*y|)
  log bwd         |gpu - ref| <= 1e-5 * (|dy| + exp(y) * sum|dy|)
Masked (-inf) inputs give exactly 0 (softmax) and -inf (log-softmax).
"""
import os

import numpy as np
import pytest

from cortexmind_amd import engine
from cortexmind_amd._lib import call
from cortexmind_amd.data import SplitMix64, c1_softmax, c4_long_softmax

from gpu_util import dev, empty

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
FIX = np.load(os.path.join(HERE, "golden", "fixtures_f64.npz"))


def fwd(x, log, off=0):
    r, c = x.shape
    dx, dy = dev(x, off), empty((r, c), offset_floats=off)
    engine.softmax.forward(dx, dy, r, c, log=log)
    return dy.numpy()


def bwd(y, g, log, off=0):
    r, c = y.shape
    dy_, dg, dd = dev(y, off), dev(g, off), empty((r, c), offset_floats=off)
    engine.softmax.backward(dy_, dg, dd, r, c, log=log)
    return dd.numpy()


def check_fwd(x, got, ref, log):
    x64 = x.astype(np.float64)
    ref64 = ref.astype(np.float64)
    fin = np.isfinite(ref64)
    if log:
        m = np.max(np.where(np.isfinite(x64), x64, -np.inf), axis=1, keepdims=True)
        ls = np.abs(np.where(fin, ref64 - (x64 - m), 0.0)).max(axis=1, keepdims=True)
        tol = 1e-5 * (np.abs(np.where(np.isfinite(x64), x64 - m, 0.0)) + ls + 1.0)
        assert np.array_equal(np.isneginf(got), np.isneginf(ref))
    else:
        tol = 1e-5 * np.abs(ref64) + 1e-40
        assert np.all(got[ref == 0] == 0)
    err = np.abs(got.astype(np.float64) - ref64)
    assert np.all(err[fin] <= tol[fin]), float(np.max(err[fin] - tol[fin]))


def check_bwd(y, g, got, ref, log):
    y64, g64 = y.astype(np.float64), g.astype(np.float64)
    if log:
        tol = 1e-5 * (np.abs(g64) + np.exp(y64) * np.abs(g64).sum(axis=1, keepdims=True))
    else:
        tol = 1e-5 * np.abs(y64) * (np.abs(g64) + np.abs(g64 * y64).sum(axis=1, keepdims=True))
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    assert np.all(err <= tol + 1e-38), float(np.max(err - tol))


@pytest.mark.parametrize("log", [False, True])
def test_c1_forward(hip, orc, log):
    x = c1_softmax()
    got = fwd(x, log)
    check_fwd(x, got, orc.softmax_fwd(x, log), log)
    if not log:
        assert np.all(np.abs(got.astype(np.float64).sum(axis=1) - 1.0) <= 1e-5)


@pytest.fixture(scope="module")
def c4():
    return c4_long_softmax()


@pytest.mark.parametrize("log", [False, True])
def test_c4_forward_backward(hip, orc, c4, log):
    """C4 at full size [64, 131072], 10% -inf per row: the split-row kernels."""
    x, g = c4
    got = fwd(x, log)
    ref = orc.softmax_fwd(x, log)
    check_fwd(x, got, ref, log)
    masked = np.isneginf(x)
    if log:
        assert np.all(np.isneginf(got[masked]))
    else:
        assert np.all(got[masked] == 0.0)
        assert np.all(np.abs(got.astype(np.float64).sum(axis=1) - 1.0) <= 1e-5)
    # backward from the reference forward output (finite y only for log mode,
    # where -inf rows of y give exp(y) = 0)
    y = ref
    dgot = bwd(y, g, log)
    dref = orc.softmax_bwd(y, g, log)
    if log:
        fin = np.isfinite(y)
        assert np.all(np.isfinite(dgot[fin]))
        y = np.where(fin, y, np.float32(-1e30))
    check_bwd(y, g, dgot, dref, log)


SHAPES = [(3, 17), (4, 300), (7, 4096), (5, 4100), (2, 10000), (1, 1), (9, 64), (33, 1024),
          (2, 65536 + 8)]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
@pytest.mark.parametrize("log", [False, True])
@pytest.mark.parametrize("off", [0, 1])
def test_shapes(hip, orc, shape, log, off):
    r, c = shape
    g = SplitMix64(r * 131 + c)
    x = g.normal((r, c), 0.0, 6.0)
    if c >= 10:
        x[g.mask_rows(r, c, c // 10)] = -np.inf
    got = fwd(x, log, off)
    ref = orc.softmax_fwd(x, log)
    check_fwd(x, got, ref, log)
    dyv = g.normal((r, c))
    y = np.where(np.isfinite(ref), ref, np.float32(-1e30)) if log else ref
    check_bwd(y, dyv, bwd(y, dyv, log, off), orc.softmax_bwd(y, dyv, log), log)


@pytest.mark.parametrize("name", ["sm_small", "sm_mask"])
@pytest.mark.parametrize("mode", ["soft", "log"])
def test_float64_fixtures(hip, name, mode):
    """Against float64 torch answers committed under tests/golden/."""
    x = FIX[f"{name}_x"]
    g = FIX[f"{name}_dy"]
    y64 = FIX[f"{name}_{mode}_y"]
    dx64 = FIX[f"{name}_{mode}_dx"]
    log = mode == "log"
    got = fwd(x, log)
    fin = np.isfinite(y64)
    if log:
        tol = 1e-5 * (np.abs(np.where(fin, y64, 0)) + 1.0)
    else:
        tol = 1e-5 * np.abs(y64) + 1e-30
    assert np.all(np.abs(got[fin] - y64[fin]) <= tol[fin])
    y = np.where(fin, got, np.float32(-1e30)) if log else got
    dgot = bwd(y, g, log)
    scale = np.abs(g).sum(axis=1, keepdims=True) + np.abs(g)
    assert np.all(np.abs(dgot - dx64) <= 1e-5 * scale + 1e-30)


def test_constant_and_fully_masked_rows(hip):
    x = np.full((3, 4096), 2.5, np.float32)
    x[1, :] = -np.inf
    got = fwd(x, False)
    assert np.all(got[0] == np.float32(1.0 / 4096))
    # an all -inf row is 0/0 in the reference composition (max starts at -FLT_MAX)
    assert np.all(np.isnan(got[1]))


def test_xent(hip, orc):
    g = SplitMix64(0x1E)
    logits = g.normal((4096, 10), 0.0, 3.0)
    labels = g.randint(4096, 10)
    dl_, dlab, dloss, ddl = dev(logits), dev(labels), empty((1,)), empty((4096, 10))
    engine.train.softmax_xent(dl_, dlab, dloss, ddl, 4096, 10)
    loss_ref, dl_ref = orc.softmax_xent(logits, labels)
    assert abs(dloss.numpy()[0] - loss_ref) <= 1e-5 * abs(loss_ref)
    assert np.all(np.abs(ddl.numpy() - dl_ref) <= 1e-5 * (np.abs(dl_ref) + 1.0 / 4096) )
    # float64 fixture
    lg, lb = FIX["xent_logits"], FIX["xent_labels"]
    a, b_, c_, d_ = dev(lg), dev(lb), empty((1,)), empty(lg.shape)
    engine.train.softmax_xent(a, b_, c_, d_, *lg.shape)
    assert abs(c_.numpy()[0] - FIX["xent_loss"][0]) <= 1e-5 * FIX["xent_loss"][0]
    assert np.all(np.abs(d_.numpy() - FIX["xent_dlogits"]) <= 1e-6)


def test_xent_bad_label_gives_nan(hip):
    logits = np.zeros((300, 4), np.float32)
    labels = np.zeros(300, np.int32)
    labels[123] = 4
    a, b_, c_, d_ = dev(logits), dev(labels), empty((1,)), empty((300, 4))
    engine.train.softmax_xent(a, b_, c_, d_, 300, 4)
    assert np.isnan(c_.numpy()[0])
