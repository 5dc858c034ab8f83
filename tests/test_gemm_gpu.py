"""Parity of the gfx950 fp32 MFMA GEMM with the CPU oracle (a restatement of
matrix_t::matmul, source/CortexMind/framework/Engine/AVX2/matrix.cpp:75-147,
plus transposed copies for the forms the reference lacks).

Bar: |gpu - ref| <= 1e-5 * (|A| |B|)_ij per element (summation order
differs; both are fp32).  Epilogues (bias add, ReLU, ReLU gate) are exact
operations applied after the sum.
"""
import numpy as np
import pytest

from cortexmind_amd import engine
from cortexmind_amd._lib import ACT_NONE, ACT_RELU, E_INVALID, lib
from cortexmind_amd.data import SplitMix64

from gpu_util import dev, empty

pytestmark = pytest.mark.gpu


def stored(a, trans):
    return np.ascontiguousarray(a.T) if trans else a


def run(a_op, b_op, ta, tb, bias=None, act=ACT_NONE, gate=None):
    m, k = a_op.shape
    n = b_op.shape[1]
    da, db = dev(stored(a_op, ta)), dev(stored(b_op, tb))
    dc = empty((m, n))
    engine.gemm(da, db, dc, m, k, n, ta, tb, bias=dev(bias) if bias is not None else None, act=act,
                gate=dev(gate) if gate is not None else None)
    return dc.numpy()


def bound(a_op, b_op):
    return 1e-5 * (np.abs(a_op.astype(np.float64)) @ np.abs(b_op.astype(np.float64))) + 1e-30


SHAPES = [(128, 128, 128), (64, 32, 48), (33, 17, 65), (1, 1, 1), (256, 784, 1024),
          (512, 1024, 10), (1024, 512, 10), (300, 10, 1024), (784, 2048, 1024), (130, 4100, 7)]


@pytest.mark.parametrize("m,k,n", SHAPES, ids=lambda v: str(v))
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_gemm_vs_oracle(hip, orc, m, k, n, ta, tb):
    g = SplitMix64(m * 7919 + k * 31 + n + 1000 * ta + 2000 * tb)
    a = g.normal((m, k))
    b = g.normal((k, n))
    got = run(a, b, ta, tb)
    ref = orc.gemm(stored(a, ta), stored(b, tb), bool(ta), bool(tb))
    assert np.all(np.abs(got - ref) <= bound(a, b))


def test_matmul_mirror_name(hip, orc):
    g = SplitMix64(9)
    a, b = g.uniform((100, 60), -1, 1), g.uniform((60, 36), -1, 1)
    da, db, dc = dev(a), dev(b), empty((100, 36))
    engine.matrix_t.matmul(da, db, dc, 100, 60, 36)
    assert np.all(np.abs(dc.numpy() - orc.matmul(a, b)) <= bound(a, b))


@pytest.mark.parametrize("m,k,n", [(4096, 784, 1024), (4096, 1024, 1024), (1024, 4096, 1024)])
def test_gemm_full_size_float64(hip, m, k, n):
    """C5's large products at full size, against float64 numpy."""
    g = SplitMix64(m + k + n)
    a = g.uniform((m, k), 0.0, 1.0)
    b = g.normal((k, n), 0.0, float(np.sqrt(2.0 / k)))
    got = run(a, b, 0, 0)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    assert np.all(np.abs(got - ref) <= bound(a, b))


@pytest.mark.parametrize("m,k,n", [(4096, 256, 4096), (4100, 300, 4095)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_gemm_large_grid_float64(hip, m, k, n, ta, tb):
    """Grids of >= 1024 tiles take the four-wave kernel; ragged edges included."""
    g = SplitMix64(m + 3 * k + 7 * n + 11 * ta + 13 * tb)
    a = g.normal((m, k))
    b = g.normal((k, n))
    bias = g.normal((n,), 0.0, 0.5)
    got = run(a, b, ta, tb, bias=bias, act=ACT_RELU)
    z = a.astype(np.float64) @ b.astype(np.float64) + bias.astype(np.float64)
    ref = np.maximum(z, 0.0)
    assert np.all(np.abs(got - ref) <= bound(a, b) + 1e-6 * np.abs(bias)[None, :])


def _pin(variant):
    assert lib().cxm_gemm_f32_kernel(variant) == 0


@pytest.mark.parametrize("m,k,n", [(128, 128, 128), (256, 384, 512), (512, 1024, 256), (2048, 784, 1536),
                                   (128, 40, 256)], ids=lambda v: str(v))
@pytest.mark.parametrize("tb", [0, 1])
def test_ring_same_bits_as_kc(hip, m, k, n, tb):
    """The direct-to-LDS ring (variant 7) and the k-contiguous kernel
    (variant 1) sum each output over k in the same order, so A B and A B^T
    agree bitwise; both within the bound of the float64 product.  Shapes
    whose K both kernels split alike (none, or 1024 four ways): the ring
    rounds a split's range to 128 k, the other kernel to 32.  K = 784 and 40
    end in a partial stage, of which the ring multiplies only the whole 8-k
    blocks and the other kernel zero-fills the rest."""
    g = SplitMix64(m + 5 * k + 9 * n + tb)
    a, b = g.normal((m, k)), g.normal((k, n))
    try:
        _pin(7)
        r7 = run(a, b, 0, tb)
        _pin(1)
        r1 = run(a, b, 0, tb)
    finally:
        _pin(-1)
    assert np.array_equal(r7.view(np.uint32), r1.view(np.uint32))
    assert np.all(np.abs(r7 - a.astype(np.float64) @ b.astype(np.float64)) <= bound(a, b))


@pytest.mark.parametrize("m,k,n", [(256, 4096, 256), (384, 512, 640), (300, 512, 260), (36, 256, 516),
                                   (784, 4096, 1024), (300, 784, 260), (128, 8, 128), (256, 4104, 256)],
                         ids=lambda v: str(v))
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_ring_all_forms_float64(hip, m, k, n, ta, tb):
    """Variant 7 pinned for every stored form with the bias + ReLU epilogue;
    256 x 4096 x 256 has 4 tiles and splits K 16 ways (256 each); 300 x 260,
    36 x 516 and 784 x 1024 (the MLP's first weight gradient) end in partial
    tiles, whose rows or columns past the operand load clamped duplicates;
    K = 784, 8 and 4104 (a split whose last range is 8 k) end in a partial
    32-k stage, of which only the whole 8-k blocks are multiplied."""
    g = SplitMix64(31 * m + k + 7 * n + 3 * ta + tb)
    a, b = g.normal((m, k)), g.normal((k, n))
    bias = g.normal((n,), 0.0, 0.5)
    try:
        _pin(7)
        got = run(a, b, ta, tb, bias=bias, act=ACT_RELU)
    finally:
        _pin(-1)
    ref = np.maximum(a.astype(np.float64) @ b.astype(np.float64) + bias.astype(np.float64), 0.0)
    assert np.all(np.abs(got - ref) <= bound(a, b) + 1e-6 * np.abs(bias)[None, :])


def test_kernel_pin_argument(hip):
    assert lib().cxm_gemm_f32_kernel(8) == E_INVALID
    assert lib().cxm_gemm_f32_kernel(-2) == E_INVALID
    assert lib().cxm_gemm_f32_kernel(-1) == 0


def test_epilogue_bias_relu_gate(hip, orc):
    g = SplitMix64(17)
    a, b = g.normal((200, 96)), g.normal((96, 72))
    bias = g.normal((72,), 0.0, 0.5)
    z = orc.bcast_row(orc.matmul(a, b), bias, 0)
    got = run(a, b, 0, 0, bias=bias, act=ACT_RELU)
    tol = bound(a, b)
    relu_ref = np.where(0 > z, 0, z)
    assert np.all(np.abs(got - relu_ref) <= tol)
    assert np.all(got >= 0)
    gate = g.normal((200, 72))
    got_g = run(a, b, 0, 0, gate=gate)
    ref_g = orc.matmul(a, b) * (gate > 0)
    assert np.all(np.abs(got_g - ref_g) <= tol)
    assert np.all(got_g[gate <= 0] == 0)


def test_bad_arguments(hip):
    assert lib().cxm_gemm_f32(None, None, None, 4, 4, 4, 0, 0, None, 0, None, None) == E_INVALID
    d = empty((16,))
    assert lib().cxm_gemm_f32(d.ptr, d.ptr, d.ptr, 4, 4, 4, 0, 0, None, 7, None, None) == E_INVALID


@pytest.mark.parametrize("m,k,n,ta,tb", [(4096, 1024, 10, 0, 0), (300, 512, 16, 0, 0), (129, 1020, 7, 0, 0),
                                         (65, 4, 12, 0, 0), (1, 1024, 1, 0, 0), (1024, 4096, 10, 1, 0), (4096, 10, 1024, 0, 1),
                                         (4096, 10, 1024, 0, 0), (77, 100, 3, 0, 0), (64, 333, 16, 1, 0),
                                         (50, 16, 36, 0, 1)])
def test_thin_products(hip, orc, m, k, n, ta, tb):
    """Shapes with a dimension <= 16 (the MLP's 10-class layer) run thin
    kernels instead of MFMA tiles; same bar, with their epilogues."""
    g = SplitMix64(m + 3 * k + 7 * n + ta + 2 * tb)
    a, b = g.normal((m, k)), g.normal((k, n))
    got = run(a, b, ta, tb)
    ref = orc.gemm(stored(a, ta), stored(b, tb), bool(ta), bool(tb))
    assert np.all(np.abs(got - ref) <= bound(a, b))
    if not ta:
        bias = g.normal((n,), 0.0, 0.5)
        gate = g.normal((m, n))
        z = orc.bcast_row(ref, bias, 0)
        got_b = run(a, b, ta, tb, bias=bias, act=ACT_RELU)
        assert np.all(np.abs(got_b - np.where(0 > z, 0, z)) <= bound(a, b))
        got_g = run(a, b, ta, tb, gate=gate)
        assert np.all(np.abs(got_g - ref * (gate > 0)) <= bound(a, b))
        assert np.all(got_g[gate <= 0] == 0)
