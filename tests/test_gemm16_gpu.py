"""bf16 / fp16 matmul (nv::Matrix::matmul's 16-bit cublasGemmEx branches,
Engine/CUDA/matrix.cu:112-159) through cxm_matmul_t / cxm_gemm_t.

cuBLAS cannot run here and no reference test pins its 16-bit results, so
the check is the mathematics: the float64 product of the 16-bit inputs
(widened exactly by the oracle's convert()).  The kernel accumulates in
fp32 and rounds once to the 16-bit output, so the bar per element is
  |got - C64| <= 0.5 ulp16(max(|got|, |C64|)) + 1e-5 * (|A| |B|)_ij
(the rounding to 16 bits plus an fp32 accumulation allowance).
"""
import numpy as np
import pytest

from cortexmind_amd._lib import DT_BF16, DT_F16, DT_F32, E_INVALID, call, lib

from cortexmind_amd.data import SplitMix64
from gpu_util import dev

pytestmark = pytest.mark.gpu

DTS = [DT_BF16, DT_F16]
MANT = {DT_BF16: 7, DT_F16: 10}
EMIN = {DT_BF16: -126, DT_F16: -14}


def ulp16(x, dt):
    x = np.abs(np.asarray(x, np.float64))
    e = np.floor(np.log2(np.where(x > 0, x, 1.0)))
    e = np.maximum(e, EMIN[dt])
    return np.exp2(e - MANT[dt])


def rand16(g, shape, dt, orc, scale=1.0):
    f = g.normal(shape, 0.0, scale).astype(np.float32)
    h = orc.convert(f.ravel(), DT_F32, dt).reshape(shape)
    return h, orc.convert(h.ravel(), dt, DT_F32).astype(np.float64).reshape(shape)


def run(a16, b16, m, k, n, dt, ta=0, tb=0, off=0):
    da, db = dev(a16, off), dev(b16, off)
    dc = dev(np.zeros((m, n), np.uint16), off)
    call("cxm_gemm_t", da.ptr, db.ptr, dc.ptr, m, k, n, ta, tb, dt, None)
    return dc.numpy()


def check(got16, a64, b64, dt, orc):
    c64 = a64 @ b64
    absab = np.abs(a64) @ np.abs(b64)
    got = orc.convert(got16.ravel(), dt, DT_F32).astype(np.float64).reshape(c64.shape)
    tol = 0.5 * ulp16(np.maximum(np.abs(got), np.abs(c64)), dt) + 1e-5 * absab
    err = np.abs(got - c64)
    assert np.all(np.isfinite(got))
    assert np.all(err <= tol), (float(np.max(err - tol)), np.unravel_index(np.argmax(err - tol), err.shape))


SHAPES = [(128, 64, 128), (256, 192, 384), (130, 70, 129), (1, 1, 1), (7, 300, 5), (33, 17, 65),
          (512, 1024, 256), (4096, 784, 1024)]


@pytest.mark.parametrize("dt", DTS, ids=["bf16", "f16"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_matmul_nn(hip, orc, dt, shape):
    m, k, n = shape
    g = SplitMix64(17 * m + 5 * k + n + dt)
    a16, a64 = rand16(g, (m, k), dt, orc)
    b16, b64 = rand16(g, (k, n), dt, orc)
    da, db = dev(a16), dev(b16)
    dc = dev(np.zeros((m, n), np.uint16))
    call("cxm_matmul_t", da.ptr, db.ptr, dc.ptr, m, k, n, dt, None)
    check(dc.numpy(), a64, b64, dt, orc)


@pytest.mark.parametrize("dt", DTS, ids=["bf16", "f16"])
@pytest.mark.parametrize("ta,tb", [(1, 0), (0, 1), (1, 1)])
@pytest.mark.parametrize("shape", [(128, 128, 128), (200, 136, 72), (131, 67, 93), (1024, 512, 768)],
                         ids=lambda s: "x".join(map(str, s)))
def test_gemm_transposed(hip, orc, dt, ta, tb, shape):
    m, k, n = shape
    g = SplitMix64(31 * m + 7 * k + n + 3 * ta + tb + dt)
    a16, a64 = rand16(g, (k, m) if ta else (m, k), dt, orc)
    b16, b64 = rand16(g, (n, k) if tb else (k, n), dt, orc)
    got = run(a16, b16, m, k, n, dt, ta, tb)
    check(got, a64.T if ta else a64, b64.T if tb else b64, dt, orc)


@pytest.mark.parametrize("dt", DTS, ids=["bf16", "f16"])
def test_misaligned_pointers(hip, orc, dt):
    """Bases off 16-byte alignment take the element-wise staging loads."""
    m, k, n = 96, 80, 136
    g = SplitMix64(4242 + dt)
    a16, a64 = rand16(g, (m, k), dt, orc)
    b16, b64 = rand16(g, (k, n), dt, orc)
    check(run(a16, b16, m, k, n, dt, off=3), a64, b64, dt, orc)


@pytest.mark.parametrize("dt", DTS, ids=["bf16", "f16"])
def test_exact_small_integers(hip, orc, dt):
    """Small integers: every product and partial sum is exact in fp32 and
    the result fits the 16-bit type, so the output is exact."""
    m, k, n = 64, 96, 80
    rng = np.random.default_rng(dt)
    a = rng.integers(-3, 4, (m, k)).astype(np.float32)
    b = rng.integers(-3, 4, (k, n)).astype(np.float32)
    c = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32)
    assert np.abs(c).max() <= 256  # exact in bf16 (8 significant bits) and f16
    got = run(orc.convert(a.ravel(), DT_F32, dt).reshape(m, k), orc.convert(b.ravel(), DT_F32, dt).reshape(k, n),
              m, k, n, dt)
    assert np.array_equal(orc.convert(got.ravel(), dt, DT_F32).reshape(m, n), c)


def test_f32_dtype_forwards(hip):
    m, k, n = 70, 50, 90
    g = SplitMix64(99)
    a = g.normal((m, k)).astype(np.float32)
    b = g.normal((k, n)).astype(np.float32)
    da, db = dev(a), dev(b)
    c1, c2 = dev(np.zeros((m, n), np.float32)), dev(np.zeros((m, n), np.float32))
    call("cxm_matmul_t", da.ptr, db.ptr, c1.ptr, m, k, n, DT_F32, None)
    call("cxm_matmul_f32", da.ptr, db.ptr, c2.ptr, m, k, n, None)
    assert np.array_equal(c1.numpy().view(np.uint32), c2.numpy().view(np.uint32))


def test_bad_arguments(hip):
    a = dev(np.zeros(16, np.uint16))
    assert lib().cxm_gemm_t(a.ptr, a.ptr, a.ptr, 4, 4, 4, 0, 0, 7, None) == E_INVALID
    assert lib().cxm_gemm_t(a.ptr, a.ptr, a.ptr, 4, 0, 4, 0, 0, DT_BF16, None) == E_INVALID
    assert lib().cxm_gemm_t(None, a.ptr, a.ptr, 4, 4, 4, 0, 0, DT_BF16, None) == E_INVALID
    assert lib().cxm_gemm_t(a.ptr, a.ptr, a.ptr, 0, 4, 4, 0, 0, DT_BF16, None) == 0


def _kernel(k):
    call("cxm_gemm16_kernel", k)


@pytest.mark.parametrize("dt", DTS, ids=["bf16", "f16"])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("shape", [(512, 384, 768), (512, 128, 256), (256, 1024, 384)],
                         ids=lambda s: "x".join(map(str, s)))
def test_kernels_agree_bitwise(hip, orc, dt, ta, tb, shape):
    """The 128x128 and 256x256 register-staged kernels and the 256 and 128
    four-stage direct-to-LDS kernels accumulate each output over k in the
    same order (32x32x16 MFMA blocks in k order), so they give the same
    bits.  K of 384, 128 and 1024 take the ring's eight-step loop zero,
    one and four times with and without its four-step tail; B stored
    [K,N] (tb = 0) goes through the transpose reads, A stored [K,M]
    (ta = 1) through the 16-bit transpose first.  N = 384 is not a
    multiple of 256, so kernel 2 falls back to kernel 1 there."""
    m, k, n = shape
    g = SplitMix64(77 + 4 * ta + 2 * tb + dt + k)
    a16, a64 = rand16(g, (k, m) if ta else (m, k), dt, orc)
    b16, b64 = rand16(g, (n, k) if tb else (k, n), dt, orc)
    outs = []
    try:
        for kern in (0, 1, 2, 3):
            _kernel(kern)
            outs.append(run(a16, b16, m, k, n, dt, ta, tb))
    finally:
        _kernel(-1)
    check(outs[0], a64.T if ta else a64, b64.T if tb else b64, dt, orc)
    for o in outs[1:]:
        assert np.array_equal(outs[0], o)


@pytest.mark.parametrize("dt", DTS, ids=["bf16", "f16"])
@pytest.mark.parametrize("tb", [0, 1])
def test_ring128_default_path(hip, orc, dt, tb):
    """4096 x 1024 x 1024: 64 tiles of 256x256, too few for the chip, so the
    automatic choice is the 128 ring (256 workgroups), B read as stored."""
    m, k, n = 4096, 1024, 1024
    g = SplitMix64(6160 + dt + tb)
    a16, a64 = rand16(g, (m, k), dt, orc)
    b16, b64 = rand16(g, (n, k) if tb else (k, n), dt, orc)
    check(run(a16, b16, m, k, n, dt, 0, tb), a64, b64.T if tb else b64, dt, orc)


@pytest.mark.parametrize("dt", DTS, ids=["bf16", "f16"])
def test_large_default_path(hip, orc, dt):
    """4096 x 1024 x 2048 NN: 128 tiles of 256x256, so the automatic choice
    is the 256 direct-load kernel, B read as stored."""
    m, k, n = 4096, 1024, 2048
    g = SplitMix64(5150 + dt)
    a16, a64 = rand16(g, (m, k), dt, orc)
    b16, b64 = rand16(g, (k, n), dt, orc)
    check(run(a16, b16, m, k, n, dt), a64, b64, dt, orc)


def test_kernel_choice_argument(hip):
    assert lib().cxm_gemm16_kernel(4) == E_INVALID
    assert lib().cxm_gemm16_kernel(-2) == E_INVALID
    assert lib().cxm_gemm16_kernel(-1) == 0
