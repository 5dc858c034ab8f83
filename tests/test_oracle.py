"""Pins the CPU oracle (oracle/cxm_oracle.c) before it is trusted as the
parity checker of the HIP path.

The reference ships no tests, golden vectors or fixtures (its tests/*.cpp are
comment stubs), and its own reduce.cpp/broadcast.cpp/matrix.cpp cannot be
compiled here without stand-ins for MSVC __forceinline, Intel SVML and TLX.
So every oracle function is pinned by checks that do not retype its formula:

* hand-derived known answers (tests/golden/kat_oracle.json) whose values only
  come out right with the reference's exact fold/lane/panel order;
* exact arithmetic: small-integer inputs, where every order gives the exact
  integer sum, so a dropped tail, lane or panel shows;
* library routines: numpy float32 elementwise ops (IEEE single rounding) and
  float64 reductions/matmul; numpy's axis-0 float32 reduction, which adds
  rows in order exactly like reduce.cpp:51-62;
* brute force for max/argmax (order-free; first index wins on ties);
* float64 torch answers for the compositions the reference lacks
  (tests/golden/fixtures_f64.npz, written by tests/golden/make_fixtures.py);
* closed forms and invariants (softmax rows sum to 1, constant rows give 1/N,
  masked entries give exactly 0 / -inf).
"""
import json
import math
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
KAT = json.load(open(os.path.join(HERE, "golden", "kat_oracle.json")))
FIX = np.load(os.path.join(HERE, "golden", "fixtures_f64.npz"))


def f32(v):
    return np.array(v, dtype=np.float32)


def hexf(v: float) -> str:
    return hex(int(np.float32(v).view(np.uint32)))


def ulp_dist(a, b):
    """Distance in units in the last place between float32 arrays."""
    ai = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    bi = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    ai = np.where(ai < 0, -(ai & 0x7FFFFFFF), ai)
    bi = np.where(bi < 0, -(bi & 0x7FFFFFFF), bi)
    return np.abs(ai - bi)


# ------------------------------------------------------------------ sum

@pytest.mark.parametrize("case", KAT["sum_flat"], ids=lambda c: c["name"])
def test_sum_flat_kat(orc, case):
    # lane_fold_pairs: lanes (l, l+4) pair first: (2^24 + -2^24) + (1+1) + ... = 0+2+2+2 = 6;
    #   a plain left-to-right sum gives 3 (each +1 after 2^24 rounds away).
    # lanes_accumulate_across_blocks: lane 0 holds 2^24 + 1 -> 2^24 (ties to even),
    #   lane 1 holds 1; fold: (2^24 + 1) + 0 -> 2^24.  Folding each block first gives 2^24 + 2.
    # tail_added_after_fold: fold gives 2^24, each tail 1 rounds away; summing the tail
    #   first (3) gives 2^24 + 4.
    # short_is_sequential: 1 + 2^24 -> 2^24, + 1 -> 2^24; pairing the ones first gives 2^24 + 2.
    z = orc.reduce_flat("sum", f32(case["x"]))
    assert z[0] == np.float32(case["expect"])


@pytest.mark.parametrize("n", [0, 1, 5, 7, 8, 9, 15, 16, 17, 63, 64, 65, 1000, 4099])
def test_sum_flat_small_integers_exact(orc, n):
    rng = np.random.default_rng(n)
    x = rng.integers(-100, 101, size=n).astype(np.float32)
    z = orc.reduce_flat("sum", x)
    assert z[0] == np.float32(int(x.astype(np.int64).sum()))


@pytest.mark.parametrize("n", [3, 8, 1000, 65537, 1 << 20])
def test_sum_flat_vs_float64(orc, n):
    rng = np.random.default_rng(100 + n)
    x = rng.uniform(-1, 1, n).astype(np.float32)
    z = orc.reduce_flat("sum", x)[0]
    exact = np.sum(x.astype(np.float64))
    # n/8 sequential adds per lane: error <= (n/8 + 3) * eps32 * sum|x|
    bound = (n / 8 + 3) * 2.0 ** -24 * np.sum(np.abs(x.astype(np.float64)))
    assert abs(float(z) - exact) <= bound


@pytest.mark.parametrize("outer,dim,inner", [(1, 7, 3), (2, 5, 9), (1, 257, 33), (3, 64, 17), (1, 4, 4096)])
def test_sum_axis_inner_matches_numpy_rowwise_order(orc, outer, dim, inner):
    # numpy reduces axis 1 of a C-ordered [outer, dim, inner] array by adding
    # slices d = 0, 1, 2, ... into the output in float32: the same order as
    # reduce.cpp:44-62, so the results are bit-identical.
    rng = np.random.default_rng(outer * 1000 + dim + inner)
    x = rng.normal(size=(outer, dim, inner)).astype(np.float32)
    z = orc.reduce_axis("sum", x, outer, dim, inner)
    ref = np.add.reduce(x, axis=1, dtype=np.float32).ravel()
    assert np.array_equal(z, ref)


@pytest.mark.parametrize("outer,dim,inner", [(5, 9, 1), (3, 1024, 1), (2, 3, 7), (1, 1000, 1)])
def test_sum_axis_integers_exact(orc, outer, dim, inner):
    rng = np.random.default_rng(7 + outer + dim + inner)
    x = rng.integers(-50, 51, size=(outer, dim, inner)).astype(np.float32)
    z = orc.reduce_axis("sum", x, outer, dim, inner)
    ref = x.astype(np.int64).sum(axis=1).ravel().astype(np.float32)
    assert np.array_equal(z, ref)


def test_sum_axis_row_equals_flat_per_row(orc):
    # reduce.cpp:31-36: inner==1 runs the flat sum on every row.
    x = KAT["sum_flat"][0]["x"]
    rows = np.array([x, x[::-1]], np.float32)
    z = orc.reduce_axis("sum", rows, 2, 8, 1)
    assert z[0] == 6.0 and z[1] == orc.reduce_flat("sum", rows[1])[0]


# ----------------------------------------------------------------- mean

def test_mean_axis_reciprocal_body_division_tail(orc):
    # 9 outputs, each a row [1,2,2] summing to 5.  reduce.cpp:77-80 multiplies
    # the first 8 by rn(1/3) = 0x3eaaaaab: 5 * 0.333333343 = 1.66666672 rounds
    # to 0x3fd55556; reduce.cpp:81-83 divides the 9th: rn(5/3) = 0x3fd55555.
    case = KAT["mean_axis"][0]
    x = np.tile(f32(case["row"]), case["outer"])
    z = orc.reduce_axis("mean", x, case["outer"], case["dim"], case["inner"])
    assert all(hexf(v) == case["expect_body_hex"] for v in z[:8])
    assert hexf(z[8]) == case["expect_tail_hex"]


@pytest.mark.parametrize("n", [1, 3, 8, 4096, 1 << 16])
def test_mean_flat_is_sum_over_n(orc, n):
    rng = np.random.default_rng(n)
    x = rng.integers(-100, 101, size=n).astype(np.float32)
    z = orc.reduce_flat("mean", x)[0]
    s = int(x.astype(np.int64).sum())
    assert z == np.float32(np.float32(s) / np.float32(n))


# ------------------------------------------------------------ max / argmax

@pytest.mark.parametrize("outer,dim,inner", [(1, 1, 1), (1, 13, 1), (7, 100, 1), (1, 9, 5), (4, 33, 17), (2, 8, 8)])
def test_max_argmax_brute_force(orc, outer, dim, inner):
    rng = np.random.default_rng(outer + 10 * dim + 100 * inner)
    # quantised values so that ties are frequent; no -0.0 and no NaN
    x = (rng.integers(-20, 21, size=(outer, dim, inner)) * 0.25).astype(np.float32)
    zmax = orc.reduce_axis("max", x, outer, dim, inner)
    zarg = orc.reduce_axis("argmax", x, outer, dim, inner)
    assert np.array_equal(zmax, x.max(axis=1).ravel())
    assert np.array_equal(zarg, x.argmax(axis=1).ravel().astype(np.int32))  # first occurrence


@pytest.mark.parametrize("n", [1, 7, 8, 9, 31, 1000])
def test_max_argmax_flat_brute_force(orc, n):
    rng = np.random.default_rng(1000 + n)
    x = (rng.integers(-5, 6, size=n) * 0.5).astype(np.float32)
    assert orc.reduce_flat("max", x)[0] == x.max()
    assert orc.reduce_flat("argmax", x)[0] == int(np.argmax(x))


def test_max_kats(orc):
    c0, c1 = KAT["max"]
    z = orc.reduce_flat("max", f32([float(v) for v in c0["x"]]))
    assert hexf(z[0]) == c0["expect_hex"]  # -FLT_MAX, reduce.cpp:206
    z = orc.reduce_axis("max", f32([float(v) for v in c1["x"]]), c1["outer"], c1["dim"], c1["inner"])
    assert np.all(np.isneginf(z))


@pytest.mark.parametrize("case", KAT["argmax"], ids=lambda c: c["name"])
def test_argmax_kats(orc, case):
    assert orc.reduce_flat("argmax", f32(case["x"]))[0] == case["expect"]


# --------------------------------------------------- elementwise ops

@pytest.mark.parametrize("op,npf", [(0, np.add), (1, np.subtract), (2, np.multiply), (3, np.divide)])
def test_binary_bcast_scalar_vs_numpy_float32(orc, op, npf):
    # numpy float32 arithmetic is IEEE single-rounded: the reference's
    # _mm256_{add,sub,mul,div}_ps and scalar tails round the same way.
    rng = np.random.default_rng(op)
    x = rng.normal(size=(13, 29)).astype(np.float32)
    y = rng.uniform(0.5, 2.0, size=(13, 29)).astype(np.float32)
    r = rng.uniform(0.5, 2.0, size=29).astype(np.float32)
    c = rng.uniform(0.5, 2.0, size=13).astype(np.float32)
    assert np.array_equal(orc.binary(x, y, op), npf(x, y))
    assert np.array_equal(orc.bcast_row(x, r, op), npf(x, r[None, :]))
    assert np.array_equal(orc.bcast_col(x, c, op), npf(x, c[:, None]))
    assert np.array_equal(orc.scalar(x, 0.37, op), npf(x, np.float32(0.37)))


def test_binary_max_min(orc):
    rng = np.random.default_rng(3)
    x = rng.normal(size=1000).astype(np.float32)
    y = rng.normal(size=1000).astype(np.float32)
    assert np.array_equal(orc.binary(x, y, 4), np.maximum(x, y))
    assert np.array_equal(orc.binary(x, y, 5), np.minimum(x, y))


def test_relu_special_values(orc):
    # max(0, x) = (0 > x) ? 0 : x: -0.0 and NaN pass through (functions.hpp:372-374)
    x = f32([-0.0, np.nan, -1.0, 2.5, 0.0, -np.inf, np.inf])
    z = orc.unary(x, 1)
    assert np.signbit(z[0]) and z[0] == 0
    assert np.isnan(z[1])
    assert z[2] == 0 and not np.signbit(z[2])
    assert z[3] == 2.5 and z[4] == 0 and z[5] == 0 and z[6] == np.inf
    rng = np.random.default_rng(5)
    v = rng.normal(size=10000).astype(np.float32)
    assert np.array_equal(orc.unary(v, 1), np.maximum(v, np.float32(0)))


@pytest.mark.parametrize("act,ref", [(2, lambda d: 1.0 / (1.0 + np.exp(-d))), (3, np.tanh), (4, np.exp)])
def test_transcendentals_within_2ulp_of_float64(orc, act, ref):
    rng = np.random.default_rng(act)
    x = np.concatenate([rng.normal(0, 4, 200000), np.linspace(-20, 20, 100001)]).astype(np.float32)
    if act == 4:
        x = x[x < 80]
    z = orc.unary(x, act)
    with np.errstate(over="ignore"):
        exact = ref(x.astype(np.float64)).astype(np.float32)
    assert ulp_dist(z, exact).max() <= 2


# -------------------------------------------------------------- softmax

@pytest.mark.parametrize("name", ["sm_small", "sm_mask"])
@pytest.mark.parametrize("mode", ["soft", "log"])
def test_softmax_vs_torch_float64(orc, name, mode):
    x = FIX[f"{name}_x"]
    dy = FIX[f"{name}_dy"]
    log = mode == "log"
    y = orc.softmax_fwd(x, log)
    ref = FIX[f"{name}_{mode}_y"]
    fin = np.isfinite(ref)
    assert np.array_equal(np.isfinite(y), fin)
    if log:
        assert np.all(np.isneginf(y[~fin]))
        assert np.allclose(y[fin], ref[fin], rtol=1e-5, atol=1e-5)
    else:
        assert np.allclose(y, ref, rtol=1e-5, atol=1e-7)
    dx = orc.softmax_bwd(y, dy, log)
    refdx = FIX[f"{name}_{mode}_dx"]
    scale = np.abs(refdx).max()
    assert np.allclose(dx, refdx, rtol=1e-4, atol=1e-5 * scale)


def test_softmax_invariants(orc):
    rng = np.random.default_rng(11)
    x = (rng.normal(size=(6, 1000)) * 8).astype(np.float32)
    x[0] = 3.25  # constant row -> exactly 1/N after exp(0)=1, sum=N (exact), 1/N
    x[1, ::3] = -np.inf
    y = orc.softmax_fwd(x)
    assert np.all(y[0] == np.float32(1.0) / np.float32(1000))
    assert np.all(y[1, ::3] == 0)
    assert np.allclose(y.astype(np.float64).sum(axis=1), 1.0, atol=1e-5)
    yl = orc.softmax_fwd(x, log=True)
    assert np.all(np.isneginf(yl[1, ::3]))
    # shift invariance: adding a power of two that keeps x exact
    y2 = orc.softmax_fwd(x + np.float32(64.0))
    assert np.allclose(y2, y, rtol=1e-5, atol=1e-7)


def test_affine_act_vs_torch_float64(orc):
    x, s, b, dy = FIX["aff_x"], FIX["aff_scale"], FIX["aff_bias"], FIX["aff_dy"]
    for act, an in ((1, "relu"), (2, "sigmoid"), (3, "tanh")):
        y = orc.affine_act_fwd(x, s, b, act)
        assert np.allclose(y, FIX[f"aff_{an}_y"], rtol=3e-7, atol=1e-7), an
        dx, ds, db = orc.affine_act_bwd(x, s, y, dy, act)
        assert np.allclose(dx, FIX[f"aff_{an}_dx"], rtol=1e-5, atol=1e-6), an
        assert np.allclose(ds, FIX[f"aff_{an}_dscale"], rtol=1e-5, atol=1e-5), an
        assert np.allclose(db, FIX[f"aff_{an}_dbias"], rtol=1e-5, atol=1e-5), an


def test_affine_relu_forward_bit_exact_two_roundings(orc):
    # forward relu is pure IEEE mul, add, select: numpy float32 gives the same bits
    rng = np.random.default_rng(9)
    x = rng.normal(size=(7, 45)).astype(np.float32)
    s = rng.uniform(0.5, 1.5, 45).astype(np.float32)
    b = rng.normal(0, 0.1, 45).astype(np.float32)
    y = orc.affine_act_fwd(x, s, b, 1)
    assert np.array_equal(y, np.maximum((x * s) + b, np.float32(0)))


# --------------------------------------------------------------- matmul

def test_matmul_k_panel_kat(orc):
    # K=264, A = ones, B[:,0] = [2^24] + [1]*263.  Panel 0 (k<256): fma chain
    # 2^24 + 1 + ... stays 2^24 (each +1 ties to even).  Panel 1: 8 ones = 8.
    # C = 2^24 + 8 = 16777224 exactly.  One long chain would give 2^24; a
    # 128-wide panel would give 2^24 + 136.
    k = KAT["matmul"][0]["k"]
    a = np.ones((1, k), np.float32)
    b = np.ones((k, 3), np.float32)
    b[0, 0] = 2.0 ** 24
    c = orc.matmul(a, b)
    assert c[0, 0] == np.float32(KAT["matmul"][0]["expect"])
    assert c[0, 1] == k


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (9, 17, 13), (33, 300, 65), (64, 784, 10)])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True)])
def test_gemm_vs_float64(orc, m, k, n, ta, tb):
    rng = np.random.default_rng(m * k + n)
    a = rng.normal(size=(k, m) if ta else (m, k)).astype(np.float32)
    b = rng.normal(size=(n, k) if tb else (k, n)).astype(np.float32)
    c = orc.gemm(a, b, ta, tb)
    A = (a.T if ta else a).astype(np.float64)
    B = (b.T if tb else b).astype(np.float64)
    ref = A @ B
    bound = 1e-5 * (np.abs(A) @ np.abs(B))
    assert np.all(np.abs(c - ref) <= bound)


def test_matmul_small_integers_exact(orc):
    rng = np.random.default_rng(2)
    a = rng.integers(-8, 9, size=(20, 600)).astype(np.float32)
    b = rng.integers(-8, 9, size=(600, 30)).astype(np.float32)
    assert np.array_equal(orc.matmul(a, b), (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32))


# ------------------------------------------------------------------ MLP

def test_softmax_xent_vs_torch(orc):
    loss, dl = orc.softmax_xent(FIX["xent_logits"], FIX["xent_labels"])
    assert math.isclose(loss, float(FIX["xent_loss"][0]), rel_tol=1e-6)
    assert np.allclose(dl, FIX["xent_dlogits"], rtol=1e-5, atol=1e-7)


def test_sgd_two_roundings(orc):
    w = f32([1.0, -2.0, 3.0])
    g = f32([0.5, 0.25, -1.0])
    assert np.array_equal(orc.sgd(w, g, 0.01), w - g * np.float32(0.01))


def test_mlp_two_steps_vs_torch(orc):
    x, lab = FIX["mlp_x"], FIX["mlp_labels"]
    params = {k: FIX[f"mlp_init_{k}"].astype(np.float32).copy() for k in ("w1", "b1", "w2", "b2", "w3", "b3")}
    losses = [orc.mlp_step(x, lab, params, 0.01) for _ in range(2)]
    assert np.allclose(losses, FIX["mlp_losses"], rtol=1e-5)
    for k, v in params.items():
        ref = FIX[f"mlp_final_{k}"]
        assert np.allclose(v, ref, rtol=1e-4, atol=1e-6), k


# ------------------------------------------------------- elementwise math

def _round_f32(fr):
    """Nearest float32 to an exact rational (ties to even)."""
    from fractions import Fraction
    c = np.float32(float(fr))
    best = None
    for cand in (np.nextafter(c, np.float32(-np.inf)), c, np.nextafter(c, np.float32(np.inf))):
        d = abs(Fraction(float(cand)) - fr)
        key = (d, int(np.float32(cand).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, cand)
    return np.float32(best[1])


def test_wise_exact_ops_vs_numpy(orc):
    # square/abs/neg are exact or single-rounded; numpy float32 ufuncs are IEEE.
    rng = np.random.default_rng(41)
    x = np.concatenate([rng.normal(0, 1e3, 5000), [0.0, -0.0, np.inf, -np.inf, 3e19, -3e19]]).astype(np.float32)
    with np.errstate(over="ignore"):
        assert np.array_equal(orc.wise(x, orc.FN_SQUARE).view(np.uint32), np.square(x).view(np.uint32))
    assert np.array_equal(orc.wise(x, orc.FN_ABS).view(np.uint32), np.abs(x).view(np.uint32))
    assert np.array_equal(orc.wise(x, orc.FN_NEG).view(np.uint32), np.negative(x).view(np.uint32))


def test_wise_correctly_rounded_ops_vs_numpy(orc):
    # sqrt and 1/x are correctly rounded in IEEE arithmetic (numpy float32)
    rng = np.random.default_rng(42)
    x = np.abs(rng.normal(0, 50, 20000)).astype(np.float32) + np.float32(1e-30)
    assert np.array_equal(orc.wise(x, orc.FN_SQRT), np.sqrt(x))
    y = np.concatenate([x, -x]).astype(np.float32)
    assert np.array_equal(orc.wise(y, orc.FN_RCP), np.float32(1.0) / y)
    assert np.array_equal(orc.wise(y, orc.FN_INVERSE), np.float32(1.0) / y)
    # rsqrt = 1/sqrt(x): two correctly rounded steps stay within 1 ulp of exact
    exact = (1.0 / np.sqrt(x.astype(np.float64))).astype(np.float32)
    assert ulp_dist(orc.wise(x, orc.FN_RSQRT), exact).max() <= 1


def test_wise_sign_table(orc):
    x = f32([3.5, -2.0, 0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45])
    z = orc.wise(x, orc.FN_SIGN)
    assert z.tolist()[:6] == [1.0, -1.0, 0.0, 0.0, 1.0, -1.0]
    assert z[6] == 0.0 and not np.signbit(z[6])  # ordered compares: NaN -> +0
    assert not np.signbit(z[3])  # sign(-0) = +0
    assert z[7] == 1.0 and z[8] == -1.0  # denormals keep their sign
    v = np.random.default_rng(43).normal(size=1000).astype(np.float32)
    assert np.array_equal(orc.wise(v, orc.FN_SIGN), np.sign(v))


@pytest.mark.parametrize("fn,lo,hi,ref", [
    ("FN_LOG", 1e-30, 1e30, np.log), ("FN_EXP", -87.0, 88.0, np.exp),
    ("FN_SIN", -100.0, 100.0, np.sin), ("FN_COS", -100.0, 100.0, np.cos),
    ("FN_ERF", -6.0, 6.0, None)])
def test_wise_transcendentals_within_1ulp_of_float64(orc, fn, lo, hi, ref):
    import scipy.special
    rng = np.random.default_rng(44)
    if fn == "FN_LOG":
        x = np.exp(rng.uniform(np.log(lo), np.log(hi), 50000)).astype(np.float32)
    else:
        x = rng.uniform(lo, hi, 50000).astype(np.float32)
    f = scipy.special.erf if ref is None else ref
    exact = f(x.astype(np.float64)).astype(np.float32)
    assert ulp_dist(orc.wise(x, getattr(orc, fn)), exact).max() <= 1


def test_pow_vs_float64(orc):
    rng = np.random.default_rng(45)
    x = rng.uniform(0.01, 10, 20000).astype(np.float32)
    y = rng.uniform(-6, 6, 20000).astype(np.float32)
    exact = np.power(x.astype(np.float64), y.astype(np.float64)).astype(np.float32)
    assert ulp_dist(orc.binary(x, y, orc.POW), exact).max() <= 1
    e2 = np.power(x.astype(np.float64), np.float64(np.float32(2.5))).astype(np.float32)
    assert ulp_dist(orc.scalar(x, 2.5, orc.POW), e2).max() <= 1
    # IEEE special cases of pow
    sx = f32([-2.0, -2.0, 0.0, 1.0, 5.0, np.nan])
    sy = f32([3.0, 0.5, -1.0, np.nan, 0.0, 0.0])
    z = orc.binary(sx, sy, orc.POW)
    assert z[0] == -8.0 and np.isnan(z[1]) and z[2] == np.inf and z[3] == 1.0 and z[4] == 1.0 and z[5] == 1.0


def test_lerp_single_fma_rounding(orc):
    # exact rational x + v2*(v1 - x) with (v1 - x) rounded to float32 first,
    # rounded once: a two-rounding mul+add or an unrounded difference fails
    from fractions import Fraction
    rng = np.random.default_rng(46)
    x = rng.normal(0, 10, 600).astype(np.float32)
    v1, v2 = np.float32(3.3), np.float32(0.7)
    z = orc.lerp(x, v1, v2)
    d = (v1 - x).astype(np.float32)
    for i in range(x.size):
        exact = Fraction(float(v2)) * Fraction(float(d[i])) + Fraction(float(x[i]))
        assert z[i] == _round_f32(exact), i


def test_clamp_vs_numpy_clip(orc):
    rng = np.random.default_rng(47)
    x = rng.normal(0, 3, 10000).astype(np.float32)
    assert np.array_equal(orc.clamp(x, -1.5, 2.0), np.clip(x, np.float32(-1.5), np.float32(2.0)))
    z = orc.clamp(f32([np.nan, -np.inf, np.inf]), -1.0, 1.0)
    assert z.tolist() == [-1.0, -1.0, 1.0]  # _mm256_max_ps(NaN, lo) = lo


def test_gather_vs_numpy_indexing(orc):
    rng = np.random.default_rng(48)
    x = rng.normal(size=1000).astype(np.float32)
    xi = rng.integers(-1000, 1000, 1000).astype(np.int32)
    idx = rng.integers(0, 1000, 5000).astype(np.int32)
    assert np.array_equal(orc.gather(x, idx), x[idx])
    assert np.array_equal(orc.gather(xi, idx), xi[idx])
    bad = np.array([-1, 1000, 5], np.int32)
    zf, zi = orc.gather(x, bad), orc.gather(xi, bad)
    assert np.isnan(zf[0]) and np.isnan(zf[1]) and zf[2] == x[5]
    assert zi.tolist() == [-(2 ** 31), -(2 ** 31), xi[5]]


# ------------------------------------------------- min, argmin, norms, var

@pytest.mark.parametrize("outer,dim,inner", [(1, 1, 1), (1, 13, 1), (7, 100, 1), (1, 9, 5), (4, 33, 17), (2, 8, 8)])
def test_min_argmin_brute_force(orc, outer, dim, inner):
    rng = np.random.default_rng(7 * outer + 10 * dim + 100 * inner)
    x = (rng.integers(-20, 21, size=(outer, dim, inner)) * 0.25).astype(np.float32)
    assert np.array_equal(orc.reduce_axis("min", x, outer, dim, inner), x.min(axis=1).ravel())
    assert np.array_equal(orc.reduce_axis("argmin", x, outer, dim, inner),
                          x.argmin(axis=1).ravel().astype(np.int32))  # first occurrence


@pytest.mark.parametrize("n", [1, 7, 8, 9, 31, 1000])
def test_min_argmin_flat_brute_force(orc, n):
    rng = np.random.default_rng(2000 + n)
    x = (rng.integers(-5, 6, size=n) * 0.5).astype(np.float32)
    assert orc.reduce_flat("min", x)[0] == x.min()
    assert orc.reduce_flat("argmin", x)[0] == int(np.argmin(x))


def test_min_start_values(orc):
    # flat and row forms start from FLT_MAX (reduce.cpp:255, 271), the column
    # form from slice 0 (reduce.cpp:285-293)
    inf = f32([np.inf] * 12)
    assert hexf(orc.reduce_flat("min", inf)[0]) == "0x7f7fffff"
    assert hexf(orc.reduce_axis("min", inf, 3, 4, 1)[0]) == "0x7f7fffff"
    assert np.all(np.isposinf(orc.reduce_axis("min", inf, 1, 3, 4)))
    assert orc.reduce_flat("argmin", inf)[0] == 0


@pytest.mark.parametrize("outer,dim,inner", [(1, 7, 3), (2, 5, 9), (1, 257, 33), (3, 64, 17)])
def test_norm1_axis_matches_numpy_rowwise_order(orc, outer, dim, inner):
    # |slice 0| then |slice d| added in order: numpy's axis-1 float32 reduce of |x|
    rng = np.random.default_rng(3 * outer + dim + inner)
    x = rng.normal(size=(outer, dim, inner)).astype(np.float32)
    ref = np.add.reduce(np.abs(x), axis=1, dtype=np.float32).ravel()
    assert np.array_equal(orc.reduce_axis("norm1", x, outer, dim, inner), ref)


@pytest.mark.parametrize("outer,dim,inner", [(1, 1000, 1), (5, 9, 1), (2, 3, 7), (1, 77, 12)])
def test_norms_small_integers_exact(orc, outer, dim, inner):
    # |x| and x*x of small integers and their sums are exact in float32, in any order
    rng = np.random.default_rng(11 + outer + dim + inner)
    x = rng.integers(-40, 41, size=(outer, dim, inner)).astype(np.float32)
    xi = x.astype(np.int64)
    n1 = np.abs(xi).sum(axis=1).ravel().astype(np.float32)
    n2 = np.sqrt((xi * xi).sum(axis=1).ravel().astype(np.float32))
    assert np.array_equal(orc.reduce_axis("norm1", x, outer, dim, inner), n1)
    assert np.array_equal(orc.reduce_axis("norm2", x, outer, dim, inner), n2)
    if inner == 1 and outer == 1:
        assert orc.reduce_flat("norm1", x)[0] == n1[0]
        assert orc.reduce_flat("norm2", x)[0] == n2[0]


@pytest.mark.parametrize("n", [5, 4099, 1 << 16])
def test_norms_vs_float64(orc, n):
    x = np.random.default_rng(n).normal(size=n).astype(np.float32)
    d = x.astype(np.float64)
    assert abs(orc.reduce_flat("norm1", x)[0] - np.abs(d).sum()) <= 1e-5 * np.abs(d).sum()
    assert abs(orc.reduce_flat("norm2", x)[0] - np.sqrt((d * d).sum())) <= 1e-5 * np.sqrt((d * d).sum())


def test_var_axis_reciprocal_body_division_tail(orc):
    # 9 columns, each (0.5, 2.5, 3.0): the column mean is exactly 2 and the
    # squared deviations sum to exactly 3.5.  reduce.cpp:173-182 multiplies
    # the first 8 outputs by rn(1/3): 3.5 * 0.333333343 rounds to 0x3f955556;
    # the 9th divides: rn(3.5/3) = 0x3f955555.  Rows divide (reduce.cpp:135).
    x = np.repeat(f32([0.5, 2.5, 3.0]), 9).reshape(3, 9)
    z = orc.reduce_axis("var", x, 1, 3, 9)
    assert all(hexf(v) == "0x3f955556" for v in z[:8]) and hexf(z[8]) == "0x3f955555"
    zr = orc.reduce_axis("var", f32([0.5, 2.5, 3.0] * 4), 4, 3, 1)
    assert all(hexf(v) == "0x3f955555" for v in zr)
    assert hexf(orc.reduce_flat("var", f32([0.5, 2.5, 3.0]))[0]) == "0x3f955555"
    s = orc.reduce_axis("stdv", x, 1, 3, 9)
    assert np.array_equal(s, np.sqrt(z))  # stdv = sqrt(var), reduce.cpp:190-202


@pytest.mark.parametrize("outer,dim,inner", [(1, 4099, 1), (3, 1000, 1), (1, 500, 40), (2, 37, 9)])
def test_var_stdv_vs_float64(orc, outer, dim, inner):
    rng = np.random.default_rng(outer + dim + inner)
    x = rng.normal(3.0, 2.0, size=(outer, dim, inner)).astype(np.float32)
    d = x.astype(np.float64)
    v = d.var(axis=1).ravel()  # population variance
    assert np.all(np.abs(orc.reduce_axis("var", x, outer, dim, inner) - v) <= 1e-5 * v)
    assert np.all(np.abs(orc.reduce_axis("stdv", x, outer, dim, inner) - np.sqrt(v)) <= 1e-5 * np.sqrt(v))
    f = x.ravel()
    assert abs(orc.reduce_flat("var", f)[0] - f.astype(np.float64).var()) <= 1e-5 * f.astype(np.float64).var()


def test_var_closed_forms(orc):
    assert orc.reduce_flat("var", f32([7.25] * 1001))[0] == 0.0  # constant
    assert orc.reduce_flat("var", f32([-3.0, 3.0] * 64))[0] == 9.0  # +-c: c^2
    assert orc.reduce_flat("stdv", f32([-3.0, 3.0] * 64))[0] == 3.0
    assert np.isnan(orc.reduce_flat("var", np.zeros(0, np.float32))[0])  # 0/0


@pytest.mark.parametrize("act", [1, 2, 3])
def test_act_bwd_is_affine_bwd_with_unit_scale(orc, act):
    # dx of the (already pinned) affine backward with scale 1 is dy*act'(y)
    # exactly (the product with 1 is exact), so act_bwd must match it bit for bit
    rng = np.random.default_rng(60 + act)
    x = rng.normal(size=(7, 33)).astype(np.float32)
    y = orc.unary(x, act) if act != 1 else np.maximum(x, 0).astype(np.float32)
    dy = rng.normal(size=(7, 33)).astype(np.float32)
    dx_aff, _, _ = orc.affine_act_bwd(x, np.ones(33, np.float32), y, dy, act)
    assert np.array_equal(orc.act_bwd(y, dy, act), dx_aff)
    if act == 1:  # relu' = [y > 0]: zero where y <= 0, dy elsewhere
        assert np.array_equal(orc.act_bwd(y, dy, act), np.where(y > 0, dy, np.float32(0) * dy))


# ------------------------------------------------------------ 16-bit casts

def test_bf16_f16_widening_exhaustive(orc):
    # every 16-bit pattern: bf16 widens to bits << 16; f16 widens as numpy's IEEE float16
    h = np.arange(65536, dtype=np.uint16)
    wb = orc.convert(h, orc.DT_BF16, orc.DT_F32)
    assert np.array_equal(wb.view(np.uint32), h.astype(np.uint32) << 16)
    wf = orc.convert(h, orc.DT_F16, orc.DT_F32)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(wf), nan) and np.array_equal(wf[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    # round trips are the identity on non-NaN patterns
    assert np.array_equal(orc.convert(wb, orc.DT_F32, orc.DT_BF16)[~np.isnan(wb)], h[~np.isnan(wb)])
    assert np.array_equal(orc.convert(wf, orc.DT_F32, orc.DT_F16)[~nan], h[~nan])


def test_f32_to_bf16_round_to_nearest_even(orc):
    # exact integer rounding of the 32-bit pattern to its top 16 bits, ties to even
    rng = np.random.default_rng(71)
    u = rng.integers(0, 2 ** 32, 200000, dtype=np.uint64).astype(np.uint32)
    u = u[(u & 0x7FFFFFFF) < 0x7F800000]  # finite
    u = np.concatenate([u, np.array([0x3F808000, 0x3F818000, 0x3F807FFF, 0x7F7FFFFF, 0x00008000], np.uint32)])
    f = u.view(np.float32)
    got = orc.convert(f, orc.DT_F32, orc.DT_BF16).astype(np.uint64)
    hi, lo = u.astype(np.uint64) >> 16, u.astype(np.uint64) & 0xFFFF
    exp = hi + ((lo > 0x8000) | ((lo == 0x8000) & (hi & 1 == 1))).astype(np.uint64)
    assert np.array_equal(got, exp)  # 0x7F7FFFFF rounds up to 0x7F80 (inf), as RNE does
    nanb = orc.convert(np.array([np.nan, -np.nan], np.float32), orc.DT_F32, orc.DT_BF16)
    assert np.all(np.isnan(orc.convert(nanb, orc.DT_BF16, orc.DT_F32)))


def test_f32_to_f16_matches_numpy(orc):
    rng = np.random.default_rng(72)
    f = np.concatenate([rng.normal(0, 100, 100000), rng.normal(0, 1e-5, 10000),
                        [65504.0, 65520.0, 1e6, -1e6, 6e-8, 0.0, -0.0, np.inf, -np.inf]]).astype(np.float32)
    assert np.array_equal(orc.convert(f, orc.DT_F32, orc.DT_F16), f.astype(np.float16).view(np.uint16))
