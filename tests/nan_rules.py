"""The library's NaN / signed-zero rule for max, min, argmax and argmin
(include/cxm_hip.h, reductions), restated in numpy for the tests.

`arg_loop` is the reference's axis loop (Engine/AVX2/reduce.cpp:483-521 for
argmax, 590-617 for argmin): start from element 0, take strictly better
values.  `arg_rule` is the vectorised statement of the same rule (NaN first
element -> 0, else the first best over the non-NaN elements, +0 == -0);
tests/test_nan_rules.py checks the two against each other."""
import numpy as np


def arg_loop(op, v):
    best, idx = v[0], 0
    for k in range(1, len(v)):
        if (v[k] > best) if op == "argmax" else (v[k] < best):
            best, idx = v[k], k
    return idx


def arg_rule(op, a):
    """a: [slices, n] float32; the index per slice."""
    a = np.asarray(a, np.float32)
    nan = np.isnan(a)
    fill = -np.inf if op == "argmax" else np.inf
    b = np.where(nan, np.float32(fill), a)
    m = b.max(axis=1) if op == "argmax" else b.min(axis=1)
    hit = (a == m[:, None])  # NaN never equal; +0 == -0
    idx = np.argmax(hit, axis=1)
    return np.where(nan[:, 0], 0, idx).astype(np.int32)


def value_rule(op, a, start=None):
    """a: [slices, n]; IEEE 754-2019 maximum / minimum per slice, with the
    start value (the flat and row forms' -FLT_MAX / FLT_MAX) folded in."""
    a = np.asarray(a, np.float32)
    if start is not None:
        a = np.concatenate([a, np.full((a.shape[0], 1), start, np.float32)], axis=1)
    nan = np.isnan(a).any(axis=1)
    m = (a.max(axis=1) if op == "max" else a.min(axis=1)).astype(np.float32)
    z = a == 0
    has_pos = (z & ~np.signbit(a)).any(axis=1)
    has_neg = (z & np.signbit(a)).any(axis=1)
    zero = m == 0
    if op == "max":
        m = np.where(zero, np.where(has_pos, np.float32(0.0), np.float32(-0.0)), m)
    else:
        m = np.where(zero, np.where(has_neg, np.float32(-0.0), np.float32(0.0)), m)
    return np.where(nan, np.float32(np.nan), m).astype(np.float32)
