"""CPU check of tests/nan_rules.py: the vectorised argmax / argmin rule
against the reference's own loop (best = element 0, strictly better values
replace it), and the IEEE maximum / minimum restatement against a pairwise
fold with math's rules, on small inputs full of NaNs, infinities and signed
zeros."""
import math

import numpy as np
import pytest

from nan_rules import arg_loop, arg_rule, value_rule

VALS = np.float32([np.nan, 0.0, -0.0, 1.0, -1.0, 2.0, -2.0, np.inf, -np.inf])


@pytest.mark.parametrize("op", ["argmax", "argmin"])
def test_arg_rule_is_the_reference_loop(op):
    rng = np.random.default_rng(5)
    a = VALS[rng.integers(0, len(VALS), size=(20000, 7))]
    want = np.array([arg_loop(op, v) for v in a], np.int32)
    assert np.array_equal(arg_rule(op, a), want)


def ieee_fold(op, v):
    """maximum / minimum by pairs: NaN wins, +0 above -0 (max), -0 below +0 (min)."""
    m = v[0]
    for x in v[1:]:
        if math.isnan(m) or math.isnan(x):
            m = float("nan")
        elif x == m == 0.0:
            neg = math.copysign(1.0, x) < 0 and math.copysign(1.0, m) < 0
            pos = math.copysign(1.0, x) > 0 and math.copysign(1.0, m) > 0
            if op == "max":
                m = -0.0 if neg else 0.0
            else:
                m = 0.0 if pos else -0.0
        else:
            m = max(m, x) if op == "max" else min(m, x)
    return np.float32(m)


@pytest.mark.parametrize("op", ["max", "min"])
def test_value_rule_is_ieee_maximum(op):
    rng = np.random.default_rng(6)
    a = VALS[rng.integers(0, len(VALS), size=(20000, 6))]
    got = value_rule(op, a)
    want = np.array([ieee_fold(op, [float(t) for t in v]) for v in a], np.float32)
    same = (np.isnan(got) & np.isnan(want)) | (got.view(np.uint32) == want.view(np.uint32))
    assert same.all()
