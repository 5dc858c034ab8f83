"""Parity of the gfx950 MLP training step (cxm_mlp3_step_f32) with the CPU
oracle's step (oracle/cxm_oracle.c: orc_mlp_step, composed of the reference
primitives) and with float64 torch answers committed under tests/golden/.

Bars: per-step loss within 1e-5 relative of the oracle; weights after the
steps within 1e-4 relative to the size of the update path (fp32 GEMM sums
differ in order, and the difference compounds over steps).
"""
import os

import numpy as np
import pytest

from cortexmind_amd import engine
from cortexmind_amd.data import c5_mlp

from gpu_util import dev, empty

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
FIX = np.load(os.path.join(HERE, "golden", "fixtures_f64.npz"))


def gpu_steps(x, labels, params, lr, steps):
    b, d0 = x.shape
    d1, d2, d3 = params["w1"].shape[1], params["w2"].shape[1], params["w3"].shape[1]
    net = engine.Mlp3(b, d0, d1, d2, d3)
    dx, dlab, dloss = dev(x), dev(labels), empty((1,))
    dp = {k: dev(v) for k, v in params.items()}
    losses = []
    for _ in range(steps):
        net.step(dx, dlab, dp, lr, dloss)
        losses.append(float(dloss.numpy()[0]))
    net.close()
    return losses, {k: v.numpy() for k, v in dp.items()}


def test_mlp_vs_oracle_reduced_batch(hip, orc):
    """C5 layer sizes (784 -> 1024 -> 1024 -> 10), batch 256, 3 steps."""
    x, labels, params = c5_mlp(batch=256)
    losses, final = gpu_steps(x, labels, params, 0.01, 3)
    ref = {k: v.copy() for k, v in params.items()}
    ref_losses = [orc.mlp_step(x, labels, ref, 0.01) for _ in range(3)]
    for got, want in zip(losses, ref_losses):
        assert abs(got - want) <= 1e-5 * abs(want), (losses, ref_losses)
    for k in ref:
        scale = np.abs(params[k]).max() + 1e-3
        assert np.max(np.abs(final[k] - ref[k])) <= 1e-4 * scale, k
    assert ref_losses[-1] < ref_losses[0]


def test_mlp_float64_fixture(hip):
    """Two steps of a 49 -> 32 -> 32 -> 10 MLP against float64 torch."""
    x, labels = FIX["mlp_x"], FIX["mlp_labels"]
    params = {k: FIX[f"mlp_init_{k}"].astype(np.float32) for k in ["w1", "b1", "w2", "b2", "w3", "b3"]}
    losses, final = gpu_steps(x, labels, params, 0.01, 2)
    for got, want in zip(losses, FIX["mlp_losses"]):
        assert abs(got - want) <= 1e-5 * abs(want)
    for k in params:
        assert np.max(np.abs(final[k] - FIX[f"mlp_final_{k}"])) <= 1e-5 * (np.abs(FIX[f"mlp_final_{k}"]).max() + 1e-3), k


def test_mlp_full_size_ten_steps(hip):
    """C5 at full size: batch 4096, 10 SGD steps; loss finite and falling,
    first loss close to ln(10) for He-normal weights on U(0,1) inputs."""
    x, labels, params = c5_mlp()
    losses, final = gpu_steps(x, labels, params, 0.01, 10)
    assert all(np.isfinite(losses))
    assert losses[-1] < losses[0]
    assert all(np.all(np.isfinite(v)) for v in final.values())
