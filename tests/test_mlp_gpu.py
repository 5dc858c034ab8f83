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
from cortexmind_amd.data import SplitMix64, c5_mlp

from gpu_util import dev, empty

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
FIX = np.load(os.path.join(HERE, "golden", "fixtures_f64.npz"))


def gpu_steps(x, labels, params, lr, steps, side=None):
    """`steps` fused steps; with `side`, the number of side workgroups of
    each step's paired weight-gradient launch goes into that list."""
    b, d0 = x.shape
    d1, d2, d3 = params["w1"].shape[1], params["w2"].shape[1], params["w3"].shape[1]
    net = engine.Mlp3(b, d0, d1, d2, d3)
    dx, dlab, dloss = dev(x), dev(labels), empty((1,))
    dp = {k: dev(v) for k, v in params.items()}
    losses = []
    for _ in range(steps):
        net.step(dx, dlab, dp, lr, dloss)
        losses.append(float(dloss.numpy()[0]))
        if side is not None:
            side.append(net.last_side())
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


def test_mlp_full_size_ten_steps_vs_oracle(hip, orc):
    """C5 exactly as configured: batch 4096, 784 -> 1024 -> 1024 -> 10, He-normal
    weights, zero biases, 10 SGD steps at lr 0.01, against the oracle's step
    (about 3 s per step on one CPU core).  At this batch the weight gradients
    take the split-K kernels with the fused SGD epilogue, which the reduced
    batch does not reach.  Every step's loss within 1e-5 relative; all six
    tensors after step 10 within 1e-4 of their scale.  The paired
    weight-gradient launch leaves CUs free here, so its side workgroups run
    the output layer's finish and the b1 step (asserted)."""
    x, labels, params = c5_mlp()
    ran = []
    losses, final = gpu_steps(x, labels, params, 0.01, 10, ran)
    assert all(w > 0 for w in ran), ran
    ref = {k: v.copy() for k, v in params.items()}
    ref_losses = []
    for step in range(10):
        ref_losses.append(orc.mlp_step(x, labels, ref, 0.01))
        print(f"step {step}: gpu {losses[step]:.8f} oracle {ref_losses[step]:.8f}", flush=True)
    for got, want in zip(losses, ref_losses):
        assert abs(got - want) <= 1e-5 * abs(want), (losses, ref_losses)
    # A layer's bias moves under the same gradient magnitudes as its weight
    # (b_l's gradient is a column sum of the same dZ_l that forms W_l's), so
    # both are held to 1e-4 of that layer's weight scale; the bias itself
    # starts at zero and stays near 1e-3, where its column sums cancel.
    errs = {}
    for k in ref:
        w = "w" + k[1]
        scale = max(np.abs(params[w]).max(), np.abs(ref[w]).max())
        errs[k] = (float(np.max(np.abs(final[k] - ref[k]))), 1e-4 * float(scale))
        print(f"{k}: max |gpu - oracle| {errs[k][0]:.3e} (bar {errs[k][1]:.3e})", flush=True)
    assert all(e <= bar for e, bar in errs.values()), errs
    assert all(np.isfinite(losses)) and losses[-1] < losses[0]


@pytest.mark.parametrize("batch,dims,side", [
    (100, (49, 64, 36, 3), False), (37, (20, 40, 1024, 16), False), (300, (784, 128, 96, 10), False),
    (64, (16, 24, 1028, 10), False), (16, (8, 8, 4, 1), False), (40, (784, 256, 256, 10), False),
    (520, (784, 1024, 1024, 10), False), (384, (784, 1024, 1024, 10), True), (640, (784, 1024, 1024, 10), True),
    (384, (784, 256, 1024, 10), True)], ids=lambda v: str(v))
def test_mlp_shapes_vs_oracle(hip, orc, batch, dims, side):
    """The fused output layer (d3 <= 16, d2 <= 1024, d2 % 4 == 0) at batch
    sizes off its 16-row tile, with 1, 3 and 16 classes and d2 from 4 to its
    1024 limit; d2 = 1028 takes the unfused kernels.  Batches of 40 and 520
    have a partial last 16-row head tile; their weight gradients (K = batch,
    not a multiple of 128) take the unpaired kernels, and the output layer's
    finish and the b1 step run as kernels of their own.  Batches of 384 and
    640 (multiples of 128, not of 256) pair the weight gradients on the
    ring, with split K at 640, and leave CUs free, so the paired launch's
    side workgroups run the finish and the b1 step, the latter with a
    partial last row tile of its 256-row column sums (rows >= batch
    masked); `side` asserts which path ran.  Random biases, three steps at
    lr 0.05 (0.01 from batch 384 on: at 0.05 the 1024-wide layers overshoot
    and the loss rises at step 2) against the oracle's step, same bars as
    above."""
    x, labels, params = c5_mlp(batch=batch, dims=dims)
    g = SplitMix64(77 + batch)
    for k in ("b1", "b2", "b3"):
        params[k] = g.normal(params[k].shape, 0.0, 0.1)
    lr = 0.05 if batch < 384 else 0.01
    ran = []
    losses, final = gpu_steps(x, labels, params, lr, 3, ran)
    assert all(w > 0 for w in ran) if side else all(w == 0 for w in ran), ran
    ref = {k: v.copy() for k, v in params.items()}
    ref_losses = [orc.mlp_step(x, labels, ref, lr) for _ in range(3)]
    for got, want in zip(losses, ref_losses):
        assert abs(got - want) <= 1e-5 * max(abs(want), 1e-3), (losses, ref_losses)
    for k in ref:
        w = "w" + k[1]
        scale = max(np.abs(params[w]).max(), np.abs(ref[w]).max())
        assert np.max(np.abs(final[k] - ref[k])) <= 1e-4 * scale, k


def test_mlp_pair_without_free_cus_vs_oracle(hip, orc):
    """Hidden widths of 2048: the two weight gradients (256 + 112 ring tiles)
    fill the chip, so the paired launch has no free CUs for the output
    layer's finish and the layer-1 bias step, which then run as their own
    kernels (at the C5 shape they ride on the pair's 16 free CUs).  Three
    steps at the C5 rate (lr 0.01: at 0.05 this width diverges and the
    loss amplifies rounding differences past the bar by the third step)
    against the oracle, same bars as above."""
    x, labels, params = c5_mlp(batch=128, dims=(784, 2048, 2048, 10))
    g = SplitMix64(2048)
    for k in ("b1", "b2", "b3"):
        params[k] = g.normal(params[k].shape, 0.0, 0.1)
    ran = []
    losses, final = gpu_steps(x, labels, params, 0.01, 3, ran)
    assert ran == [0, 0, 0], ran
    ref = {k: v.copy() for k, v in params.items()}
    ref_losses = [orc.mlp_step(x, labels, ref, 0.01) for _ in range(3)]
    for got, want in zip(losses, ref_losses):
        assert abs(got - want) <= 1e-5 * max(abs(want), 1e-3), (losses, ref_losses)
    for k in ref:
        w = "w" + k[1]
        scale = max(np.abs(params[w]).max(), np.abs(ref[w]).max())
        assert np.max(np.abs(final[k] - ref[k])) <= 1e-4 * scale, k
