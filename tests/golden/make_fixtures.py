"""Writes tests/golden/fixtures_f64.npz: float64 answers from torch (a
library, not the reference) for the parts of the path that the reference
lacks and therefore cannot pin itself: softmax / log-softmax and their
backward, affine+activation forward/backward, softmax cross-entropy and two
SGD steps of a small 3-layer ReLU MLP.  Inputs come from the seeded
generator in cortexmind_amd/data.py and are stored as float32 next to the
answers, so the fixture is self-contained.

Run:  python tests/golden/make_fixtures.py
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from cortexmind_amd.data import SplitMix64  # noqa: E402

torch.set_default_dtype(torch.float64)


def t64(a):
    return torch.tensor(np.asarray(a, dtype=np.float64))


def main():
    out = {}
    g = SplitMix64(0x5EED0001)

    # softmax / log-softmax, small dense and masked long-ish rows
    sm_small = g.normal((3, 17), 0.0, 4.0)
    sm_mask = g.normal((4, 300), 0.0, 8.0)
    sm_mask[g.mask_rows(4, 300, 30)] = -np.inf
    for name, x in (("sm_small", sm_small), ("sm_mask", sm_mask)):
        dy = g.normal(x.shape)
        out[f"{name}_x"] = x
        out[f"{name}_dy"] = dy
        for mode, fn in (("soft", torch.softmax), ("log", torch.log_softmax)):
            xt = t64(x).requires_grad_(True)
            y = fn(xt, dim=1)
            y.backward(t64(dy))
            out[f"{name}_{mode}_y"] = y.detach().numpy()
            out[f"{name}_{mode}_dx"] = xt.grad.numpy()

    # affine + activation
    m, n = 5, 37
    ax = g.normal((m, n))
    ascale = g.uniform((n,), 0.5, 1.5)
    abias = g.normal((n,), 0.0, 0.1)
    ady = g.normal((m, n))
    out.update(aff_x=ax, aff_scale=ascale, aff_bias=abias, aff_dy=ady)
    acts = {"relu": torch.relu, "sigmoid": torch.sigmoid, "tanh": torch.tanh}
    for an, fn in acts.items():
        xt = t64(ax).requires_grad_(True)
        st = t64(ascale).requires_grad_(True)
        bt = t64(abias).requires_grad_(True)
        y = fn(xt * st + bt)
        y.backward(t64(ady))
        out[f"aff_{an}_y"] = y.detach().numpy()
        out[f"aff_{an}_dx"] = xt.grad.numpy()
        out[f"aff_{an}_dscale"] = st.grad.numpy()
        out[f"aff_{an}_dbias"] = bt.grad.numpy()

    # softmax cross-entropy
    lg = g.normal((6, 10), 0.0, 2.0)
    lab = g.randint(6, 10)
    lt = t64(lg).requires_grad_(True)
    loss = torch.nn.functional.cross_entropy(lt, torch.tensor(lab.astype(np.int64)))
    loss.backward()
    out.update(xent_logits=lg, xent_labels=lab, xent_loss=np.array([loss.item()]),
               xent_dlogits=lt.grad.numpy())

    # two SGD steps of a 49->32->32->10 ReLU MLP
    b, dims, lr = 16, (49, 32, 32, 10), 0.01
    mx = g.uniform((b, dims[0]), 0.0, 1.0)
    mlab = g.randint(b, dims[-1])
    params = {}
    for li in range(3):
        params[f"w{li + 1}"] = g.normal((dims[li], dims[li + 1]), 0.0, float(np.sqrt(2.0 / dims[li])))
        params[f"b{li + 1}"] = np.zeros(dims[li + 1], np.float32)
    out["mlp_x"] = mx
    out["mlp_labels"] = mlab
    for k, v in params.items():
        out[f"mlp_init_{k}"] = v
    P = {k: t64(v).requires_grad_(True) for k, v in params.items()}
    losses = []
    for _ in range(2):
        h1 = torch.relu(t64(mx) @ P["w1"] + P["b1"])
        h2 = torch.relu(h1 @ P["w2"] + P["b2"])
        logits = h2 @ P["w3"] + P["b3"]
        loss = torch.nn.functional.cross_entropy(logits, torch.tensor(mlab.astype(np.int64)))
        for p in P.values():
            p.grad = None
        loss.backward()
        losses.append(loss.item())
        with torch.no_grad():
            for p in P.values():
                p -= lr * p.grad
    out["mlp_losses"] = np.array(losses)
    for k, p in P.items():
        out[f"mlp_final_{k}"] = p.detach().numpy()

    np.savez_compressed(os.path.join(HERE, "fixtures_f64.npz"), **out)
    print("wrote", len(out), "arrays")


if __name__ == "__main__":
    main()
