"""Shared test inputs: the reference QuantLinear's state and the reference's pruned
LeNet300 checkpoint (from the committed fixture)."""
from pathlib import Path

import numpy as np
import torch

from oracle import fourbit_oracle as O

ROOT = Path(__file__).resolve().parents[1]


def reference_state(N, K, seed, bias=True):
    """State of the reference QuantLinear (layers.py:11-31): weight, s, Q, Theta, mask."""
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(N, K, generator=g) * 0.02
    theta = torch.randn(N, K, generator=g) * 2
    mask = (torch.rand(N, K, generator=g) > 0.25).float()
    _, s, _ = O.quantlinear_commit_weight(w, theta, mask)
    sd = {"weight": w, "s": s, "Q": torch.floor(w / s), "Theta": theta, "mask": mask}
    if bias:
        sd["bias"] = torch.randn(N, generator=g)
    return sd


LENET = ROOT / "tests" / "golden" / "models" / "lenet300_sparse.npz"


def lenet300_from_fixture():
    """nn.Sequential(Flatten, Linear(784,300), ReLU, Linear(300,100), ReLU, Linear(100,10))
    with the reference checkpoint's weights (QuantNetworkTest.py:29-44)."""
    z = np.load(LENET)
    net = torch.nn.Sequential(torch.nn.Flatten(), torch.nn.Linear(784, 300), torch.nn.ReLU(),
                              torch.nn.Linear(300, 100), torch.nn.ReLU(),
                              torch.nn.Linear(100, 10))
    with torch.no_grad():
        for name in ("1", "3", "5"):
            shape = tuple(z[f"l{name}_shape"])
            w = np.zeros(int(np.prod(shape)), np.float32)
            w[z[f"l{name}_idx"]] = z[f"l{name}_val"]
            net[int(name)].weight.copy_(torch.from_numpy(w.reshape(shape)))
            net[int(name)].bias.copy_(torch.from_numpy(z[f"l{name}_bias"]))
    return net
