"""Writes tests/golden/models/lenet300_sparse.npz from the reference's pruned LeNet300 checkpoint.

Source: the reference repository's
``Python_Jenks_Test/Jenks_Tests/Best_Results_HPO/LeNet300/best_2025-12-09_18-58-19_MNIST_LeNet300.pth``,
a ``state_dict`` of ``nn.Sequential(Flatten, Linear(784,300), ReLU, Linear(300,100), ReLU,
Linear(100,10))`` (keys ``1.*``, ``3.*``, ``5.*``; the architecture of
``QuantNetworkTest.py:29-44``).  It is read with ``torch.load(weights_only=True)``, which
executes nothing from the file.  The fixture keeps the data only: per layer the shape, the
flat indices and fp32 values of the non-zero weights, and the fp32 bias.  That is the
whole checkpoint, losslessly, in ~35 KB (the weights are ~98% zero).

Run in a checkout that has the reference next to it:
    python tests/golden/make_lenet300.py [path/to/checkpoint.pth]
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
DEFAULT = Path("/root/reference/Python_Jenks_Test/Jenks_Tests/Best_Results_HPO/LeNet300/"
               "best_2025-12-09_18-58-19_MNIST_LeNet300.pth")
LAYERS = ("1", "3", "5")


def main(src: Path) -> None:
    sd = torch.load(src, weights_only=True, map_location="cpu")
    out = {}
    for name in LAYERS:
        w = sd[f"{name}.weight"].float().numpy()
        flat = w.reshape(-1)
        nz = np.flatnonzero(flat).astype(np.int32)
        out[f"l{name}_shape"] = np.array(w.shape, np.int32)
        out[f"l{name}_idx"] = nz
        out[f"l{name}_val"] = flat[nz].astype(np.float32)
        out[f"l{name}_bias"] = sd[f"{name}.bias"].float().numpy()
    np.savez_compressed(HERE / "models" / "lenet300_sparse.npz", **out)
    total = sum(int(np.prod(out[f"l{n}_shape"])) for n in LAYERS)
    nnz = sum(out[f"l{n}_idx"].size for n in LAYERS)
    print(f"wrote models/lenet300_sparse.npz: {nnz} non-zeros of {total} weights "
          f"(sparsity {1 - nnz / total:.5f})")


if __name__ == "__main__":
    main(Path(sys.argv[1]) if len(sys.argv) > 1 else DEFAULT)
