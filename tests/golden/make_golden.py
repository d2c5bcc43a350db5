"""Writes the golden fixtures under tests/golden/ from the CPU oracle.

The oracle is pinned independently (tests/test_oracle.py); these fixtures freeze its
outputs on small seeded inputs so that the native packers, the device decoder and the
GEMV are checked against stored vectors on the GPU box too.  Regenerate only when a
format definition changes on purpose:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import fourbit_oracle as O  # noqa: E402


def student_t(gen, shape, nu=5.0, std=0.02):
    # t = z / sqrt(chi2_nu / nu), scaled to the requested std (var of t_nu = nu/(nu-2))
    z = torch.randn(shape, generator=gen, dtype=torch.float64)
    chi = torch.distributions.Chi2(torch.tensor(nu, dtype=torch.float64))
    torch.manual_seed(int(torch.randint(0, 2**31 - 1, (1,), generator=gen)))
    c = chi.sample(shape)
    return (z / torch.sqrt(c / nu) * (std / np.sqrt(nu / (nu - 2)))).float()


def case_gf4(gen, N, K, B, fwht_block=0):
    w = (torch.randn(N, K, generator=gen) * 0.02).numpy()
    # a few structured groups: all-zero, constant, few distinct values
    w[0, :128] = 0.0
    w[1, 128:256] = 0.0625
    w[2, :128] = np.resize(np.array([-0.03, 0.01, 0.02], np.float32), 128)
    if fwht_block:
        w = O.rotate_weights(w, fwht_block)
    codes, book = O.gf4_quantize(w)
    x = torch.randn(B, K, generator=gen).half()
    y = O.y_ref("gf4", codes, book, x, fwht_block)
    return dict(w=w, codes=O.pack_nibbles(codes), codebook=book, x=x.view(torch.int16).numpy(),
                y=y.numpy(), fwht_block=np.int32(fwht_block))


def case_e2m1(gen, N, K, B):
    w = student_t(gen, (N, K)).numpy()
    w[0, :32] = 0.0
    w[1, 32:64] = np.float32(2.0 ** -129)  # tiny group: E8M0 clamps at 2^-127
    x = torch.randn(B, K, generator=gen)
    n_out = max(1, round(0.001 * K))
    pos = torch.randperm(K, generator=gen)[:n_out]
    x[:, pos] *= 20.0
    x = x.bfloat16()
    codes, scales = O.e2m1_quantize(w)
    y = O.y_ref("e2m1", codes, scales, x)
    return dict(w=w, codes=O.pack_nibbles(codes), scales=scales, x=x.view(torch.int16).numpy(),
                y=y.numpy(), fwht_block=np.int32(0))


def main():
    gen = torch.Generator().manual_seed(0)
    cases = {
        "gf4_n24_k512_b3": case_gf4(gen, 24, 512, 3),
        "gf4_fwht256_n16_k768_b1": case_gf4(gen, 16, 768, 1, fwht_block=256),
        "gf4_fwht4096_n8_k4096_b2": case_gf4(gen, 8, 4096, 2, fwht_block=4096),
        "e2m1_n24_k512_b4": case_e2m1(gen, 24, 512, 4),
        "e2m1_n40_k1152_b1": case_e2m1(gen, 40, 1152, 1),
    }
    for name, d in cases.items():
        np.savez_compressed(HERE / f"{name}.npz", **d)
        print(name, {k: v.shape for k, v in d.items()})


if __name__ == "__main__":
    main()
