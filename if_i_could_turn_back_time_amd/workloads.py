"""Benchmark workloads: the layer shapes of the five benchmark configurations and their
seeded synthetic inputs, shared by ``bench.py`` and the GPU parity tests.

Every generator draws from a CPU ``torch.Generator`` seeded 0, in the order weights,
outlier masks, activations:

- ``cfg1`` (GF4 4096x4096; also the GF4 half of the batch-8/16 configuration):
  ``W = 0.02 N(0,1)``, ``x = N(0,1)``.
- ``cfg2`` (E2M1 Llama-7B shapes; also the E2M1 half of the batch-8/16 configuration):
  ``W`` Student-t with 5 degrees of freedom scaled to std 0.02 (``t * 0.02 / sqrt(5/3)``),
  ``x = N(0,1)`` with ``round(0.001 K)`` seeded positions multiplied by 20.
- ``cfg4`` (70B MLP shapes): ``W = 0.015 N(0,1)`` with a seeded 0.5% of the entries
  replaced by ``N(0, (8 * 0.015)^2)`` (the "heavy-tail component at 8 sigma").
- The rotated configuration uses ``cfg1``'s distribution; the rotation is applied by the
  packer (weights) and the kernel (x).
"""
from __future__ import annotations

import math

import torch

# name -> (fmt, K, N, B, generator, rotated)
WORKLOADS = {
    "gf4_k8192_n28672_b1": ("gf4", 8192, 28672, 1, "cfg4", False),
    "gf4_k28672_n8192_b1": ("gf4", 28672, 8192, 1, "cfg4", False),
    "gf4_k8192_n28672_b2": ("gf4", 8192, 28672, 2, "cfg4", False),
    "gf4_k8192_n28672_b4": ("gf4", 8192, 28672, 4, "cfg4", False),
    "gf4_k28672_n8192_b2": ("gf4", 28672, 8192, 2, "cfg4", False),
    "gf4_k28672_n8192_b4": ("gf4", 28672, 8192, 4, "cfg4", False),
    "gf4_k4096_n4096_b1": ("gf4", 4096, 4096, 1, "cfg1", False),
    "e2m1_k4096_n4096_b1": ("e2m1", 4096, 4096, 1, "cfg2", False),
    "e2m1_k4096_n11008_b1": ("e2m1", 4096, 11008, 1, "cfg2", False),
    "e2m1_k11008_n4096_b1": ("e2m1", 11008, 4096, 1, "cfg2", False),
    "gf4fwht_k4096_n4096_b1": ("gf4", 4096, 4096, 1, "cfg1", True),
    "gf4fwht_k4096_n11008_b1": ("gf4", 4096, 11008, 1, "cfg1", True),
    "gf4fwht_k11008_n4096_b1": ("gf4", 11008, 4096, 1, "cfg1", True),
    # small-batch dense contraction (batch 8 / 16): E2M1 as cfg2, GF4 as cfg1
    "e2m1_k8192_n8192_b8": ("e2m1", 8192, 8192, 8, "cfg2", False),
    "e2m1_k8192_n8192_b16": ("e2m1", 8192, 8192, 16, "cfg2", False),
    "e2m1_k8192_n28672_b8": ("e2m1", 8192, 28672, 8, "cfg2", False),
    "e2m1_k8192_n28672_b16": ("e2m1", 8192, 28672, 16, "cfg2", False),
    "gf4_k8192_n8192_b8": ("gf4", 8192, 8192, 8, "cfg1", False),
    "gf4_k8192_n8192_b16": ("gf4", 8192, 8192, 16, "cfg1", False),
    "gf4_k8192_n28672_b8": ("gf4", 8192, 28672, 8, "cfg1", False),
    "gf4_k8192_n28672_b16": ("gf4", 8192, 28672, 16, "cfg1", False),
    # batch 16 over the Llama-7B down projection (K = 11008, 3 K-slices of x on one row tile
    # per CU): the shape the split-K plan is for
    "gf4_k11008_n4096_b16": ("gf4", 11008, 4096, 16, "cfg1", False),
    "e2m1_k11008_n4096_b16": ("e2m1", 11008, 4096, 16, "cfg2", False),
    # the reference's own 4-bit weight (QuantLinear.commit) as GF4 integer-level codebooks
    "int4ref_k8192_n28672_b1": ("int4ref", 8192, 28672, 1, "cfg4", False),
}
DEFAULT = "gf4_k8192_n28672_b1"
# the configuration the reference's CPU dequantize-then-matmul path is quoted on
CPU_CONFIG = "gf4_k4096_n4096_b1"


def synth_weight(kind: str, N: int, K: int, g: torch.Generator) -> torch.Tensor:
    """fp32 ``[N, K]`` weights of generator ``kind``, drawn from ``g``."""
    if kind == "cfg4":
        w = torch.randn(N, K, generator=g) * 0.015
        m = torch.rand(N, K, generator=g) < 0.005
        w[m] = torch.randn(int(m.sum()), generator=g) * (8 * 0.015)
    elif kind == "cfg2":
        nu = 5
        z = torch.randn(N, K, generator=g)
        chi = torch.zeros(N, K)
        for _ in range(nu):
            chi += torch.randn(N, K, generator=g) ** 2
        w = z / torch.sqrt(chi / nu) * (0.02 / math.sqrt(nu / (nu - 2)))
    elif kind in ("cfg1", "cfg3"):
        w = torch.randn(N, K, generator=g) * 0.02
    else:
        raise ValueError(f"unknown generator {kind!r}")
    return w.contiguous()


def synth_x(kind: str, B: int, K: int, g: torch.Generator) -> torch.Tensor:
    """fp32 ``[B, K]`` activations of generator ``kind`` (cast by the caller)."""
    x = torch.randn(B, K, generator=g)
    if kind == "cfg2":
        n_out = max(1, round(0.001 * K))
        pos = torch.randperm(K, generator=g)[:n_out]
        x[:, pos] *= 20.0
    return x


def synth(kind: str, N: int, K: int, B: int, xdtype, seed: int = 0):
    """Weights then activations of one workload from one generator seeded ``seed``."""
    g = torch.Generator().manual_seed(seed)
    w = synth_weight(kind, N, K, g)
    x = synth_x(kind, B, K, g)
    return w, x.to(xdtype)


def x_dtype(fmt: str):
    """Activation dtype of a format's configurations: fp16 for GF4, bf16 for E2M1."""
    return torch.float16 if fmt in ("gf4", "int4ref") else torch.bfloat16


def algorithmic_bytes(fmt: str, N: int, K: int, B: int, xbytes: int = 2, ybytes: int = 2) -> int:
    """Bytes one call must move, each counted once: nibbles + codebooks (GF4: 16 fp16
    per 128-group) or E8M0 scales (E2M1: one byte per 32-group) + x + y."""
    meta = N * (K // 128) * 32 if fmt in ("gf4", "int4ref") else N * (K // 32)
    return N * K // 2 + meta + B * K * xbytes + B * N * ybytes
