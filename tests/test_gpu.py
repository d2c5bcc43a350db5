"""GPU parity: device decode bit-exact vs the oracle, fused GEMV within the north-star
tolerance |y - y_ref| <= 1e-2 + 1e-3 |y_ref| (y_ref = oracle dequantize-then-F.linear in
fp32 on the CPU), all through the C ABI of libfourbit.so."""
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import fourbit_oracle as O
from if_i_could_turn_back_time_amd import _capi as C
from if_i_could_turn_back_time_amd import PackedWeight, QuantLinear, quantize_module
from model_fixtures import lenet300_from_fixture, reference_state

pytestmark = pytest.mark.gpu
ROOT = Path(__file__).resolve().parents[1]
GOLDEN = sorted((ROOT / "tests" / "golden").glob("*.npz"))
ATOL, RTOL = 1e-2, 1e-3
DEV = "cuda:0"


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def within_tol(y, yref, extra_rel=0.0):
    y = y.detach().float().cpu()
    yref = yref.detach().float().cpu()
    err = (y - yref).abs()
    bound = ATOL + (RTOL + extra_rel) * yref.abs()
    return bool((err <= bound).all()), float(err.max()), float((err / (yref.abs() + 1e-6)).max())


def oracle_y(pw: PackedWeight, x: torch.Tensor) -> torch.Tensor:
    codes = O.unpack_nibbles(pw.codes.numpy())
    meta = pw.meta.numpy().view(np.uint16) if pw.fmt == C.FMT_GF4 else pw.meta.numpy()
    return O.y_ref(pw.fmt_name, codes, meta, x.cpu(), pw.fwht_block)


def test_cuda_device_present():
    assert torch.cuda.is_available()
    say("device", torch.cuda.get_device_name(0))
    assert C.lib() is not None


@pytest.mark.parametrize("path", GOLDEN, ids=lambda p: p.stem)
def test_golden_decode_and_gemv(path):
    d = np.load(path)
    fmt = "gf4" if "codebook" in d else "e2m1"
    say("golden", path.stem)
    N, K = d["w"].shape
    meta = torch.from_numpy(d["codebook"].view(np.int16) if fmt == "gf4" else d["scales"])
    pw = PackedWeight(fmt, N, K, torch.from_numpy(d["codes"]), meta, int(d["fwht_block"]), DEV)
    # device decode, bit-exact
    deq = pw.dequant_device(torch.float32).cpu()
    ref = O.dequant_f32(fmt, O.unpack_nibbles(d["codes"]),
                        d["codebook"] if fmt == "gf4" else d["scales"])
    assert torch.equal(deq.view(torch.int32), ref.view(torch.int32))
    # GEMV against the stored y
    xdt = torch.float16 if fmt == "gf4" else torch.bfloat16
    x = torch.from_numpy(d["x"]).view(xdt).to(DEV)
    y = pw.gemv(x, out_dtype=torch.float32)
    torch.cuda.synchronize()
    ok, emax, _ = within_tol(y, torch.from_numpy(d["y"]))
    assert ok, f"max abs err {emax}"


@pytest.mark.parametrize("fmt", ["gf4", "e2m1"])
@pytest.mark.parametrize("N,K", [(1, 128), (3, 256), (65, 384), (33, 4096), (17, 11008),
                                 (9, 8192), (5, 28672)])
def test_decode_bit_exact_shapes(fmt, N, K):
    say("decode", fmt, N, K)
    gen = torch.Generator().manual_seed(N * 7 + K)
    w = torch.randn(N, K, generator=gen) * 0.02
    pw = PackedWeight.quantize(w, fmt, device=DEV)
    deq = pw.dequant_device(torch.float32).cpu()
    assert torch.equal(deq.view(torch.int32), pw.dequant_host().view(torch.int32))
    if fmt == "gf4":  # fp16 output is the codebook entry itself
        d16 = pw.dequant_device(torch.float16).cpu()
        assert torch.equal(d16.float(), deq)
    else:
        db = pw.dequant_device(torch.bfloat16).cpu()
        assert torch.equal(db.float(), deq)


@pytest.mark.parametrize("fmt,xdt", [("gf4", torch.float16), ("e2m1", torch.bfloat16),
                                     ("e2m1", torch.float16)])
@pytest.mark.parametrize("B", [1, 2, 3, 4, 8, 16])
@pytest.mark.parametrize("N,K", [(1, 128), (7, 256), (64, 1024), (130, 4096), (48, 11008),
                                 (40, 28672)])
def test_gemv_vs_oracle(fmt, xdt, B, N, K):
    say("gemv", fmt, xdt, B, N, K)
    gen = torch.Generator().manual_seed(B * 1000 + N + K)
    w = torch.randn(N, K, generator=gen) * 0.02
    pw = PackedWeight.quantize(w, fmt, device=DEV)
    x = torch.randn(B, K, generator=gen)
    x[:, :: max(1, K // 7)] *= 20.0  # outliers
    x = x.to(xdt)
    yref = oracle_y(pw, x)
    for ydt, extra in ((torch.float32, 0.0), (torch.float16, 2.0 ** -11),
                       (torch.bfloat16, 2.0 ** -8)):
        y = pw.gemv(x.to(DEV), out_dtype=ydt)
        torch.cuda.synchronize()
        ok, emax, _ = within_tol(y, yref, extra)
        assert ok, f"{ydt}: max abs err {emax}"


@pytest.mark.parametrize("B", [1, 2, 4])
@pytest.mark.parametrize("N,K,block", [(64, 4096, 4096), (96, 11008, 256), (32, 1024, 256),
                                       (16, 512, 2), (24, 2048, 32), (40, 3072, 512),
                                       (48, 2048, 1024), (20, 6144, 2048), (24, 28672, 4096)])
def test_gemv_fwht_vs_oracle(B, N, K, block):
    say("fwht", B, N, K, block)
    gen = torch.Generator().manual_seed(N + K + block)
    w = torch.randn(N, K, generator=gen) * 0.02
    pw = PackedWeight.quantize(w, "gf4", fwht_block=block, device=DEV)
    x = torch.randn(B, K, generator=gen).half()
    yref = oracle_y(pw, x)
    y = pw.gemv(x.to(DEV), out_dtype=torch.float32)
    torch.cuda.synchronize()
    ok, emax, _ = within_tol(y, yref)
    assert ok, f"max abs err {emax}"
    # rotation invariance: the rotated 4-bit layer approximates the unrotated product
    # (quantization error of 16 Jenks levels is ~7% rms of the weight)
    ydense = x.float() @ w.t()
    rel = ((y.cpu() - ydense).pow(2).mean() / ydense.pow(2).mean()).sqrt()
    assert rel < 0.15


@pytest.mark.parametrize("B", [5, 8, 16])
@pytest.mark.parametrize("N,K,block", [(96, 11008, 256), (64, 4096, 4096), (40, 8192, 4096)])
def test_gemv_fwht_large_batch_vs_oracle(B, N, K, block):
    """Rotated layers at larger batches: K = 11008 (256-blocks) runs three K-slices, the
    last one ragged; 4096-blocks keep an fp32 copy of each batch row in LDS, so batches
    that do not fit run in row chunks inside fb_gemv."""
    say("fwht large batch", B, N, K, block)
    gen = torch.Generator().manual_seed(7 * N + K + B)
    w = torch.randn(N, K, generator=gen) * 0.02
    pw = PackedWeight.quantize(w, "gf4", fwht_block=block, device=DEV)
    x = torch.randn(B, K, generator=gen).half()
    yref = oracle_y(pw, x)
    for ydt in (torch.float32, torch.float16):
        y = pw.gemv(x.to(DEV), out_dtype=ydt)
        torch.cuda.synchronize()
        ok, emax, _ = within_tol(y, yref, 2.0 ** -11 if ydt == torch.float16 else 0.0)
        assert ok, f"{ydt}: max abs err {emax}"


@pytest.mark.parametrize("B", [1, 4, 16])
@pytest.mark.parametrize("N,K,block", [(64, 4096, 4096), (48, 11008, 256)])
def test_gemv_e2m1_fwht_vs_oracle(B, N, K, block):
    """E2M1 weights with a rotation (fp16 x): the same in-kernel rotation feeding the
    E2M1 decode; also through QuantLinear(fmt='e2m1', hadamard=block)."""
    say("e2m1 fwht", B, N, K, block)
    gen = torch.Generator().manual_seed(3 * N + K + B)
    w = torch.randn(N, K, generator=gen) * 0.02
    pw = PackedWeight.quantize(w, "e2m1", fwht_block=block, device=DEV)
    x = torch.randn(B, K, generator=gen).half()
    yref = oracle_y(pw, x)
    y = pw.gemv(x.to(DEV), out_dtype=torch.float32)
    torch.cuda.synchronize()
    ok, emax, _ = within_tol(y, yref)
    assert ok, f"max abs err {emax}"
    lin = torch.nn.Linear(K, N, bias=False)
    with torch.no_grad():
        lin.weight.copy_(w)
    q = QuantLinear(lin, fmt="e2m1", hadamard=block).to(DEV)
    yq = q(x.to(DEV))
    torch.cuda.synchronize()
    ok, emax, _ = within_tol(yq, yref, 2.0 ** -11)
    assert ok, f"QuantLinear: max abs err {emax}"


@pytest.mark.parametrize("fmt", ["gf4", "e2m1"])
def test_special_inputs(fmt):
    say("special", fmt)
    N, K = 50, 1024
    w = torch.randn(N, K) * 0.02
    pw = PackedWeight.quantize(w, fmt, device=DEV)
    xdt = torch.float16 if fmt == "gf4" else torch.bfloat16
    W = pw.dequant_device(torch.float32)
    # one-hot x recovers a dequantized column exactly (fp32 output)
    for col in (0, 127, 128, K - 1):
        x = torch.zeros(1, K, dtype=xdt, device=DEV)
        x[0, col] = 1
        y = pw.gemv(x, out_dtype=torch.float32)
        assert torch.equal(y[0], W[:, col])
    # zero input -> exact zeros
    y = pw.gemv(torch.zeros(2, K, dtype=xdt, device=DEV), out_dtype=torch.float32)
    assert torch.count_nonzero(y) == 0
    # linearity
    x1 = torch.randn(1, K, device=DEV).to(xdt)
    x2 = torch.randn(1, K, device=DEV).to(xdt)
    y12 = pw.gemv(torch.cat([x1, x2]), out_dtype=torch.float32)
    ysum = pw.gemv((x1.float() + x2.float()).to(xdt), out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert (ysum[0] - (y12[0] + y12[1])).abs().max() < 1e-2


@pytest.mark.parametrize("fmt,N,K", [("gf4", 28672, 8192), ("gf4", 8192, 28672),
                                     ("e2m1", 11008, 4096), ("e2m1", 4096, 11008)])
def test_full_size_vs_torch_reference(fmt, N, K):
    """Config-size layers: GEMV vs torch fp32 matmul of the device-decoded weight (itself
    checked bit-exact against the host decode on sampled rows), plus sampled rows
    against the CPU oracle."""
    say("full", fmt, N, K)
    gen = torch.Generator().manual_seed(0)
    w = torch.randn(N, K, generator=gen) * 0.015
    pw = PackedWeight.quantize(w, fmt, device=DEV)
    xdt = torch.float16 if fmt == "gf4" else torch.bfloat16
    W = pw.dequant_device(torch.float32)
    rows = torch.randint(0, N, (16,), generator=gen)
    host = pw.dequant_host()
    assert torch.equal(W[rows].cpu(), host[rows])
    for B in (1, 2, 4, 8, 16):
        x = torch.randn(B, K, generator=gen).to(xdt)
        y = pw.gemv(x.to(DEV), out_dtype=torch.float32)
        y2 = pw.gemv(x.to(DEV), out_dtype=torch.float32)  # workspace reuse, same bits
        assert torch.equal(y, y2)
        yref = (x.to(DEV).float() @ W.t())
        torch.cuda.synchronize()
        ok, emax, _ = within_tol(y, yref)
        assert ok, f"B={B}: max abs err {emax}"
        ysub = torch.nn.functional.linear(x.float(), host[rows])
        ok, emax, _ = within_tol(y[:, rows], ysub)
        assert ok, f"B={B} oracle rows: max abs err {emax}"


def test_quantlinear_forward_gpu():
    say("quantlinear")
    lin = torch.nn.Linear(1024, 300)
    for fmt, xdt in (("gf4", torch.float16), ("e2m1", torch.bfloat16), ("gf4", torch.float32)):
        q = QuantLinear(lin, fmt=fmt).to(DEV)
        x = torch.randn(2, 3, 1024, device=DEV).to(xdt)   # batch 6 > 4: two launches
        y = q(x)
        assert y.shape == (2, 3, 300) and y.dtype == xdt
        W = q.dequantized_weight()
        xin = x.reshape(-1, 1024).cpu().float()
        if fmt == "gf4":
            xin = xin.half().float()
        yref = torch.nn.functional.linear(xin, W, lin.bias.detach())
        extra = {torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8, torch.float32: 0.0}[xdt]
        ok, emax, _ = within_tol(y.reshape(-1, 300), yref, extra)
        assert ok, f"{fmt}/{xdt}: {emax}"


def oracle_weight(q: QuantLinear) -> torch.Tensor:
    """Oracle decode of a QuantLinear's packed buffers, cut to in_features."""
    codes = O.unpack_nibbles(q.codes.cpu().numpy())
    meta = q.meta.cpu().numpy().view(np.uint16) if q.fmt == "gf4" else q.meta.cpu().numpy()
    return O.dequant_f32(q.fmt, codes, meta)[:, :q.in_features]


def test_c_abi_gpu_caller():
    """The C ABI from a native C++ caller with no Python or torch (tests/c/abi_gpu.cpp,
    built by build_lib): hipMalloc'd buffers, its own stream, weights packed by the host
    packers, fb_gemv, and y checked against an fp64 host product of the exact decode
    (GF4 fp16 x batch 3 with a partial row tile; E2M1 bf16 x batch 16; E2M1 batch 8 on the
    native FP4 path, fb_gemv_mx, with a hipMalloc'd workspace)."""
    say("native C++ caller")
    exe = Path(__file__).resolve().parent / "c" / "abi_gpu"
    if not exe.exists():  # build() makes it with the library (and fails loudly if it cannot)
        pytest.skip("tests/c/abi_gpu not built: run __graft_entry__.build()")
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    print(r.stdout, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().endswith("ok")


def test_quantlinear_batch_edges_gpu():
    """Batch edges of the forward: an empty batch gives an empty output (no launch), 33
    rows run as chunks of 16 + 16 + 1, and a 3-D input keeps its leading shape; every
    row is checked against the oracle's decode + fp32 F.linear."""
    say("batch edges")
    g = torch.Generator().manual_seed(33)
    lin = torch.nn.Linear(512, 80)
    for fmt, xdt in (("gf4", torch.float16), ("e2m1", torch.bfloat16)):
        q = QuantLinear(lin, fmt=fmt).to(DEV)
        W = oracle_weight(q).float()
        y0 = q(torch.empty(0, 512, device=DEV, dtype=xdt))
        assert y0.shape == (0, 80) and y0.dtype == xdt
        for shape in ((33, 512), (1, 1, 512), (2, 17, 512)):
            x = torch.randn(*shape, generator=g).to(xdt)
            y = q(x.to(DEV))
            torch.cuda.synchronize()
            assert y.shape == (*shape[:-1], 80)
            yref = torch.nn.functional.linear(x.reshape(-1, 512).float(), W, lin.bias.detach())
            extra = {torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8}[xdt]
            ok, emax, _ = within_tol(y.reshape(-1, 80), yref, extra)
            assert ok, f"{fmt} {shape}: max abs err {emax}"


def test_quantlinear_hadamard_forward_gpu():
    """QuantLinear(hadamard=True) on 24 rows (launches of 16 + 8 rows; the 4096-wide
    rotation runs each in row chunks that fit LDS) against the oracle's rotated product
    plus bias; commit() rotates the packed weight back, and F.linear with it agrees."""
    say("quantlinear hadamard")
    g = torch.Generator().manual_seed(4096)
    lin = torch.nn.Linear(4096, 96)
    q = QuantLinear(lin, hadamard=True).to(DEV)
    assert q.fwht_block == 4096
    x = torch.randn(2, 12, 4096, generator=g).half()
    y = q(x.to(DEV))
    torch.cuda.synchronize()
    assert y.shape == (2, 12, 96) and y.dtype == torch.float16
    codes = O.unpack_nibbles(q.codes.cpu().numpy())
    meta = q.meta.cpu().numpy().view(np.uint16)
    yref = O.y_ref("gf4", codes, meta, x.reshape(-1, 4096), 4096) + lin.bias.detach()
    ok, emax, _ = within_tol(y.reshape(-1, 96), yref, 2.0 ** -10)
    assert ok, f"max abs err {emax}"
    q.commit()
    ycommit = torch.nn.functional.linear(x.reshape(-1, 4096).float(), q.weight.detach().cpu(),
                                         lin.bias.detach())
    ok, emax, _ = within_tol(y.reshape(-1, 96), ycommit, 2.0 ** -9)
    assert ok, f"vs committed weight: max abs err {emax}"


def test_ragged_k_masked_forward_gpu():
    """in_features = 300 (x zero-padded to 384 for the kernel), 70% of weights masked."""
    say("ragged K / masked")
    g = torch.Generator().manual_seed(21)
    lin = torch.nn.Linear(300, 100)
    mask = (torch.rand(100, 300, generator=g) > 0.7).float()
    for fmt, xdt in (("gf4", torch.float16), ("e2m1", torch.bfloat16)):
        q = QuantLinear(lin, mask=mask, fmt=fmt).to(DEV)
        x = torch.randn(5, 300, generator=g).to(xdt)
        y = q(x.to(DEV))
        W = oracle_weight(q)
        assert (W[mask == 0] == 0).all()
        yref = torch.nn.functional.linear(x.float(), W, lin.bias.detach())
        ok, emax, _ = within_tol(y, yref)
        assert ok, f"{fmt}: {emax}"


def test_from_reference_forward_gpu():
    """The reference QuantLinear's committed 4-bit weight (layers.py:39-45) through the
    GEMV: within tolerance of the oracle decode, and of F.linear with the reference's own
    fp32 committed weight once the fp16 rounding of the codebook entries (|rel| <= 2^-11
    per weight) is allowed for."""
    say("from_reference")
    for N, K in ((96, 256), (40, 200)):
        sd = reference_state(N, K, seed=N + K)
        Wq, _, _ = O.quantlinear_commit_weight(sd["weight"], sd["Theta"], sd["mask"])
        q = QuantLinear.from_reference(sd).to(DEV)
        x = torch.randn(3, K).half()
        y = q(x.to(DEV))
        ok, emax, _ = within_tol(y, torch.nn.functional.linear(x.float(), oracle_weight(q),
                                                               sd["bias"]))
        assert ok, f"oracle {N}x{K}: {emax}"
        yref = torch.nn.functional.linear(x.float(), Wq, sd["bias"])
        bound = ATOL + RTOL * yref.abs() + 2.0 ** -11 * (x.float().abs() @ Wq.abs().T)
        err = (y.float().cpu() - yref).abs()
        assert bool((err <= bound).all()), f"reference {N}x{K}: {float(err.max())}"


def test_brecq_replace_forward_gpu():
    """brecq's AdaRound layer (brecq.py:59-92) packed by replace_forward: with |alpha|
    saturating the gate, the packed forward matches the reference's soft forward
    F.linear(x, clamp(mask*(W_floor+h), qmin, qmax)*delta) up to fp16 codebook rounding."""
    from types import SimpleNamespace
    from if_i_could_turn_back_time_amd import replace_forward
    say("brecq replace_forward")
    g = torch.Generator().manual_seed(31)
    lin = torch.nn.Linear(256, 64)
    delta = lin.weight.data.abs().amax(dim=1, keepdim=True) / 7
    W = lin.weight.data / delta
    alpha = torch.sign(torch.randn(64, 256, generator=g)) * 4.0
    wq = SimpleNamespace(W_floor=torch.floor(W), alpha=alpha, mask=torch.ones(64, 256),
                         quantizer=SimpleNamespace(delta=delta, qmin=-8, qmax=7))
    lin.weight_quantizer = wq
    lin = lin.to(DEV)
    replace_forward(lin)
    x = torch.randn(4, 256, generator=g).half()
    y = lin(x.to(DEV))
    h = torch.clamp(torch.sigmoid(alpha) * 1.2 - 0.1, 0, 1)
    Wsoft = torch.clamp(wq.mask * (wq.W_floor + h), -8, 7) * delta
    bias = lin.bias.detach().cpu()
    yref = torch.nn.functional.linear(x.float(), Wsoft, bias)
    bound = ATOL + RTOL * yref.abs() + 2.0 ** -11 * (x.float().abs() @ Wsoft.abs().T)
    err = (y.float().cpu() - yref).abs()
    assert bool((err <= bound).all()), float(err.max())


def test_lenet300_fixture_forward_gpu():
    """The reference's pruned LeNet300 (784-300-100-10, ~98% zeros) with every Linear
    swapped for the packed layer (GF4 with masks, and E2M1): each layer's GEMV within
    tolerance of the oracle decode on that layer's own input, batch 40 (3 launches of
    <= 16 rows per layer)."""
    say("lenet300")
    g = torch.Generator().manual_seed(41)
    x = torch.rand(40, 1, 28, 28, generator=g)
    for fmt in ("gf4", "e2m1"):
        q = quantize_module(lenet300_from_fixture(), fmt=fmt).to(DEV)
        h = x.flatten(1)
        for i in (1, 3, 5):
            y = q[i](h.to(DEV))
            # GF4 takes x in fp16 (rounded here too); E2M1 rounds fp32 x to bf16 in the
            # layer, which the 2^-8 relative allowance covers
            xin = h.half().float() if fmt == "gf4" else h.float()
            Wo = oracle_weight(q[i])
            yref = torch.nn.functional.linear(xin, Wo, q[i].bias.detach().cpu())
            bound = ATOL + RTOL * yref.abs()
            if fmt == "e2m1":
                bound = bound + 2.0 ** -8 * (xin.abs() @ Wo.abs().T)
            err = (y.float().cpu() - yref).abs()
            assert bool((err <= bound).all()), f"{fmt} layer {i}: {float(err.max())}"
            h = torch.relu(yref)
        logits = q(x.to(DEV)).float().cpu()
        assert logits.shape == (40, 10) and torch.isfinite(logits).all()


def _structured_weights(g, N, K):
    w = torch.randn(N, K, generator=g) * 0.02
    w[0, :128] = 0.0                                          # all zeros
    w[1, :128] = 0.0625                                       # constant
    w[2, :128] = torch.tensor([-0.03, 0.01, 0.02]).repeat(43)[:128]   # 3 distinct values
    w[3] = torch.round(w[3] * 200) / 200                      # heavy ties
    w[4, :128] = torch.randn(128, generator=g) * 1e3          # wide range
    w[4, 128:256] = torch.randn(128, generator=g) * 1e-30     # tiny normals
    w[5, :64] = -0.0                                          # signed zeros
    w[5, 64:128] = torch.randn(64, generator=g) * 1e-40       # fp32 subnormals
    w[6, :128] = torch.arange(128, dtype=torch.float32)       # 128 distinct, sorted
    w[7, :128] = -torch.arange(128, dtype=torch.float32)      # reverse sorted
    return w


@pytest.mark.parametrize("density", [None, 1.0, 0.9, 0.3, 0.05, 0.0])
def test_gpu_packer_bit_exact_vs_host(density):
    """fb_quantize_gf4_gpu produces the host packer's bytes (fb_quantize_gf4 without a
    mask, fb_quantize_gf4_masked with one): structured groups, ties, signed zeros, a wide
    dynamic range, and every kept count from 0 to 128 across the masked cases."""
    say("gpu packer", density)
    g = torch.Generator().manual_seed(61)
    N, K = 72, 1024
    w = _structured_weights(g, N, K)
    keep = None
    if density is not None:
        keep = torch.rand(N, K, generator=g) < density
        for r in range(8, 8 + 40):                            # kept counts 0..117 in steps of 3
            keep[r, :128] = torch.arange(128) < 3 * (r - 8)
    hc, hb = C.quantize_gf4(w, 8, keep)
    dc, db = C.quantize_gf4_gpu(w.to(DEV), None if keep is None else keep.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(dc.cpu(), hc)
    assert torch.equal(db.cpu(), hb)
    # and the oracle's bytes on the same weights
    wn = w.numpy()
    oc, ob = (O.gf4_quantize(wn) if keep is None
              else O.gf4_quantize_masked(wn, keep.numpy()))
    assert np.array_equal(O.unpack_nibbles(dc.cpu().numpy()), oc)
    assert np.array_equal(db.cpu().numpy().view(np.uint16), ob)


def test_gpu_packer_rejects_nonfinite():
    w = torch.zeros(2, 128)
    w[1, 3] = float("inf")
    with pytest.raises(RuntimeError, match="non-finite"):
        C.quantize_gf4_gpu(w.to(DEV))
    keep = torch.ones(2, 128, dtype=torch.bool)
    keep[1, 3] = False                                        # masked: never read
    C.quantize_gf4_gpu(w.to(DEV), keep.to(DEV))


def test_quantlinear_gpu_packer_matches_host_on_lenet300():
    """QuantLinear(packer='gpu') on the pruned LeNet300 (masked, ragged in_features):
    the same packed buffers as the host packer."""
    say("lenet300 gpu packer")
    host = quantize_module(lenet300_from_fixture())
    gpu = quantize_module(lenet300_from_fixture().to(DEV), packer="gpu")
    for i in (1, 3, 5):
        assert torch.equal(gpu[i].codes.cpu(), host[i].codes)
        assert torch.equal(gpu[i].meta.cpu(), host[i].meta)
        assert torch.equal(gpu[i].wdev.cpu(), host[i].wdev)


def test_gemv_in_hip_graph_replays_match_eager():
    """fb_gemv captured in a HIP graph (it records kernel launches only: no memset nodes,
    no workspace): several replays, with eager work and synchronisations between them,
    each equal to the eager result, bit for bit."""
    say("hip graph")
    g = torch.Generator().manual_seed(71)
    for fmt, N, K, B, fb in (("gf4", 4096, 2048, 1, 0), ("e2m1", 3000, 1024, 4, 0),
                             ("gf4", 2048, 4096, 2, 4096)):
        w = torch.randn(N, K, generator=g) * 0.02
        pw = PackedWeight.quantize(w, fmt, fwht_block=fb, device=DEV)
        xdt = torch.float16 if fmt == "gf4" else torch.bfloat16
        x = torch.randn(B, K, generator=g).to(xdt).to(DEV)
        y = torch.empty(B, N, dtype=torch.float32, device=DEV)
        pw.gemv(x, out=y)
        torch.cuda.synchronize()
        eager = y.clone()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            pw.gemv(x, out=y)  # warm-up on the capture stream
            torch.cuda.synchronize()
            with torch.cuda.graph(graph, stream=s):
                pw.gemv(x, out=y)
        torch.cuda.synchronize()
        for rep in range(4):
            y.fill_(float("nan"))                      # eager work between replays
            x2 = (x.float() * 2).to(xdt)               # unrelated eager kernel
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(y, eager), f"{fmt} fb={fb} replay {rep}"
            assert x2.shape == x.shape


def test_concurrent_streams_match_serial():
    """Calls on two streams at once (two layers, interleaved launches) give the same bits as
    the same calls one after the other: the library keeps no state between calls."""
    say("two streams")
    g = torch.Generator().manual_seed(81)
    layers = []
    for fmt, N, K in (("gf4", 8192, 4096), ("e2m1", 6000, 8192)):
        pw = PackedWeight.quantize(torch.randn(N, K, generator=g) * 0.02, fmt, device=DEV,
                                   packer="gpu" if fmt == "gf4" else "host")
        xdt = torch.float16 if fmt == "gf4" else torch.bfloat16
        xs = [torch.randn(2, K, generator=g).to(xdt).to(DEV) for _ in range(6)]
        layers.append((pw, xs))
    serial = [[pw.gemv(x, out_dtype=torch.float32) for x in xs] for pw, xs in layers]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [[None] * 6 for _ in layers]
    for i in range(6):
        for j, ((pw, xs), s) in enumerate(zip(layers, streams)):
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                outs[j][i] = pw.gemv(xs[i], out_dtype=torch.float32)
    torch.cuda.synchronize()
    for j in range(2):
        for i in range(6):
            assert torch.equal(outs[j][i], serial[j][i]), (j, i)


def test_gpu_e2m1_packer_bit_exact_vs_host():
    """fb_quantize_e2m1_gpu produces the host packer's bytes: random rows, exact rounding
    midpoints (ties to the even index), saturation, signed zeros, all-zero groups, fp32
    subnormals and large magnitudes."""
    say("gpu e2m1 packer")
    g = torch.Generator().manual_seed(91)
    N, K = 40, 1024
    w = torch.randn(N, K, generator=g) * 0.02
    grid = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])
    mids = torch.tensor([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0])
    w[0, :32] = torch.cat([grid, -grid, mids, -mids, torch.tensor([6.0, 5.99, 7.0, 12.0,
                                                                    -0.0, 0.0, 0.1, -0.3, 4.5,
                                                                    5.5])])[:32]
    w[1, :32] = 0.0
    w[2, :32] = -0.0
    w[3] = torch.randn(K, generator=g) * 1e-40            # subnormal fp32
    w[4] = torch.randn(K, generator=g) * 1e30
    w[5, :32] = mids.repeat(5)[:32] * 2.0 ** -20          # midpoints at another scale
    hc, hs = C.quantize_e2m1(w)
    dc, ds = C.quantize_e2m1_gpu(w.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(dc.cpu(), hc)
    assert torch.equal(ds.cpu(), hs)
    oc, osc = O.e2m1_quantize(w.numpy())
    assert np.array_equal(O.unpack_nibbles(dc.cpu().numpy()), oc)
    assert np.array_equal(ds.cpu().numpy(), osc)
