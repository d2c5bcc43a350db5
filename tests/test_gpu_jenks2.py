"""GPU two-class Jenks (fb_jenks2_gpu) against the oracle and its host twin, bit for bit: the
split, the GVF and the mask, on the reference's pruned LeNet300 weights (the arrays its
Linear_Mask / Bias_Mask prune, cuda_helpers.py:378-411) and on random arrays across the
256-element block and 65536-element superblock edges; the per-filter version likewise."""
import sys
import time

import numpy as np
import pytest
import torch

from oracle import fourbit_oracle as O
from if_i_could_turn_back_time_amd import _capi as C
from if_i_could_turn_back_time_amd import bias_mask, linear_mask
from model_fixtures import lenet300_from_fixture

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _inputs():
    rng = np.random.default_rng(11)
    net = lenet300_from_fixture()
    for i in (1, 3, 5):
        yield f"lenet300.{i}.weight", net[i].weight.detach().numpy()
        yield f"lenet300.{i}.bias", net[i].bias.detach().numpy()
    for n in (1, 2, 3, 255, 256, 257, 4096, 65535, 65536, 65537, 131073, 1000003):
        w = (rng.standard_normal(n) * 0.02).astype(np.float32)
        if n > 8:
            w[rng.integers(0, n, n // 4)] = 0.0
            w[rng.integers(0, n, n // 8)] = -0.0
        yield f"random{n}", w
    yield "constant", np.full(3000, -0.125, np.float32)
    yield "two-levels", np.repeat(np.array([1.0, -2.0], np.float32), 777)


@pytest.mark.parametrize("case", list(range(20)))
def test_jenks2_gpu_bit_exact_vs_host(case):
    name, w = list(_inputs())[case]
    say("jenks2", name, w.size)
    wt = torch.from_numpy(np.ascontiguousarray(w))
    keep_h, split_h, gvf_h = C.jenks2_host(wt)
    keep_g, split_g, gvf_g = C.jenks2_gpu(wt.to(DEV))
    keep_o, split_o, gvf_o, _ = O.jenks2(w)
    assert split_g == split_h == split_o, name
    assert (np.float64(gvf_g).view(np.int64) == np.float64(gvf_h).view(np.int64)
            == np.float64(gvf_o).view(np.int64)), name
    assert torch.equal(keep_g.cpu(), keep_h), name
    assert np.array_equal(keep_g.cpu().numpy().astype(bool), keep_o), name


def test_linear_mask_on_device_matches_host():
    """linear_mask / bias_mask on ROCm tensors return what they return on the CPU."""
    net = lenet300_from_fixture()
    for i in (1, 3, 5):
        mh, gh = linear_mask(net[i].weight.detach())
        md, gd = linear_mask(net[i].weight.detach().to(DEV))
        assert torch.equal(mh, md) and gh == gd and md.device.type == "cpu"
        bh, _ = bias_mask(net[i].bias.detach())
        bd, _ = bias_mask(net[i].bias.detach().to(DEV))
        assert torch.equal(bh, bd)


def test_jenks2_gpu_large_array():
    """A 32M-value array (an 8192 x 4096 layer): bit-exact against the host twin; the
    GPU time is printed (the reference's one-thread-per-split kernel is O(n^2))."""
    g = torch.Generator().manual_seed(3)
    w = torch.randn(8192 * 4096, generator=g) * 0.02
    w[torch.rand(w.numel(), generator=g) < 0.5] = 0.0
    keep_h, split_h, gvf_h = C.jenks2_host(w)
    wd = w.to(DEV)
    C.jenks2_gpu(wd)                                   # warm-up
    torch.cuda.synchronize()
    t = time.perf_counter()
    keep_g, split_g, gvf_g = C.jenks2_gpu(wd)
    torch.cuda.synchronize()
    say(f"jenks2 gpu 32M values: {(time.perf_counter() - t) * 1e3:.1f} ms (incl. workspace "
        "allocation and the host copy of split / GVF)")
    assert split_g == split_h and gvf_g == gvf_h
    assert torch.equal(keep_g.cpu(), keep_h)


def _filter_inputs():
    """Convolution weights [out, in, kh, kw]: LeNet-5, VGG, AlexNet-stem and ResNet-stem
    filter sizes, the per-filter maximum of 1024 values, ties, signed zeros and constant
    filters."""
    rng = np.random.default_rng(12)
    # one filter per lane for 1024 or more filters of at most 25 values (2100 filters: a
    # partial last workgroup; 1 and 4 values), else one filter per one-wave workgroup (25
    # values in 6 filters; 26 values, the smallest size never run per lane)
    for shape in ((6, 1, 5, 5), (64, 64, 3, 3), (64, 3, 11, 11), (64, 3, 7, 7), (2, 3, 32, 32),
                  (7, 5, 1, 1), (3, 2, 16, 17), (3, 3, 2, 13), (300, 7, 3, 3), (7, 3, 2, 13),
                  (1024, 2, 1, 1), (40, 30, 2, 2), (64, 32, 5, 5)):
        yield f"random{shape}", (rng.standard_normal(shape) * 0.05).astype(np.float32)
    w = (np.round(rng.standard_normal((32, 16, 3, 3)) * 2) / 4).astype(np.float32)
    w[::3] = 0.0
    w[1::5, :, ::2] = -0.0
    w[2] = 0.7
    yield "ties", w


@pytest.mark.parametrize("case", list(range(14)))
def test_jenks2_filters_gpu_bit_exact_vs_host(case):
    """fb_jenks2_filters_gpu (the reference's Conv_Mask, cuda_helpers.py:333-376) against
    the oracle and its host twin, bit for bit, on every filter: split, GVF and mask."""
    name, w = list(_filter_inputs())[case]
    say("jenks2 filters", name)
    w2 = torch.from_numpy(w.reshape(w.shape[0] * w.shape[1], -1))
    keep_h, split_h, gvf_h = C.jenks2_filters_host(w2)
    keep_g, split_g, gvf_g = C.jenks2_filters_gpu(w2.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(split_g.cpu(), split_h), name
    assert torch.equal(gvf_g.cpu().view(torch.int64), gvf_h.view(torch.int64)), name
    assert torch.equal(keep_g.cpu(), keep_h), name
    keep_o, split_o, gvf_o = O.jenks2_filters(w2.numpy())
    assert np.array_equal(split_g.cpu().numpy(), split_o), name
    assert np.array_equal(gvf_g.cpu().numpy().view(np.int64), gvf_o.view(np.int64)), name
    assert np.array_equal(keep_g.cpu().numpy().astype(bool), keep_o), name


def test_conv_mask_on_device_matches_host():
    """conv_mask keeps the mask on the weights' device (as the reference's Conv_Mask does)
    and gives the host's mask and GVF list; a 512 x 512 x 3 x 3 layer is timed."""
    from if_i_could_turn_back_time_amd import jenks
    g = torch.Generator().manual_seed(5)
    w = torch.randn(512, 512, 3, 3, generator=g) * 0.05
    mh, gh = jenks.conv_mask(w)
    wd = w.to(DEV)
    jenks.conv_mask(wd)                                # warm-up
    torch.cuda.synchronize()
    t = time.perf_counter()
    md, gd = jenks.conv_mask(wd)
    torch.cuda.synchronize()
    say(f"conv_mask 512x512x3x3 on the GPU: {(time.perf_counter() - t) * 1e3:.2f} ms (incl. the "
        "finiteness check and the GVF copy to the host)")
    assert md.device.type == "cuda" and md.dtype == torch.float32
    assert torch.equal(md.cpu(), mh) and gd == gh


def _reference_var_f64(v):
    """The reference kernels' per-split SSD (cuda_helpers.py:85-118, :151-184: serial class
    means, then serial squared deviations), in float64."""
    v = np.asarray(v, np.float64)
    n = v.size
    var = np.zeros(n)
    for idx in range(n):
        m1 = v[:idx].sum() / idx if idx else 0.0
        m2 = v[idx:].sum() / (n - idx)
        var[idx] = ((v[:idx] - m1) ** 2).sum() + ((v[idx:] - m2) ** 2).sum()
    return var


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_jenks2_ssd_gpu_bit_exact_vs_oracle_and_host(dtype):
    """fb_jenks2_ssd_gpu (the per-split SSD the reference's optimizers bind,
    jenks_optimization_cuda / jenks_optimization_biases_cuda) against the oracle's
    jenks2_ssd rounded to the dtype and the host twin, bit for bit, across the block and
    superblock edges, with ties and signed zeros; and within float64 rounding of the
    reference kernels' own two-pass sums on a short array."""
    rng = np.random.default_rng(31)
    npdt = np.float32 if dtype == torch.float32 else np.float64
    for n in (1, 2, 255, 256, 257, 4096, 65535, 65536, 65537, 131073, 1000003):
        say("jenks2 ssd", dtype, n)
        w = (rng.standard_normal(n) * 0.02).astype(npdt)
        if n > 8:
            w[rng.integers(0, n, n // 4)] = 0.0
            w[rng.integers(0, n, n // 8)] = -0.0
        v = np.sort(w, kind="stable")
        vt = torch.from_numpy(v)
        got = C.jenks2_ssd(vt.to(DEV))
        torch.cuda.synchronize()
        assert got.dtype == dtype and got.device.type == "cuda" and got.shape == (n,)
        g = got.cpu().numpy()
        assert np.array_equal(g.view(np.uint8), O.jenks2_ssd(v).astype(npdt).view(np.uint8)), n
        assert np.array_equal(g.view(np.uint8), C.jenks2_ssd(vt).numpy().view(np.uint8)), n
    v = np.sort((rng.standard_t(3, size=300) * 0.05).astype(npdt))
    ref = _reference_var_f64(v)
    got = C.jenks2_ssd(torch.from_numpy(v).to(DEV)).cpu().numpy().astype(np.float64)
    tol = (1e-5 if dtype == torch.float32 else 1e-9) * ref[0]
    assert np.allclose(got, ref, rtol=0, atol=tol)


def test_reference_optimizer_call_pattern_binds_unchanged():
    """The reference's JenksSGD steps (custom_optimizer.py:130-139 for weights, :162-167 for
    biases) and Conv_Mask (cuda_helpers.py:349-359) run as written against module_weights,
    module_bias and module_conv: output shapes, dtypes and devices are the reference's, the
    values are the oracle's per-split SSD, and var.argmin() is the mask path's split."""
    from if_i_could_turn_back_time_amd import module_bias, module_conv, module_weights
    g = torch.Generator().manual_seed(41)
    W = (torch.randn(300, 100, generator=g) * 0.05).to(DEV)
    grad = torch.randn(300, 100, generator=g).to(DEV) * 0.01
    s_W = torch.abs(torch.mul(W, grad))
    WB_cuda_sorted, WB_cuda_indices = s_W.flatten().sort()
    WB_cuda_sorted = WB_cuda_sorted.reshape(s_W.shape)
    var = module_weights.jenks_optimization_cuda(WB_cuda_sorted)
    var_min = var.argmin().item()
    assert var.shape == (30000,) and var.dtype == torch.float32 and var.is_cuda
    srt = WB_cuda_sorted.reshape(-1).cpu().numpy()
    assert np.array_equal(var.cpu().numpy(), O.jenks2_ssd(srt).astype(np.float32))
    _, split, _, _ = O.jenks2(s_W.reshape(-1).cpu().numpy())
    ssd64 = O.jenks2_ssd(srt)
    assert var_min == int(np.argmin(var.cpu().numpy()))
    assert ssd64[var_min] <= ssd64[split] * (1 + 1e-6)        # equal up to the fp32 rounding
    b = (torch.randn(100, generator=g) * 0.05).to(DEV).double()
    B_cuda_sorted, _ = torch.abs(b).sort()
    vb = module_bias.jenks_optimization_biases_cuda(B_cuda_sorted)
    assert vb.shape == (100,) and vb.dtype == torch.float64
    assert np.array_equal(vb.cpu().numpy(), O.jenks2_ssd(B_cuda_sorted.cpu().numpy()))
    Wc = (torch.randn(16, 8, 3, 3, generator=g) * 0.05).to(DEV)
    flat = Wc.view(16 * 8, -1)
    sorted_weights, _ = torch.sort(flat, dim=1)
    weights_sorted = sorted_weights.view(16, 8, 3, 3).contiguous()
    vc = module_conv.jenks_optimization_cuda_conv(weights_sorted)
    assert vc.shape == (16 * 8 * 9,) and vc.dtype == torch.float32
    ref = np.stack([O.jenks2_ssd(r) for r in sorted_weights.cpu().numpy()]).astype(np.float32)
    assert np.array_equal(vc.cpu().numpy().reshape(128, 9), ref)
    _, cs, _ = O.jenks2_filters(flat.cpu().numpy())
    mins = vc.view(16, 8, -1).min(dim=2).indices.cpu().numpy().reshape(-1)
    ssds = [O.jenks2_ssd(r) for r in sorted_weights.cpu().numpy()]
    for f in range(128):
        assert ssds[f][mins[f]] <= ssds[f][cs[f]] * (1 + 1e-6) + 1e-30
    with pytest.raises(RuntimeError, match="contiguous"):
        module_weights.jenks_optimization_cuda(WB_cuda_sorted.t())
    with pytest.raises(RuntimeError, match="not implemented"):
        module_weights.jenks_optimization_cuda(WB_cuda_sorted.half())


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_jenks2_ssd_filters_gpu_bit_exact(dtype):
    """fb_jenks2_ssd_filters_gpu against the host twin and the oracle per filter, bit for
    bit, at the per-filter size edges (1, 9, 25, a 256-block and past it, the maximum)."""
    rng = np.random.default_rng(32)
    npdt = np.float32 if dtype == torch.float32 else np.float64
    for nf, n in ((3000, 9), (700, 25), (5, 1), (9, 256), (9, 257), (4, C.JENKS2_FILTER_MAX)):
        say("jenks2 ssd filters", dtype, nf, n)
        w = np.sort((rng.standard_normal((nf, n)) * 0.05).astype(npdt), axis=1)
        w[::7, : n // 2] = 0.0
        got = C.jenks2_ssd_filters(torch.from_numpy(w).to(DEV))
        torch.cuda.synchronize()
        assert got.dtype == dtype and got.is_cuda
        g = got.cpu().numpy()
        host = C.jenks2_ssd_filters(torch.from_numpy(w)).numpy()
        assert np.array_equal(g.view(np.uint8), host.view(np.uint8))
        for f in range(0, nf, max(1, nf // 25)):
            assert np.array_equal(g[f], O.jenks2_ssd(w[f]).astype(npdt)), (nf, n, f)
