"""GPU two-class Jenks (fb_jenks2_gpu) against its host twin, bit for bit: the split, the
GVF and the mask, on the reference's pruned LeNet300 weights (the arrays its Linear_Mask /
Bias_Mask prune, cuda_helpers.py:378-411) and on random arrays across the 256-element block
and 65536-element superblock edges.  The host twin is itself checked against the oracle
(tests/test_host.py)."""
import sys
import time

import numpy as np
import pytest
import torch

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
    assert split_g == split_h, name
    assert np.float64(gvf_g).view(np.int64) == np.float64(gvf_h).view(np.int64), name
    assert torch.equal(keep_g.cpu(), keep_h), name


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
    its host twin, bit for bit, on every filter: split, GVF and mask."""
    name, w = list(_filter_inputs())[case]
    say("jenks2 filters", name)
    w2 = torch.from_numpy(w.reshape(w.shape[0] * w.shape[1], -1))
    keep_h, split_h, gvf_h = C.jenks2_filters_host(w2)
    keep_g, split_g, gvf_g = C.jenks2_filters_gpu(w2.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(split_g.cpu(), split_h), name
    assert torch.equal(gvf_g.cpu().view(torch.int64), gvf_h.view(torch.int64)), name
    assert torch.equal(keep_g.cpu(), keep_h), name


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
