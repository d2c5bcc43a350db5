"""The allocation-free entry point fb_gemv_noalloc (its rotation scratch is a fixed device
array, not a workspace argument) against fb_gemv with a caller workspace, through the C
ABI: two calls in a row, the second with a smaller input, each bitwise equal to fb_gemv's
result and within the north-star tolerance of the oracle's product."""
import ctypes
import sys

import numpy as np
import pytest
import torch

from oracle import fourbit_oracle as O
from if_i_could_turn_back_time_amd import _capi as C
from if_i_could_turn_back_time_amd import PackedWeight

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _run(fmt, N, K, B, block, seed):
    print("noalloc", fmt, N, K, B, block, flush=True)
    sys.stdout.flush()
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(N, K, generator=g) * 0.02
    pw = PackedWeight.quantize(w, fmt, fwht_block=block, device=DEV)
    xdt = torch.float16 if (fmt == "gf4" or block) else torch.bfloat16
    x = torch.randn(B, K, generator=g).to(xdt)
    shape = pw.shape(B, xdt, torch.float32)
    xd = x.to(DEV)
    sp = torch.cuda.current_stream().cuda_stream
    L = C.lib()
    need = C.workspace_bytes(shape)
    ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=DEV)
    y_ws = torch.full((B, N), float("nan"), device=DEV)
    assert L.fb_gemv(pw.wdev.data_ptr(), xd.data_ptr(), y_ws.data_ptr(), ctypes.byref(shape),
                     ws.data_ptr(), need, sp) == 0
    y_na = torch.full((B, N), float("nan"), device=DEV)
    assert L.fb_gemv_noalloc(pw.wdev.data_ptr(), xd.data_ptr(), y_na.data_ptr(),
                             ctypes.byref(shape), sp) == 0
    torch.cuda.synchronize()
    assert torch.equal(y_na, y_ws)
    codes = O.unpack_nibbles(pw.codes.numpy())
    meta = pw.meta.numpy().view(np.uint16) if fmt == "gf4" else pw.meta.numpy()
    yref = O.y_ref(fmt, codes, meta, x, block)
    err = (y_na.cpu() - yref).abs()
    assert bool((err <= 1e-2 + 1e-3 * yref.abs()).all()), float(err.max())
    return need


def test_noalloc_two_calls_second_smaller():
    # rotated: x is rotated into the scratch (256 KiB, then 32 KiB)
    assert _run("gf4", 2048, 8192, 16, 4096, 1) == 16 * 8192 * 2
    assert _run("gf4", 1024, 4096, 4, 4096, 2) == 4 * 4096 * 2
    # a 256-wide rotation and E2M1 weights, then a call that needs no scratch
    assert _run("e2m1", 520, 11008, 8, 256, 3) == 8 * 11008 * 2
    assert _run("gf4", 300, 1024, 2, 0, 4) == 0


def test_noalloc_rejects_shapes_beyond_its_scratch():
    L = C.lib()
    buf = torch.zeros(64, dtype=torch.uint8, device=DEV)
    big = C.make_shape(64, 65536, 16, C.FMT_GF4, 4096)    # 2 MiB of rotated x
    assert L.fb_gemv_noalloc(buf.data_ptr(), buf.data_ptr(), buf.data_ptr(),
                             ctypes.byref(big), None) == -15
    assert "scratch" in C.strerror(-15)
