"""The native FP4 path (fb_gemv_mx): E2M1 weights on v_mfma_scale_f32_16x16x128_f8f6f4, with
x split into two MX-E4M3 terms.  No counterpart in the reference, whose product is F.linear
on the dequantized weight (layers.py:36-38); the path is the matrix cores' native FP4 mode
for the small-batch contraction.

- The split (fb_mx_split) against the oracle's mx_split_x, byte for byte.
- The GEMV against the product of the device-decoded weight (bit-identical to the host and
  oracle decodes, checked on sampled rows) with the oracle's split of x, in fp64: the
  MFMA's fp32 accumulation is the only difference allowed, |err| <= 2^-16 sum |w x|.
- The GEMV against the exact product (bf16 x, unsplit) within the north star's tolerance,
  |y - y_ref| <= 1e-2 + 1e-3 |y_ref|: config 5a's shapes and generator (Student-t weights,
  bf16 x with 20x outliers), the split-K and sliced plans, ragged rows, every output dtype.
"""
import ctypes
import sys

import numpy as np
import pytest
import torch

from oracle import fourbit_oracle as O
from if_i_could_turn_back_time_amd import _capi as C
from if_i_could_turn_back_time_amd import PackedWeight, QuantLinear
from if_i_could_turn_back_time_amd import workloads as WL

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
ATOL, RTOL = 1e-2, 1e-3
ACC_REL = 2.0 ** -16  # fp32 accumulation against fp64, relative to sum |w x|


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _x_cases(B, K, kind, seed):
    g = torch.Generator().manual_seed(seed)
    x = WL.synth_x("cfg2", B, K, g).float()
    if kind == "edges":
        x[0, :32] = 0.0                                   # an all-zero block
        x[0, 32:64] *= 1e-30                              # tiny values
        if B > 1:
            x[1, :64] *= 1e30                             # huge values
            x[1, 64:96] = torch.linspace(-3e4, 3e4, 32)   # a wide block
            x[1, 96] = -3.0e38
        x[0, 128:160] = torch.tensor(2.0) ** torch.arange(-20, 12).float()  # 31 binades
    return x.to(torch.bfloat16)


@pytest.mark.parametrize("B,K,kind", [(1, 128, "plain"), (3, 1024, "edges"), (16, 4096, "edges"),
                                      (16, 11008, "plain"), (8, 8192, "plain")],
                         ids=lambda v: str(v))
def test_mx_split_bit_exact_vs_oracle(B, K, kind):
    say("mx split", B, K, kind)
    x = _x_cases(B, K, kind, B * 7 + K)
    shape = C.make_shape(64, K, B, C.FMT_E2M1, 0, C.DT_BF16, C.DT_F32)
    codes, scales = C.mx_split(x.to(DEV), shape)
    torch.cuda.synchronize()
    oc, osc = O.mx_split_x(x.float().numpy())
    assert np.array_equal(scales.cpu().numpy(), osc)
    assert np.array_equal(codes.cpu().numpy(), oc)


@pytest.mark.parametrize("order", ["sorted", "shuffled"])
def test_mx_split_every_bf16_value(order):
    """Every finite bf16 value (65,280 bit patterns, as x of 15 rows of 4,352) through the
    split, against the oracle's split byte for byte.  In pattern order each 32-value block
    holds neighbouring values of one sign, so every value meets term 0's rounding at its own
    block's scale; shuffled (seeded), the blocks span up to the whole exponent range, so
    small values round to E4M3 subnormals or zero at a large block's scale and term 1 picks
    them up."""
    p = np.arange(65536, dtype=np.uint32)
    p = p[((p >> 7) & 0xFF) != 0xFF]
    assert p.size == 15 * 4352
    if order == "shuffled":
        p = np.random.default_rng(5).permutation(p)
    x = torch.from_numpy(p.astype(np.uint16).view(np.int16).reshape(15, 4352)).view(torch.bfloat16)
    say("mx split, every bf16 value,", order)
    shape = C.make_shape(64, 4352, 15, C.FMT_E2M1, 0, C.DT_BF16, C.DT_F32)
    codes, scales = C.mx_split(x.to(DEV), shape)
    torch.cuda.synchronize()
    oc, osc = O.mx_split_x(x.float().numpy())
    bad = np.argwhere(scales.cpu().numpy() != osc)
    assert bad.size == 0, f"scale bytes differ at (term, row, block) {bad[:8].tolist()}"
    bad = np.argwhere(codes.cpu().numpy() != oc)
    assert bad.size == 0, f"codes differ at (term, row, k) {bad[:8].tolist()}"


_PW = {}


def _packed(N, K):
    key = (N, K)
    if key not in _PW:
        _PW.clear()
        torch.cuda.empty_cache()
        w = WL.synth_weight("cfg2", N, K, torch.Generator().manual_seed(N + K))
        pw = PackedWeight.quantize(w, "e2m1", device=DEV, packer="gpu")
        W = pw.dequant_device(torch.float32)
        rows = torch.randint(0, N, (16,), generator=torch.Generator().manual_seed(N))
        host = torch.stack([torch.from_numpy(pw.dequant_host_row(int(r))) for r in rows])
        assert torch.equal(W[rows].cpu().view(torch.int32), host.view(torch.int32))
        _PW[key] = (pw, W, rows)
    return _PW[key]


def _check_mx(N, K, B, kind="plain"):
    pw, W, rows = _packed(N, K)
    x = _x_cases(B, K, kind, 1000 + B)
    xd = x.to(DEV)
    y = pw.gemv_mx(xd, out_dtype=torch.float32)
    # the oracle's split in fp64, times the decoded weight in fp64 (on the GPU)
    oc, osc = O.mx_split_x(x.float().numpy())
    xs = torch.from_numpy(O.mx_terms_value(oc, osc)).to(DEV)
    W64 = W.double()
    y_mx = xs @ W64.t()
    mag = xs.abs() @ W64.abs().t()
    y_exact = xd.double() @ W64.t()
    torch.cuda.synchronize()
    ratio = float(((y.double() - y_mx).abs() / (mag + 1e-300)).max())
    say(f"  max |y - y_mx| / sum|w x| = {ratio:.3g} (2^{np.log2(max(ratio, 1e-300)):.1f})")
    assert bool(((y.double() - y_mx).abs() <= ACC_REL * mag + 1e-30).all()), ratio
    err = (y.double() - y_exact).abs()
    assert bool((err <= ATOL + RTOL * y_exact.abs()).all()), float(err.max())
    # sampled rows: the oracle's own decode of the packed codes and its split product
    codes = O.unpack_nibbles(pw.codes[rows].numpy())
    y_o = torch.from_numpy(O.y_ref_mx(codes, pw.meta[rows].numpy(), x.float().numpy()))
    mag_o = torch.from_numpy(np.abs(O.mx_terms_value(oc, osc)) @
                             np.abs(O.e2m1_dequant(codes, pw.meta[rows].numpy())).astype(np.float64).T)
    assert bool(((y[:, rows].double().cpu() - y_o).abs() <= ACC_REL * mag_o + 1e-30).all())
    # the same call again gives the same bits; narrower outputs are y rounded
    assert torch.equal(pw.gemv_mx(xd, out_dtype=torch.float32), y)
    for dt, ulp in ((torch.bfloat16, 2.0 ** -8), (torch.float16, 2.0 ** -11)):
        yn = pw.gemv_mx(xd, out_dtype=dt).double()
        ok = (yn - y.double()).abs() <= ulp * y.double().abs() + 1e-7
        assert bool((ok | ~torch.isfinite(y.to(dt).double())).all()), dt


@pytest.mark.parametrize("N,K,B,kind", [
    (96, 128, 1, "plain"), (100, 1024, 3, "edges"), (4096, 4096, 1, "plain"),
    (4096, 4096, 8, "edges"), (130, 28672, 4, "plain"),
    # config 5a: E2M1 with bf16 x at batch 8 / 16 (one slice, K-slices), and the split-K plan
    (8192, 8192, 8, "plain"), (8192, 8192, 16, "plain"), (28672, 8192, 8, "plain"),
    (28672, 8192, 16, "plain"), (4096, 11008, 16, "plain"),
    # K-slices whose last slice ends inside a 512 span (its staged groups past K read zeros)
    (12288, 11008, 16, "edges"),
], ids=lambda v: str(v))
def test_gemv_mx_vs_oracle(N, K, B, kind):
    say("gemv mx", N, K, B, kind)
    _check_mx(N, K, B, kind)


def test_gemv_mx_against_the_bf16_path():
    """The native FP4 path and the exact-decode bf16 path agree within the tolerance on
    config 5a's layer, and their difference is the split's (zero where the split is exact)."""
    pw, W, _ = _packed(8192, 8192)
    x = _x_cases(16, 8192, "plain", 5).to(DEV)
    y_mx = pw.gemv_mx(x, out_dtype=torch.float32)
    y_bf = pw.gemv(x, out_dtype=torch.float32)
    torch.cuda.synchronize()
    err = (y_mx - y_bf).abs()
    assert bool((err <= ATOL + RTOL * y_bf.abs()).all()), float(err.max())
    say(f"  fp4 mfma vs bf16 mfma: max abs diff {float(err.max()):.3g}")


def test_quantlinear_fp4_mfma():
    """QuantLinear(..., fp4_mfma=True): forward on any leading shape and dtype against the
    default path, backward through the decoded weight, and the formats it refuses."""
    torch.manual_seed(0)
    lin = torch.nn.Linear(1000, 300)
    q = QuantLinear(lin, fmt="e2m1", fp4_mfma=True).to(DEV)
    ref = QuantLinear(lin, fmt="e2m1").to(DEV)
    x = torch.randn(3, 7, 1000, device=DEV)
    for dt in (torch.bfloat16, torch.float32):
        y = q(x.to(dt))
        y0 = ref(x.to(torch.bfloat16).to(dt))
        assert y.shape == (3, 7, 300) and y.dtype == dt
        err = (y.float() - y0.float()).abs()
        assert bool((err <= ATOL + 2e-2 * y0.float().abs()).all()), float(err.max())
    xg = x.to(torch.bfloat16).requires_grad_(True)
    q(xg).float().sum().backward()
    xg0 = x.to(torch.bfloat16).requires_grad_(True)
    ref(xg0).float().sum().backward()
    assert torch.equal(xg.grad, xg0.grad)
    with pytest.raises(ValueError):
        QuantLinear(lin, fmt="gf4", fp4_mfma=True)
    with pytest.raises(ValueError):
        QuantLinear(torch.nn.Linear(1024, 64), fmt="e2m1", hadamard=True, fp4_mfma=True)


def test_gemv_mx_workspace_contract():
    """fb_gemv_mx refuses a missing, short or misaligned workspace with its error code and
    writes nothing; a larger one is fine."""
    pw, W, _ = _packed(96, 128)
    x = torch.randn(2, 128).to(torch.bfloat16).to(DEV)
    y = torch.full((2, 96), 7.0, device=DEV)
    shape = pw.shape(2, torch.bfloat16, torch.float32)
    need = C.mx_workspace_bytes(shape)
    assert need == (2 * 128 * 2 + 255) // 256 * 256 + 256
    L = C.lib()
    ws = torch.empty(need + 512, dtype=torch.uint8, device=DEV)
    args = (C._ptr(pw.wdev), C._ptr(x), C._ptr(y), ctypes.byref(shape))
    st = C._stream(x.device)
    assert L.fb_gemv_mx(*args, None, need, st) == -1                     # FB_ERR_NULL
    assert L.fb_gemv_mx(*args, C._ptr(ws), need - 1, st) == -8           # FB_ERR_WORKSPACE
    assert L.fb_gemv_mx(*args, C._ptr(ws) + 16, need, st) == -7          # FB_ERR_ALIGN
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())
    assert L.fb_gemv_mx(*args, C._ptr(ws), need + 512, st) == 0
    torch.cuda.synchronize()
    yref = x.double() @ W.double().t()
    assert bool(((y.double() - yref).abs() <= ATOL + RTOL * yref.abs()).all())


@pytest.mark.parametrize("N,K,B", [(8192, 8192, 8), (4096, 11008, 16), (100, 1024, 3)],
                         ids=lambda v: str(v))
def test_gemv_mx_presplit_equals_gemv_mx(N, K, B):
    """One split (fb_mx_split), then fb_gemv_mx_presplit: the bits of fb_gemv_mx with a
    workspace; without one (split-K shapes run their K-slices in turn) within the tolerance
    of the exact product.  Two layers on the same split each give their own result."""
    say("presplit", N, K, B)
    pw, W, _ = _packed(N, K)
    x = _x_cases(B, K, "plain", 77).to(DEV)
    shape = pw.shape(B, torch.bfloat16, torch.float32)
    xs = C.mx_split_raw(x, shape)
    y_mx = pw.gemv_mx(x, out_dtype=torch.float32)
    y_ps = C.gemv_mx_presplit(pw.wdev, xs, torch.empty(B, N, device=DEV), shape)
    torch.cuda.synchronize()
    assert torch.equal(y_ps, y_mx)
    y_nows = torch.empty(B, N, device=DEV)
    C.check(C.lib().fb_gemv_mx_presplit(C._ptr(pw.wdev), C._ptr(xs), C._ptr(y_nows),
                                        ctypes.byref(shape), None, 0, C._stream(x.device)))
    yref = x.double() @ W.double().t()
    torch.cuda.synchronize()
    assert bool(((y_nows.double() - yref).abs() <= ATOL + RTOL * yref.abs()).all())
    # a second layer on the same split (64 rows of another weight)
    w2 = WL.synth_weight("cfg2", 64, K, torch.Generator().manual_seed(9))
    pw2 = PackedWeight.quantize(w2, "e2m1", device=DEV, packer="gpu")
    sh2 = pw2.shape(B, torch.bfloat16, torch.float32)
    y2 = C.gemv_mx_presplit(pw2.wdev, xs, torch.empty(B, 64, device=DEV), sh2)
    assert torch.equal(y2, pw2.gemv_mx(x, out_dtype=torch.float32))


def test_fp4_mfma_shared_matches_each_layer():
    """Three E2M1 layers on one input (q/k/v-like), one split per 16 rows: each output has
    the bits of the layer's own fp4_mfma forward; with autograd on x it runs each layer on
    its own and the gradients are the layers' own."""
    from if_i_could_turn_back_time_amd import fp4_mfma_shared
    torch.manual_seed(1)
    lins = [torch.nn.Linear(1024, n) for n in (512, 256, 256)]
    qs = [QuantLinear(l, fmt="e2m1", fp4_mfma=True).to(DEV) for l in lins]
    x = torch.randn(2, 19, 1024, device=DEV).to(torch.bfloat16)  # 38 rows: 3 chunks
    ys = fp4_mfma_shared(qs, x)
    for q, y in zip(qs, ys):
        assert torch.equal(y, q(x))
    xg = x.clone().requires_grad_(True)
    outs = fp4_mfma_shared(qs, xg)
    sum(o.float().sum() for o in outs).backward()
    xg0 = x.clone().requires_grad_(True)
    sum(q(xg0).float().sum() for q in qs).backward()
    assert torch.equal(xg.grad, xg0.grad)
    with pytest.raises(ValueError):
        fp4_mfma_shared([qs[0], QuantLinear(torch.nn.Linear(1024, 64), fmt="gf4").to(DEV)], x)


def test_gemv_mx_in_hip_graph_replays_match_eager():
    """fb_gemv_mx captured in a HIP graph (its split and GEMV kernels; the workspace is cached
    by the PackedWeight before capture, and no memset is recorded): several replays with
    eager work between them, each equal to the eager result bit for bit."""
    for N, K, B in ((4096, 2048, 8), (4096, 11008, 16)):
        say("mx graph", N, K, B)
        pw, W, _ = _packed(N, K)
        x = _x_cases(B, K, "plain", 3).to(DEV)
        y = torch.empty(B, N, dtype=torch.float32, device=DEV)
        pw.gemv_mx(x, out=y)
        torch.cuda.synchronize()
        eager = y.clone()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            pw.gemv_mx(x, out=y)
            torch.cuda.synchronize()
            with torch.cuda.graph(graph, stream=s):
                pw.gemv_mx(x, out=y)
        torch.cuda.synchronize()
        for rep in range(4):
            y.fill_(float("nan"))
            x2 = (x.float() * 3).to(torch.bfloat16)
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(y, eager), (N, K, B, rep)
            assert x2.shape == x.shape


def test_gemv_mx_two_streams_match_serial():
    """Two layers' fb_gemv_mx calls interleaved on two streams, each layer with its own
    workspace, give the bits of the same calls one after the other."""
    g = torch.Generator().manual_seed(5)
    layers = []
    for N, K in ((4096, 4096), (3000, 8192)):
        pw = PackedWeight.quantize(WL.synth_weight("cfg2", N, K, g), "e2m1", device=DEV,
                                   packer="gpu")
        xs = [_x_cases(4, K, "plain", 50 + i).to(DEV) for i in range(5)]
        layers.append((pw, xs))
    serial = [[pw.gemv_mx(x, out_dtype=torch.float32) for x in xs] for pw, xs in layers]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [[None] * 5 for _ in layers]
    for i in range(5):
        for j, ((pw, xs), s) in enumerate(zip(layers, streams)):
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):  # a layer's calls (and its workspace) stay on one stream
                outs[j][i] = pw.gemv_mx(xs[i], out_dtype=torch.float32)
    torch.cuda.synchronize()
    for j in range(2):
        for i in range(5):
            assert torch.equal(outs[j][i], serial[j][i]), (j, i)
