"""GPU parity at the benchmark configurations' own shapes and input generators, plus the
edges of the product's contract: weight streams past 2 GiB, E2M1 scale bytes at the
fp16 limits, fp16 activation range checks and the backward pass of the packed linear.

Full-size layers are checked on every row against torch's fp32 product of the
device-decoded weight (itself compared bit for bit with the host decode on sampled rows),
and on sampled rows against the oracle's dequantize-then-F.linear.  The tolerance is the
north star's: |y - y_ref| <= 1e-2 + 1e-3 |y_ref|.  The batched product these replace is the
reference's F.linear (layers.py:36-38) and linear_kernel_batch
(CUDA_C_Code/include/layers.h:9828-9839)."""
import sys

import numpy as np
import pytest
import torch

from oracle import fourbit_oracle as O
from if_i_could_turn_back_time_amd import _capi as C
from if_i_could_turn_back_time_amd import PackedWeight, QuantLinear
from if_i_could_turn_back_time_amd import workloads as WL
from if_i_could_turn_back_time_amd.linear import E2M1_F16_SCALES

pytestmark = pytest.mark.gpu
ATOL, RTOL = 1e-2, 1e-3
DEV = "cuda:0"


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def within_tol(y, yref, extra_rel=0.0):
    y = y.float().cpu()
    yref = yref.float().cpu()
    err = (y - yref).abs()
    return bool((err <= ATOL + (RTOL + extra_rel) * yref.abs()).all()), float(err.max())


_CACHE = {}


def packed(fmt, K, N, kind):
    """Packed weight of one generator/shape; one layer is kept at a time (the batch
    variants of a shape run one after another)."""
    key = (fmt, K, N, kind)
    if key not in _CACHE:
        _CACHE.clear()
        torch.cuda.empty_cache()
        w = WL.synth_weight(kind, N, K, torch.Generator().manual_seed(0))
        # the GPU Jenks packer gives the host packer's bytes (test_gpu_packer_bit_exact_vs_host)
        pw = PackedWeight.quantize(w, fmt, device=DEV, packer="gpu")
        W = pw.dequant_device(torch.float32)
        rows = torch.randint(0, N, (24,), generator=torch.Generator().manual_seed(N + K))
        host = torch.stack([torch.from_numpy(pw.dequant_host_row(int(r))) for r in rows])
        assert torch.equal(W[rows].cpu().view(torch.int32), host.view(torch.int32))
        _CACHE[key] = (pw, W, rows, host)
    return _CACHE[key]


def check_layer(fmt, K, N, B, kind, xdt=None):
    pw, W, rows, host = packed(fmt, K, N, kind)
    g = torch.Generator().manual_seed(1000 + B)
    x = WL.synth_x(kind, B, K, g).to(xdt or WL.x_dtype(fmt))
    xd = x.to(DEV)
    y = pw.gemv(xd, out_dtype=torch.float32)
    y16 = pw.gemv(xd, out_dtype=x.dtype)
    yref = xd.float() @ W.t()
    torch.cuda.synchronize()
    ok, emax = within_tol(y, yref)
    assert ok, f"all rows vs device decode: max abs err {emax}"
    extra = 2.0 ** -11 if x.dtype == torch.float16 else 2.0 ** -8
    ok, emax = within_tol(y16, yref, extra)
    assert ok, f"{x.dtype} output: max abs err {emax}"
    # sampled rows against the oracle's own decode and fp32 F.linear
    codes = O.unpack_nibbles(pw.codes[rows].numpy())
    meta = pw.meta[rows].numpy()
    Wo = O.dequant_f32(fmt, codes, meta.view(np.uint16) if fmt == "gf4" else meta)
    assert torch.equal(Wo, host)
    ok, emax = within_tol(y[:, rows], torch.nn.functional.linear(x.float(), Wo))
    assert ok, f"oracle rows: max abs err {emax}"
    # the same call again gives the same bits
    assert torch.equal(pw.gemv(xd, out_dtype=torch.float32), y)


# Config 5: the small-batch dense contraction, E2M1 (Student-t weights, bf16 x with 20x
# outliers) and GF4 (N(0, 0.02) weights, fp16 x).
@pytest.mark.parametrize("fmt,K,N,kind,B", [
    ("e2m1", 8192, 8192, "cfg2", 8), ("e2m1", 8192, 8192, "cfg2", 16),
    ("e2m1", 8192, 28672, "cfg2", 8), ("e2m1", 8192, 28672, "cfg2", 16),
    ("gf4", 8192, 8192, "cfg1", 8), ("gf4", 8192, 8192, "cfg1", 16),
    ("gf4", 8192, 28672, "cfg1", 8), ("gf4", 8192, 28672, "cfg1", 16),
    # batch 16 over the Llama-7B down projection: the split-K plan's shape
    ("e2m1", 11008, 4096, "cfg2", 16), ("gf4", 11008, 4096, "cfg1", 16),
], ids=lambda v: str(v))
def test_config5_small_batch(fmt, K, N, kind, B):
    say("config 5", fmt, K, N, B)
    check_layer(fmt, K, N, B, kind)


# Batches 2-16 on the 8-wave plan with several row tiles per workgroup (GF4, short rows: up to
# 64 units per workgroup), one K-slice and two: 4096 -> 11008 owns 2-3 row tiles per workgroup,
# 4096 -> 28672 seven.
@pytest.mark.parametrize("K,N,B", [(4096, 11008, 4), (4096, 11008, 16), (4096, 28672, 2),
                                   (3968, 11003, 3)],  # ragged rows, K not a multiple of 512
                         ids=lambda v: str(v))
def test_gf4_batch_several_tiles_per_8wave_workgroup(K, N, B):
    say("gf4 8-wave batch", K, N, B)
    check_layer("gf4", K, N, B, "cfg1")


def staged_slices(fmt, K, N, B, xdt):
    """Slices of the plan fb_gemv takes for this shape (fb_phase_plan of the diagnostic
    library, built beside the product one); 0: each wave stages the x of its own spans."""
    import ctypes
    from pathlib import Path
    T_lib = ctypes.CDLL(str(Path(C.__file__).resolve().parent / "libfourbit_trace.so"))
    ip = ctypes.POINTER(ctypes.c_int)
    T_lib.fb_phase_plan.argtypes = [ctypes.POINTER(C.FbShape), ip, ip, ip, ip, ip, ip]
    s = C.make_shape(N, K, B, C.FMT_GF4 if fmt == "gf4" else C.FMT_E2M1, 0, xdt, C.DT_F16)
    v = [ctypes.c_int() for _ in range(6)]
    assert T_lib.fb_phase_plan(ctypes.byref(s), *[ctypes.byref(a) for a in v]) == 0
    return v[2].value


# Batches whose x the staged plan would cut into K-slices, on the plan where each of the 8
# waves stages the x of its own spans: several row tiles per workgroup (up to 7), a K that ends inside
# a span (11008 = 21.5 spans), ragged rows, one span per wave (E2M1), batches that are not a
# power of two, fp16 x, and a layer that split-K would otherwise take (16384 -> 4096).
@pytest.mark.parametrize("fmt,K,N,B,xdt", [
    ("gf4", 8192, 8192, 12, torch.float16), ("e2m1", 8192, 8192, 12, torch.bfloat16),
    ("gf4", 11008, 4001, 8, torch.float16), ("e2m1", 11008, 4001, 12, torch.float16),
    ("e2m1", 4096, 11008, 16, torch.bfloat16), ("gf4", 28672, 8192, 3, torch.float16),
    ("e2m1", 16384, 4096, 16, torch.bfloat16), ("gf4", 8192, 16384, 16, torch.float16),
    ("e2m1", 8192, 28672, 12, torch.bfloat16),  # 7 row tiles per workgroup
    ("e2m1", 3584, 28672, 16, torch.bfloat16),  # 7 spans: wave 7 owns none (zero slots)
], ids=lambda v: str(v).replace("torch.", ""))
def test_waves_stage_their_own_spans(fmt, K, N, B, xdt):
    say("own-span plan", fmt, K, N, B, xdt)
    assert staged_slices(fmt, K, N, B, C.DT_F16 if xdt == torch.float16 else C.DT_BF16) == 0
    check_layer(fmt, K, N, B, "cfg1" if fmt == "gf4" else "cfg2", xdt=xdt)


# E2M1 with fp16 activations on the 8-wave batch plans: one K-slice at batch 8, each wave
# staging its own spans at batch 16.
@pytest.mark.parametrize("B", [8, 16])
def test_e2m1_fp16_x_batch_8wave(B):
    say("e2m1 fp16 x 8-wave batch", B)
    check_layer("e2m1", 8192, 8192, B, "cfg2", xdt=torch.float16)


# Config 4: the 70B MLP shapes with the 0.5% heavy tail at 8 sigma (wide Jenks codebooks).
@pytest.mark.parametrize("K,N,B", [
    (8192, 28672, 1), (8192, 28672, 2), (8192, 28672, 4),
    (28672, 8192, 1), (28672, 8192, 2), (28672, 8192, 4),
], ids=lambda v: str(v))
def test_config4_heavy_tail(K, N, B):
    say("config 4", K, N, B)
    check_layer("gf4", K, N, B, "cfg4")


# Config 2: Llama-7B shapes in E2M1 with Student-t weights and activation outliers.
@pytest.mark.parametrize("K,N", [(4096, 4096), (4096, 11008), (11008, 4096)],
                         ids=lambda v: str(v))
def test_config2_student_t(K, N):
    say("config 2", K, N)
    check_layer("e2m1", K, N, 1, "cfg2")


# Config 1: the GF4 4096 x 4096 layer at batch 1 (the CPU baseline's configuration).
def test_config1_gf4_full_size():
    say("config 1", 4096, 4096)
    check_layer("gf4", 4096, 4096, 1, "cfg1")


def check_layer_rot(fmt, K, N, block, kind):
    """A rotated layer at full size, batch 1: every row against the device-decoded weight
    W' (rotated basis) times x' = H_b x / sqrt(b) (the oracle's fp64 rotation, as fp32) in
    fp32 torch; sampled rows against the oracle's own decode; the same bits twice."""
    g = torch.Generator().manual_seed(0)
    w = WL.synth_weight(kind, N, K, g)
    x = WL.synth_x(kind, 1, K, g).half()      # rotations take fp16 x
    pw = PackedWeight.quantize(w, fmt, fwht_block=block, device=DEV,
                               packer="gpu" if fmt == "gf4" else "host")
    assert pw.f16_exact
    W = pw.dequant_device(torch.float32)
    xr = O.rotate_x(x, block)
    xd = x.to(DEV)
    y = pw.gemv(xd, out_dtype=torch.float32)
    y16 = pw.gemv(xd, out_dtype=torch.float16)
    yref = xr.to(DEV) @ W.t()
    torch.cuda.synchronize()
    ok, emax = within_tol(y, yref)
    assert ok, f"all rows vs device decode: max abs err {emax}"
    ok, emax = within_tol(y16, yref, 2.0 ** -11)
    assert ok, f"fp16 output: max abs err {emax}"
    rows = torch.randint(0, N, (24,), generator=torch.Generator().manual_seed(N + K))
    codes = O.unpack_nibbles(pw.codes[rows].numpy())
    meta = pw.meta[rows].numpy()
    meta = meta.view(np.uint16) if fmt == "gf4" else meta
    Wo = O.dequant_f32(fmt, codes, meta)
    assert torch.equal(W[rows].cpu().view(torch.int32), Wo.view(torch.int32))
    ok, emax = within_tol(y[:, rows], O.y_ref(fmt, codes, meta, x, block))
    assert ok, f"oracle rows: max abs err {emax}"
    assert torch.equal(pw.gemv(xd, out_dtype=torch.float32), y)


# Config 3: the Llama-7B shapes in GF4 with the fused Walsh-Hadamard rotation, at full size
# (4096 -> 11008 runs the 8-wave rotated batch-1 plan with 2-3 row tiles per workgroup), and
# one E2M1 layer through the same rotated kernel.
@pytest.mark.parametrize("fmt,K,N,block,kind", [
    ("gf4", 4096, 4096, 4096, "cfg1"), ("gf4", 4096, 11008, 4096, "cfg1"),
    ("gf4", 11008, 4096, 256, "cfg1"), ("e2m1", 4096, 11008, 4096, "cfg2"),
], ids=lambda v: str(v))
def test_config3_rotated_full_size(fmt, K, N, block, kind):
    say("config 3", fmt, K, N, block)
    check_layer_rot(fmt, K, N, block, kind)


def _random_packed(fmt, N, K, seed):
    """A packed weight of random codes and random codebooks / scale bytes (no packing
    run: the shape is too large for the Jenks packer to be quick)."""
    g = torch.Generator().manual_seed(seed)
    codes = torch.randint(0, 256, (N, K // 2), dtype=torch.uint8, generator=g)
    if fmt == "gf4":
        meta = (torch.randn(N, K // 128, 16, generator=g) * 0.02).half().view(torch.int16)
    else:
        meta = torch.randint(118, 124, (N, K // 32), dtype=torch.uint8, generator=g)
    return PackedWeight(fmt, N, K, codes, meta, 0, DEV)


@pytest.mark.parametrize("fmt", ["gf4", "e2m1"])
def test_batch1_more_row_tiles_than_threads(fmt):
    """Batch 1 over a short K and a very long N: each 8-wave (512-thread) workgroup owns
    more row tiles than it has threads (N = 2,200,000, K = 512: 137,500 tiles, 538 per
    workgroup on 256 CUs), so the per-tile unit counters are cleared by a strided loop.
    Every row is checked against the device-decoded weight times x in fp32 torch, sampled
    rows against the oracle's decode, and the same call twice gives the same bits."""
    N, K = 2_200_000, 512
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    T = (N + 15) // 16
    say("tiles > threads", fmt, N, K, "tiles per workgroup", -(-T // min(T, cus)))
    pw = _random_packed(fmt, N, K, 17)
    xdt = torch.float16 if fmt == "gf4" else torch.bfloat16
    x = torch.randn(1, K, generator=torch.Generator().manual_seed(3)).to(xdt)
    xd = x.to(DEV)
    y = torch.full((1, N), float("nan"), device=DEV)
    pw.gemv(xd, out=y)
    W = pw.dequant_device(torch.float32)
    yref = xd.float() @ W.t()
    torch.cuda.synchronize()
    del W
    assert bool(torch.isfinite(y).all()), "outputs left unwritten"
    ok, emax = within_tol(y, yref)
    assert ok, f"all rows vs device decode: max abs err {emax}"
    rows = torch.randint(0, N, (32,), generator=torch.Generator().manual_seed(4))
    rows[0], rows[1] = N - 1, (T - 1) * 16 - 1       # the last tile and the one before
    codes = O.unpack_nibbles(pw.codes[rows].numpy())
    meta = pw.meta[rows].numpy()
    Wo = O.dequant_f32(fmt, codes, meta.view(np.uint16) if fmt == "gf4" else meta)
    ok, emax = within_tol(y[:, rows], torch.nn.functional.linear(x.float(), Wo))
    assert ok, f"oracle rows: max abs err {emax}"
    y2 = torch.full((1, N), float("nan"), device=DEV)
    pw.gemv(xd, out=y2)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)


@pytest.mark.parametrize("N", [11008, 14336])
def test_gf4_batch1_several_tiles_per_8wave_workgroup(N):
    """GF4 batch 1 at K = 4096 with more row tiles T than CUs: the plan runs one 8-wave
    workgroup per CU (the max-ILP copy of the kernel), each owning T // CUs row tiles and the
    first T % CUs one more (2-3 tiles at N = 11008 and 3-4 at N = 14336 on 256 CUs)."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    T = N // 16
    say("8-wave plan", N, "tiles", T, "CUs", cus)
    if T <= cus:
        pytest.skip(f"{cus} CUs: {T} row tiles give one tile per workgroup")
    check_layer("gf4", 4096, N, 1, "cfg1")


def test_weight_stream_past_2gib():
    """A GF4 layer whose device stream is 2.25 GiB (49152 x 65536): every 16-row tile and
    512-wide span holds the same block, so every row tile must give the same outputs, bit
    for bit, including the tiles stored past 2^31 bytes, and they must match the fp32
    product of the block's decode with the span-summed x."""
    say("2 GiB stream")
    N, K = 49152, 65536
    g = torch.Generator().manual_seed(5)
    blk = PackedWeight.quantize(torch.randn(16, 512, generator=g) * 0.02, "gf4")
    assert blk.wdev.numel() == 6144
    shape = C.make_shape(N, K, 1, C.FMT_GF4, 0, C.DT_F16, C.DT_F32)
    nbytes = C.device_bytes(shape)
    assert nbytes > 2 ** 31
    wdev = blk.wdev.to(DEV).repeat(nbytes // 6144)
    x = torch.randn(1, K, generator=g).half()
    y = torch.empty(1, N, dtype=torch.float32, device=DEV)
    C.gemv(wdev, x.to(DEV), y, shape)
    torch.cuda.synchronize()
    tiles = y.view(-1, 16)
    assert torch.equal(tiles, tiles[:1].expand_as(tiles)), "row tiles differ"
    Wb = blk.dequant_host().double()
    xs = x.double().view(-1, 512).sum(dim=0)
    yref = (Wb @ xs).float()
    ok, emax = within_tol(tiles[0], yref)
    assert ok, f"max abs err {emax}"
    del wdev


def _e2m1_weight_with_scales(scales):
    """[len(scales), 128] weights whose first 32-group gets E8M0 byte s (amax 6 * 2^(s-127))
    with values on the E2M1 grid, the rest scale byte 127."""
    grid = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])
    rows = []
    for i, s in enumerate(scales):
        r = torch.zeros(128)
        v = torch.cat([grid, -grid]).repeat(2) * 2.0 ** (s - 127)
        r[:32] = v
        r[32:] = torch.cat([grid, -grid]).repeat(6)[:96]
        rows.append(r)
    return torch.stack(rows)


def test_e2m1_scale_bytes_at_fp16_limits():
    """E8M0 bytes 0, 103, 104, 140, 141: the device decode is exact (fp32) for all; the
    GEMV with bf16 x matches the fp32 product; with fp16 x the weights decode to fp16,
    which is exact only for bytes 104..140, and PackedWeight refuses the others."""
    say("e2m1 scale limits")
    for s in (0, 103, 104, 140, 141):
        w = _e2m1_weight_with_scales([s] * 16)
        pw = PackedWeight.quantize(w, "e2m1", device=DEV)
        assert int(pw.meta[0, 0]) == s
        W = pw.dequant_device(torch.float32).cpu()
        assert torch.equal(W, pw.dequant_host())
        assert torch.equal(W, w)
        x = torch.randn(2, 128, generator=torch.Generator().manual_seed(s)).to(torch.bfloat16)
        y = pw.gemv(x.to(DEV), out_dtype=torch.float32).cpu()
        # E8M0 byte 0 (2^-127) is taken as 0 by the GEMV's converter: values below 2^-124
        # do not reach the output
        Wk = W.clone()
        if s == 0:
            Wk[:, :32] = 0
        ok, emax = within_tol(y, x.float() @ Wk.t())
        assert ok, f"byte {s} bf16: {emax}"
        exact16 = E2M1_F16_SCALES[0] <= s <= E2M1_F16_SCALES[1]
        assert pw.f16_exact == exact16
        xh = x.half()
        if exact16:
            y = pw.gemv(xh.to(DEV), out_dtype=torch.float32).cpu()
            ok, emax = within_tol(y, xh.float() @ W.t())
            assert ok, f"byte {s} fp16: {emax}"
        else:
            with pytest.raises(ValueError, match="fp16"):
                pw.gemv(xh.to(DEV), out_dtype=torch.float32)


def test_fp16_range_checks():
    """GF4 and rotated layers stage x in fp16.  With range_check on, a bf16 activation
    beyond 65504 raises, as does a rotation block whose L2 norm reaches 65504; by default
    (no host sync) such an overflow shows as non-finite outputs."""
    say("fp16 range")
    lin = torch.nn.Linear(4096, 32)
    q = QuantLinear(lin).to(DEV)
    assert q.range_check is False
    x = torch.randn(2, 4096, device=DEV, dtype=torch.bfloat16)
    q(x)
    x[1, 7] = 70000.0
    assert not torch.isfinite(q(x)).all()
    q.range_check = True
    with pytest.raises(ValueError, match="fp16 range"):
        q(x)
    qr = QuantLinear(lin, hadamard=True).to(DEV)
    qr.range_check = True
    xh = torch.randn(1, 4096, device=DEV, dtype=torch.float16)
    qr(xh)
    xh[0, :4] = 40000.0                                     # block norm 80000
    with pytest.raises(ValueError, match="norm"):
        qr(xh)
    qe = QuantLinear(lin, fmt="e2m1").to(DEV)
    qe.range_check = True
    qe(x)                                                   # bf16 x: no fp16 staging


@pytest.mark.parametrize("K,N,hadamard", [(4096, 4096, True), (11008, 4096, True),
                                          (8192, 1024, False)])
def test_quantlinear_graph_capture_replays(K, N, hadamard):
    """QuantLinear's forward captured in a HIP graph at batch 8 and replayed: a rotated
    layer (x rotated once into the module's cached workspace, then the GEMV) and a plain
    one.  Every replay, with the program's own eager work and synchronisations between
    them, gives the eager forward's bits for the input then in the static buffer; the
    graph records no allocation or memset of the workspace (the module caches an
    uninitialised one, and the forward makes no host sync)."""
    say("graph capture", K, N, hadamard)
    B = 8
    g = torch.Generator().manual_seed(K + N)
    q = QuantLinear(torch.nn.Linear(K, N), hadamard=hadamard, packer="gpu").to(DEV)
    xs = [torch.randn(B, K, generator=g).half().to(DEV) for _ in range(4)]
    eager = []
    for x in xs:
        eager.append(q(x))
    torch.cuda.synchronize()
    static_x = xs[0].clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        q(static_x)                                        # the stream's own workspace
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):               # s's workspace, made above
        static_y = q(static_x)
    for rep in range(3):
        for i, x in enumerate(xs):
            static_x.copy_(x)
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(static_y, eager[i]), f"replay {rep}, input {i}"
            # eager work of the program's own between replays (on the default stream,
            # with that stream's workspace)
            junk = q(xs[(i + 1) % len(xs)])
            assert torch.equal(junk, eager[(i + 1) % len(xs)])
            torch.cuda.synchronize()


@pytest.mark.parametrize("fmt,K,hadamard", [("gf4", 1024, False), ("e2m1", 1024, False),
                                            ("gf4", 300, False), ("gf4", 4096, True),
                                            ("gf4", 11008, True), ("e2m1", 2048, 256)])
def test_backward_matches_linear_with_decoded_weight(fmt, K, hadamard):
    """The packed linear is differentiable in x and bias as F.linear with the frozen
    committed weight is (layers.py:34-35): grad_x = grad_y W (W the committed weight, i.e.
    the decode rotated back for a rotated layer) and grad_bias = sum of grad_y.  The
    forward with grad enabled gives the same bits as without."""
    say("backward", fmt, K, hadamard)
    g = torch.Generator().manual_seed(K)
    N = 96
    lin = torch.nn.Linear(K, N)
    q = QuantLinear(lin, fmt=fmt, hadamard=hadamard).to(DEV)
    xdt = torch.float16 if fmt == "gf4" else torch.bfloat16
    x = torch.randn(3, 5, K, generator=g).to(xdt).to(DEV).requires_grad_(True)
    gy = torch.randn(3, 5, N, generator=g).to(xdt).to(DEV)
    y = q(x)
    with torch.no_grad():
        y_nograd = q(x)
    assert torch.equal(y.detach(), y_nograd)
    y.backward(gy)
    q.commit()                                              # weight = exact committed decode
    Wc = q.weight.detach().float()
    gx_ref = (gy.float().reshape(-1, N) @ Wc).reshape(3, 5, K)
    ok, emax = within_tol(x.grad, gx_ref, 2.0 ** -8 if xdt == torch.bfloat16 else 2.0 ** -10)
    assert ok, f"grad_x: max abs err {emax}"
    gb_ref = gy.float().reshape(-1, N).sum(0)
    ok, emax = within_tol(q.bias.grad, gb_ref, 2.0 ** -8)
    assert ok, f"grad_bias: {emax}"


@pytest.mark.parametrize("N,K,B,block", [(4096, 4096, 8, 4096), (96, 11008, 16, 256),
                                         (520, 8192, 4, 4096), (64, 4096, 4, 2048)])
def test_rotated_batch_with_and_without_workspace(N, K, B, block):
    """Rotated batches of B*K >= 16384 values rotate x once into the workspace (an extra
    small kernel; at batch 16 with K = 11008 the GEMV after it also runs its K-parts side by
    side through the workspace), else (no workspace passed) in every workgroup's prologue:
    both within tolerance of the oracle's rotated product, and of each other."""
    import ctypes
    say("rotate once", N, K, B, block)
    g = torch.Generator().manual_seed(N + K + B)
    w = torch.randn(N, K, generator=g) * 0.02
    pw = PackedWeight.quantize(w, "gf4", fwht_block=block, device=DEV)
    x = torch.randn(B, K, generator=g).half()
    codes = O.unpack_nibbles(pw.codes.numpy())
    yref = O.y_ref("gf4", codes, pw.meta.numpy().view(np.uint16), x, block)
    shape = pw.shape(B, torch.float16, torch.float32)
    need = C.workspace_bytes(shape)
    # the rotated x, then (batch 16 at K = 11008) the split-K parts' sums
    assert need == B * K * 2 or need == B * K * 2 + 4 * B * N * 4
    xd = x.to(DEV)
    ys = {}
    for mode in ("workspace", "none"):
        y = torch.full((B, N), float("nan"), device=DEV)
        ws = torch.zeros(need, dtype=torch.uint8, device=DEV) if mode == "workspace" else None
        rc = C.lib().fb_gemv(pw.wdev.data_ptr(), xd.data_ptr(), y.data_ptr(), ctypes.byref(shape),
                             None if ws is None else ws.data_ptr(), need if ws is not None else 0,
                             torch.cuda.current_stream().cuda_stream)
        assert rc == 0
        torch.cuda.synchronize()
        ok, emax = within_tol(y, yref)
        assert ok, f"{mode}: max abs err {emax}"
        ys[mode] = y.cpu()
    ok, emax = within_tol(ys["workspace"], ys["none"])
    assert ok, emax


@pytest.mark.parametrize("fmt,N,ydt,K", [("gf4", 4096, torch.float16, 11008),
                                         ("e2m1", 4096, torch.bfloat16, 11008),
                                         ("gf4", 1000, torch.float32, 11008),
                                         ("e2m1", 72, torch.float16, 11008),
                                         ("gf4", 200, torch.bfloat16, 28672),
                                         ("e2m1", 512, torch.float32, 28672)])
def test_splitk_against_slices_and_oracle(fmt, N, ydt, K):
    """Batch 16 at K = 11008 (22 spans: parts of 6, 6, 6 and 4) runs its K-parts side by side
    through the workspace and adds their fp32 sums in part order; at K = 28672 (56 spans,
    x of 917 KB in 6 slices) in eight parts of 7.  Checked: within tolerance of the sliced
    plan (no workspace) and of the device-decoded weight x fp32 torch on all rows, the same
    bits on a second call (the last part sums only its own spans), and sampled rows against
    the oracle's exact decode.  The reference's batched product it replaces is
    layers.h:9828-9839 / layers.py:36-38."""
    import ctypes
    B = 16
    P = 4 if K == 11008 else 8
    say("split-K", fmt, N, K, B, ydt)
    g = torch.Generator().manual_seed(N + 7)
    w = torch.randn(N, K, generator=g) * 0.02
    pw = PackedWeight.quantize(w, fmt, device=DEV, packer="gpu" if fmt == "gf4" else "host")
    xdt = torch.float16 if fmt == "gf4" else torch.bfloat16
    x = (torch.randn(B, K, generator=g) * 0.5).to(xdt).to(DEV)
    shape = pw.shape(B, xdt, ydt)
    need = C.workspace_bytes(shape)
    assert need == P * B * N * 4   # the parts' fp32 sums
    ws = torch.full((need,), 0xFF, dtype=torch.uint8, device=DEV)   # no zero-fill needed
    L = C.lib()
    sp = torch.cuda.current_stream().cuda_stream
    outs = []
    for ws_ptr, nws in ((ws.data_ptr(), need), (ws.data_ptr(), need), (None, 0)):
        y = torch.full((B, N), float("nan"), dtype=ydt, device=DEV)
        assert L.fb_gemv(pw.wdev.data_ptr(), x.data_ptr(), y.data_ptr(), ctypes.byref(shape),
                         ws_ptr, nws, sp) == 0
        outs.append(y)
    torch.cuda.synchronize()
    y_sk, y_sk2, y_sl = outs
    assert torch.equal(y_sk, y_sk2)
    W = pw.dequant_device(torch.float32)
    yref = x.float() @ W.t()
    extra = 4e-3 if ydt != torch.float32 else 0.0   # the output's own rounding
    ok, emax = within_tol(y_sk, yref, extra)
    assert ok, f"split-K vs torch: {emax}"
    ok, emax = within_tol(y_sk, y_sl.float(), extra)
    assert ok, f"split-K vs slices: {emax}"
    rows = torch.randint(0, N, (8,), generator=g)
    host = pw.dequant_host()[rows]
    ok, emax = within_tol(y_sk[:, rows], torch.nn.functional.linear(x.cpu().float(), host), extra)
    assert ok, f"split-K vs oracle decode: {emax}"


def test_one_workspace_shared_across_shapes_and_paths():
    """One uninitialised workspace (sized for the largest call) serves split-K calls of
    different shapes and part counts, a rotated call whose x' lands where the other shapes'
    part sums were, and the native FP4 path, interleaved and repeated: every call gives the
    bits of the same call on a fresh workspace, whatever the previous calls left in it."""
    import ctypes
    g = torch.Generator().manual_seed(77)
    cases = []
    for fmt, N, K, B, block in (("gf4", 1000, 11008, 16, 0), ("e2m1", 520, 28672, 16, 0),
                                ("gf4", 640, 11008, 16, 256), ("gf4", 96, 11008, 12, 0)):
        w = torch.randn(N, K, generator=g) * 0.02
        pw = PackedWeight.quantize(w, fmt, fwht_block=block, device=DEV,
                                   packer="gpu" if fmt == "gf4" else "host")
        xdt = torch.float16 if fmt == "gf4" else torch.bfloat16
        x = torch.randn(B, K, generator=g).to(xdt).to(DEV)
        cases.append((pw, x, pw.shape(B, xdt, torch.float32)))
    L = C.lib()
    sp = torch.cuda.current_stream().cuda_stream
    need = max(C.workspace_bytes(sh) for _, _, sh in cases)
    mx_sh = cases[1][2]
    need = max(need, C.mx_workspace_bytes(mx_sh))
    shared = torch.full((need,), 0x7F, dtype=torch.uint8, device=DEV)

    def call(i, ws, mx=False):
        pw, x, sh = cases[i]
        y = torch.full((sh.B, sh.N), float("nan"), device=DEV)
        f = L.fb_gemv_mx if mx else L.fb_gemv
        assert f(pw.wdev.data_ptr(), x.data_ptr(), y.data_ptr(), ctypes.byref(sh),
                 ws.data_ptr(), ws.numel(), sp) == 0
        return y

    fresh = {}
    for i in range(len(cases)):
        fresh[i] = call(i, torch.empty(need, dtype=torch.uint8, device=DEV))
    fresh["mx"] = call(1, torch.empty(need, dtype=torch.uint8, device=DEV), mx=True)
    order = [0, 1, 2, 3, "mx", 2, 0, 3, 1, "mx", 0]
    for k in order:
        y = call(1, shared, mx=True) if k == "mx" else call(k, shared)
        torch.cuda.synchronize()
        assert torch.equal(y, fresh[k]), f"case {k}"
    for i, (pw, x, sh) in enumerate(cases):
        W = pw.dequant_device(torch.float32)
        xr = O.rotate_x(x.cpu(), pw.fwht_block).to(DEV) if pw.fwht_block else x.float()
        ok, emax = within_tol(fresh[i], xr @ W.t())
        assert ok, f"case {i}: max abs err {emax}"
