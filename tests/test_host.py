"""CPU tests of the product's host side: the C ABI loads and exports what
include/fourbit.h declares, argument validation, and the native packers / layout
transform against the oracle and the golden fixtures (bit-exact)."""
import ctypes
import re
import shutil
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import fourbit_oracle as O
from if_i_could_turn_back_time_amd import _capi as C
from if_i_could_turn_back_time_amd import PackedWeight, QuantLinear, fwht_block_for, quantize_module
from model_fixtures import lenet300_from_fixture, reference_state

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = sorted((ROOT / "tests" / "golden").glob("*.npz"))
RNG = np.random.default_rng(7)


def test_abi_exports_every_declared_symbol():
    header = (ROOT / "include" / "fourbit.h").read_text()
    declared = set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(fb_\w+)\(", header, re.M))
    assert declared == set(C.EXPORTED)
    L = C.lib()
    for name in declared:
        assert getattr(L, name) is not None
    assert L.fb_abi_version() == C.ABI_VERSION


def test_diagnostic_trace_library_exports():
    """libfourbit_trace.so (the GEMV with per-wave phase timestamps, read by
    `bench.py --phase-trace`) exports the same C ABI plus its diagnostic entry points (the
    phase buffer, the launch plan, the launch-floor kernels of the GEMV and of the FP4 path's
    split, the forced split-K part count, the x fill-rate kernel); the product library exports
    none of those."""
    path = Path(C.__file__).resolve().parent / "libfourbit_trace.so"
    T = ctypes.CDLL(str(path))
    for name in C.EXPORTED:
        assert getattr(T, name) is not None
    assert T.fb_phase_trace_set is not None and T.fb_phase_plan is not None
    assert T.fb_phase_floor is not None
    T.fb_phase_trace_set.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    assert T.fb_phase_trace_set(None, 0) == 0  # host-side only: needs no GPU
    T.fb_phase_floor.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    assert T.fb_phase_floor(None, None) == -1  # validated before any device call
    assert T.fb_phase_force_parts(3) == -2 and T.fb_phase_force_parts(0) == 0
    T.fb_phase_mx_floor.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_size_t, ctypes.c_void_p]
    assert T.fb_phase_mx_floor(None, None, None, None, None, 0, None) == -1
    T.fb_phase_xfill.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                 ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    assert T.fb_phase_xfill(None, 16, 1024, 1, 1, None, None) == -1
    one = ctypes.c_char_p(b"x")  # any non-null pointer: the shape is checked before any launch
    for xb, nt, passes in ((24, 1024, 1), (512 * 1024, 1024, 1), (16, 256, 1), (16, 512, 3)):
        assert T.fb_phase_xfill(one, xb, nt, passes, 1, one, None) == -2
    for name in ("fb_phase_trace_set", "fb_phase_plan", "fb_phase_floor", "fb_phase_force_parts",
                 "fb_phase_mx_floor", "fb_phase_xfill"):
        with pytest.raises(AttributeError):
            getattr(C.lib(), name)


def test_batch1_plans_over_a_shape_sweep():
    """The GEMV's launch plan (fb_phase_plan of the diagnostic library, host-side: without a
    GPU it plans for 256 CUs, an MI355X's count) over batch-1 shapes up to N = 4.2M: every
    valid shape gets a plan, batch-1 layers that fit one K-slice run one 8-wave workgroup
    per CU (the largest fall back to 16 waves or K-slices), and the row tiles are split
    evenly (tq or tq + 1 per workgroup, covering every tile once).  Shapes of short K and
    long N give workgroups more row tiles than threads, whose per-tile unit counters the
    kernel clears with a strided loop; the GPU suite runs such a shape (N = 2,200,000,
    K = 512: 538 tiles per 512-thread workgroup)."""
    T_lib = ctypes.CDLL(str(Path(C.__file__).resolve().parent / "libfourbit_trace.so"))
    ip = ctypes.POINTER(ctypes.c_int)
    T_lib.fb_phase_plan.argtypes = [ctypes.POINTER(C.FbShape), ip, ip, ip, ip, ip, ip]
    over = []
    for fmt in (C.FMT_GF4, C.FMT_E2M1):
        xdt = C.DT_F16 if fmt == C.FMT_GF4 else C.DT_BF16
        for K in (128, 512, 2048, 4096, 8192):
            for N in (1, 16, 4095, 65536, 2_200_000, 4_200_000):
                s = C.make_shape(N, K, 1, fmt, 0, xdt, C.DT_F32)
                v = [ctypes.c_int() for _ in range(6)]
                assert T_lib.fb_phase_plan(ctypes.byref(s), *[ctypes.byref(a) for a in v]) == 0
                grid, waves, slices, tq, tr, parts = (a.value for a in v)
                assert parts == 0
                T = (N + 15) // 16
                assert grid == min(T, 256) and waves in (8, 16) and slices >= 1, (fmt, K, N)
                assert grid * tq + tr == T and 0 <= tr < grid
                if N < 65536 or K * N < 2 ** 30:  # x and the slots fit one slice, 8 waves
                    assert waves == 8 and slices == 1, (fmt, K, N)
                if slices == 1 and tq + (tr > 0) > waves * 64:
                    over.append((fmt, K, N, tq + (tr > 0)))
    assert (C.FMT_GF4, 512, 2_200_000, 538) in over
    assert (C.FMT_E2M1, 512, 2_200_000, 538) in over


def test_small_batch_wave_plans():
    """Batches 2-16 (fb_phase_plan, host-side, 256 CUs): unrotated GF4 and E2M1 layers of at
    most 2 row tiles per CU (GF4: or at most 64 units per workgroup) whose x fits one
    K-slice, or two of at most 2 units per wave each, run one 8-wave workgroup per CU;
    layers of more units, rotated layers and x that needs more or larger K-slices keep
    16-wave workgroups.  Where the staged plan needs K-slices, each wave owns two or more
    units (GF4: spans) and a workgroup at most 4 row tiles (8 at batch 8-16), the 8 waves stage
    the x of their own spans instead (kSpanX, reported as 0 slices)."""
    T_lib = ctypes.CDLL(str(Path(C.__file__).resolve().parent / "libfourbit_trace.so"))
    ip = ctypes.POINTER(ctypes.c_int)
    T_lib.fb_phase_plan.argtypes = [ctypes.POINTER(C.FbShape), ip, ip, ip, ip, ip, ip]

    def plan(fmt, K, N, B, fb=0, xdt=None):
        if xdt is None:
            xdt = C.DT_F16 if fmt == C.FMT_GF4 else C.DT_BF16
        s = C.make_shape(N, K, B, fmt, fb, xdt, C.DT_F16)
        v = [ctypes.c_int() for _ in range(6)]
        assert T_lib.fb_phase_plan(ctypes.byref(s), *[ctypes.byref(a) for a in v]) == 0
        return v[1].value, v[2].value  # waves, slices

    for K, N, B in ((8192, 8192, 2), (8192, 8192, 8), (4096, 4096, 4), (28672, 8192, 2)):
        assert plan(C.FMT_GF4, K, N, B) == (8, 1), (K, N, B)
        assert plan(C.FMT_E2M1, K, N, B) == (8, 1), (K, N, B)
        assert plan(C.FMT_E2M1, K, N, B, xdt=C.DT_F16) == (8, 1), (K, N, B)
    assert plan(C.FMT_GF4, 8192, 28672, 2)[0] == 16  # 7 row tiles of 16 spans: 112 units
    assert plan(C.FMT_GF4, 4096, 11008, 4) == (8, 1)  # 3 row tiles of 8 spans: 24 units
    assert plan(C.FMT_GF4, 4096, 28672, 4) == (8, 1)  # 56 units
    assert plan(C.FMT_GF4, 4096, 28672, 16)[0] == 16  # 28 units per slice
    assert plan(C.FMT_E2M1, 4096, 11008, 4)[0] == 16  # E2M1: at most 2 row tiles per CU
    # x in K-slices: each wave stages its own spans instead
    assert plan(C.FMT_GF4, 8192, 8192, 16) == (8, 0)
    assert plan(C.FMT_E2M1, 8192, 8192, 16) == (8, 0)
    assert plan(C.FMT_GF4, 11008, 4096, 8) == (8, 0)
    assert plan(C.FMT_GF4, 28672, 8192, 4) == (8, 0)
    assert plan(C.FMT_GF4, 28672, 8192, 8) == (8, 0)
    assert plan(C.FMT_GF4, 8192, 28672, 16) == (8, 0)  # 7 row tiles at batch 16
    assert plan(C.FMT_E2M1, 4096, 11008, 16) == (8, 0)  # E2M1: one span per wave
    assert plan(C.FMT_GF4, 8192, 28672, 8) == (8, 0)  # 7 row tiles at batch 8
    assert plan(C.FMT_E2M1, 3584, 28672, 16) == (8, 0)  # 7 spans: one wave owns none
    # ... but not with more than 4 row tiles below batch 8, GF4 with one span per wave, one
    # unit per wave, or where split-K (over fewer than 4 spans per wave) takes the layer
    assert plan(C.FMT_GF4, 28672, 28672, 4)[1] != 0
    assert plan(C.FMT_GF4, 4096, 11008, 16) == (8, 2)  # 12 units per slice
    assert plan(C.FMT_E2M1, 4096, 4096, 16)[1] != 0
    assert plan(C.FMT_GF4, 11008, 4096, 16)[1] != 0
    assert plan(C.FMT_GF4, 4096, 4096, 2, fb=4096)[0] == 16  # rotated in the kernel


def test_batch_plans_over_a_shape_sweep():
    """Every valid batch 2-16 shape gets a plan (fb_phase_plan, host-side, 256 CUs): the row
    tiles are split evenly over the grid, 8-wave workgroups take at most two K-slices and no
    split-K parts, split-K plans (K >= 10240 only) run 2, 4 or 8 parts, and plans whose waves
    stage their own spans (0 slices) have 8 waves and at most 4 row tiles per workgroup (8
    at batch 8-16)."""
    T_lib = ctypes.CDLL(str(Path(C.__file__).resolve().parent / "libfourbit_trace.so"))
    ip = ctypes.POINTER(ctypes.c_int)
    T_lib.fb_phase_plan.argtypes = [ctypes.POINTER(C.FbShape), ip, ip, ip, ip, ip, ip]
    seen = set()
    for fmt, xdt in ((C.FMT_GF4, C.DT_F16), (C.FMT_E2M1, C.DT_BF16), (C.FMT_E2M1, C.DT_F16)):
        for B in (2, 3, 4, 8, 16):
            for K in (128, 512, 4096, 8192, 11008, 28672):
                for N in (1, 64, 4096, 11008, 28672):
                    s = C.make_shape(N, K, B, fmt, 0, xdt, C.DT_F16)
                    v = [ctypes.c_int() for _ in range(6)]
                    assert T_lib.fb_phase_plan(ctypes.byref(s), *[ctypes.byref(a) for a in v]) == 0
                    grid, waves, slices, tq, tr, parts = (a.value for a in v)
                    T = (N + 15) // 16
                    assert waves in (8, 16) and slices >= 0, (fmt, B, K, N)
                    assert grid * tq + tr == T and 0 <= tr < grid, (fmt, B, K, N)
                    if slices == 0:
                        assert waves == 8 and not parts, (fmt, B, K, N)
                        assert tq + (tr > 0) <= (8 if B >= 8 else 4), (fmt, B, K, N)
                    if waves == 8 and not parts:
                        assert slices <= 2, (fmt, B, K, N)
                    if parts:
                        assert K >= 10240 and parts in (2, 4, 8), (fmt, B, K, N)
                    seen.add((waves, slices, bool(parts)))
    # every kind of plan occurs in the sweep
    assert {(8, 0, False), (8, 1, False), (8, 2, False), (16, 1, False)} <= seen
    assert any(w == 16 and sl > 1 for w, sl, _ in seen)
    assert any(p for _, _, p in seen)


@pytest.mark.parametrize("kw,err", [
    (dict(K=100), -2), (dict(K=0), -2), (dict(N=0), -2), (dict(B=0), -2),
    (dict(group=64), -3), (dict(fmt=7), -4), (dict(x_dtype=C.DT_BF16), -5),
    (dict(y_dtype=9), -5), (dict(fwht_block=3), -6), (dict(fwht_block=8192), -6),
    (dict(K=8192, fwht_block=8192), -6),
])
def test_validate_errors(kw, err):
    s = dict(N=64, K=1024, B=1, group=128, fmt=C.FMT_GF4, fwht_block=0, x_dtype=C.DT_F16,
             y_dtype=C.DT_F16)
    s.update(kw)
    sh = C.FbShape(**s)
    assert C.lib().fb_validate(ctypes.byref(sh)) == err
    assert "fourbit" in C.strerror(err)


def test_gemv_validation_needs_no_gpu():
    sh = C.make_shape(64, 1024, 17)
    buf = ctypes.c_char_p(b"x" * 64)
    assert C.lib().fb_gemv(buf, buf, buf, ctypes.byref(sh), None, 0, None) == -9  # batch 17
    sh = C.make_shape(64, 1024, 1)
    assert C.lib().fb_gemv(None, buf, buf, ctypes.byref(sh), None, 0, None) == -1
    sh.group = 32
    assert C.lib().fb_gemv(buf, buf, buf, ctypes.byref(sh), None, 0, None) == -3


def test_quantizers_reject_nonfinite():
    w = torch.zeros(2, 128)
    w[1, 5] = float("nan")
    with pytest.raises(RuntimeError, match="non-finite"):
        C.quantize_gf4(w)
    with pytest.raises(RuntimeError, match="non-finite"):
        C.quantize_e2m1(w)


def _weights(kind, N, K):
    if kind == "normal":
        return (RNG.normal(size=(N, K)) * 0.02).astype(np.float32)
    if kind == "heavy":
        w = RNG.normal(size=(N, K)) * 0.015
        m = RNG.random(size=(N, K)) < 0.005
        w[m] = RNG.normal(size=m.sum()) * 8 * 0.015
        return w.astype(np.float32)
    if kind == "sparse":  # ~98% zeros like the reference's pruned checkpoints
        w = RNG.normal(size=(N, K)) * 0.05
        w[RNG.random(size=(N, K)) < 0.98] = 0.0
        return w.astype(np.float32)
    if kind == "few":
        return RNG.choice(np.float32([-0.5, 0.0, 0.125, 3.0]), size=(N, K)).astype(np.float32)
    raise ValueError(kind)


@pytest.mark.parametrize("kind", ["normal", "heavy", "sparse", "few"])
def test_native_gf4_bit_exact_vs_oracle(kind):
    w = _weights(kind, 6, 768)
    codes, book = C.quantize_gf4(torch.from_numpy(w), nthreads=3)
    oc, ob = O.gf4_quantize(w)
    assert np.array_equal(O.unpack_nibbles(codes.numpy()), oc)
    assert np.array_equal(book.numpy().view(np.uint16), ob)


@pytest.mark.parametrize("kind", ["normal", "heavy", "sparse", "few"])
def test_native_e2m1_bit_exact_vs_oracle(kind):
    w = _weights(kind, 16, 1024)
    w[0, :32] *= 1e-30  # denormal / tiny groups hit the E8M0 clamp
    codes, sc = C.quantize_e2m1(torch.from_numpy(w), nthreads=4)
    oc, osc = O.e2m1_quantize(w)
    assert np.array_equal(O.unpack_nibbles(codes.numpy()), oc)
    assert np.array_equal(sc.numpy(), osc)


@pytest.mark.parametrize("block", [2, 256, 4096])
def test_native_fwht_bit_exact_vs_oracle(block):
    w = _weights("normal", 3, 8192)
    assert np.array_equal(C.fwht_rows(torch.from_numpy(w), block).numpy(),
                          O.rotate_weights(w, block))


@pytest.mark.parametrize("fmt", [C.FMT_GF4, C.FMT_E2M1])
@pytest.mark.parametrize("N,K", [(1, 128), (3, 384), (65, 256), (7, 11008 // 43 * 2)])
def test_device_layout_roundtrip(fmt, N, K):
    codes = torch.from_numpy(RNG.integers(0, 256, size=(N, K // 2), dtype=np.uint8))
    if fmt == C.FMT_GF4:
        meta = torch.from_numpy(RNG.integers(0, 2**16, size=(N, K // 128, 16), dtype=np.uint16)
                                .view(np.int16))
    else:
        meta = torch.from_numpy(RNG.integers(0, 255, size=(N, K // 32), dtype=np.uint8))
    sh = C.make_shape(N, K, 1, fmt)
    dev = C.to_device_layout(codes, meta, sh)
    tiles, spans = -(-N // 16), -(-(K // 128) // 4)
    assert dev.numel() == tiles * spans * (6144 if fmt == C.FMT_GF4 else 4352)
    c2, m2 = C.from_device_layout(dev, sh)
    assert torch.equal(c2, codes) and torch.equal(m2, meta)


def test_gf4_table_solver_exhaustive_bytes():
    """Every byte value in every table slot decodes back through the v_perm model."""
    for trial in range(300):
        T = RNG.integers(0, 256, 16, dtype=np.uint8)
        if trial < 256:
            T[trial % 16] = trial  # sweep each byte value through a slot
        codes = torch.zeros(1, 64, dtype=torch.uint8)
        book = torch.from_numpy((T.astype(np.uint16) | (T[::-1].astype(np.uint16) << 8))
                                .view(np.int16)[None, None, :].copy())
        sh = C.make_shape(1, 128, 1, C.FMT_GF4)
        _, b2 = C.from_device_layout(C.to_device_layout(codes, book, sh), sh)
        assert torch.equal(b2, book)


@pytest.mark.parametrize("path", GOLDEN, ids=lambda p: p.stem)
def test_golden_fixture_native_and_oracle(path):
    d = np.load(path)
    w, fb = d["w"], int(d["fwht_block"])
    fmt = "gf4" if "codebook" in d else "e2m1"
    N, K = w.shape
    # the oracle still reproduces its stored outputs
    if fmt == "gf4":
        oc, ob = O.gf4_quantize(w)
        assert np.array_equal(O.pack_nibbles(oc), d["codes"])
        assert np.array_equal(ob, d["codebook"])
        meta = torch.from_numpy(d["codebook"].view(np.int16))
        x = torch.from_numpy(d["x"]).view(torch.float16)
    else:
        oc, os_ = O.e2m1_quantize(w)
        assert np.array_equal(O.pack_nibbles(oc), d["codes"])
        assert np.array_equal(os_, d["scales"])
        meta = torch.from_numpy(d["scales"])
        x = torch.from_numpy(d["x"]).view(torch.bfloat16)
    y = O.y_ref(fmt, O.unpack_nibbles(d["codes"]), d["codebook"] if fmt == "gf4" else d["scales"],
                x, fb)
    assert torch.equal(y, torch.from_numpy(d["y"]))
    # the native packer (on the already rotated weight) reproduces the stored codes
    pw = PackedWeight.quantize(torch.from_numpy(w), fmt)
    assert np.array_equal(pw.codes.numpy(), d["codes"])
    assert torch.equal(pw.meta, meta)
    # exact host decode
    deq = pw.dequant_host()
    assert torch.equal(deq, O.dequant_f32(fmt, O.unpack_nibbles(d["codes"]),
                                          d["codebook"] if fmt == "gf4" else d["scales"]))


def test_fwht_block_rule():
    assert fwht_block_for(4096) == 4096
    assert fwht_block_for(11008) == 256
    assert fwht_block_for(28672) == 4096
    assert fwht_block_for(8192) == 4096


def test_quantlinear_api_on_cpu():
    lin = torch.nn.Linear(256, 48)
    q = QuantLinear(lin)                         # reference ctor: (linear_module, bitwidth, mask)
    assert q.weight.shape == (48, 256) and not q.weight.requires_grad
    assert q.codes.shape == (48, 128) and q.meta.shape == (48, 2, 16)
    with pytest.raises(RuntimeError, match="GPU"):
        q(torch.randn(2, 256))
    # like F.linear, an input whose last dimension is not in_features is refused (here
    # before the device check): [2, 512] would otherwise reshape to 4 rows of 256
    for bad in (torch.randn(2, 512), torch.randn(256, 2), torch.tensor(1.0)):
        with pytest.raises(RuntimeError, match="in_features=256"):
            q(bad)
    with pytest.raises(ValueError):
        QuantLinear(lin, bitwidth=8)
    # commit(): weight becomes the exact decode of the packed codes
    q.commit()
    assert q.hard_quant
    assert torch.equal(q.weight.data, q.dequantized_weight())
    # state_dict round trip rebuilds the device stream
    sd = q.state_dict()
    assert {"codes", "meta", "fb_header", "weight", "bias"} <= set(sd)
    q2 = QuantLinear(torch.nn.Linear(256, 48), fmt="e2m1")
    q2.load_state_dict(sd)
    assert q2.fmt == "gf4" and torch.equal(q2.wdev, q.wdev)
    # hadamard: committed weight is rotated back to the original basis
    qh = QuantLinear(lin, hadamard=True)
    assert qh.fwht_block == 256
    qh.commit()
    assert (qh.weight - lin.weight).abs().max() < 0.05


def test_quantize_module_swaps_linears_and_keeps_masks():
    net = torch.nn.Sequential(torch.nn.Linear(128, 64), torch.nn.ReLU(), torch.nn.Linear(64 * 2, 8))
    with torch.no_grad():
        net[0].weight[:, :64] = 0.0
    q = quantize_module(net, fmt="e2m1")
    assert isinstance(q[0], QuantLinear) and isinstance(q[2], QuantLinear)
    assert isinstance(net[0], torch.nn.Linear) and not isinstance(net[0], QuantLinear)
    assert torch.equal(q[0].mask[:, :64], torch.zeros(64, 64))
    assert (q[0].dequantized_weight()[:, :64] == 0).all()


def test_workspace_contract():
    """fb_gemv's workspace holds x rotated once per call (rotated shapes of at least 16384
    activation values, B*K*2 rounded up to 256) and, for the split-K plan, the K-parts' fp32
    sums after it (P*B*N*4: unrotated batches whose sliced plan needs 3 or more slices of a
    long K over few row tiles); 0 bytes otherwise.  Invalid shapes report 0 and are still
    rejected by fb_gemv."""
    for B in (1, 4, 16):
        assert C.workspace_bytes(C.make_shape(8192, 28672, B)) == 0
    # 11008 -> 4096 at batch 16: 3 slices of 1 row tile each -> 4 parts side by side
    assert C.workspace_bytes(C.make_shape(4096, 11008, 16)) == 4 * 16 * 4096 * 4
    assert C.workspace_bytes(C.make_shape(4096, 11008, 16, C.FMT_E2M1, 0, C.DT_BF16)) == \
        4 * 16 * 4096 * 4
    assert C.workspace_bytes(C.make_shape(4096, 11008, 8)) == 0      # 2 slices
    assert C.workspace_bytes(C.make_shape(8192, 8192, 16)) == 0      # K too short
    # rotated once, then split-K on the rotated x: both, the sums after x'
    assert C.workspace_bytes(C.make_shape(96, 11008, 16, C.FMT_GF4, 256)) == \
        16 * 11008 * 2 + 4 * 16 * 96 * 4
    assert C.workspace_bytes(C.make_shape(4096, 4096, 3, C.FMT_GF4, 4096)) == 0
    assert C.workspace_bytes(C.make_shape(4096, 4096, 4, C.FMT_GF4, 4096)) == 4 * 4096 * 2
    assert C.workspace_bytes(C.make_shape(4096, 11008, 2, C.FMT_GF4, 256)) == 44032
    assert C.workspace_bytes(C.make_shape(4096, 11008, 1, C.FMT_GF4, 256)) == 0
    assert C.workspace_bytes(C.make_shape(64, 100, 4, C.FMT_GF4, 4096)) == 0   # invalid K
    buf = ctypes.c_char_p(b"x" * 64)
    big = C.make_shape(8192, 28672, 17)
    assert C.lib().fb_gemv(buf, buf, buf, ctypes.byref(big), None, 0, None) == -9


def test_magic_division_identity():
    """The GEMV kernel divides by runtime values with one multiply-high and one compare:
    q = hi32(n * m), m = floor(2^32 / d) (2^32 - 1 for d = 1), then q + 1 if (q + 1) d <= n.
    Exhaustive over small n and d, sampled up to n < 2^30."""
    import random
    rnd = random.Random(5)

    def magic(d):
        return 0xFFFFFFFF if d == 1 else (1 << 32) // d

    def fdiv(n, d):
        q = (n * magic(d)) >> 32
        return q + 1 if (q + 1) * d <= n else q

    for d in list(range(1, 257)) + [1000, 4093, 32767, 32768, 65535]:
        for n in list(range(0, 3000)) + [rnd.randrange(0, 1 << 30) for _ in range(300)]:
            assert fdiv(n, d) == n // d, (n, d)


# ----------------------------------------------------------------------------- masks, levels
@pytest.mark.parametrize("density", [0.0, 0.02, 0.3, 0.9, 1.0])
def test_native_gf4_masked_bit_exact_vs_oracle(density):
    g = torch.Generator().manual_seed(int(density * 100))
    w = torch.randn(12, 512, generator=g) * 0.02
    keep = torch.rand(12, 512, generator=g) < density
    keep[0] = True                                      # a fully kept row
    w[~keep] = float("nan")                             # masked values are never read
    codes, book = C.quantize_gf4(w, 4, keep)
    oc, ob = O.gf4_quantize_masked(w.numpy(), keep.numpy())
    assert np.array_equal(O.unpack_nibbles(codes.numpy()), oc)
    assert np.array_equal(book.numpy().view(np.uint16), ob)
    c0, b0 = C.quantize_gf4(w[:1], 4)                   # no mask: fb_quantize_gf4
    assert torch.equal(codes[:1], c0) and torch.equal(book[:1], b0)


def test_native_pack_levels_bit_exact_and_errors():
    g = torch.Generator().manual_seed(2)
    N, K = 10, 384
    lev = (torch.randint(-8, -6, (N, K // 128, 1), generator=g)
           + torch.randint(0, 16, (N, K // 128, 128), generator=g)).reshape(N, K).float()
    lev[0, :128] = -0.0
    s = torch.rand(N, generator=g) * 0.01 + 1e-4
    codes, book = C.pack_levels_gf4(lev, s, 3)
    oc, ob = O.levels_to_gf4(lev.numpy(), s.numpy())
    assert np.array_equal(O.unpack_nibbles(codes.numpy()), oc)
    assert np.array_equal(book.numpy().view(np.uint16), ob)
    bad = lev.clone()
    bad[4, 0], bad[4, 1] = -8, 8
    with pytest.raises(RuntimeError, match="span more than 16"):
        C.pack_levels_gf4(bad, s)
    bad = lev.clone()
    bad[4, 7] = 1.5
    with pytest.raises(RuntimeError, match="non-integer"):
        C.pack_levels_gf4(bad, s)
    with pytest.raises(RuntimeError, match="scale"):
        C.pack_levels_gf4(lev, torch.zeros(N))
    with pytest.raises(RuntimeError, match="fp16 range"):
        C.pack_levels_gf4(lev, torch.full((N,), 1e4))


def test_quantlinear_ragged_k_keeps_masked_and_padding_zero():
    """in_features not a multiple of 128: the packed weight is zero-padded to the next
    multiple; masked and padded entries decode to exactly 0 (GF4) and the kept
    values of a group are unaffected by the padding."""
    g = torch.Generator().manual_seed(4)
    lin = torch.nn.Linear(300, 40)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(40, 300, generator=g) * 0.02)
    mask = (torch.rand(40, 300, generator=g) > 0.7).float()
    q = QuantLinear(lin, mask=mask)
    assert q.k_pack == 384 and q.codes.shape == (40, 192) and q.meta.shape == (40, 3, 16)
    full = C.dequant_host(q.codes, q.meta, q._shape())
    assert (full[:, 300:] == 0).all()
    dq = q.dequantized_weight()
    assert dq.shape == (40, 300) and (dq[mask == 0] == 0).all()
    wp = torch.nn.functional.pad(lin.weight.data * mask, (0, 84))
    keep = torch.nn.functional.pad(mask != 0, (0, 84))
    oc, ob = O.gf4_quantize_masked(wp.numpy(), keep.numpy())
    assert np.array_equal(O.unpack_nibbles(q.codes.numpy()), oc)
    qe = QuantLinear(lin, mask=mask, fmt="e2m1")
    assert (qe.dequantized_weight()[mask == 0] == 0).all()
    with pytest.raises(ValueError):
        QuantLinear(lin, hadamard=True)


@pytest.mark.parametrize("K", [256, 200])
def test_from_reference_decodes_the_committed_weight(K):
    sd = reference_state(24, K, seed=K)
    Wq, _, _ = O.quantlinear_commit_weight(sd["weight"], sd["Theta"], sd["mask"])
    q = QuantLinear.from_reference(sd)
    assert q.fmt == "gf4" and q.k_pack == 256
    assert torch.equal(q.weight.data, Wq)                       # the reference's commit
    dq = q.dequantized_weight()
    assert torch.equal(dq, Wq.half().float())                   # fp16 of it, value for value
    assert torch.equal(q.bias.data, sd["bias"])
    # Jenks-16 on the committed weight finds the same grid (<= 16 values per group)
    q2 = QuantLinear(q, mask=sd["mask"])
    assert torch.equal(q2.dequantized_weight(), dq)
    # the state_dict round trip keeps the level codebooks
    q3 = QuantLinear(torch.nn.Linear(K, 24), pack=False)
    q3.load_state_dict(q.state_dict())
    assert torch.equal(q3.wdev, q.wdev)


def test_load_state_dict_takes_the_reference_layers_own_state():
    """A reference QuantLinear's state_dict (layers.py:23-31) loads into the drop-in, in
    a model as in a bare layer, and packs exactly as from_reference does; without a mask the
    reference's default (all ones) applies; mismatched shapes are load errors."""
    sd = reference_state(24, 256, seed=3)
    q = QuantLinear(torch.nn.Linear(256, 24), fmt="e2m1", pack=False)
    q.load_state_dict(sd)
    ref = QuantLinear.from_reference(sd)
    assert q.fmt == "gf4" and torch.equal(q.wdev, ref.wdev)
    assert torch.equal(q.weight.data, ref.weight.data) and torch.equal(q.mask, sd["mask"])
    net = torch.nn.Sequential(torch.nn.Flatten(), QuantLinear(torch.nn.Linear(256, 24), pack=False))
    net.load_state_dict({f"1.{k}": v for k, v in sd.items()})
    assert torch.equal(net[1].wdev, ref.wdev)
    nomask = {k: v for k, v in sd.items() if k != "mask"}
    q2 = QuantLinear(torch.nn.Linear(256, 24), pack=False)
    q2.load_state_dict(nomask)
    assert torch.equal(q2.mask, torch.ones(24, 256))
    ones = dict(sd, mask=torch.ones(24, 256))
    assert torch.equal(q2.wdev, QuantLinear.from_reference(ones).wdev)
    with pytest.raises(RuntimeError, match="does not match"):
        QuantLinear(torch.nn.Linear(128, 24), pack=False).load_state_dict(sd)


def test_load_into_fp4_mfma_module_drops_the_fp4_path_for_other_formats():
    """A module built for the native FP4 path (fp4_mfma=True: unrotated E2M1 only) that
    loads another format -- the reference layer's own state (packed as GF4), a packed GF4
    or a rotated E2M1 checkpoint -- runs that format's exact-decode path afterwards instead
    of refusing its next forward; an unrotated E2M1 checkpoint keeps the FP4 path."""
    g = torch.Generator().manual_seed(4)
    lin = torch.nn.Linear(256, 24)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(24, 256, generator=g) * 0.02)

    def fresh():
        q = QuantLinear(lin, fmt="e2m1", fp4_mfma=True)
        assert q.fp4_mfma
        return q

    q = fresh()
    q.load_state_dict(reference_state(24, 256, seed=3))
    assert q.fmt == "gf4" and not q.fp4_mfma
    q = fresh()
    q.load_state_dict(QuantLinear(lin, fmt="gf4").state_dict())
    assert q.fmt == "gf4" and not q.fp4_mfma
    q = fresh()
    q.load_state_dict(QuantLinear(lin, fmt="e2m1", hadamard=True).state_dict())
    assert q.fmt == "e2m1" and q.fwht_block == 256 and not q.fp4_mfma
    q = fresh()
    q.load_state_dict(QuantLinear(lin, fmt="e2m1").state_dict())
    assert q.fmt == "e2m1" and q.fwht_block == 0 and q.fp4_mfma


def test_backward_decodes_in_chunks_of_row_tiles():
    """The backward pass decodes the weight a chunk of 16-row tiles at a time: the row
    offsets into the device stream are whole tiles, and the rows from a tile on are the
    stream of the layer without its first rows (the layout is tile-major)."""
    from if_i_could_turn_back_time_amd import linear as LN
    for fmt, bb in ((C.FMT_GF4, 6144), (C.FMT_E2M1, 4352)):
        N, K = 80, 1152
        codes = torch.from_numpy(RNG.integers(0, 256, size=(N, K // 2), dtype=np.uint8))
        meta = (torch.from_numpy(RNG.integers(0, 2**16, size=(N, K // 128, 16),
                                              dtype=np.uint16).view(np.int16))
                if fmt == C.FMT_GF4 else
                torch.from_numpy(RNG.integers(0, 255, size=(N, K // 32), dtype=np.uint8)))
        full = C.to_device_layout(codes, meta, C.make_shape(N, K, 1, fmt))
        for r0 in (16, 48):
            sh = C.make_shape(N - r0, K, 1, fmt)
            assert C.tile_offset(sh, r0) == (r0 // 16) * 3 * bb
            tail = C.to_device_layout(codes[r0:], meta[r0:], sh)
            off = C.tile_offset(sh, r0)
            assert torch.equal(full[off:off + tail.numel()], tail)
    with pytest.raises(ValueError):
        C.tile_offset(C.make_shape(64, 512, 1, C.FMT_GF4), 8)
    assert LN.BACKWARD_CHUNK_BYTES // (8192 * 4) // 16 * 16 == 2048


def test_replace_forward_packs_adaround_levels():
    from types import SimpleNamespace
    from if_i_could_turn_back_time_amd import adaround_levels, pack_quantized_linears
    g = torch.Generator().manual_seed(8)
    lin = torch.nn.Linear(200, 32)
    delta = torch.rand(32, 1, generator=g) * 0.01 + 1e-3
    W = lin.weight.data / delta
    wq = SimpleNamespace(W_floor=torch.floor(W), alpha=torch.randn(32, 200, generator=g) * 4,
                         mask=(lin.weight.data != 0).float(),
                         quantizer=SimpleNamespace(delta=delta, qmin=-8, qmax=7))
    lin.weight_quantizer = wq
    net = torch.nn.Sequential(lin, torch.nn.ReLU())
    pack_quantized_linears(net)
    lv, d = adaround_levels(wq)
    assert torch.equal(lv, O.adaround_hard_levels(wq.W_floor, wq.alpha, wq.mask, -8, 7))
    pw = lin.packed_weight
    dec = pw.dequant_host()[:, :200]
    assert torch.equal(dec, (delta * lv).half().float())
    with pytest.raises(RuntimeError, match="GPU"):
        net(torch.randn(2, 200))


# ----------------------------------------------------------------------------- LeNet300
def test_lenet300_fixture_packs_and_round_trips():
    """The reference's pruned LeNet300 checkpoint: sparsity equals the reference's own log
    (0.97860, sparisty_log_2025-12-09_18-58-19_0.99_SGD_Agg_80.txt); packed with masks
    from the zero weights, every pruned weight decodes to exactly 0 and groups with at most
    15 distinct kept values decode exactly (fp16); the packed state_dict survives
    torch.save / torch.load(weights_only=True)."""
    import io
    net = lenet300_from_fixture()
    ws = [net[i].weight.data for i in (1, 3, 5)]
    zeros = sum(int((w == 0).sum()) for w in ws)
    assert round(zeros / sum(w.numel() for w in ws), 5) == 0.97860
    q = quantize_module(net, fmt="gf4")
    for i, w in zip((1, 3, 5), ws):
        dq = q[i].dequantized_weight()
        assert (dq[w == 0] == 0).all()
        assert int((dq != 0).sum()) <= int((w != 0).sum())
        kp = q[i].k_pack
        wp = torch.nn.functional.pad(w, (0, kp - w.shape[1])).reshape(w.shape[0], -1, 128)
        few = torch.tensor([len(torch.unique(grp[grp != 0])) <= 15 for grp in wp.reshape(-1, 128)])
        exact = (dq.half().float() == w.half().float())
        exact = torch.nn.functional.pad(exact, (0, kp - w.shape[1]), value=True)
        assert exact.reshape(-1, 128)[few].all()
        oc, ob = O.gf4_quantize_masked(torch.nn.functional.pad(w, (0, kp - w.shape[1])).numpy(),
                                       torch.nn.functional.pad(w != 0, (0, kp - w.shape[1])).numpy())
        assert np.array_equal(O.unpack_nibbles(q[i].codes.numpy()), oc)
        assert np.array_equal(q[i].meta.numpy().view(np.uint16), ob)
    buf = io.BytesIO()
    torch.save(q.state_dict(), buf)
    buf.seek(0)
    sd = torch.load(buf, weights_only=True)
    fresh = quantize_module(lenet300_from_fixture(), fmt="e2m1", pack=False)
    fresh.load_state_dict(sd)
    for i in (1, 3, 5):
        assert fresh[i].fmt == "gf4"
        assert torch.equal(fresh[i].wdev, q[i].wdev)
        assert torch.equal(fresh[i].dequantized_weight(), q[i].dequantized_weight())


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not on PATH")
def test_c_abi_from_c(tmp_path):
    """The host-side C ABI called from C, as a native binding would: tests/c/abi_host.c is
    compiled with gcc against include/fourbit.h (-Wall -Wextra -Werror), linked to the
    built libfourbit.so, and checks known answers of validation, both packers, integer
    levels, the FWHT and the device-layout round trip."""
    C.lib()  # the library is built
    root = Path(__file__).resolve().parents[1]
    exe = tmp_path / "abi_host"
    libdir = C.LIB_PATH.parent
    subprocess.run(["gcc", "-std=c99", "-O1", "-Wall", "-Wextra", "-Werror",
                    f"-I{root / 'include'}", str(root / "tests" / "c" / "abi_host.c"),
                    "-o", str(exe), f"-L{libdir}", "-l:libfourbit.so",
                    f"-Wl,-rpath,{libdir}", "-lm"], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip() == "ok"


def _sanitizers_available(tmp_path) -> bool:
    src = tmp_path / "probe.c"
    src.write_text("int main(void) { return 0; }\n")
    r = subprocess.run(["gcc", "-fsanitize=address,undefined", str(src), "-o",
                        str(tmp_path / "probe")], capture_output=True)
    return r.returncode == 0


@pytest.mark.skipif(shutil.which("gcc") is None or shutil.which("g++") is None,
                    reason="gcc/g++ not on PATH")
def test_host_packers_under_address_and_ub_sanitizers(tmp_path):
    """The host side (csrc/fourbit_host.cpp alone: packers, integer levels, FWHT, layout
    transform, decode, two-class split) built with -fsanitize=address,undefined and driven
    by tests/c/sanitize_host.c over edge shapes and inputs; any memory error, leak or
    undefined operation fails the run."""
    if not _sanitizers_available(tmp_path):
        pytest.skip("this toolchain has no AddressSanitizer / UBSan runtime")
    root = Path(__file__).resolve().parents[1]
    inc = [f"-I{root / 'include'}", f"-I{root / 'if_i_could_turn_back_time_amd' / 'csrc'}"]
    san = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-fno-omit-frame-pointer", "-g", "-O1"]
    drv, host, exe = tmp_path / "drv.o", tmp_path / "host.o", tmp_path / "sanitize_host"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Wextra", "-Werror", *san, *inc, "-c",
                    str(root / "tests" / "c" / "sanitize_host.c"), "-o", str(drv)], check=True)
    subprocess.run(["g++", "-std=c++17", "-ffp-contract=off", *san, *inc, "-c",
                    str(root / "if_i_could_turn_back_time_amd" / "csrc" / "fourbit_host.cpp"),
                    "-o", str(host)], check=True)
    subprocess.run(["g++", "-fsanitize=address,undefined", str(drv), str(host), "-o", str(exe),
                    "-lpthread", "-lm"], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300,
                       env={"ASAN_OPTIONS": "detect_leaks=1", "PATH": "/usr/bin:/bin"})
    assert r.returncode == 0, r.stderr[-4000:]
    assert r.stdout.strip() == "ok"


def test_bench_refuses_several_gpus():
    """bench.py runs on one GPU: --gpus N > 1 exits non-zero with a message, before any
    GPU work (this runs without a GPU)."""
    root = Path(__file__).resolve().parents[1]
    r = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)


# ----------------------------------------------------------------------------- contract edges
def test_workgroup_offsets_fit_32_bits():
    """The GEMV addresses a workgroup's blocks with 32-bit offsets from its first block.
    fb_validate caps a layer at 2^31 - 1 groups of 128 (96 bytes each in GF4, at most
    192 GiB), so with one workgroup per CU a workgroup spans at most 192 GiB / CUs plus one
    row tile (<= 192 MiB): less than 2^31 bytes on any device with 128 CUs or more (MI355X
    has 256), whatever the layer's total size.  fb_gemv returns FB_ERR_SHAPE otherwise."""
    groups = 2 ** 31 - 1
    for K in (1 << 24, 1 << 20, 1 << 14, 128 * 3):
        N = min(groups // (K // 128), 1 << 26)
        sh = C.make_shape(N, K, 1)
        assert C.lib().fb_validate(ctypes.byref(sh)) == 0
        if N < (1 << 26):
            sh_over = C.make_shape(N + 1, K, 1)
            assert C.lib().fb_validate(ctypes.byref(sh_over)) == -2
        for cus in (128, 256, 304):
            T = (N + 15) // 16
            GS = (K // 128 + 3) // 4
            grid = min(T, cus)
            assert -(-T // grid) * GS * 6144 < 2 ** 31, (K, cus)
    # a stream past 2 GiB is a valid shape (the GPU test runs one)
    big = C.make_shape(49152, 65536, 1)
    assert C.device_bytes(big) > 2 ** 31


def test_e2m1_fp16_exact_scale_range():
    """E2M1 decodes to fp16 exactly when 0.5 * 2^(s-127) >= 2^-24 and 6 * 2^(s-127) <= 65504,
    i.e. E8M0 bytes 104..140; PackedWeight records it from the packed scales."""
    from if_i_could_turn_back_time_amd.linear import E2M1_F16_SCALES, e2m1_scales_fit_f16
    lo, hi = E2M1_F16_SCALES
    assert 0.5 * 2.0 ** (lo - 127) == 2.0 ** -24 and 0.5 * 2.0 ** (lo - 1 - 127) < 2.0 ** -24
    assert 6 * 2.0 ** (hi - 127) <= 65504 < 6 * 2.0 ** (hi + 1 - 127)
    for s, ok in ((0, False), (103, False), (104, True), (127, True), (140, True),
                  (141, False), (255, False)):
        meta = torch.full((2, 4), 127, dtype=torch.uint8)
        meta[1, 2] = s
        assert e2m1_scales_fit_f16(meta) == ok, s
    w = torch.randn(16, 256) * 0.02
    assert PackedWeight.quantize(w, "e2m1").f16_exact
    w[3, :32] *= 2.0 ** 23                                  # amax ~ 2^18: byte >= 141
    assert not PackedWeight.quantize(w, "e2m1").f16_exact


@pytest.mark.parametrize("block", [2, 16, 256, 4096])
def test_backward_fwht_matches_oracle(block):
    """The device-side FWHT of the packed linear's backward (torch ops, any device) is
    the oracle's normalised Sylvester transform."""
    from if_i_could_turn_back_time_amd.linear import _fwht_last_dim
    K = max(2 * block, 512)
    t = torch.from_numpy(RNG.standard_normal((3, K)).astype(np.float32))
    got = _fwht_last_dim(t, block)
    ref = torch.from_numpy(O.fwht_rows(t.double().numpy(), block)).float()
    assert torch.allclose(got, ref, atol=1e-5, rtol=1e-5)


# ----------------------------------------------------------------------------- two-class Jenks
def _jenks2_inputs():
    from model_fixtures import lenet300_from_fixture
    net = lenet300_from_fixture()
    yield "lenet300.1.weight", net[1].weight.detach().numpy()      # 300 x 784, ~98% zeros
    yield "lenet300.3.weight", net[3].weight.detach().numpy()
    yield "lenet300.5.bias", net[5].bias.detach().numpy()
    for n in (1, 2, 3, 255, 256, 257, 4096, 65535, 65536, 65537, 131073):
        w = (RNG.standard_normal(n) * 0.02).astype(np.float32)
        if n > 8:
            w[RNG.integers(0, n, n // 4)] = 0.0
            w[RNG.integers(0, n, n // 8)] = -0.0
        yield f"random{n}", w
    yield "constant", np.full(1000, 0.5, np.float32)


def test_jenks2_host_bit_exact_vs_oracle():
    """fb_jenks2_host gives the oracle's split, GVF bits and mask (its arithmetic and
    association order are the oracle's), on the reference's pruned LeNet300 weights and
    on random arrays across the 256-element block and 65536-element superblock edges."""
    for name, w in _jenks2_inputs():
        keep_o, split_o, gvf_o, _ = O.jenks2(w)
        keep_h, split_h, gvf_h = C.jenks2_host(torch.from_numpy(np.ascontiguousarray(w)))
        assert split_h == split_o, name
        assert np.float64(gvf_h).view(np.int64) == np.float64(gvf_o).view(np.int64), name
        assert np.array_equal(keep_h.numpy(), keep_o.reshape(-1)), name


def test_jenks2_host_errors_and_mask_api():
    L = C.lib()
    k = ctypes.c_char_p(b"x" * 8)
    sp, gv = ctypes.c_int64(0), ctypes.c_double(0)
    w = torch.tensor([1.0, float("nan")])
    assert L.fb_jenks2_host(w.data_ptr(), 2, k, ctypes.byref(sp), ctypes.byref(gv)) == -10
    assert L.fb_jenks2_host(w.data_ptr(), 0, k, ctypes.byref(sp), ctypes.byref(gv)) == -2
    assert L.fb_jenks2_host(None, 2, k, ctypes.byref(sp), ctypes.byref(gv)) == -1
    from if_i_could_turn_back_time_amd import bias_mask, linear_mask
    W = torch.randn(30, 20) * 0.02
    m, gvf = linear_mask(W)                         # cuda_helpers.py:378-395 return types
    assert m.shape == W.shape and m.dtype == torch.float32 and m.device.type == "cpu"
    assert isinstance(gvf, float) and 0.0 <= gvf <= 1.0
    keep, split, _, _ = O.jenks2(W.numpy())
    assert torch.equal(m.reshape(-1).bool(), torch.from_numpy(keep))
    mb, _ = bias_mask(torch.randn(10))
    assert mb.shape == (10,)
    with pytest.raises(ValueError):
        bias_mask(W)


def _jenks2_filter_inputs():
    """Convolution weights as [filters, values per filter]: LeNet-5 / VGG / AlexNet filter
    sizes, the per-filter maximum (1024, four 256-blocks), ties, signed zeros and constant
    filters."""
    for shape in ((6, 1, 5, 5), (16, 8, 3, 3), (8, 3, 11, 11), (2, 2, 16, 16), (2, 1, 32, 32),
                  (5, 3, 1, 1), (3, 3, 1, 2), (2, 2, 17, 17)):
        w = (RNG.standard_normal(shape) * 0.05).astype(np.float32)
        yield f"random{shape}", w.reshape(shape[0] * shape[1], -1)
    w = (np.round(RNG.standard_normal((40, 9)) * 2) / 4).astype(np.float32)   # ties
    w[::3] = 0.0
    w[1::5, ::2] = -0.0
    w[2] = 0.7                                                            # constant filter
    yield "ties", w


def test_jenks2_filters_host_bit_exact_vs_oracle():
    """fb_jenks2_filters_host gives, for every filter, the oracle's split, GVF bits and
    mask (the whole-array rule on each filter alone)."""
    for name, w in _jenks2_filter_inputs():
        keep_o, split_o, gvf_o = O.jenks2_filters(w)
        keep_h, split_h, gvf_h = C.jenks2_filters_host(torch.from_numpy(w), nthreads=3)
        assert np.array_equal(split_h.numpy(), split_o), name
        assert np.array_equal(gvf_h.numpy().view(np.int64), gvf_o.view(np.int64)), name
        assert np.array_equal(keep_h.numpy(), keep_o), name


def test_jenks2_filters_host_errors_and_conv_mask_api():
    L = C.lib()
    buf = torch.zeros(64, dtype=torch.float64)
    p = buf.data_ptr()
    w = torch.tensor([[1.0, float("nan")]])
    assert L.fb_jenks2_filters_host(w.data_ptr(), 1, 2, p, p, p, 1) == -10
    w = torch.zeros(2, 4)
    assert L.fb_jenks2_filters_host(w.data_ptr(), 0, 4, p, p, p, 1) == -2
    assert L.fb_jenks2_filters_host(w.data_ptr(), 2, 0, p, p, p, 1) == -2
    assert L.fb_jenks2_filters_host(w.data_ptr(), 1, C.JENKS2_FILTER_MAX + 1, p, p, p, 1) == -2
    assert L.fb_jenks2_filters_host(w.data_ptr(), 2, 4, p, p, p, 0) == -12
    assert L.fb_jenks2_filters_host(None, 2, 4, p, p, p, 1) == -1
    assert L.fb_jenks2_filters_gpu(None, 2, 4, p, p, p, None) == -1     # no device call
    assert L.fb_jenks2_filters_gpu(w.data_ptr(), 2, 2000, p, p, p, None) == -2
    from if_i_could_turn_back_time_amd import jenks
    W = torch.randn(8, 4, 3, 3) * 0.05
    m, gvf = jenks.conv_mask(W)                     # cuda_helpers.py:333-376 return types
    assert m.shape == W.shape and m.dtype == torch.float32
    assert len(gvf) == 8 and len(gvf[0]) == 4 and isinstance(gvf[0][0], float)
    keep, split, g = O.jenks2_filters(W.reshape(32, 9).numpy())
    assert torch.equal(m.reshape(32, 9).bool(), torch.from_numpy(keep))
    with pytest.raises(ValueError):
        jenks.conv_mask(torch.randn(4, 9))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_jenks2_ssd_host_bit_exact_vs_oracle(dtype):
    """fb_jenks2_ssd_host (the reference's per-split SSD interface, jenks_optimization_cuda /
    jenks_optimization_biases_cuda) gives the oracle's jenks2_ssd, rounded to the input's
    dtype, bit for bit: across the 256-value block and 65,536-value superblock edges, with
    ties and signed zeros, and on unsorted input (taken in the order given)."""
    rng = np.random.default_rng(21)
    npdt = np.float32 if dtype == torch.float32 else np.float64
    for n in (1, 2, 255, 256, 257, 4097, 65536, 65537, 200003):
        w = (rng.standard_t(3, size=n) * 0.05).astype(npdt)
        if n > 8:
            w[rng.integers(0, n, n // 5)] = 0.0
            w[rng.integers(0, n, n // 9)] = -0.0
        v = np.sort(w, kind="stable")
        got = C.jenks2_ssd(torch.from_numpy(v))
        assert got.dtype == dtype and got.shape == (n,)
        ref = O.jenks2_ssd(v).astype(npdt)
        assert np.array_equal(got.numpy().view(np.uint8), ref.view(np.uint8)), n
        # the fp64 SSDs' first argmin is the mask path's split on the same (float32) values
        # (the rounded vector's argmin may fall on a split that rounding made equal)
        if dtype == torch.float32:
            assert int(np.argmin(O.jenks2_ssd(v))) == C.jenks2_host(torch.from_numpy(v))[1]
    u = np.array([3.0, -2.0, 0.5, 0.5, 9.0], npdt)
    assert np.array_equal(C.jenks2_ssd(torch.from_numpy(u)).numpy(), O.jenks2_ssd(u).astype(npdt))


def test_jenks2_ssd_filters_host_and_errors():
    """fb_jenks2_ssd_filters_host: every filter's row is the oracle's jenks2_ssd of that
    filter, bit for bit (fp32 and fp64), at the per-filter size edges; argument errors are
    codes, and the reference-shaped drop-ins refuse CPU tensors as CHECK_INPUT does."""
    rng = np.random.default_rng(22)
    for npdt, tdt in ((np.float32, torch.float32), (np.float64, torch.float64)):
        for n in (1, 9, 25, 256, 257, C.JENKS2_FILTER_MAX):
            w = np.sort((rng.standard_normal((7, n)) * 0.05).astype(npdt), axis=1, kind="stable")
            got = C.jenks2_ssd_filters(torch.from_numpy(w), nthreads=3)
            assert got.dtype == tdt and got.shape == (7, n)
            ref = np.stack([O.jenks2_ssd(r) for r in w]).astype(npdt)
            assert np.array_equal(got.numpy().view(np.uint8), ref.view(np.uint8)), n
    L = C.lib()
    arena = np.zeros(1 << 12, np.uint8)
    p = arena.ctypes.data + (-arena.ctypes.data) % 256  # aligned host address: never read
    assert L.fb_jenks2_ssd_host(p, 0, C.DT_F32, p) == -2
    assert L.fb_jenks2_ssd_host(p, 4, C.DT_F16, p) == -5
    assert L.fb_jenks2_ssd_host(None, 4, C.DT_F32, p) == -1
    assert L.fb_jenks2_ssd_filters_host(p, 2, C.JENKS2_FILTER_MAX + 1, C.DT_F32, p, 1) == -2
    assert L.fb_jenks2_ssd_filters_host(p, 2, 4, C.DT_BF16, p, 1) == -5
    assert L.fb_jenks2_ssd_filters_host(p, 2, 4, C.DT_F64, p, 0) == -12
    assert L.fb_jenks2_ssd_gpu(p, 4, C.DT_F32, p, None, 0, None) == -1   # no device call
    assert L.fb_jenks2_ssd_gpu(p + 8, 4, C.DT_F32, p, p, 1 << 20, None) == -7
    assert L.fb_jenks2_ssd_filters_gpu(p, 2, 2000, C.DT_F32, p, None) == -2
    need = ctypes.c_size_t(0)
    assert L.fb_jenks2_ssd_workspace(1 << 20, ctypes.byref(need)) == 0 and need.value > 0
    assert L.fb_jenks2_ssd_gpu(p, 1 << 20, C.DT_F32, p, p, need.value - 1, None) == -8
    from if_i_could_turn_back_time_amd import module_bias, module_conv, module_weights
    with pytest.raises(RuntimeError, match="CUDA"):
        module_weights.jenks_optimization_cuda(torch.zeros(4, 4))
    with pytest.raises(RuntimeError, match="CUDA"):
        module_bias.jenks_optimization_biases_cuda(torch.zeros(4))
    with pytest.raises(RuntimeError, match="CUDA"):
        module_conv.jenks_optimization_cuda_conv(torch.zeros(2, 2, 3, 3))


def test_gemv_noalloc_validation_needs_no_gpu():
    """fb_gemv_noalloc checks the shape and its scratch need before any device call: a
    rotated call of more than 524288 activation values (1 MiB of fp16) is FB_ERR_SCRATCH."""
    L = C.lib()
    buf = ctypes.c_char_p(b"x" * 64)
    big = C.make_shape(64, 65536, 16, C.FMT_GF4, 4096)
    assert L.fb_gemv_noalloc(buf, buf, buf, ctypes.byref(big), None) == -15
    assert "scratch" in C.strerror(-15)
    assert L.fb_gemv_noalloc(buf, buf, buf, None, None) == -1
    bad = C.make_shape(64, 100, 1)
    assert L.fb_gemv_noalloc(buf, buf, buf, ctypes.byref(bad), None) == -2


def test_gemv_mx_validation_needs_no_gpu():
    """fb_gemv_mx checks the shape, pointers and workspace before any device call, and the
    workspace is the split (B*K*2 + 8*B*K/128, each rounded up to 256) plus the split-K
    parts' sums of the same plan as fb_gemv's."""
    L = C.lib()
    arena = np.zeros(1 << 16, np.uint8)
    base = arena.ctypes.data
    p = base + (-base) % 256  # 256-byte aligned host addresses: never dereferenced here
    s = C.make_shape(4096, 11008, 16, C.FMT_E2M1, 0, C.DT_BF16, C.DT_F32)
    split = 16 * 11008 * 2 + (16 * 86 * 8 + 255) // 256 * 256
    assert L.fb_mx_split_bytes(ctypes.byref(s)) == split
    assert L.fb_mx_workspace_bytes(ctypes.byref(s)) == split + L.fb_workspace_bytes(ctypes.byref(s))
    assert L.fb_workspace_bytes(ctypes.byref(s)) == 4 * 16 * 4096 * 4  # split-K, P = 4
    call = lambda sh, ws, n: L.fb_gemv_mx(p, p, p, ctypes.byref(sh), ws, n, None)
    assert call(s, p, split - 1) == -8                                   # FB_ERR_WORKSPACE
    assert call(s, None, split) == -1                                    # FB_ERR_NULL
    assert call(s, p + 16, 1 << 30) == -7                                # FB_ERR_ALIGN
    for kw, code in (({"x_dtype": C.DT_F16}, -5), ({"fmt": C.FMT_GF4, "x_dtype": C.DT_F16}, -4),
                     ({"fwht_block": 256}, -6), ({"B": 17}, -9), ({"K": 100}, -2)):
        sh = C.make_shape(**{**dict(N=4096, K=11008, B=16, fmt=C.FMT_E2M1, fwht_block=0,
                                    x_dtype=C.DT_BF16, y_dtype=C.DT_F32), **kw})
        assert call(sh, p, 1 << 30) == code, kw
        assert L.fb_mx_workspace_bytes(ctypes.byref(sh)) == 0
        assert L.fb_mx_split(p, p, ctypes.byref(sh), None) == code
    assert L.fb_mx_split(p, p + 16, ctypes.byref(s), None) == -7


def test_gemv_mx_presplit_validation_needs_no_gpu():
    """fb_gemv_mx_presplit: the shape checks of fb_gemv_mx, a 256-byte aligned split, and an
    optional workspace (the split-K parts' sums only)."""
    L = C.lib()
    arena = np.zeros(1 << 16, np.uint8)
    base = arena.ctypes.data
    p = base + (-base) % 256
    s = C.make_shape(4096, 11008, 16, C.FMT_E2M1, 0, C.DT_BF16, C.DT_F32)
    assert L.fb_mx_presplit_workspace_bytes(ctypes.byref(s)) == L.fb_workspace_bytes(ctypes.byref(s))
    s8 = C.make_shape(4096, 8192, 8, C.FMT_E2M1, 0, C.DT_BF16, C.DT_F32)
    assert L.fb_mx_presplit_workspace_bytes(ctypes.byref(s8)) == 0
    call = lambda sh, xs: L.fb_gemv_mx_presplit(p, xs, p, ctypes.byref(sh), None, 0, None)
    assert call(s, None) == -1
    assert call(s, p + 16) == -7
    sh = C.make_shape(4096, 11008, 16, C.FMT_E2M1, 0, C.DT_F16, C.DT_F32)
    assert call(sh, p) == -5
    sh = C.make_shape(4096, 11008, 16, C.FMT_E2M1, 256, C.DT_BF16, C.DT_F32)
    assert call(sh, p) == -6
