"""ctypes binding of libfourbit.so (the C ABI declared in ``include/fourbit.h``).

The reference binds its native code with ``torch.utils.cpp_extension.load_inline`` and
torch::Tensor signatures (``Python_Jenks_Test/Jenks_Tests/cuda_helpers.py:42-62``);
here the boundary is a plain C ABI: tensors cross it as ``data_ptr()`` integers, the
HIP stream as ``torch.cuda.current_stream().cuda_stream``, and every non-zero status
becomes a ``RuntimeError`` carrying ``fb_strerror`` (the reference's ``TORCH_CHECK``
failures surface the same way, ``cuda_helpers.py:72-78``).

There is no fallback: if the library is missing, every call raises.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().with_name("libfourbit.so")

FMT_GF4, FMT_E2M1 = 0, 1
DT_F16, DT_BF16, DT_F32, DT_F64 = 0, 1, 2, 3
FMT_BY_NAME = {"gf4": FMT_GF4, "e2m1": FMT_E2M1}
GROUP_BY_FMT = {FMT_GF4: 128, FMT_E2M1: 32}
# bytes of one device-stream block (16 rows x 512 K-elements): fourbit_layout.h
BLOCK_BYTES = {FMT_GF4: 6144, FMT_E2M1: 4352}
DTYPE_CODE = {torch.float16: DT_F16, torch.bfloat16: DT_BF16, torch.float32: DT_F32}
ABI_VERSION = 1
ERR_VALUE = -10  # FB_ERR_VALUE: non-finite / non-integer / out-of-range packer input

# every symbol include/fourbit.h declares
EXPORTED = (
    "fb_abi_version", "fb_strerror", "fb_validate", "fb_device_bytes", "fb_workspace_bytes",
    "fb_quantize_gf4", "fb_quantize_gf4_masked", "fb_pack_levels_gf4", "fb_quantize_e2m1",
    "fb_fwht_rows_f32", "fb_to_device",
    "fb_from_device", "fb_dequant_host", "fb_gemv", "fb_dequant", "fb_quantize_gf4_gpu",
    "fb_quantize_e2m1_gpu", "fb_jenks2_host", "fb_jenks2_workspace", "fb_jenks2_gpu",
    "fb_jenks2_filters_host", "fb_jenks2_filters_gpu", "fb_gemv_noalloc",
    "fb_mx_split_bytes", "fb_mx_split", "fb_mx_workspace_bytes", "fb_gemv_mx",
    "fb_gemv_mx_presplit", "fb_mx_presplit_workspace_bytes",
    "fb_jenks2_ssd_host", "fb_jenks2_ssd_workspace", "fb_jenks2_ssd_gpu",
    "fb_jenks2_ssd_filters_host", "fb_jenks2_ssd_filters_gpu",
)


class FbShape(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in
                ("N", "K", "B", "group", "fmt", "fwht_block", "x_dtype", "y_dtype")]


_lib = None


def lib() -> ctypes.CDLL:
    """Loads libfourbit.so once (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m if_i_could_turn_back_time_amd.build_lib`"
        )
    L = ctypes.CDLL(str(LIB_PATH))
    vp, i32, sz = ctypes.c_void_p, ctypes.c_int32, ctypes.c_size_t
    sp = ctypes.POINTER(FbShape)
    sigs = {
        "fb_abi_version": (i32, []),
        "fb_strerror": (ctypes.c_char_p, [ctypes.c_int]),
        "fb_validate": (ctypes.c_int, [sp]),
        "fb_device_bytes": (sz, [sp]),
        "fb_workspace_bytes": (sz, [sp]),
        "fb_quantize_gf4": (ctypes.c_int, [vp, i32, i32, vp, vp, i32]),
        "fb_quantize_gf4_masked": (ctypes.c_int, [vp, vp, i32, i32, vp, vp, i32]),
        "fb_pack_levels_gf4": (ctypes.c_int, [vp, vp, i32, i32, vp, vp, i32]),
        "fb_quantize_e2m1": (ctypes.c_int, [vp, i32, i32, vp, vp, i32]),
        "fb_fwht_rows_f32": (ctypes.c_int, [vp, i32, i32, i32, i32]),
        "fb_to_device": (ctypes.c_int, [vp, vp, vp, sp]),
        "fb_from_device": (ctypes.c_int, [vp, vp, vp, sp]),
        "fb_dequant_host": (ctypes.c_int, [vp, vp, vp, sp]),
        "fb_gemv": (ctypes.c_int, [vp, vp, vp, sp, vp, sz, vp]),
        "fb_dequant": (ctypes.c_int, [vp, vp, i32, sp, vp]),
        "fb_quantize_gf4_gpu": (ctypes.c_int, [vp, vp, i32, i32, vp, vp, vp]),
        "fb_quantize_e2m1_gpu": (ctypes.c_int, [vp, i32, i32, vp, vp, vp]),
        "fb_jenks2_host": (ctypes.c_int, [vp, ctypes.c_int64, vp, vp, vp]),
        "fb_jenks2_workspace": (ctypes.c_int, [ctypes.c_int64, ctypes.POINTER(sz)]),
        "fb_jenks2_gpu": (ctypes.c_int, [vp, ctypes.c_int64, vp, vp, vp, vp, sz, vp]),
        "fb_jenks2_filters_host": (ctypes.c_int, [vp, ctypes.c_int64, ctypes.c_int32, vp, vp, vp,
                                                  ctypes.c_int32]),
        "fb_jenks2_filters_gpu": (ctypes.c_int, [vp, ctypes.c_int64, ctypes.c_int32, vp, vp, vp,
                                                 vp]),
        "fb_gemv_noalloc": (ctypes.c_int, [vp, vp, vp, sp, vp]),
        "fb_mx_split_bytes": (sz, [sp]),
        "fb_mx_split": (ctypes.c_int, [vp, vp, sp, vp]),
        "fb_mx_workspace_bytes": (sz, [sp]),
        "fb_gemv_mx": (ctypes.c_int, [vp, vp, vp, sp, vp, sz, vp]),
        "fb_gemv_mx_presplit": (ctypes.c_int, [vp, vp, vp, sp, vp, sz, vp]),
        "fb_mx_presplit_workspace_bytes": (sz, [sp]),
        "fb_jenks2_ssd_host": (ctypes.c_int, [vp, ctypes.c_int64, i32, vp]),
        "fb_jenks2_ssd_workspace": (ctypes.c_int, [ctypes.c_int64, ctypes.POINTER(sz)]),
        "fb_jenks2_ssd_gpu": (ctypes.c_int, [vp, ctypes.c_int64, i32, vp, vp, sz, vp]),
        "fb_jenks2_ssd_filters_host": (ctypes.c_int, [vp, ctypes.c_int64, i32, i32, vp, i32]),
        "fb_jenks2_ssd_filters_gpu": (ctypes.c_int, [vp, ctypes.c_int64, i32, i32, vp, vp]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(L, name)
        fn.restype, fn.argtypes = res, args
    if L.fb_abi_version() != ABI_VERSION:
        raise RuntimeError(f"libfourbit ABI {L.fb_abi_version()} != expected {ABI_VERSION}")
    _lib = L
    return L


def strerror(code: int) -> str:
    return lib().fb_strerror(code).decode()


def check(code: int) -> None:
    if code != 0:
        raise RuntimeError(strerror(code))


def nthreads_default() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def make_shape(N, K, B=1, fmt=FMT_GF4, fwht_block=0, x_dtype=DT_F16, y_dtype=DT_F16) -> FbShape:
    return FbShape(N, K, B, GROUP_BY_FMT[fmt], fmt, fwht_block, x_dtype, y_dtype)


def _ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


def _host_contig(t: torch.Tensor, dtype) -> torch.Tensor:
    if t.device.type != "cpu":
        raise ValueError("host packers take CPU tensors")
    return t.detach().to(dtype).contiguous()


# ------------------------------------------------------------------ host packers
def quantize_gf4(w: torch.Tensor, nthreads: int | None = None, keep: torch.Tensor | None = None):
    """fp32 [N,K] -> (codes uint8 [N,K/2], codebook uint16-as-int16 [N,K/128,16]).

    ``keep`` (bool/uint8 [N,K], optional): entries where it is 0 decode to exactly 0
    (fb_quantize_gf4_masked)."""
    w = _host_contig(w, torch.float32)
    N, K = w.shape
    codes = torch.empty(N, K // 2, dtype=torch.uint8)
    book = torch.empty(N, max(K // 128, 1), 16, dtype=torch.int16)
    nt = nthreads or nthreads_default()
    if keep is None:
        check(lib().fb_quantize_gf4(_ptr(w), N, K, _ptr(codes), _ptr(book), nt))
    else:
        keep = _host_contig(keep != 0, torch.uint8)
        if keep.shape != w.shape:
            raise ValueError("keep mask must have the weight's shape")
        check(lib().fb_quantize_gf4_masked(_ptr(w), _ptr(keep), N, K, _ptr(codes),
                                           _ptr(book), nt))
    return codes, book


def pack_levels_gf4(levels: torch.Tensor, scale: torch.Tensor, nthreads: int | None = None):
    """Integer levels fp32 [N,K] and per-row scale [N] -> GF4 (codes, codebook) with
    codebook entries fp16(scale * level) (fb_pack_levels_gf4)."""
    levels = _host_contig(levels, torch.float32)
    N, K = levels.shape
    scale = _host_contig(scale.reshape(-1), torch.float32)
    if scale.numel() != N:
        raise ValueError("scale needs one entry per row")
    codes = torch.empty(N, K // 2, dtype=torch.uint8)
    book = torch.empty(N, max(K // 128, 1), 16, dtype=torch.int16)
    check(lib().fb_pack_levels_gf4(_ptr(levels), _ptr(scale), N, K, _ptr(codes), _ptr(book),
                                   nthreads or nthreads_default()))
    return codes, book


def quantize_e2m1(w: torch.Tensor, nthreads: int | None = None):
    """fp32 [N,K] -> (codes uint8 [N,K/2], scales uint8 [N,K/32])."""
    w = _host_contig(w, torch.float32)
    N, K = w.shape
    codes = torch.empty(N, K // 2, dtype=torch.uint8)
    scales = torch.empty(N, max(K // 32, 1), dtype=torch.uint8)
    check(lib().fb_quantize_e2m1(_ptr(w), N, K, _ptr(codes), _ptr(scales),
                                 nthreads or nthreads_default()))
    return codes, scales


def fwht_rows(w: torch.Tensor, block: int, nthreads: int | None = None) -> torch.Tensor:
    """Returns w with every K-block rotated: w H_b / sqrt(b) (fp64 math, fp32 result)."""
    out = _host_contig(w, torch.float32).clone()
    N, K = out.shape
    check(lib().fb_fwht_rows_f32(_ptr(out), N, K, block, nthreads or nthreads_default()))
    return out


def device_bytes(shape: FbShape) -> int:
    n = lib().fb_device_bytes(ctypes.byref(shape))
    if n == 0:
        check(lib().fb_validate(ctypes.byref(shape)))
    return n


def to_device_layout(codes: torch.Tensor, meta: torch.Tensor, shape: FbShape) -> torch.Tensor:
    """Canonical host buffers -> device weight stream (uint8 CPU tensor)."""
    codes = _host_contig(codes, torch.uint8)
    meta = meta.detach().contiguous()
    out = torch.empty(device_bytes(shape), dtype=torch.uint8)
    check(lib().fb_to_device(_ptr(codes), _ptr(meta), _ptr(out), ctypes.byref(shape)))
    return out


def from_device_layout(wdev: torch.Tensor, shape: FbShape):
    wdev = _host_contig(wdev, torch.uint8)
    codes = torch.empty(shape.N, shape.K // 2, dtype=torch.uint8)
    if shape.fmt == FMT_GF4:
        meta = torch.empty(shape.N, shape.K // 128, 16, dtype=torch.int16)
    else:
        meta = torch.empty(shape.N, shape.K // 32, dtype=torch.uint8)
    check(lib().fb_from_device(_ptr(wdev), _ptr(codes), _ptr(meta), ctypes.byref(shape)))
    return codes, meta


def dequant_host(codes: torch.Tensor, meta: torch.Tensor, shape: FbShape) -> torch.Tensor:
    codes = _host_contig(codes, torch.uint8)
    meta = meta.detach().contiguous()
    out = torch.empty(shape.N, shape.K, dtype=torch.float32)
    check(lib().fb_dequant_host(_ptr(codes), _ptr(meta), _ptr(out), ctypes.byref(shape)))
    return out


# ------------------------------------------------------------------ GPU entry points
def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def workspace_bytes(shape: FbShape) -> int:
    return lib().fb_workspace_bytes(ctypes.byref(shape))


def new_workspace(shape: FbShape, device) -> torch.Tensor | None:
    """Device workspace for fb_gemv, or None when the shape needs none.  Its contents need
    no initialisation (fb_gemv writes before it reads), so it is left uninitialised."""
    need = workspace_bytes(shape)
    return torch.empty(need, dtype=torch.uint8, device=device) if need else None


def gemv(wdev: torch.Tensor, x: torch.Tensor, y: torch.Tensor, shape: FbShape,
         workspace: torch.Tensor | None = None) -> torch.Tensor:
    """y[B,N] = x'[B,K] . W^T on the GPU (asynchronous on the current stream)."""
    if not (wdev.is_cuda and x.is_cuda and y.is_cuda):
        raise RuntimeError("fb_gemv needs device tensors (ROCm GPU)")
    if not (wdev.device == x.device == y.device):
        raise ValueError(f"fb_gemv operands are on different devices: weight {wdev.device}, "
                         f"x {x.device}, y {y.device}")
    if not (x.is_contiguous() and y.is_contiguous()):
        raise ValueError("x and y must be contiguous")
    if x.dtype not in DTYPE_CODE or y.dtype not in DTYPE_CODE:
        raise ValueError("x and y must be float16, bfloat16 or float32 tensors")
    if DTYPE_CODE[x.dtype] != shape.x_dtype or DTYPE_CODE[y.dtype] != shape.y_dtype:
        raise ValueError("x / y dtypes do not match the shape's x_dtype / y_dtype")
    if tuple(x.shape) != (shape.B, shape.K) or tuple(y.shape) != (shape.B, shape.N):
        raise ValueError(f"x {tuple(x.shape)} / y {tuple(y.shape)} do not match the shape "
                         f"(B={shape.B}, K={shape.K}, N={shape.N})")
    if wdev.numel() < device_bytes(shape):
        raise ValueError("weight stream is smaller than fb_device_bytes(shape)")
    need = workspace_bytes(shape)
    if need and (workspace is None or workspace.numel() < need):
        workspace = new_workspace(shape, x.device)
    wp = _ptr(workspace) if need else None
    with torch.cuda.device(x.device):  # HIP launches on the current device
        check(lib().fb_gemv(_ptr(wdev), _ptr(x), _ptr(y), ctypes.byref(shape), wp, need,
                            _stream(x.device)))
    return y


def _check_gemv_operands(name, wdev, x, y, shape):
    if not (wdev.is_cuda and x.is_cuda and y.is_cuda):
        raise RuntimeError(f"{name} needs device tensors (ROCm GPU)")
    if not (wdev.device == x.device == y.device):
        raise ValueError(f"{name} operands are on different devices: weight {wdev.device}, "
                         f"x {x.device}, y {y.device}")
    if not (x.is_contiguous() and y.is_contiguous()):
        raise ValueError("x and y must be contiguous")
    if x.dtype not in DTYPE_CODE or y.dtype not in DTYPE_CODE:
        raise ValueError("x and y must be float16, bfloat16 or float32 tensors")
    if DTYPE_CODE[x.dtype] != shape.x_dtype or DTYPE_CODE[y.dtype] != shape.y_dtype:
        raise ValueError("x / y dtypes do not match the shape's x_dtype / y_dtype")
    if tuple(x.shape) != (shape.B, shape.K) or tuple(y.shape) != (shape.B, shape.N):
        raise ValueError(f"x {tuple(x.shape)} / y {tuple(y.shape)} do not match the shape "
                         f"(B={shape.B}, K={shape.K}, N={shape.N})")
    if wdev.numel() < device_bytes(shape):
        raise ValueError("weight stream is smaller than fb_device_bytes(shape)")


def _mx_refuse(shape: FbShape) -> None:
    check(lib().fb_validate(ctypes.byref(shape)))
    raise ValueError("the native FP4 path takes E2M1 weights, bfloat16 x, no rotation and "
                     "batch <= 16")


def mx_workspace_bytes(shape: FbShape) -> int:
    """Workspace of fb_gemv_mx (0: the shape is not one the native FP4 path takes)."""
    return lib().fb_mx_workspace_bytes(ctypes.byref(shape))


def gemv_mx(wdev: torch.Tensor, x: torch.Tensor, y: torch.Tensor, shape: FbShape,
            workspace: torch.Tensor | None = None) -> torch.Tensor:
    """E2M1 y[B,N] = x[B,K] . W^T on the matrix cores' native FP4 path: x (bf16) split
    into two MX-E4M3 terms, then v_mfma_scale_f32_16x16x128_f8f6f4 on the stored codes
    (asynchronous on the current stream)."""
    _check_gemv_operands("fb_gemv_mx", wdev, x, y, shape)
    need = mx_workspace_bytes(shape)
    if not need:
        _mx_refuse(shape)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    elif workspace.device != x.device:
        raise ValueError("workspace is on another device")
    with torch.cuda.device(x.device):
        check(lib().fb_gemv_mx(_ptr(wdev), _ptr(x), _ptr(y), ctypes.byref(shape),
                               _ptr(workspace), workspace.numel(), _stream(x.device)))
    return y


def mx_split_raw(x: torch.Tensor, shape: FbShape) -> torch.Tensor:
    """fb_mx_split of x (bf16 [B, K] on the GPU): the split in its device layout (uint8),
    the input of gemv_mx_presplit."""
    if not x.is_cuda or x.dtype != torch.bfloat16 or not x.is_contiguous():
        raise ValueError("x must be a contiguous bfloat16 device tensor")
    if tuple(x.shape) != (shape.B, shape.K):
        raise ValueError("x does not match the shape")
    nbytes = lib().fb_mx_split_bytes(ctypes.byref(shape))
    if not nbytes:
        _mx_refuse(shape)
    out = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
    with torch.cuda.device(x.device):
        check(lib().fb_mx_split(_ptr(x), _ptr(out), ctypes.byref(shape), _stream(x.device)))
    return out


def gemv_mx_presplit(wdev: torch.Tensor, xs: torch.Tensor, y: torch.Tensor, shape: FbShape,
                     workspace: torch.Tensor | None = None) -> torch.Tensor:
    """gemv_mx on a split made by mx_split_raw (one split for several layers with the same
    input)."""
    if not (wdev.is_cuda and xs.is_cuda and y.is_cuda):
        raise RuntimeError("fb_gemv_mx_presplit needs device tensors (ROCm GPU)")
    if not (wdev.device == xs.device == y.device):
        raise ValueError("fb_gemv_mx_presplit operands are on different devices")
    if xs.numel() < lib().fb_mx_split_bytes(ctypes.byref(shape)):
        raise ValueError("xs is smaller than fb_mx_split_bytes(shape)")
    if tuple(y.shape) != (shape.B, shape.N) or DTYPE_CODE.get(y.dtype) != shape.y_dtype:
        raise ValueError("y does not match the shape")
    if wdev.numel() < device_bytes(shape):
        raise ValueError("weight stream is smaller than fb_device_bytes(shape)")
    need = lib().fb_mx_presplit_workspace_bytes(ctypes.byref(shape))
    if need and (workspace is None or workspace.numel() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=y.device)
    wp = _ptr(workspace) if need else None
    with torch.cuda.device(y.device):
        check(lib().fb_gemv_mx_presplit(_ptr(wdev), _ptr(xs), _ptr(y), ctypes.byref(shape), wp,
                                        need, _stream(y.device)))
    return y


def mx_split(x: torch.Tensor, shape: FbShape):
    """The split fb_gemv_mx makes of x (bf16 [B, K] on the GPU): (codes uint8 [2, B, K],
    scales uint8 [2, B, K/32]) -- term t of value (b, k) and of its 32-value block."""
    out = mx_split_raw(x, shape)
    B, K = shape.B, shape.K
    soff = (B * K * 2 + 255) // 256 * 256
    terms = out[:B * K * 2].view(B, K // 128, 2, 128).permute(2, 0, 1, 3).reshape(2, B, K)
    sc = out[soff:soff + B * (K // 128) * 8].view(B, K // 128, 2, 4).permute(2, 0, 1, 3)
    return terms.contiguous(), sc.reshape(2, B, K // 32).contiguous()


def tile_offset(shape: FbShape, row: int) -> int:
    """Byte offset of row ``row`` (a multiple of 16) in the device stream: the stream is
    16-row tiles, each ``ceil(K/512)`` blocks, one after the other, so the rows from
    ``row`` on are the stream of the same layer without its first ``row`` rows."""
    if row % 16:
        raise ValueError("row offsets of the device stream are multiples of 16")
    return (row // 16) * ((shape.K // 128 + 3) // 4) * BLOCK_BYTES[shape.fmt]


def dequant_device(wdev: torch.Tensor, shape: FbShape, out_dtype=torch.float32,
                   out: torch.Tensor | None = None) -> torch.Tensor:
    """Exact device decode of the stream ``wdev`` (fb_dequant) to ``[N, K]`` of
    ``out_dtype``, into ``out`` when given (contiguous, on wdev's device)."""
    if not wdev.is_cuda:
        raise RuntimeError("fb_dequant needs a device tensor (ROCm GPU)")
    if wdev.numel() < device_bytes(shape):
        raise ValueError("weight stream is smaller than fb_device_bytes(shape)")
    if out is None:
        out = torch.empty(shape.N, shape.K, dtype=out_dtype, device=wdev.device)
    elif (tuple(out.shape) != (shape.N, shape.K) or out.dtype != out_dtype
          or out.device != wdev.device or not out.is_contiguous()):
        raise ValueError("out does not match the shape, dtype or device")
    with torch.cuda.device(wdev.device):
        check(lib().fb_dequant(_ptr(wdev), _ptr(out), DTYPE_CODE[out_dtype],
                               ctypes.byref(shape), _stream(wdev.device)))
    return out


def quantize_gf4_gpu(w: torch.Tensor, keep: torch.Tensor | None = None):
    """GF4 packing on the GPU (fb_quantize_gf4_gpu): fp32 device ``w [N,K]`` (and an
    optional keep mask) -> device ``(codes uint8 [N,K/2], codebook int16 [N,K/128,16])``,
    bit-identical to :func:`quantize_gf4`.  Raises on non-finite kept weights (checked
    with one torch reduction before the launch)."""
    if not w.is_cuda:
        raise RuntimeError("fb_quantize_gf4_gpu needs a device tensor (ROCm GPU)")
    w = w.detach().to(torch.float32).contiguous()
    N, K = w.shape
    kp = None
    if keep is not None:
        kp = (keep != 0).to(device=w.device, dtype=torch.uint8).contiguous()
        if kp.shape != w.shape:
            raise ValueError("keep mask must have the weight's shape")
        finite = torch.isfinite(w) | (kp == 0)
    else:
        finite = torch.isfinite(w)
    if not bool(finite.all()):
        raise RuntimeError(strerror(ERR_VALUE))
    codes = torch.empty(N, K // 2, dtype=torch.uint8, device=w.device)
    book = torch.empty(N, max(K // 128, 1), 16, dtype=torch.int16, device=w.device)
    with torch.cuda.device(w.device):
        check(lib().fb_quantize_gf4_gpu(_ptr(w), _ptr(kp) if kp is not None else None, N, K,
                                        _ptr(codes), _ptr(book), _stream(w.device)))
    return codes, book


def quantize_e2m1_gpu(w: torch.Tensor):
    """E2M1 packing on the GPU (fb_quantize_e2m1_gpu): fp32 device ``w [N,K]`` -> device
    ``(codes uint8 [N,K/2], scales uint8 [N,K/32])``, bit-identical to
    :func:`quantize_e2m1`.  Raises on non-finite weights."""
    if not w.is_cuda:
        raise RuntimeError("fb_quantize_e2m1_gpu needs a device tensor (ROCm GPU)")
    w = w.detach().to(torch.float32).contiguous()
    N, K = w.shape
    if not bool(torch.isfinite(w).all()):
        raise RuntimeError(strerror(ERR_VALUE))
    codes = torch.empty(N, K // 2, dtype=torch.uint8, device=w.device)
    scales = torch.empty(N, max(K // 32, 1), dtype=torch.uint8, device=w.device)
    with torch.cuda.device(w.device):
        check(lib().fb_quantize_e2m1_gpu(_ptr(w), N, K, _ptr(codes), _ptr(scales),
                                         _stream(w.device)))
    return codes, scales


# ------------------------------------------------------------------ two-class Jenks
def jenks2_host(w: torch.Tensor):
    """fb_jenks2_host over the flattened fp32 values: (keep bool [n], split, gvf)."""
    w = _host_contig(w.reshape(-1), torch.float32)
    n = w.numel()
    keep = torch.empty(n, dtype=torch.uint8)
    split = ctypes.c_int64(0)
    gvf = ctypes.c_double(0.0)
    check(lib().fb_jenks2_host(_ptr(w), n, _ptr(keep), ctypes.byref(split), ctypes.byref(gvf)))
    return keep.bool(), split.value, gvf.value


def jenks2_gpu(w: torch.Tensor):
    """fb_jenks2_gpu over the flattened fp32 values of a device tensor: (keep bool [n] on
    the device, split, gvf).  Raises on non-finite values (one torch reduction first)."""
    if not w.is_cuda:
        raise RuntimeError("fb_jenks2_gpu needs a device tensor (ROCm GPU)")
    w = w.detach().reshape(-1).to(torch.float32).contiguous()
    n = w.numel()
    if not bool(torch.isfinite(w).all()):
        raise RuntimeError(strerror(ERR_VALUE))
    with torch.cuda.device(w.device):
        need = ctypes.c_size_t(0)
        check(lib().fb_jenks2_workspace(n, ctypes.byref(need)))
        ws = torch.empty(need.value + 256, dtype=torch.uint8, device=w.device)
        off = (-ws.data_ptr()) % 256
        keep = torch.empty(n, dtype=torch.uint8, device=w.device)
        out = torch.empty(2, dtype=torch.float64, device=w.device)   # [split (int64 bits), gvf]
        split_p = out.data_ptr()
        check(lib().fb_jenks2_gpu(_ptr(w), n, _ptr(keep), split_p, split_p + 8,
                                  ws.data_ptr() + off, need.value, _stream(w.device)))
        host = out.cpu()
    split = int(host[:1].view(torch.int64).item())
    return keep.bool(), split, float(host[1].item())


JENKS2_FILTER_MAX = 1024  # FB_JENKS2_FILTER_MAX


def jenks2_filters_host(w: torch.Tensor, nthreads: int | None = None):
    """fb_jenks2_filters_host over w [nf, n] (fp32, each row one filter): (keep bool [nf, n],
    split int32 [nf], gvf float64 [nf])."""
    w = _host_contig(w, torch.float32)
    if w.dim() != 2:
        raise ValueError("w must be [filters, values per filter]")
    nf, n = w.shape
    keep = torch.empty(nf, n, dtype=torch.uint8)
    split = torch.empty(nf, dtype=torch.int32)
    gvf = torch.empty(nf, dtype=torch.float64)
    check(lib().fb_jenks2_filters_host(_ptr(w), nf, n, _ptr(keep), _ptr(split), _ptr(gvf),
                                       nthreads or nthreads_default()))
    return keep.bool(), split, gvf


def jenks2_filters_gpu(w: torch.Tensor):
    """fb_jenks2_filters_gpu over a device tensor w [nf, n]: (keep bool [nf, n], split int32
    [nf], gvf float64 [nf]), on the device.  Raises on non-finite values (one torch
    reduction first)."""
    if not w.is_cuda:
        raise RuntimeError("fb_jenks2_filters_gpu needs a device tensor (ROCm GPU)")
    w = w.detach().to(torch.float32).contiguous()
    if w.dim() != 2:
        raise ValueError("w must be [filters, values per filter]")
    if not bool(torch.isfinite(w).all()):
        raise RuntimeError(strerror(ERR_VALUE))
    nf, n = w.shape
    with torch.cuda.device(w.device):
        keep = torch.empty(nf, n, dtype=torch.uint8, device=w.device)
        split = torch.empty(nf, dtype=torch.int32, device=w.device)
        gvf = torch.empty(nf, dtype=torch.float64, device=w.device)
        check(lib().fb_jenks2_filters_gpu(_ptr(w), nf, n, _ptr(keep), _ptr(split), _ptr(gvf),
                                          _stream(w.device)))
    return keep.bool(), split, gvf


# ------------------------------------------------------------------ per-split SSD
SSD_DTYPE = {torch.float32: DT_F32, torch.float64: DT_F64}


def _ssd_operand(t: torch.Tensor, align: int) -> torch.Tensor:
    """t as a contiguous tensor of an fp32 / fp64 dtype whose data is ``align``-byte
    aligned (a copy only when it is not)."""
    if t.dtype not in SSD_DTYPE:
        raise RuntimeError(f"the per-split SSD takes float32 or float64 values, got {t.dtype}")
    t = t.detach().contiguous()
    if t.data_ptr() % align:
        t = t.clone()
    return t


def jenks2_ssd(srt: torch.Tensor) -> torch.Tensor:
    """The within-class SSD of every split of the flattened values in the order given
    (fb_jenks2_ssd_gpu on a device tensor, fb_jenks2_ssd_host on a CPU one; the same bits):
    a 1-D tensor of srt's dtype and device."""
    flat = srt.reshape(-1)
    n = flat.numel()
    if n < 1:
        raise RuntimeError("the per-split SSD needs at least one value")
    if not flat.is_cuda:
        flat = _ssd_operand(flat, 8)
        out = torch.empty(n, dtype=flat.dtype)
        check(lib().fb_jenks2_ssd_host(_ptr(flat), n, SSD_DTYPE[flat.dtype], _ptr(out)))
        return out
    flat = _ssd_operand(flat, 16)
    with torch.cuda.device(flat.device):
        need = ctypes.c_size_t(0)
        check(lib().fb_jenks2_ssd_workspace(n, ctypes.byref(need)))
        ws = torch.empty(need.value + 256, dtype=torch.uint8, device=flat.device)
        off = (-ws.data_ptr()) % 256
        out = torch.empty(n, dtype=flat.dtype, device=flat.device)
        check(lib().fb_jenks2_ssd_gpu(_ptr(flat), n, SSD_DTYPE[flat.dtype], _ptr(out),
                                      ws.data_ptr() + off, need.value, _stream(flat.device)))
    return out


def jenks2_ssd_filters(srt: torch.Tensor, nthreads: int | None = None) -> torch.Tensor:
    """Per-split SSD of every row of srt [nf, n] (each row one filter, in the order given;
    n <= JENKS2_FILTER_MAX): [nf, n] of srt's dtype and device (fb_jenks2_ssd_filters_gpu /
    fb_jenks2_ssd_filters_host, the same bits)."""
    if srt.dim() != 2:
        raise ValueError("srt must be [filters, values per filter]")
    nf, n = srt.shape
    if nf < 1 or n < 1:
        raise RuntimeError("the per-split SSD needs at least one filter of one value")
    if n > JENKS2_FILTER_MAX:
        raise RuntimeError(f"filters of more than {JENKS2_FILTER_MAX} values are not supported")
    if not srt.is_cuda:
        srt = _ssd_operand(srt, 8)
        out = torch.empty(nf, n, dtype=srt.dtype)
        check(lib().fb_jenks2_ssd_filters_host(_ptr(srt), nf, n, SSD_DTYPE[srt.dtype], _ptr(out),
                                               nthreads or nthreads_default()))
        return out
    srt = _ssd_operand(srt, 8)
    with torch.cuda.device(srt.device):
        out = torch.empty(nf, n, dtype=srt.dtype, device=srt.device)
        check(lib().fb_jenks2_ssd_filters_gpu(_ptr(srt), nf, n, SSD_DTYPE[srt.dtype], _ptr(out),
                                              _stream(srt.device)))
    return out
