"""Drop-in quantized linear layer backed by the fused 4-bit dequant-GEMV.

Mirrors the reference's ``QuantLinear`` (``Python_Jenks_Test/Jenks_Tests/
Quantization_Experiments/layers.py:11-45``): same constructor
``QuantLinear(linear_module, bitwidth=4, mask=None)``, ``forward(x)``, ``commit()`` and
``hard_quant`` flag, and the ``quantize_module`` swap helper (``utils.py:1498-1524``).
Where the reference keeps four dense fp32 ``[N,K]`` tensors (``s``, ``Q``, ``Theta``,
``mask``) and dequantizes them on every call before ``F.linear`` (``layers.py:36-38``),
this layer keeps the packed 4-bit weight (GF4 codebooks or E2M1 scales) and runs the
HIP kernel, which decodes in registers.

Extra keyword arguments: ``fmt`` ('gf4' | 'e2m1'), ``hadamard`` (False, True for the
default block, or an explicit power-of-two block: the weight is rotated offline and x
in-kernel), ``nthreads`` for the host packer and ``packer`` ('host' | 'gpu': where the
GF4 Jenks search runs; both give the same bytes).

``in_features`` need not be a multiple of the 128-wide group: the packed weight gets
zero columns up to the next multiple (masked, so they decode to exactly 0 and do not
move the last group's codebook) and ``forward`` pads x with zeros to match.
``QuantLinear.from_reference`` packs the reference layer's own committed 4-bit weight
(``layers.py:39-45``) exactly, through integer-level GF4 codebooks.
"""
from __future__ import annotations

import copy

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _capi as C

LAYOUT_VERSION = 1
MAX_GEMV_BATCH = 16
GROUP = 128


def packed_k(K: int) -> int:
    """K of the packed weight: in_features rounded up to a multiple of 128."""
    return (K + GROUP - 1) // GROUP * GROUP


def fwht_block_for(K: int) -> int:
    """Default rotation block: 4096 when it divides K, else the largest power of two
    dividing K (256 for K = 11008 = 43 * 256), capped at 4096."""
    if K % 4096 == 0:
        return 4096
    b = K & -K
    return min(b, 4096)


FP16_MAX = 65504.0
# E8M0 scale bytes whose E2M1 products are all exact fp16 values: 0.5 * 2^(s-127) >= 2^-24
# (the smallest fp16 subnormal) and 6 * 2^(s-127) <= 65504.
E2M1_F16_SCALES = (104, 140)


def e2m1_scales_fit_f16(meta: torch.Tensor) -> bool:
    """Whether every E8M0 byte of an E2M1 weight lies in ``E2M1_F16_SCALES``, i.e. the
    kernel's fp16 decode (fp16 activations) gives the exact weight values."""
    if meta.numel() == 0:
        return True
    lo, hi = int(meta.min()), int(meta.max())
    return E2M1_F16_SCALES[0] <= lo and hi <= E2M1_F16_SCALES[1]


def _fwht_last_dim(t: torch.Tensor, block: int) -> torch.Tensor:
    """Normalised blockwise Walsh-Hadamard transform along the last dim (fp32, on t's
    device): every ``block``-wide slice becomes ``H_b v / sqrt(b)``, Sylvester order."""
    lead = t.shape[:-1]
    K = t.shape[-1]
    v = t.reshape(-1, K // block, block).float()
    h = 1
    while h < block:
        v = v.reshape(v.shape[0], v.shape[1], block // (2 * h), 2, h)
        a, c = v[:, :, :, 0, :], v[:, :, :, 1, :]
        v = torch.stack((a + c, a - c), dim=3)
        h *= 2
    return (v.reshape(*lead, K) / float(block) ** 0.5)


def _workspace(cache: dict | None, nbytes: int, device: torch.device):
    """An uninitialised device workspace of at least ``nbytes`` (None for 0), kept in
    ``cache`` per (device, stream) and grown when a call needs more: fb_gemv and
    fb_gemv_mx need no initialised contents, and calls on one stream run in order, so one
    buffer serves every call of a module on that stream (including graph replays)."""
    if not nbytes:
        return None
    key = (device.index, torch.cuda.current_stream(device).cuda_stream)
    ws = cache.get(key) if cache is not None else None
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
        if cache is not None:
            cache[key] = ws
    return ws


def _gemv_chunks(wdev, N, kp, fmt, fwht_block, xk, y, fp4_mfma=False, ws_cache=None):
    f = C.FMT_BY_NAME[fmt]
    for b0 in range(0, xk.shape[0], MAX_GEMV_BATCH):
        b1 = min(b0 + MAX_GEMV_BATCH, xk.shape[0])
        shape = C.make_shape(N, kp, b1 - b0, f, fwht_block, C.DTYPE_CODE[xk.dtype],
                             C.DTYPE_CODE[y.dtype])
        if fp4_mfma:
            ws = _workspace(ws_cache, C.mx_workspace_bytes(shape), xk.device)
            C.gemv_mx(wdev, xk[b0:b1], y[b0:b1], shape, ws)
        else:
            ws = _workspace(ws_cache, C.workspace_bytes(shape), xk.device)
            C.gemv(wdev, xk[b0:b1], y[b0:b1], shape, ws)


# Most bytes of fp32 weight the backward pass decodes at once (a chunk of 16-row tiles).
BACKWARD_CHUNK_BYTES = 64 * 2**20


def _grad_x(wdev, N, kp, fmt, fwht_block, gy: torch.Tensor) -> torch.Tensor:
    """``grad_y [M, N] @ W [N, kp]`` in fp32 with W decoded on the device (fb_dequant,
    exact) a chunk of row tiles at a time: at most ``BACKWARD_CHUNK_BYTES`` of decoded
    weight exist at once, whatever the layer's size.  Chunks are added in row order."""
    f = C.FMT_BY_NAME[fmt]
    rows = max(16, BACKWARD_CHUNK_BYTES // (kp * 4) // 16 * 16)
    gyf = gy.float()
    gx = torch.zeros(gy.shape[0], kp, dtype=torch.float32, device=gy.device)
    buf = None
    for r0 in range(0, N, rows):
        r1 = min(N, r0 + rows)
        shape = C.make_shape(r1 - r0, kp, 1, f, fwht_block)
        if buf is None or buf.shape[0] != r1 - r0:
            buf = torch.empty(r1 - r0, kp, dtype=torch.float32, device=gy.device)
        W = C.dequant_device(wdev[C.tile_offset(shape, r0):], shape, torch.float32, out=buf)
        gx.addmm_(gyf[:, r0:r1], W)
    return gx


def _kernel_input(x2: torch.Tensor, K: int, fmt: str, fwht_block: int, range_check: bool,
                  f16_exact: bool, fp4_mfma: bool = False) -> torch.Tensor:
    """x [M, K] -> the kernel's activation: fp16 for GF4 and every rotation (E2M1 keeps
    fp16 / bf16, fp32 becomes bf16; on the native FP4 path every dtype becomes bf16),
    zero-padded to ``packed_k(K)``.  ``range_check`` raises where the fp16 staging would
    overflow: values beyond +-65504 in a wider x, and for a rotation any block of L2 norm
    >= 65504 (a rotated value is at most its block's norm).  It costs one reduction and a
    host sync per call, so it is off by default and skipped while a graph is captured;
    without it such an overflow shows as non-finite outputs (the staged value is inf)."""
    if fmt == "gf4" or fwht_block:
        xk = x2.to(torch.float16)
        if range_check and xk.numel() and not torch.cuda.is_current_stream_capturing():
            if x2.dtype != torch.float16 and bool((torch.isfinite(x2) & ~torch.isfinite(xk)).any()):
                raise ValueError("packed linear: activations beyond the fp16 range (+-65504); "
                                 "the GF4 and rotated kernels take fp16 x")
            if fwht_block:
                nb = K // fwht_block
                norm = xk.float().reshape(-1, nb, fwht_block).norm(dim=-1).max()
                if bool(norm >= FP16_MAX):
                    raise ValueError("packed linear: a rotation block of x has L2 norm >= 65504, "
                                     "so its rotated values may overflow fp16")
    elif fp4_mfma:
        xk = x2.to(torch.bfloat16)
    else:
        xk = x2 if x2.dtype in (torch.float16, torch.bfloat16) else x2.to(torch.bfloat16)
    if fmt == "e2m1" and xk.dtype == torch.float16 and not f16_exact:
        raise ValueError(f"packed linear: E2M1 scale bytes outside {E2M1_F16_SCALES} do not "
                         "decode exactly to fp16; pass bfloat16 activations (without a "
                         "rotation) for this weight")
    kp = packed_k(K)
    if kp != K:
        xk = F.pad(xk, (0, kp - K))
    return xk.contiguous()


class _PackedLinearFn(torch.autograd.Function):
    """``x -> x W^T`` through the fused kernel, differentiable in x (as ``F.linear`` with
    the reference's frozen committed weight is, ``layers.py:34-35``).  Backward:
    ``grad_x = grad_y W``, with W decoded on the device (fb_dequant, fp32) in chunks of row
    tiles (``_grad_x``) and, for a rotated weight W' = W H, rotated back:
    ``grad_x = (grad_y W') H``."""

    @staticmethod
    def forward(ctx, x2, wdev, N, K, fmt, fwht_block, range_check, f16_exact, fp4_mfma=False,
                ws_cache=None):
        xk = _kernel_input(x2, K, fmt, fwht_block, range_check, f16_exact, fp4_mfma)
        ydt = x2.dtype if x2.dtype in C.DTYPE_CODE else torch.float32
        y = torch.empty(x2.shape[0], N, dtype=ydt, device=x2.device)
        _gemv_chunks(wdev, N, packed_k(K), fmt, fwht_block, xk, y, fp4_mfma, ws_cache)
        ctx.save_for_backward(wdev)
        ctx.cfg = (N, K, fmt, fwht_block, x2.dtype)
        return y

    @staticmethod
    def backward(ctx, gy):
        (wdev,) = ctx.saved_tensors
        N, K, fmt, fwht_block, xdt = ctx.cfg
        gx = _grad_x(wdev, N, packed_k(K), fmt, fwht_block, gy)
        if fwht_block:
            gx = _fwht_last_dim(gx, fwht_block)
        return gx[:, :K].to(xdt), None, None, None, None, None, None, None, None, None


def packed_linear(wdev: torch.Tensor, N: int, K: int, fmt: str, fwht_block: int,
                  x: torch.Tensor, bias: torch.Tensor | None = None, *,
                  range_check: bool = False, f16_exact: bool = True,
                  fp4_mfma: bool = False, ws_cache: dict | None = None) -> torch.Tensor:
    """``F.linear(x, W, bias)`` for a packed 4-bit ``W [N, K]`` (device stream ``wdev``
    of a ``packed_k(K)``-wide weight), through fb_gemv in chunks of 16 rows of x.

    x may have any leading shape and dtype: it is cast to fp16 (GF4, or any rotation) or
    kept in fp16/bf16 (E2M1; fp32 becomes bf16) and zero-padded to ``packed_k(K)``; y
    has x's dtype (fp32 for other dtypes).  Differentiable in x (and bias): the weight is
    frozen, as the reference's committed weight is.  ``range_check`` (see
    ``_kernel_input``) raises instead of letting fp16 staging overflow, at the cost of a
    host sync; ``ws_cache`` keeps the call's fb_gemv workspace for the next calls (a dict
    the caller owns, e.g. one per module); ``f16_exact``
    (E2M1 only) says whether the weight's scales decode exactly to fp16.  ``fp4_mfma``
    (unrotated E2M1 only) runs the matrix cores' native FP4 path (fb_gemv_mx): x as bf16,
    split into two MX-E4M3 terms, which hold a bf16 value exactly unless its 32-value block
    spans more than E4M3's exponent range (fp16 and fp32 x are rounded to bf16 first).  No
    CPU path: x must be on the GPU."""
    if x.dim() == 0 or x.shape[-1] != K:
        raise RuntimeError(f"packed linear: input of shape {tuple(x.shape)} does not end in "
                           f"in_features={K}")
    if not x.is_cuda:
        raise RuntimeError("the packed 4-bit linear runs the HIP kernel: move the module and "
                           "input to a ROCm GPU")
    if fp4_mfma and (fmt != "e2m1" or fwht_block):
        raise ValueError("the native FP4 path (fp4_mfma) takes unrotated E2M1 weights")
    lead = x.shape[:-1]
    x2 = x.reshape(-1, K)
    if torch.is_grad_enabled() and x.requires_grad:
        y = _PackedLinearFn.apply(x2, wdev, N, K, fmt, fwht_block, range_check, f16_exact,
                                  fp4_mfma, ws_cache)
        if bias is not None:
            y = y + bias.to(y.dtype)
        return y.reshape(*lead, N)
    with torch.no_grad():
        y = _PackedLinearFn.forward(_NoCtx(), x2, wdev, N, K, fmt, fwht_block, range_check,
                                    f16_exact, fp4_mfma, ws_cache)
    if bias is not None:
        if torch.is_grad_enabled() and bias.requires_grad:
            y = y + bias.to(y.dtype)
        else:
            y.add_(bias.to(y.dtype))  # y is this call's own buffer
    return y.reshape(*lead, N)


class _NoCtx:
    """Stand-in for the autograd context when no graph is built."""

    def save_for_backward(self, *a):
        pass


class PackedWeight:
    """Packed 4-bit weight: canonical host buffers + the device stream, and a GEMV."""

    def __init__(self, fmt: str, N: int, K: int, codes: torch.Tensor, meta: torch.Tensor,
                 fwht_block: int = 0, device=None):
        self.fmt = C.FMT_BY_NAME[fmt]
        self.fmt_name = fmt
        self.N, self.K, self.fwht_block = N, K, fwht_block
        self.codes, self.meta = codes, meta
        self.f16_exact = self.fmt != C.FMT_E2M1 or e2m1_scales_fit_f16(meta)
        self._ws = {}
        shape = C.make_shape(N, K, 1, self.fmt, fwht_block)
        self.wdev = C.to_device_layout(codes, meta, shape)
        if device is not None:
            self.wdev = self.wdev.to(device)

    @classmethod
    def quantize(cls, w: torch.Tensor, fmt: str = "gf4", fwht_block: int = 0, device=None,
                 nthreads: int | None = None, keep: torch.Tensor | None = None,
                 packer: str = "host") -> "PackedWeight":
        """Packs fp32 ``w [N,K]``.  ``keep`` (GF4 only, no rotation): entries where it is
        0 decode to exactly 0.  ``packer='gpu'`` packs on the GPU (``device``, or cuda:0)
        with the same bytes as the host packer."""
        w = w.detach().float().cpu().contiguous()
        N, K = w.shape
        if keep is not None and (fmt != "gf4" or fwht_block):
            raise ValueError("keep masks apply to unrotated GF4 packing only")
        if packer not in ("host", "gpu"):
            raise ValueError(f"packer must be 'host' or 'gpu', got {packer!r}")
        if fwht_block:
            w = C.fwht_rows(w, fwht_block, nthreads)
        if fmt == "gf4" and packer == "gpu":
            dev = device if device is not None and torch.device(device).type == "cuda" else "cuda:0"
            codes, meta = C.quantize_gf4_gpu(w.to(dev), None if keep is None else keep.to(dev))
            codes, meta = codes.cpu(), meta.cpu()
        elif fmt == "gf4":
            codes, meta = C.quantize_gf4(w, nthreads, keep)
        elif fmt == "e2m1" and packer == "gpu":
            dev = device if device is not None and torch.device(device).type == "cuda" else "cuda:0"
            codes, meta = C.quantize_e2m1_gpu(w.to(dev))
            codes, meta = codes.cpu(), meta.cpu()
        elif fmt == "e2m1":
            codes, meta = C.quantize_e2m1(w, nthreads)
        else:
            raise ValueError(f"unknown fmt {fmt!r}")
        return cls(fmt, N, K, codes, meta, fwht_block, device)

    @classmethod
    def from_levels(cls, levels: torch.Tensor, scale: torch.Tensor, device=None,
                    nthreads: int | None = None) -> "PackedWeight":
        """Integer levels ``[N,K]`` times a per-row ``scale [N]`` as GF4 codebooks
        (fb_pack_levels_gf4): decodes to ``fp16(fp32(scale * level))``."""
        levels = levels.detach().float().cpu()
        N, K = levels.shape
        codes, meta = C.pack_levels_gf4(levels, scale, nthreads)
        return cls("gf4", N, K, codes, meta, 0, device)

    def shape(self, B: int, x_dtype: torch.dtype, y_dtype: torch.dtype) -> C.FbShape:
        return C.make_shape(self.N, self.K, B, self.fmt, self.fwht_block,
                            C.DTYPE_CODE[x_dtype], C.DTYPE_CODE[y_dtype])

    def workspace(self, shape: C.FbShape, device):
        """Cached fb_gemv workspace (uninitialised: none is needed) for this device and
        size (None when the shape needs none)."""
        need = C.workspace_bytes(shape)
        if not need:
            return None
        key = (str(device), need)
        ws = self._ws.get(key)
        if ws is None:
            ws = self._ws[key] = C.new_workspace(shape, device)
        return ws

    def gemv(self, x: torch.Tensor, out: torch.Tensor | None = None,
             out_dtype: torch.dtype | None = None) -> torch.Tensor:
        """x [B,K] (B <= 16) on the GPU -> y [B,N]."""
        B = x.shape[0]
        if x.dtype == torch.float16 and not self.f16_exact:
            raise ValueError(f"E2M1 scale bytes outside {E2M1_F16_SCALES} do not decode "
                             "exactly to fp16: use bfloat16 activations for this weight")
        ydt = out.dtype if out is not None else (out_dtype or x.dtype)
        if out is None:
            out = torch.empty(B, self.N, dtype=ydt, device=x.device)
        shape = self.shape(B, x.dtype, ydt)
        return C.gemv(self.wdev, x, out, shape, self.workspace(shape, x.device))

    def gemv_mx(self, x: torch.Tensor, out: torch.Tensor | None = None,
                out_dtype: torch.dtype | None = None) -> torch.Tensor:
        """x [B,K] (bf16, B <= 16) on the GPU -> y [B,N] on the native FP4 path
        (fb_gemv_mx; unrotated E2M1 only)."""
        B = x.shape[0]
        ydt = out.dtype if out is not None else (out_dtype or x.dtype)
        if out is None:
            out = torch.empty(B, self.N, dtype=ydt, device=x.device)
        shape = self.shape(B, x.dtype, ydt)
        need = C.mx_workspace_bytes(shape)
        key = ("mx", str(x.device), need)
        ws = self._ws.get(key)
        if ws is None and need:
            ws = self._ws[key] = torch.empty(need, dtype=torch.uint8, device=x.device)
        return C.gemv_mx(self.wdev, x, out, shape, ws)

    def dequant_device(self, out_dtype=torch.float32) -> torch.Tensor:
        return C.dequant_device(self.wdev, C.make_shape(self.N, self.K, 1, self.fmt), out_dtype)

    def dequant_host(self) -> torch.Tensor:
        return C.dequant_host(self.codes, self.meta, C.make_shape(self.N, self.K, 1, self.fmt))

    def dequant_host_row(self, r: int):
        """Exact fp32 decode of row r (numpy [K])."""
        sh = C.make_shape(1, self.K, 1, self.fmt)
        return C.dequant_host(self.codes[r:r + 1], self.meta[r:r + 1], sh)[0].numpy()

    def algorithmic_bytes(self, B: int, xbytes: int = 2, ybytes: int = 2) -> int:
        meta = self.N * (self.K // 128) * 32 if self.fmt == C.FMT_GF4 else self.N * (self.K // 32)
        return self.N * self.K // 2 + meta + B * self.K * xbytes + B * self.N * ybytes


class QuantLinear(nn.Linear):
    """4-bit quantized ``nn.Linear`` (reference: ``layers.py:11-45``)."""

    def __init__(self, linear_module: nn.Linear, bitwidth: int = 4, mask=None, *,
                 fmt: str = "gf4", hadamard=False, nthreads: int | None = None,
                 pack: bool = True, packer: str = "host", fp4_mfma: bool = False):
        super().__init__(linear_module.in_features, linear_module.out_features,
                         bias=(linear_module.bias is not None))
        if bitwidth != 4:
            raise ValueError("QuantLinear packs 4-bit weights only (bitwidth=4)")
        if fmt not in C.FMT_BY_NAME:
            raise ValueError(f"fmt must be 'gf4' or 'e2m1', got {fmt!r}")
        K = linear_module.in_features
        self.k_pack = packed_k(K)
        if hadamard and K % GROUP:
            raise ValueError("hadamard rotation needs in_features to be a multiple of 128")
        self.weight.requires_grad = False
        self.weight.data = linear_module.weight.data.clone()
        if linear_module.bias is not None:
            self.bias.data = linear_module.bias.data.clone()
        self.fmt = fmt
        self.fwht_block = (fwht_block_for(K) if hadamard is True else int(hadamard or 0))
        self.nthreads = nthreads
        self.packer = packer
        self.register_buffer("mask", None if mask is None else torch.as_tensor(mask).float())
        self.register_buffer("codes", torch.empty(0, dtype=torch.uint8))
        self.register_buffer("meta", torch.empty(0, dtype=torch.uint8))
        self.register_buffer("fb_header", torch.tensor(
            [LAYOUT_VERSION, C.FMT_BY_NAME[fmt], C.GROUP_BY_FMT[C.FMT_BY_NAME[fmt]],
             self.fwht_block], dtype=torch.int32))
        self.register_buffer("wdev", torch.empty(0, dtype=torch.uint8), persistent=False)
        self.hard_quant = False
        # unrotated E2M1 only: the matrix cores' native FP4 path (x as two MX-E4M3 terms)
        if fp4_mfma and (fmt != "e2m1" or self.fwht_block):
            raise ValueError("fp4_mfma needs fmt='e2m1' without a rotation")
        self.fp4_mfma = fp4_mfma
        # True: raise instead of letting fp16 activation staging overflow, at one host sync
        # per call for bf16 / fp32 inputs and for rotated layers (not while a graph is
        # captured).  Off by default, so the forward never syncs and can be captured in a
        # HIP graph; an overflow then shows as non-finite outputs.
        self.range_check = False
        # fb_gemv / fb_gemv_mx workspaces of this module, per (device, stream)
        self._ws_cache = {}
        self._f16_exact = True
        self.register_load_state_dict_post_hook(QuantLinear._rebuild_after_load)
        if pack:
            self.quantize()

    @classmethod
    def from_reference(cls, ref, *, nthreads: int | None = None) -> "QuantLinear":
        """Packs a reference ``QuantLinear`` (``layers.py:11-45``; the module or its
        ``state_dict`` with ``weight, s, Q, Theta, mask`` and optional ``bias``) in its
        own 4-bit format: the committed weight ``mask * s * round(Q + [h(Theta) > 0.5])``
        (``layers.py:39-45``) as integer levels with the per-row scale ``s``
        (fb_pack_levels_gf4).  The packed weight decodes to ``fp16`` of the reference's
        committed fp32 weight, element for element; ``weight`` holds that fp32 weight.
        Raises if ``mask`` is not 0/1 or a 128-group spans more than 16 levels."""
        sd = ref.state_dict() if isinstance(ref, nn.Module) else ref
        s = sd["s"].detach().float().cpu()
        Q = sd["Q"].detach().float().cpu()
        mask = sd["mask"].detach().float().cpu()
        if not bool(((mask == 0) | (mask == 1)).all()):
            raise ValueError("from_reference needs a 0/1 mask")
        N, K = Q.shape
        # layers.py:41-43
        theta = (torch.sigmoid(sd["Theta"].detach().float().cpu()) * 1.2 - .1 > 0.5).float()
        q_round = torch.round(Q + theta)
        bias = sd.get("bias")
        lin = nn.Linear(K, N, bias=bias is not None)
        with torch.no_grad():
            lin.weight.copy_(mask * s * q_round)
            if bias is not None:
                lin.bias.copy_(bias.detach().float().cpu())
        q = cls(lin, 4, mask=mask, fmt="gf4", nthreads=nthreads, pack=False)
        levels = F.pad(q_round * mask, (0, q.k_pack - K))
        q._set_packed(PackedWeight.from_levels(levels, s.reshape(-1), nthreads=nthreads))
        return q

    # -- packing ------------------------------------------------------------------
    def quantize(self) -> None:
        """(Re)packs ``weight`` (times ``mask``) into 4-bit codes + codebooks/scales.
        Unrotated GF4 keeps masked (and padding) entries at exactly 0."""
        w = self.weight.data.detach().float().cpu()
        N, K = w.shape
        keep = None
        if self.mask is not None:
            w = w * self.mask.float().cpu()
            keep = self.mask.cpu() != 0
        pad = self.k_pack - K
        if pad:
            w = F.pad(w, (0, pad))
            keep = F.pad(torch.ones(N, K, dtype=torch.bool) if keep is None else keep, (0, pad))
        if self.fmt != "gf4" or self.fwht_block:
            keep = None  # E2M1 codes zeros exactly; a rotation mixes masked and kept
        self._set_packed(PackedWeight.quantize(w, self.fmt, self.fwht_block,
                                               device=self.weight.device,
                                               nthreads=self.nthreads, keep=keep,
                                               packer=self.packer))

    pack = quantize

    def _set_packed(self, pw: PackedWeight) -> None:
        dev = self.weight.device
        self.codes = pw.codes.to(dev)
        self.meta = pw.meta.to(dev)
        self.wdev = pw.wdev.to(dev)
        self._f16_exact = self.fmt != "e2m1" or e2m1_scales_fit_f16(pw.meta)

    def _shape(self, B=1, x_dtype=torch.float16, y_dtype=torch.float16) -> C.FbShape:
        return C.make_shape(self.out_features, self.k_pack, B, C.FMT_BY_NAME[self.fmt],
                            self.fwht_block, C.DTYPE_CODE[x_dtype], C.DTYPE_CODE[y_dtype])

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys,
                              unexpected_keys, error_msgs):
        # A reference QuantLinear's own state (layers.py:23-31: weight, s, Q, Theta, mask,
        # bias) loads too: it is packed as from_reference packs it (its committed 4-bit
        # weight as GF4 integer levels), whatever format this module was built with.
        ref_keys = ("s", "Q", "Theta")
        if (all(prefix + k in state_dict for k in ref_keys)
                and prefix + "codes" not in state_dict):
            sd = {k: state_dict[prefix + k] for k in ref_keys + ("mask", "bias")
                  if prefix + k in state_dict}
            if "mask" not in sd:  # the reference's default mask is all ones
                sd["mask"] = torch.ones_like(sd["Q"])
            if ("bias" in sd) != (self.bias is not None):
                error_msgs.append(f"{prefix}bias: the module and the checkpoint disagree on "
                                  "having a bias")
                return
            if tuple(sd["Q"].shape) != (self.out_features, self.in_features):
                error_msgs.append(f"{prefix}Q: shape {tuple(sd['Q'].shape)} does not match "
                                  f"({self.out_features}, {self.in_features})")
                return
            q = QuantLinear.from_reference(sd, nthreads=self.nthreads)
            dev = self.weight.device
            with torch.no_grad():
                self.weight.data = q.weight.data.to(dev)
                if self.bias is not None:
                    self.bias.data = q.bias.data.to(dev)
            self.mask = q.mask.to(dev)
            self.fb_header = q.fb_header.clone()
            self.codes = q.codes.to(dev)
            self.meta = q.meta.to(dev)
            self.hard_quant = False
            self.fp4_mfma = False  # the reference's weight loads as GF4
            return
        # packed buffers take the checkpoint's shape/dtype (format may differ from ctor),
        # and the mask is present exactly when the checkpoint has one
        for name in ("codes", "meta", "fb_header"):
            key = prefix + name
            if key in state_dict:
                cur = getattr(self, name)
                setattr(self, name, torch.empty_like(state_dict[key], device=cur.device))
        key = prefix + "mask"
        self.mask = (torch.empty_like(state_dict[key], device=self.weight.device)
                     if key in state_dict else None)
        super()._load_from_state_dict(state_dict, prefix, local_metadata, strict, missing_keys,
                                      unexpected_keys, error_msgs)

    def _rebuild_after_load(self, incompatible_keys) -> None:
        if self.codes.numel() == 0:  # nothing packed was loaded (the load reports why)
            return
        hdr = self.fb_header.tolist()
        if hdr[0] != LAYOUT_VERSION:
            raise RuntimeError(f"packed layout version {hdr[0]} != {LAYOUT_VERSION}")
        inv = {v: k for k, v in C.FMT_BY_NAME.items()}
        self.fmt = inv[hdr[1]]
        self.fwht_block = hdr[3]
        if self.fp4_mfma and (self.fmt != "e2m1" or self.fwht_block):
            self.fp4_mfma = False  # the native FP4 path takes unrotated E2M1 weights only
        shape = self._shape()
        self.wdev = C.to_device_layout(self.codes.cpu(), self.meta.cpu(), shape).to(
            self.codes.device)
        self._f16_exact = self.fmt != "e2m1" or e2m1_scales_fit_f16(self.meta.cpu())

    # -- reference API ------------------------------------------------------------
    def dequantized_weight(self) -> torch.Tensor:
        """Exact fp32 decode of the packed weight (in the rotated basis when
        ``fwht_block`` is set)."""
        w = C.dequant_host(self.codes.cpu(), self.meta.cpu(), self._shape())
        return w[:, :self.in_features].contiguous()

    def commit(self) -> None:
        """Reference ``commit()`` (``layers.py:39-45``) stores the hard-rounded weight
        in ``weight`` and sets ``hard_quant``; here the packed weight is already hard,
        so ``weight`` receives its exact decode (rotated back when ``fwht_block``)."""
        with torch.no_grad():
            w = self.dequantized_weight()
            if self.fwht_block:
                w = C.fwht_rows(w, self.fwht_block)  # H is its own inverse
            self.weight.data.copy_(w.to(self.weight.device))
            self.hard_quant = True

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return packed_linear(self.wdev, self.out_features, self.in_features, self.fmt,
                             self.fwht_block, x, self.bias, range_check=self.range_check,
                             f16_exact=self._f16_exact,
                             fp4_mfma=self.fp4_mfma, ws_cache=self._ws_cache)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"fmt={self.fmt}, fwht_block={self.fwht_block}, bias={self.bias is not None}")


def fp4_mfma_shared(layers, x: torch.Tensor):
    """Runs several E2M1 ``QuantLinear`` layers that take the same input x (the q/k/v or
    gate/up projections of one activation) on the native FP4 path with one split of x per
    16 rows (fb_mx_split, then fb_gemv_mx_presplit per layer): ``(y_0, y_1, ...)``, each
    what ``layer(x)`` gives with ``fp4_mfma=True``.  When autograd needs x's gradient each
    layer runs on its own (the split is not differentiable; every layer's backward is).
    No counterpart in the reference, whose layers each run their own ``F.linear``."""
    layers = list(layers)
    if not layers:
        return ()
    K = layers[0].in_features
    for q in layers:
        if not isinstance(q, QuantLinear) or q.fmt != "e2m1" or q.fwht_block:
            raise ValueError("fp4_mfma_shared takes unrotated E2M1 QuantLinear layers")
        if q.in_features != K:
            raise ValueError("fp4_mfma_shared: the layers differ in in_features")
    if x.dim() == 0 or x.shape[-1] != K:
        raise RuntimeError(f"fp4_mfma_shared: input of shape {tuple(x.shape)} does not end in "
                           f"in_features={K}")
    if not x.is_cuda:
        raise RuntimeError("the packed 4-bit linear runs the HIP kernel: move the modules and "
                           "input to a ROCm GPU")
    if torch.is_grad_enabled() and (x.requires_grad or any(
            q.bias is not None and q.bias.requires_grad for q in layers)):
        return tuple(packed_linear(q.wdev, q.out_features, K, "e2m1", 0, x, q.bias,
                                   range_check=q.range_check, f16_exact=q._f16_exact,
                                   fp4_mfma=True, ws_cache=q._ws_cache) for q in layers)
    lead = x.shape[:-1]
    x2 = x.reshape(-1, K)
    kp = packed_k(K)
    xk = _kernel_input(x2, K, "e2m1", 0, False, True, fp4_mfma=True)
    ydt = x2.dtype if x2.dtype in C.DTYPE_CODE else torch.float32
    ys = [torch.empty(x2.shape[0], q.out_features, dtype=ydt, device=x.device) for q in layers]
    with torch.no_grad():
        for b0 in range(0, xk.shape[0], MAX_GEMV_BATCH):
            b1 = min(b0 + MAX_GEMV_BATCH, xk.shape[0])
            sh0 = C.make_shape(layers[0].out_features, kp, b1 - b0, C.FMT_E2M1, 0, C.DT_BF16,
                               C.DTYPE_CODE[ydt])
            xs = C.mx_split_raw(xk[b0:b1], sh0)
            for q, y in zip(layers, ys):
                sh = C.make_shape(q.out_features, kp, b1 - b0, C.FMT_E2M1, 0, C.DT_BF16,
                                  C.DTYPE_CODE[ydt])
                C.gemv_mx_presplit(q.wdev, xs, y[b0:b1], sh)
        for q, y in zip(layers, ys):
            if q.bias is not None:
                y.add_(q.bias.to(y.dtype))
    return tuple(y.reshape(*lead, q.out_features) for q, y in zip(layers, ys))


def quantize_module(module, bitwidth: int = 4, **kw):
    """Recursively swaps every ``nn.Linear`` for a ``QuantLinear`` (reference:
    ``Quantization_Experiments/utils.py:1498-1524``; masks come from existing zero
    weights so pruning is preserved).  Other layers are left as they are."""
    if isinstance(module, nn.Linear) and not isinstance(module, QuantLinear):
        mask = (module.weight.data != 0).float()
        return QuantLinear(module, bitwidth, mask=mask, **kw)
    if isinstance(module, list):
        return [quantize_module(m, bitwidth, **kw) for m in module]
    module = copy.deepcopy(module)
    for name, child in module.named_children():
        setattr(module, name, quantize_module(child, bitwidth, **kw))
    return module
