"""Two-class natural-breaks pruning masks over whole weight arrays, the reference's
``Linear_Mask`` / ``Bias_Mask`` (``Python_Jenks_Test/Jenks_Tests/cuda_helpers.py:378-411``).

The reference sorts the flattened weights, launches one CUDA thread per split index that
sums both classes serially (``jenks_optimization_cuda``, ``:151-211``; O(n^2) overall),
takes the first argmin of the within-class SSD and keeps the weights at sorted positions
from the split on.  Here the same rule runs natively in O(n) after the sort
(``fb_jenks2_gpu`` on a ROCm tensor, ``fb_jenks2_host`` on a CPU one; the two give the
same bits).  The return values have the reference's types: a float32 CPU mask of the
input's shape (1 = kept) and the goodness of variance fit as a Python float.

``conv_mask`` is the reference's ``Conv_Mask`` (``:333-376``): the same rule on every
(out, in) filter of a convolution weight on its own, over its per-filter kernel
(``jenks_optimization_cuda_conv``, ``:219-289``, one thread per filter trying every split
serially).  Here ``fb_jenks2_filters_gpu`` runs one 64-lane workgroup per filter
(``fb_jenks2_filters_host`` on the CPU), each filter bit for bit what ``jenks2`` gives on it
alone.

``module_weights``, ``module_bias`` and ``module_conv`` stand in for the reference's three
``load_inline`` extensions (``cuda_helpers.py:297-299``), which its optimizers call directly
and then take ``var.argmin()`` (``custom_optimizer.py:135-136``, ``:164-165`` and 20 more
sites; ``Conv_Mask`` at ``cuda_helpers.py:356``): each returns the SSD of every split of an
array the caller has sorted, with the reference's argument meaning, output shape and dtype
and its error behaviour (``CHECK_INPUT``: a GPU tensor, contiguous; ``AT_DISPATCH_FLOATING_
TYPES``: float32 or float64).  The SSDs come from prefix sums in O(n) (``fb_jenks2_ssd_gpu``,
``fb_jenks2_ssd_filters_gpu``) instead of one serial O(n) pass per split.
"""
from __future__ import annotations

from types import SimpleNamespace

import torch

from . import _capi as C


def jenks2(weights: torch.Tensor):
    """(keep bool tensor of ``weights``' shape, on its device; split index; GVF)."""
    if weights.is_cuda:
        keep, split, gvf = C.jenks2_gpu(weights)
    else:
        keep, split, gvf = C.jenks2_host(weights)
    return keep.reshape(weights.shape), split, gvf


def linear_mask(weights_cuda: torch.Tensor):
    """``Linear_Mask`` (``cuda_helpers.py:378-395``): mask over the flattened weights,
    reshaped to their shape, and GVF."""
    keep, _, gvf = jenks2(weights_cuda)
    return keep.to(device="cpu", dtype=torch.float32), gvf


def bias_mask(weights_cuda: torch.Tensor):
    """``Bias_Mask`` (``cuda_helpers.py:397-411``): the same rule on a 1-D tensor."""
    if weights_cuda.dim() != 1:
        raise ValueError("bias_mask takes a 1-D tensor (Linear_Mask flattens any shape)")
    keep, _, gvf = jenks2(weights_cuda)
    return keep.to(device="cpu", dtype=torch.float32), gvf


def jenks2_filters(weights: torch.Tensor):
    """Per-filter split of ``weights`` [out, in, kh, kw] (or any [..., kh, kw]): (keep bool
    tensor of ``weights``' shape, split int32 [out, in], GVF float64 [out, in]), on the
    weights' device."""
    if weights.dim() < 3:
        raise ValueError("conv weights are [out, in, kh, kw]")
    lead = weights.shape[:-2]
    w2 = weights.reshape(-1, weights.shape[-2] * weights.shape[-1])
    if weights.is_cuda:
        keep, split, gvf = C.jenks2_filters_gpu(w2)
    else:
        keep, split, gvf = C.jenks2_filters_host(w2)
    return keep.reshape(weights.shape), split.reshape(lead), gvf.reshape(lead)


def conv_mask(weights_cuda: torch.Tensor):
    """``Conv_Mask`` (``cuda_helpers.py:333-376``): a float32 mask of the weights' shape on
    their device (1 = kept) and the GVF of every filter as a nested list [out][in]."""
    if weights_cuda.dim() != 4:
        raise ValueError("conv_mask takes [out, in, kh, kw] weights")
    keep, _, gvf = jenks2_filters(weights_cuda)
    return keep.to(torch.float32), gvf.cpu().tolist()


def _check_input(t: torch.Tensor, name: str) -> None:
    """The reference's CHECK_INPUT (cuda_helpers.py:72-78) and AT_DISPATCH_FLOATING_TYPES."""
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise RuntimeError(f"{name} must be a CUDA tensor")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")
    if t.dtype not in (torch.float32, torch.float64):
        raise RuntimeError(f'"{name}" not implemented for \'{t.dtype}\'')


def jenks_optimization_cuda(WB: torch.Tensor) -> torch.Tensor:
    """``module_weights.jenks_optimization_cuda(WB)`` (``cuda_helpers.py:187-211``): for a
    sorted ``WB`` of shape ``(rows, cols, ...)``, the SSD of every split of its first
    ``rows * cols`` values, 1-D, of WB's dtype and device."""
    _check_input(WB, "WB")
    if WB.dim() < 2:
        raise RuntimeError("WB must have at least two dimensions (rows, cols)")
    n = WB.shape[0] * WB.shape[1]
    return C.jenks2_ssd(WB.reshape(-1)[:n])


def jenks_optimization_biases_cuda(B: torch.Tensor) -> torch.Tensor:
    """``module_bias.jenks_optimization_biases_cuda(B)`` (``cuda_helpers.py:122-146``): the
    SSD of every split of the first ``B.size(0)`` values of a sorted ``B``, 1-D, of B's
    dtype and device."""
    _check_input(B, "B")
    if B.dim() < 1:
        raise RuntimeError("B must have at least one dimension")
    return C.jenks2_ssd(B.reshape(-1)[:B.shape[0]])


def jenks_optimization_cuda_conv(WB: torch.Tensor) -> torch.Tensor:
    """``module_conv.jenks_optimization_cuda_conv(WB)`` (``cuda_helpers.py:258-289``): for
    ``WB [C0, C1, kh, kw]`` with each (c0, c1) filter's ``kh * kw`` values sorted, the SSD of
    every split of every filter, flat ``[C0 * C1 * kh * kw]`` in WB's order, of WB's dtype
    and device.  Filters of at most 1024 values."""
    _check_input(WB, "WB")
    if WB.dim() != 4:
        raise RuntimeError("WB must be [in_channels, out_channels, rows, cols]")
    c0, c1, kh, kw = WB.shape
    return C.jenks2_ssd_filters(WB.reshape(c0 * c1, kh * kw)).reshape(-1)


module_weights = SimpleNamespace(jenks_optimization_cuda=jenks_optimization_cuda)
module_bias = SimpleNamespace(jenks_optimization_biases_cuda=jenks_optimization_biases_cuda)
module_conv = SimpleNamespace(jenks_optimization_cuda_conv=jenks_optimization_cuda_conv)
