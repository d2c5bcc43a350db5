"""Caller side of the packed 4-bit linear for the reference's brecq/AdaRound pipeline.

The reference's BRECQ pass (``Quantization_Experiments/brecq.py:613-654``) gives every
``nn.Linear`` an ``AdaRoundQuantizer`` (``:59-92``) as ``module.weight_quantizer`` and
swaps its forward with ``replace_forward`` (``:305-331``), which rebuilds the fp32 weight
``clamp(mask * (W_floor + h(alpha)), qmin, qmax) * delta`` on every call before
``F.linear``.  ``replace_forward`` here takes such a module after reconstruction, packs the
hard-rounded integer levels with the per-row ``delta`` as GF4 codebooks
(``fb_pack_levels_gf4``: codebook entry ``fp16(fp32(delta * level))``) and routes forward
through the fused GEMV.  At 4 bits ``[qmin, qmax] = [-8, 7]`` is exactly 16 levels, so
every group fits; wider bit widths are rejected when a 128-group spans more than 16.

Hard rounding rounds ``h`` as the reference's ``QuantLinear.commit`` rounds its gate
(``layers.py:41``): ``h > 0.5`` adds one level.  Where ``alpha`` has converged to the
clip's flat parts (``|alpha| >~ 2.4``), ``h`` is already exactly 0 or 1 and the packed
layer computes the reference's soft forward.  ``nn.Conv2d`` modules keep the reference
forward (the GEMV serves linear layers).
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from .linear import PackedWeight, packed_k, packed_linear


def adaround_levels(weight_quantizer) -> tuple[torch.Tensor, torch.Tensor]:
    """Hard integer levels ``[N, K]`` (fp32) and per-row scale ``[N]`` of an AdaRound
    quantizer: ``clamp(mask * (W_floor + [clip(sigmoid(alpha)*1.2-0.1, 0, 1) > 0.5]),
    qmin, qmax)`` and ``delta`` (``brecq.py:81-92``; per-tensor delta is broadcast)."""
    wq = weight_quantizer
    q = wq.quantizer
    w_floor = wq.W_floor.detach().float().cpu()
    alpha = wq.alpha.detach().float().cpu()
    mask = wq.mask.detach().float().cpu()
    if w_floor.dim() != 2:
        raise ValueError("only linear (2-D) weights are packed")
    h = torch.clamp(torch.sigmoid(alpha) * 1.2 - 0.1, 0, 1)
    levels = torch.clamp(mask * (w_floor + (h > 0.5).float()), q.qmin, q.qmax)
    delta = torch.as_tensor(q.delta).detach().float().cpu().reshape(-1)
    N = levels.shape[0]
    if delta.numel() == 1:
        delta = delta.expand(N).contiguous()
    elif delta.numel() != N:
        raise ValueError("delta must be per-tensor or per-output-row")
    return levels, delta


def replace_forward(module: nn.Linear, *, nthreads: int | None = None) -> nn.Linear:
    """Packs ``module.weight_quantizer`` and sets ``module.forward`` to the fused GEMV
    (drop-in for ``brecq.replace_forward``, ``brecq.py:305-331``, on ``nn.Linear``).
    The packed weight lives on ``module.weight``'s device as ``module.packed_weight``."""
    if not isinstance(module, nn.Linear):
        raise TypeError("replace_forward packs nn.Linear modules")
    levels, delta = adaround_levels(module.weight_quantizer)
    N, K = levels.shape
    levels = F.pad(levels, (0, packed_k(K) - K))
    dev = module.weight.device
    pw = PackedWeight.from_levels(levels, delta, device=dev if dev.type == "cuda" else None,
                                  nthreads=nthreads)
    module.packed_weight = pw

    def new_forward(x):
        return packed_linear(pw.wdev, N, K, "gf4", 0, x, module.bias)

    module.forward = new_forward
    return module


def pack_quantized_linears(model: nn.Module, *, nthreads: int | None = None) -> nn.Module:
    """``replace_forward`` on every ``nn.Linear`` of ``model`` that carries a
    ``weight_quantizer`` (the state ``copy_block_with_quantizers`` leaves,
    ``brecq.py:333-369``); returns ``model``."""
    for m in model.modules():
        if isinstance(m, nn.Linear) and hasattr(m, "weight_quantizer"):
            replace_forward(m, nthreads=nthreads)
    return model
