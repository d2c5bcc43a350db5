"""MI355X-native fused 4-bit dequant-GEMV (GF4 Jenks codebooks / E2M1), drop-in for the
quantized linear layer of jvap2/If_I_could_turn_back_time.

Python host code over PyTorch-ROCm; compute in hand-written gfx950 HIP kernels behind the
C ABI of ``libfourbit.so`` (``include/fourbit.h``).
"""
from .linear import PackedWeight, QuantLinear, fwht_block_for, quantize_module  # noqa: F401
from . import _capi  # noqa: F401

__all__ = ["PackedWeight", "QuantLinear", "fwht_block_for", "quantize_module"]
