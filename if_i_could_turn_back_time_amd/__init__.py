"""MI355X-native fused 4-bit dequant-GEMV (GF4 Jenks codebooks / E2M1), drop-in for the
quantized linear layer of jvap2/If_I_could_turn_back_time.

Python host code over PyTorch-ROCm; compute in hand-written gfx950 HIP kernels behind the
C ABI of ``libfourbit.so`` (``include/fourbit.h``).
"""
from .linear import (PackedWeight, QuantLinear, fp4_mfma_shared, fwht_block_for,  # noqa: F401
                     packed_k, packed_linear, quantize_module)
from .brecq import adaround_levels, pack_quantized_linears, replace_forward  # noqa: F401
from .jenks import (bias_mask, jenks2, linear_mask, module_bias, module_conv,  # noqa: F401
                    module_weights)
from . import _capi  # noqa: F401

__all__ = ["PackedWeight", "QuantLinear", "fp4_mfma_shared", "fwht_block_for", "packed_k",
           "packed_linear",
           "quantize_module", "adaround_levels", "pack_quantized_linears", "replace_forward",
           "jenks2", "linear_mask", "bias_mask", "module_weights", "module_bias",
           "module_conv"]
