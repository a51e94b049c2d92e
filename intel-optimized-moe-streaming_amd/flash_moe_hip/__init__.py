"""flash_moe_hip -- MI355X (gfx950) quantized-expert hot path.

GGUF Q3_K/Q4_K/Q5_K/Q6_K/Q8_0 dequantization fused with the routed-expert
SwiGLU FFN, as hand-written HIP kernels behind a C ABI
(``include/moe_quant_hip.h``, ``libmoe_quant_hip.so``).  The Python layer
mirrors the reference's ``flash_moe`` interface for this path:

  native_expert   NativeExpert, load_native_expert, SUPPORTED_TYPES
  dequant         dequant_to_f16, dequantize, dequantize_to, dequant_device, GGML_BLOCK_INFO
  router          ExpertRouter, synthetic_router, softmax_all_experts
  moe_layer       run_moe_layer, run_moe_sequence
  backend         HipExpertBackend (HBM-resident expert layers)
  shared_expert   SharedExpert
  layer_store     ExpertLayer (stacked GGUF expert tensors in HBM)
  moe_gpu         MoeRunner (device-tensor fused calls)

Importing the package does not load the library; the first call does, and
raises if it is missing.
"""
from .key import ExpertKey
from .quant_types import GGML_BLOCK_INFO, GGML_TYPE_IDS, SUPPORTED_TYPES, block_info, name_of

__all__ = ["ExpertKey", "GGML_BLOCK_INFO", "GGML_TYPE_IDS", "SUPPORTED_TYPES", "block_info", "name_of"]
