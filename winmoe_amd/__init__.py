"""winmoe_amd -- MI355X-native MoE expert-layer path of WinMoE.

Router softmax/top-K, raw GGUF block dequantisation (Q8_0, Q2_K, Q3_K, Q4_K,
Q5_K, Q6_K) fused into the gate/up/down expert products, SwiGLU and the
routing-weighted combine with the shared expert, as hand-written gfx950 HIP
kernels behind the C-ABI of include/winmoe_hip.h.
"""
from ._lib import (BLOCK_BYTES, BLOCK_ELEMS, F16, F32, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0, QUANT_TYPES,  # noqa: F401
                   TYPE_IDS, TYPE_NAMES, WinMoEError, load)
from .moe import (ExpertPool, MoELayer, SharedExpert, decode_stack, dequant_q4k_block, dequant_q8_0_row, dequantize,  # noqa: F401
                  expert_ffn,
                  matrix_bytes, q8_0_matvec, quant_matvec, quantize, quantize_into, router_logits,
                  router_topk)

__version__ = "0.1.0"
