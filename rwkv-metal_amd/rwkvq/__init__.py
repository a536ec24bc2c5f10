"""rwkvq -- MI355X (gfx950) group-affine quantized-linear path for rwkv-metal models.

Ops (MLX names): quantize, dequantize, quantized_matmul, pack_codes,
unpack_codes, grouped_qmv; BoundQmm / GroupedQmv bind a product once for
repeated runs.  Modules: QuantizedLinear, QuantizedEmbedding,
quantize (mlx.nn.quantize).  LoRA engine: LoRALinear, add_lora,
quantize_base_model, BIG_QUANT_TARGETS, save_lora / load_lora / merge_lora.
Packed checkpoints: rwkvq.io.save_quantized / load_quantized.  The .rwkvq
(rwkv-quant sb6) base: RwkvqLinear, RwkvqNativeLinear, RwkvqHybridLinear,
add_lora_rwkvq, load_sidecar.
All compute runs in librwkvq_hip.so; tensors must be on the GPU.
"""
from .ops import (VALID_BITS, VALID_GROUP_SIZES, BoundQmm, GroupedQmv, dequantize, grouped_qmv,
                  lora_down, lora_grads, pack_codes, qlora_fused, quantize, quantized_embedding, quantized_matmul,
                  quantized_matmul_lora, unpack_codes)
from .nn import QuantizedEmbedding, QuantizedLinear, is_quantizable
from .nn import quantize as quantize_model
from . import io, sb6
from .sb6 import RwkvqHybridLinear, RwkvqLinear, RwkvqNativeLinear, add_lora_rwkvq, load_sidecar
from .lora import (BIG_QUANT_TARGETS, CMIX_TARGETS, TMIX_TARGETS, LoRALinear, add_lora,
                   load_lora, lora_state, merge_lora, quantize_base_model, save_lora)

__all__ = [
    "VALID_BITS", "VALID_GROUP_SIZES", "quantize", "dequantize", "quantized_matmul",
    "quantized_embedding", "quantized_matmul_lora", "lora_down", "lora_grads", "qlora_fused",
    "pack_codes", "unpack_codes", "grouped_qmv", "GroupedQmv", "BoundQmm", "QuantizedLinear", "QuantizedEmbedding",
    "is_quantizable", "quantize_model", "BIG_QUANT_TARGETS", "TMIX_TARGETS", "CMIX_TARGETS",
    "LoRALinear", "add_lora", "quantize_base_model", "lora_state", "save_lora", "load_lora",
    "merge_lora", "io", "sb6", "RwkvqLinear", "RwkvqNativeLinear", "RwkvqHybridLinear",
    "add_lora_rwkvq", "load_sidecar",
]
