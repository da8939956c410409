"""combsengine_amd -- MI355X (gfx950) fused GGUF dequant-matmul.

A drop-in replacement for the quantized linear layer of asqrzk/CombsEngine
(engine/core/combs-models/src/qlinear.rs + qmatmul.rs): weights stay in their
GGUF block layout (Q4_0/Q5_0/Q8_0/Q4_K/Q5_K/Q6_K) in device memory and are
dequantised inside hand-written HIP kernels for gfx950 behind a C ABI
(include/combs_qlinear.h).  This package is the host-side mirror of the
reference's seam; the compute lives only in lib/libcombs_qlinear.so.
"""
from .qlinear import (  # noqa: F401
    Activation, BadShape, Linear, ModelError, QuantFormat, QuantLinearOp, QuantTensor, QuantWeight, gated_up,
    multi_forward,
    block_bytes, block_values, dequantize_gpu, quantize, tensor_byte_size, try_quant_linear,
)
from .gguf import GgufSource  # noqa: F401,E402
