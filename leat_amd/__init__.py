"""leat_amd: MI355X-native (gfx950, wave64) kernels for leat's quantized-weight linear layers.

A drop-in for leat's `leat.ops` / `leat.kernels` hot path (GGUF Q4_K/Q6_K/Q8_0 matvec for
single-stream and batched decode, prefill matmul, MoE experts) over a ctypes C ABI
(include/leatmi.h) to hand-written HIP kernels, on torch-ROCm tensors.
"""

from leat_amd.quant import BLOCK, GGMLType, QTensor, from_blocks

__all__ = ["BLOCK", "GGMLType", "QTensor", "from_blocks"]
