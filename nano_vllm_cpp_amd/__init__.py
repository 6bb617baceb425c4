"""MI355X (gfx950) fused per-layer ops of Nano_vLLM_cpp: embedding gather with
in-kernel Q8_0/K-quant dequant, residual-add + RMSNorm, Qwen3 QK-norm + NeoX
RoPE, and SiLU*up.  Kernels and the C ABI live in libnvf_ops.so (csrc/,
include/nvf_ops.h); `ops` is the Python front end."""
from . import ops  # noqa: F401

__all__ = ["ops"]
