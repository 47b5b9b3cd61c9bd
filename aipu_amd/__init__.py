"""aipu_amd -- MI355X (gfx950) implementation of the AIPU Q4_K GEMM core.

Hot path: ggml Q4_K super-block dequant -> fp32 MAC -> bf16 out (plus the Q6_K / Q8_0 / F16
decoders, the SwiGLU expert and the MoE decode step), as hand-written HIP kernels behind the
C ABI in include/aipu_q4k.h.

Modules
  aipu_amd.device             torch-tensor API (device tensors in/out, stream-ordered)
  aipu_amd.q4k_ref            drop-in for tools/q4k_ref.py's entry points (numpy in/out)
  aipu_amd.glm_model_q4k_ref  drop-in for the hot-path entry points of tools/glm_model_q4k_ref.py
  aipu_amd.build              hipcc build of libaipu_q4k.so (gfx950)
"""
from ._lib import (MODE_FAST, MODE_REF, TYPE_BF16, TYPE_F16, TYPE_Q4_K, TYPE_Q6_K, TYPE_Q8_0, AipuError,
                   AipuLibraryMissing, lib)

__all__ = ["MODE_FAST", "MODE_REF", "TYPE_BF16", "TYPE_F16", "TYPE_Q4_K", "TYPE_Q6_K", "TYPE_Q8_0", "AipuError",
           "AipuLibraryMissing", "lib"]
