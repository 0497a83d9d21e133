"""swarmllm_amd — SwarmLLM's quantized matmul path (candle QTensor / QMatMul
over GGUF Q8_0, Q4_K, Q6_K, IQ4_NL, MXFP4) as hand-written HIP kernels for
AMD Instinct MI355X (gfx950), behind the C ABI of include/qmm.h."""

from ._lib import QmmError, lib  # noqa: F401
from .qtensor import (MOE_CARD_ONE_ROW_MAX_TOKENS, GgmlDType, QMatMul, QTensor, fill_normal,  # noqa: F401
                      forward_glu, glu, mmq_few_rows_line, moe_forward, moe_prompt_on_tensor_cores,
                      moe_uses_prompt_kernel, prepare, prepared, set_force_dmmv)

__all__ = ["MOE_CARD_ONE_ROW_MAX_TOKENS", "GgmlDType", "QMatMul", "QTensor", "QmmError", "fill_normal", "forward_glu",
           "glu", "lib", "mmq_few_rows_line", "moe_forward", "moe_prompt_on_tensor_cores", "moe_uses_prompt_kernel",
           "prepare", "prepared", "set_force_dmmv"]
