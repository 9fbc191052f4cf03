"""vdn_fp8 -- the fp8 quantized-linear path of the VDN-H3 DiT blocks, MI355X-native.

`vdn_fp8.fp8_linear` mirrors the reference module `src.models.ops.fp8_linear`;
`vdn_fp8.lora` mirrors `src.inference.utils.lora`; `vdn_fp8.fused_block` fuses the
block's pre-norm (`src.models.ops.fused_block`) with the quantization that follows it;
`vdn_fp8.softmax_attention` holds the QK-norm + rope pass (`_qk_prep`,
`src.models.softmax_attention.kernels`). All compute is in libvdnfp8.so
(hand-written HIP for gfx950, C ABI in include/vdn_fp8.h).
"""
from .fp8_linear import (FP8_DTYPE, MIN_WIDTH, SKIP_END_BLOCKS, _FP8_MAX, Fp8Linear,
                         convert_linear_to_fp8, gelu_quantize, per_tensor_gemm, quantize_activation,
                         quantize_rows, quantize_rows_reference, requantize_weight,
                         set_index_checks, swiglu_quantize, swiglu_quantize_activation)
from .fused_block import fast_block_forward, fast_ff_forward, post, pre, pre_quantize
from .lora import load_external_lora, merge_lora_and_convert, merge_lora_state
from .softmax_attention import qk_prep

__all__ = [
    "FP8_DTYPE", "MIN_WIDTH", "SKIP_END_BLOCKS", "_FP8_MAX", "Fp8Linear", "convert_linear_to_fp8", "gelu_quantize",
    "per_tensor_gemm", "quantize_activation", "quantize_rows", "quantize_rows_reference",
    "requantize_weight", "swiglu_quantize", "swiglu_quantize_activation", "load_external_lora",
    "merge_lora_and_convert", "merge_lora_state", "pre_quantize", "qk_prep", "pre", "post",
    "fast_ff_forward", "fast_block_forward", "set_index_checks",
]
