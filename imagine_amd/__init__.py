"""MI355X (gfx950) W8A8 linear family: per-token INT8 quantization, INT8 MFMA
GEMM with fused dequant epilogue, M<=2 GEMV, behind the C ABI in include/w8a8.h.

Drop-in for the reference crate's ``int8_linear`` operator
(inference/src/cuda_linear.rs:311-317).
"""
from . import _lib
from .glue import (adaln, gated_residual, int8_linear_modulated, modulated_norm, modulated_norm_quant,
                   quantize_rowwise_modulated, rms_rope, rms_rope1, apply_rope, apply_rope1, rms_rope_, rms_rope1_,
                   apply_rope_, apply_rope1_)
from .ops import (apply_residual, convrot_rotate, dequantize_linear, gemm_dequant, gemm_dequant_residual,
                  gemm_config, gemm_dequant_xq, gemm_i32, gemv_dequant, input_act, quantize_rowwise_act, gemv_dequant_residual, int8_linear,
                  quantize_convrot_weight, quantize_rowwise, quantize_rowwise_convrot, quantize_tensorwise, route,
                  row_scales)

__all__ = ["int8_linear", "quantize_rowwise", "row_scales", "gemv_dequant", "gemv_dequant_residual",
           "gemm_config", "input_act", "quantize_rowwise_act", "gemm_dequant", "gemm_dequant_residual", "gemm_dequant_xq", "gemm_i32", "dequantize_linear",
           "apply_residual", "convrot_rotate", "quantize_rowwise_convrot", "quantize_tensorwise",
           "quantize_convrot_weight", "route", "adaln", "modulated_norm", "modulated_norm_quant", "gated_residual", "rms_rope", "rms_rope1", "apply_rope", "apply_rope1", "rms_rope_", "rms_rope1_", "apply_rope_", "apply_rope1_", "int8_linear_modulated",
           "quantize_rowwise_modulated", "_lib"]
