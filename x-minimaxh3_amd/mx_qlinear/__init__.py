"""mx_qlinear: the MI355X (gfx950) quantized DiT linear path.

Per-token INT8 activation quantization (optionally fused with adaLN), INT8 x INT8 -> INT32
GEMMs on CDNA4 matrix cores with fused dequant / bias / tanh-GELU / re-quant epilogues, and
W4A8 GEMMs, with the ConvRot (regular Hadamard) rotation and the GELU / SwiGLU input
activations folded into the quantizer, behind the reference's Comfy-Kitchen function names and its quantized-linear
module contract. All compute runs in hand-written HIP kernels (libmx_qlinear.so, C ABI in
include/mx_qlinear.h); there is no CPU path.
"""

from .ops import (  # noqa: F401
    FfnWorkspace,
    PreparedSwiGLUFc1,
    adaln,
    adaln_quantize_int8,
    apply_input_act,
    dequantize_int4_grouped_to_int8,
    dequantize_w4a8_int8_weight,
    fused_down_gated_residual,
    h3_mlp_,
    int8_ffn_gelu,
    int8_gemv_dequant,
    int8_swiglu_fc1,
    int8_linear,
    int8_linear_gated_residual_,
    int8_linear_prequantized,
    mm_int8,
    prepare_int8_weight,
    prepare_swiglu_fc1,
    quantize_int8_convrot_weight,
    quantize_int8_rowwise,
    quantize_int8_rowwise_convrot,
    quantize_w4a8_int8_weight,
    rms_adaln,
    rms_adaln_quantize_int8,
    rotate_int8_convrot_weight,
    segment_row_map,
    swiglu_mlp_gated_residual_,
    w4a8_grouped_linear,
    PreparedW4A8Grouped,
    prepare_w4a8_grouped,
    w4a8_int8_linear,
)
from .checkpoint import (  # noqa: F401
    MappingTensorSource,
    SafeTensorSource,
    audit_quantized_layer,
    quant_linear,
    save_checkpoint,
)
from .modules import (  # noqa: F401
    ComfyQuantSpec,
    ConvRotInt8Linear,
    ConvRotW4A8Linear,
    PreparedConvRotInt8Input,
    W4A8QuantSpec,
    inspect_quantized_layers,
    int8_kernel,
    w4a8_kernel,
)

__version__ = "0.1.0"
