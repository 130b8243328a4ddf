"""MI355X-native per-layer quantization path of int_crush_converter.

Public names mirror the reference package ``converter`` (its ``__init__.py``)
for the hot path: rotation, RTN scales, PiSO scales, packing, DLR Hessians,
GPTQ / LDLQ layers, the pipeline and the value types.  The reference's
SmoothQuant / SmoothRot / SVD helpers are outside this path and not
exported.  All arithmetic runs in the gfx950 HIP library
``libicq.so`` (see ``include/ic_abi.h``); there is no CPU fallback.
"""

from .rotation import rotate_weights, rotate_activations, rotate_hessian, make_hadamard_regular, get_hadamard
from .packing import pack_int4, unpack_int4, validate_int4_range
from .scales import (
    calculate_scales,
    quantize_weights,
    calculate_scales_int8,
    quantize_weights_int8,
    calculate_scales_asymmetric,
    quantize_weights_asymmetric,
    calculate_scales_int8_asymmetric,
    quantize_weights_int8_asymmetric,
)
from .piso import (
    compute_piso_scales_int8,
    compute_piso_scales_int8_asymmetric,
    compute_piso_scales_int4,
    compute_piso_scales_int4_asymmetric,
)
from .config import INT4_SCALE_DIVISOR, INT8_SCALE_DIVISOR
from .dlr import (
    is_dlr,
    validate_dlr,
    woodbury_inverse,
    dlr_to_dense,
    transform_dlr_for_smoothquant,
    permute_dlr,
    make_dlr_dict,
)
from .gptq import gptq_quantize_layer, gptq_quantize_layer_rtn
from .ldlq import ldlq_quantize_layer
from .calibration_io import load_calibration, build_name_map, get_hessian, get_per_channel_amax
from .pipeline import quantize_model, should_skip
from .types import QuantizationResult, QuantizeConfig, ProgressInfo, ProgressSummary, ProgressCallback

__all__ = [
    "rotate_weights", "rotate_activations", "rotate_hessian", "make_hadamard_regular", "get_hadamard",
    "pack_int4", "unpack_int4", "validate_int4_range",
    "calculate_scales", "quantize_weights", "calculate_scales_int8", "quantize_weights_int8",
    "calculate_scales_asymmetric", "quantize_weights_asymmetric",
    "calculate_scales_int8_asymmetric", "quantize_weights_int8_asymmetric",
    "INT4_SCALE_DIVISOR", "INT8_SCALE_DIVISOR",
    "is_dlr", "validate_dlr", "woodbury_inverse", "dlr_to_dense", "transform_dlr_for_smoothquant",
    "permute_dlr", "make_dlr_dict",
    "gptq_quantize_layer", "gptq_quantize_layer_rtn", "ldlq_quantize_layer",
    "load_calibration", "build_name_map", "get_hessian", "get_per_channel_amax",
    "quantize_model", "should_skip",
    "QuantizationResult", "QuantizeConfig", "ProgressInfo", "ProgressSummary", "ProgressCallback",
    "compute_piso_scales_int8", "compute_piso_scales_int8_asymmetric",
    "compute_piso_scales_int4", "compute_piso_scales_int4_asymmetric",
]
