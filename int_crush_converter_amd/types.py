"""Value types of the public API.

Field names, order and defaults match ``converter/types.py:11-306`` of the
reference so that callers can construct and read them unchanged.  Note the
library default ``rot_size=256`` (the CLI default is 0).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Protocol

import torch


@dataclass
class QuantizeConfig:
    """All options of :func:`quantize_model` (reference ``types.py:11-160``)."""

    input_path: str
    output_dir: str
    rot_size: int = 256
    perm_group_size: int = 128
    quant_group_size: int = 128
    use_permuquant: bool = False
    tau: float = 0.0
    skip_patterns: list[str] | None = None
    exclude_patterns: list[str] | None = None
    calibration_path: str | None = None
    quant_method: str = "rtn"
    gptq_block_size: int = 128
    damping: float = 0.01
    hessian_method: str = "hinv"
    int_bits: int = 4
    ldlq_iterations: int = 1
    greedy_passes: int = 0
    rank_threshold: float = 0.01
    comfy_compat: bool = False
    comfy_int8_fast: bool = False
    asymmetric: bool = False
    clipping_ratios: list[float] | None = None
    piso_scales: bool = False
    quality_report_path: str | None = None
    smoothquant: bool = False
    smooth_alpha: float = 0.5
    seed: int = 42
    smoothrot: bool = False
    smoothrot_alpha: float | None = None
    force_smoothrot_w4: bool = False
    svd_rank: int = 0


@dataclass
class QuantizationResult:
    """One quantized layer (reference ``types.py:163-199``).

    ``quantized_W`` holds int8 codes ([-8, 7] for INT4, [-128, 127] for INT8),
    ``scales`` the fp16 dequantisation scales [out, 1] and ``zero_points`` the
    int8 zero-points [out, 1] or ``None`` for symmetric formats.
    """

    quantized_W: torch.Tensor
    scales: torch.Tensor
    zero_points: torch.Tensor | None = None
    mse: float = 0.0
    max_err: float = 0.0
    method_used: str = ""
    fallbacks: list[str] = field(default_factory=list)


@dataclass(frozen=True)
class ProgressInfo:
    """Per-layer progress event; ``current_layer`` counts from 1."""

    current_layer: int
    total_layers: int
    layer_name: str
    layer_shape: tuple[int, ...]
    elapsed_seconds: float
    estimated_remaining_seconds: float
    method: str
    mse: float


@dataclass(frozen=True)
class ProgressSummary:
    """Final event, delivered once after the output file is written."""

    total_layers: int
    skipped_layers: int
    permuted_layers: int
    gptq_layers: int
    rtn_fallback_layers: int
    smoothquant_layers: int
    svd_layers: int
    elapsed_seconds: float
    input_size_gb: float
    output_size_gb: float
    compression_ratio: float


class ProgressCallback(Protocol):
    """Synchronous callback; an exception raised by it aborts the run."""

    def __call__(self, info: ProgressInfo | ProgressSummary) -> None: ...
