"""Command line (same flags as ``converter/cli.py:130-322``).

    python -m int_crush_converter_amd -i in.safetensors -o out/ --rot-size 256 \\
        -c cal.pt --quant-method gptq
"""

from __future__ import annotations

import argparse
import logging
import os
import sys

from .log import logger
from .pipeline import quantize_model
from .types import ProgressInfo, ProgressSummary, QuantizeConfig


def _configure_cli_logging(level: int) -> None:
    handler = logging.StreamHandler()
    handler.setFormatter(logging.Formatter("%(message)s"))
    logger.addHandler(handler)
    logger.setLevel(level)


class _PerLayerFilter(logging.Filter):
    """Drops the per-layer 'Quantizing ...' line while progress lines are printed."""

    def filter(self, record: logging.LogRecord) -> bool:
        return not (record.levelno == logging.INFO and record.getMessage().startswith("Quantizing "))


def _fmt_secs(s: float) -> str:
    return f"{int(s // 60)}m{int(s % 60):02d}s" if s >= 60 else f"{s:.0f}s"


def _cli_progress_callback(info) -> None:
    if isinstance(info, ProgressInfo):
        pct = info.current_layer / info.total_layers * 100
        print(f"  [{pct:5.1f}%] {info.layer_name}\n           {info.method:15s} MSE={info.mse:<12.6f} "
              f"ETA {_fmt_secs(info.estimated_remaining_seconds)}", file=sys.stderr)
    elif isinstance(info, ProgressSummary):
        el = info.elapsed_seconds
        el_s = f"{int(el // 60)}m{int(el % 60):02d}s" if el >= 60 else f"{el:.1f}s"
        print(f"\nQuantized {info.total_layers} layers in {el_s}, {info.compression_ratio:.1f}x compression",
              file=sys.stderr)


def build_parser() -> argparse.ArgumentParser:
    p = argparse.ArgumentParser(description="Quantize a model using INT-Crush + PermuQuant + GPTQ/LDLQ")
    p.add_argument("-i", "--input", required=True, help="Input safetensors file")
    p.add_argument("-o", "--output", required=True, help="Output directory")
    p.add_argument("--rot-size", type=int, default=0,
                   help="Regular Hadamard group size (0=no rotation, power of 4 for Regular Hadamard, any power "
                        "of 2 for Sylvester fallback. Default: 0)")
    p.add_argument("--int-bits", type=int, default=4, choices=[4, 8], help="Quantization bit-width (default: 4)")
    p.add_argument("--perm-group-size", type=int, default=128, help="PermuQuant acceptance group size")
    p.add_argument("--quant-group-size", type=int, default=128,
                   help="RTN quantization group size (validated; quantization is per row)")
    p.add_argument("--permuquant", action="store_true", help="Enable PermuQuant channel reordering")
    p.add_argument("--tau", type=float, default=0.0, help="PermuQuant acceptance threshold (default: 0.0)")
    p.add_argument("--skip-patterns", type=str, default=None,
                   help="Comma-separated skip patterns (default: embed,norm,modulation,lm_head,output,proj_out)")
    p.add_argument("--exclude-patterns", type=str, default=None,
                   help="Comma-separated additional patterns to exclude from quantization")
    p.add_argument("-c", "--calibration", type=str, default=None, help="Path to .pt calibration file (for GPTQ)")
    p.add_argument("--quant-method", type=str, default="rtn", choices=["rtn", "gptq", "ldlq"],
                   help="Quantization method (default: rtn)")
    p.add_argument("--gptq-block-size", type=int, default=128, help="GPTQ block size (default: 128)")
    p.add_argument("--damping", type=float, default=0.01, help="GPTQ/LDLQ damping ratio (default: 0.01)")
    p.add_argument("--hessian-method", type=str, default="hinv", choices=["hinv", "cholesky"],
                   help="Hessian preparation for GPTQ: 'hinv' (full inverse) or 'cholesky' (factor of H^-1)")
    p.add_argument("--ldlq-iterations", type=int, default=1, help="LDLQ iterations with scale refinement")
    p.add_argument("--greedy-passes", type=int, default=0, help="Greedy local search passes after LDLQ")
    p.add_argument("--rank-threshold", type=float, default=0.01, help="Eigenvalue threshold for low-rank greedy")
    p.add_argument("--comfy-compat", action="store_true", help="Write .comfy_quant (ComfyUI INT8 format)")
    p.add_argument("--comfy-int8-fast", action="store_true", help="Write comfy_quant for ComfyUI-INT8-Fast")
    p.add_argument("--piso", action="store_true", help="PiSO data-aware per-row scales (needs --calibration)")
    p.add_argument("--asymmetric", action="store_true", help="Asymmetric quantization (scale + zero-point)")
    p.add_argument("--clipping-ratios", type=str, default=None,
                   help="Comma-separated clipping ratios searched for the lowest-MSE scale per row")
    p.add_argument("--verbose", "-v", action="store_true", help="Show detailed output")
    p.add_argument("--quiet", "-q", action="store_true", help="Only warnings and errors")
    p.add_argument("--quality-report", type=str, default=None, metavar="REPORT.json",
                   help="Write per-layer quantization metrics as JSON")
    p.add_argument("--smoothquant", action="store_true", help="SmoothQuant (not part of this build)")
    p.add_argument("--smooth-alpha", type=float, default=0.5, help="SmoothQuant migration strength")
    p.add_argument("--smoothrot", action="store_true", help="Smooth-then-rotate (not part of this build)")
    p.add_argument("--smoothrot-alpha", type=float, default=None, help="SmoothRot migration strength")
    p.add_argument("--force-smoothrot-w4", action="store_true", help="Force smooth-then-rotate for W4")
    p.add_argument("--no-progress", action="store_true", default=False, help="Disable per-layer progress")
    p.add_argument("--seed", type=int, default=42, metavar="N", help="Random seed (default: 42, -1 to disable)")
    p.add_argument("--svd-rank", type=int, default=0, metavar="R", help="SVD-absorbed rank (not part of this build)")
    return p


def main(argv: list[str] | None = None) -> None:
    parser = build_parser()
    args = parser.parse_args(argv)
    level = logging.WARNING if args.quiet else (logging.DEBUG if args.verbose else logging.INFO)
    _configure_cli_logging(level)
    if args.rot_size != 0 and (args.rot_size & (args.rot_size - 1)) != 0:
        parser.error(f"--rot-size must be 0 or a power of 2, got {args.rot_size}")
    if args.comfy_compat and args.int_bits != 8:
        parser.error("--comfy-compat requires --int-bits 8")
    if args.comfy_int8_fast and args.int_bits != 8:
        parser.error("--comfy-int8-fast requires --int-bits 8")
    if args.smoothquant and args.rot_size > 0:
        args.smoothrot = True
    if args.smoothrot:
        if args.rot_size == 0:
            parser.error("--smoothrot requires --rot-size > 0")
        args.smoothquant = True
    split = lambda s: [p.strip() for p in s.split(",")] if s else None  # noqa: E731
    ratios = [float(x.strip()) for x in args.clipping_ratios.split(",")] if args.clipping_ratios else None
    report = args.quality_report
    if report and os.sep not in report and "/" not in report:
        report = os.path.join(args.output, report)
    config = QuantizeConfig(
        input_path=args.input, output_dir=args.output, rot_size=args.rot_size,
        perm_group_size=args.perm_group_size, quant_group_size=args.quant_group_size,
        use_permuquant=args.permuquant, tau=args.tau, skip_patterns=split(args.skip_patterns),
        exclude_patterns=split(args.exclude_patterns), calibration_path=args.calibration,
        quant_method=args.quant_method, gptq_block_size=args.gptq_block_size, damping=args.damping,
        hessian_method=args.hessian_method, int_bits=args.int_bits, ldlq_iterations=args.ldlq_iterations,
        greedy_passes=args.greedy_passes, rank_threshold=args.rank_threshold, comfy_compat=args.comfy_compat,
        comfy_int8_fast=args.comfy_int8_fast, piso_scales=args.piso, asymmetric=args.asymmetric,
        clipping_ratios=ratios, smoothquant=args.smoothquant, smooth_alpha=args.smooth_alpha,
        quality_report_path=report, seed=args.seed, smoothrot=args.smoothrot,
        smoothrot_alpha=args.smoothrot_alpha, force_smoothrot_w4=args.force_smoothrot_w4, svd_rank=args.svd_rank,
    )
    callback = None
    if not args.no_progress and not args.quiet:
        callback = _cli_progress_callback
        logger.addFilter(_PerLayerFilter())
    quantize_model(config, progress_callback=callback)


if __name__ == "__main__":
    main()
