"""``quantize_model``: safetensors in, quantised safetensors out (API of
``converter/pipeline.py``).

Same validation, output tensor names, dtypes and ``int_crush.*`` metadata as
the reference for the methods this build implements (RTN, GPTQ, LDLQ with
greedy search, ConvRot rotation, PermuQuant, PiSO scales, 2-D / 3-D / DLR
Hessians).
Each layer goes to the GPU once: the per-layer step (``layer.py``) rotates,
quantises, verifies and packs there; only the stored tensors come back to
host memory.  Options that belong to other subsystems of the reference
(SmoothQuant / SmoothRot, SVD-absorbed) raise ``NotImplementedError``.
"""

from __future__ import annotations

import copy
import json
import os
import time
import warnings

import torch
from safetensors.torch import load_file, save_file

from .calibration_io import build_name_map, get_hessian, get_permutation, is_dlr, load_calibration
from .config import DEFAULT_SKIP_PATTERNS
from .log import logger
from .types import ProgressCallback, ProgressInfo, ProgressSummary, QuantizeConfig
from . import _native as nat
from . import layer as _layer


def should_skip(name: str, skip_patterns: list[str]) -> bool:
    """True when a (lower-cased) layer name contains any skip pattern."""
    low = name.lower()
    return any(p in low for p in skip_patterns)


def _validate(config: QuantizeConfig) -> QuantizeConfig:
    """Validation and implicit couplings of converter/pipeline.py:173-250."""
    if config.quant_method not in ("rtn", "gptq", "ldlq"):
        raise ValueError(f"quant_method must be 'rtn', 'gptq', or 'ldlq', got '{config.quant_method}'")
    if config.quant_method == "gptq" and not config.calibration_path:
        raise ValueError("GPTQ requires --calibration path to a .pt file")
    if config.quant_method == "ldlq" and not config.calibration_path:
        warnings.warn(
            "LDLQ: no calibration data provided; will fall back to "
            "H = W^T W / M (weight-only). This can perform worse than RTN. "
            "Pass --calibration for best results.")
    if config.rot_size > 0 and (config.rot_size & (config.rot_size - 1)) != 0:
        raise ValueError(f"rot_size must be 0 (no rotation) or a power of 2, got {config.rot_size}")
    if config.perm_group_size < 32 or (config.perm_group_size & (config.perm_group_size - 1)) != 0:
        raise ValueError(f"perm_group_size must be a power of 2 >= 32, got {config.perm_group_size}")
    if config.quant_group_size < 32 or (config.quant_group_size & (config.quant_group_size - 1)) != 0:
        raise ValueError(f"quant_group_size must be a power of 2 >= 32, got {config.quant_group_size}")
    if config.int_bits not in (4, 8):
        raise ValueError(f"int_bits must be 4 or 8, got {config.int_bits}")
    if config.smoothquant and config.int_bits == 4:
        logger.warning("SmoothQuant is designed for W8A8 (INT8) quantization. With INT4 weight-only "
                       "quantization, the benefit is limited. Consider using --int-bits 8 with --smoothquant.")
    config = copy.copy(config)
    if config.smoothrot and config.int_bits == 4 and not config.force_smoothrot_w4:
        logger.warning("SmoothRot is automatically disabled at W4; use --force-smoothrot-w4 to override.")
        config.smoothrot = False
    if config.smoothquant and config.rot_size > 0:
        config.smoothrot = True
    if config.smoothrot:
        if config.rot_size == 0:
            raise ValueError("SmoothRot requires rot_size > 0")
        config.smoothquant = True
    if config.svd_rank < 0:
        raise ValueError(f"svd_rank must be >= 0, got {config.svd_rank}")
    if config.rot_size > 4096:
        raise ValueError(f"rot_size {config.rot_size} exceeds the supported maximum 4096")
    for flag, what in [(config.smoothquant, "SmoothQuant / SmoothRot (--smoothquant, --smoothrot)"),
                       (config.svd_rank > 0, "SVD-absorbed (--svd-rank)")]:
        if flag:
            raise NotImplementedError(f"{what} is not part of this build's quantization path")
    return config


def _metadata(config: QuantizeConfig, shapes, skip_patterns) -> dict[str, str]:
    """int_crush.* metadata (converter/pipeline.py:417-487); ``shapes`` maps
    tensor names to shapes, in the input's order."""
    is_int8 = config.int_bits == 8
    method_base = "int_crush_permuq" if config.use_permuquant else "int_crush"
    method = f"{method_base}_{config.quant_method}" if config.quant_method in ("gptq", "ldlq") else method_base
    asym = config.asymmetric or (config.quant_method == "gptq" and not is_int8)
    md = {
        "int_crush.format_version": "3" if not is_int8 else "1",
        "int_crush.method": method,
        "int_crush.rot_size": str(config.rot_size),
        "int_crush.scale_type": "per_row_asymmetric" if asym else "per_row",
        "int_crush.hadamard_type": "regular",
        "int_crush.packing_order": "native" if is_int8 else "little",
    }
    if config.exclude_patterns:
        md["int_crush.exclude_patterns"] = ",".join(config.exclude_patterns)
    if config.rot_size > 0:
        padded = {}
        for name, shape in shapes.items():
            if len(shape) == 2 and not should_skip(name, skip_patterns) and shape[1] % config.rot_size:
                padded[name] = str(shape[1])
        if padded:
            md["int_crush.padded_layers"] = ";".join(f"{k}={v}" for k, v in padded.items())
    if config.use_permuquant:
        md["int_crush.permuquant"] = "true"
        md["int_crush.permuquant_tau"] = str(config.tau)
    if config.quant_method == "gptq":
        md["int_crush.gptq_block_size"] = str(config.gptq_block_size)
        md["int_crush.damping_ratio"] = str(config.damping)
    elif config.quant_method == "ldlq":
        md["int_crush.ldlq_block_size"] = str(config.gptq_block_size)
        md["int_crush.damping_ratio"] = str(config.damping)
        md["int_crush.ldlq_iterations"] = str(config.ldlq_iterations)
        if config.greedy_passes > 0:
            md["int_crush.greedy_passes"] = str(config.greedy_passes)
            md["int_crush.rank_threshold"] = str(config.rank_threshold)
    return md


def _comfy_tensor(name: str, config: QuantizeConfig, fmt: bool) -> tuple[str, torch.Tensor]:
    prefix = name.rsplit(".weight", 1)[0]
    data = {"format": "int8_tensorwise"} if fmt else {"per_row": True}
    if config.rot_size > 0:
        data["convrot"] = True
        data["convrot_groupsize"] = config.rot_size
    blob = json.dumps(data, separators=(",", ":")) if fmt else json.dumps(data)
    return f"{prefix}.comfy_quant", torch.tensor(list(blob.encode("utf-8")), dtype=torch.uint8)


def _permuquant(name: str, W_work: torch.Tensor, orig_in: int, config: QuantizeConfig, calibration, name_map,
                state: dict):
    """PermuQuant step (converter/pipeline.py:572-615): permutes the first
    orig_in columns of W_work in place; returns (perm or None, whether it
    came from the calibration file)."""
    from . import permuquant as _pq
    layer_name = name_map.get(name) if name_map else None
    cal_perm = None
    if layer_name is not None and calibration is not None:
        cal_perm = get_permutation(calibration, layer_name)
    if cal_perm is not None:
        of = min(orig_in, cal_perm.shape[0])
        ps = cal_perm[:of]
        if ps.numel() and ps.max() < of and ps.min() >= 0 and ps.unique().numel() == ps.numel():
            W_work[:, :of] = _pq.permute_columns(W_work[:, :of], ps)
            state["permuted"] += 1
            logger.debug("PermuQuant applied (from calibration)")
            return ps.to(W_work.device), True
        logger.warning("Calibration permutation out of bounds, falling back to weight-only")
    W_orig = W_work[:, :orig_in]
    # per-row INT4 for every method: the acceptance check uses the same granularity
    # (sweep_alpha without activation statistics: one alpha, 0.0)
    gs = W_orig.shape[1] if config.int_bits == 4 else config.perm_group_size
    perm, accepted, Wp = _pq.weight_only_permutation(W_orig, gs, config.tau, config.int_bits)
    if not accepted:
        logger.debug("PermuQuant skipped (no improvement)")
        return None, False
    W_work[:, :orig_in] = Wp
    state["permuted"] += 1
    logger.debug("PermuQuant applied (alpha=%.2f)", 0.0)
    return perm, False


def _piso(name: str, tensor: torch.Tensor, W_work: torch.Tensor, outliers: int, config: QuantizeConfig,
          calibration, name_map, state: dict):
    """PiSO scales of one layer (pipeline.py:286-360): on the rotated weights
    as loaded (no outlier zeroing) with the calibration's Hessian diagonal
    zero-padded to the rotated width.  INT8: symmetric scales; INT4:
    asymmetric scales and zero-points.  A failed search leaves the layer
    without PiSO, as in the reference.  Returns (scales, zero-points or None)."""
    from .calibration_io import get_hessian_diag
    from . import piso as _piso_mod
    layer_name = name_map.get(name)
    if layer_name is None:
        return None
    h = get_hessian_diag(calibration, layer_name, tensor.shape[1])
    if h is None:
        return None
    if outliers:
        from .rotation import rotate_rows_gpu
        Wr = rotate_rows_gpu(nat.to_gpu(tensor), config.rot_size if config.rot_size > 0 else 1)
    else:
        Wr = W_work          # nothing was zeroed: the same rotated weights
    h = nat.to_gpu(h).float()
    if h.shape[0] < Wr.shape[1]:
        h = torch.nn.functional.pad(h, (0, Wr.shape[1] - h.shape[0]))
    try:
        if config.int_bits == 8:
            res = (_piso_mod.compute_piso_scales_int8(Wr, h), None)
        else:
            res = _piso_mod.compute_piso_scales_int4_asymmetric(Wr, h)
    except (ValueError, torch.cuda.OutOfMemoryError) as exc:
        logger.warning("PiSO failed for %s: %s", layer_name, exc)
        return None
    state["piso"] += 1
    if res[1] is not None:
        state["piso_zp"] += 1
    return res


def quantize_layer(name: str, tensor: torch.Tensor, config: QuantizeConfig, calibration, name_map,
                   state: dict) -> _layer.LayerOutput:
    """One layer of the pipeline loop on the GPU; ``state`` carries counters and
    one-time warnings across layers."""
    is_int8 = config.int_bits == 8
    W_work, nz = _layer.prepare_weights(tensor, config.rot_size)
    outliers = int(nz.item())
    if outliers:
        logger.warning("Zeroed %d outlier weight values in %s (|W| > %.0f)", outliers, name, 1000.0)
    fallbacks: list[str] = []
    packed = None
    piso = None
    if config.piso_scales and calibration is not None:
        piso = _piso(name, tensor, W_work, outliers, config, calibration, name_map, state)
    perm, perm_from_cal = None, False
    if config.use_permuquant:
        perm, perm_from_cal = _permuquant(name, W_work, tensor.shape[1], config, calibration, name_map, state)
    if config.quant_method in ("gptq", "ldlq"):
        layer_name = name_map.get(name) if name_map else None
        hessian = None
        if layer_name is not None and calibration is not None:
            hessian = get_hessian(calibration, layer_name, tensor.shape, device=nat.device())
        rot_h = 0
        if hessian is not None:
            md = calibration.get("metadata", {}) or {}
            already = md.get("hessian_rotated", False)
            cal_rot = md.get("rot_size", 0)
            if already and cal_rot and int(cal_rot) != config.rot_size and not state.get("rot_warned"):
                logger.warning("Calibration rot_size=%s != converter rot_size=%d. Hessian is in the wrong "
                               "rotation space.", cal_rot, config.rot_size)
                state["rot_warned"] = True
            if not already and config.rot_size > 0:
                rot_h = config.rot_size
            if is_dlr(hessian) and rot_h:
                # rotation densifies a DLR Hessian (rotation.py:181-184)
                from .dlr import dlr_to_dense
                from .rotation import rotate_hessian_gpu
                hessian = rotate_hessian_gpu(dlr_to_dense(hessian["D"], hessian["U"]), rot_h)
                rot_h = 0
            if perm is not None and not perm_from_cal:
                # re-permute the Hessian for a self-computed permutation (pipeline.py:728-756)
                from . import permuquant as _pq
                from .rotation import rotate_hessian_gpu
                if is_dlr(hessian):
                    from .dlr import make_dlr_dict, permute_dlr
                    hessian = make_dlr_dict(*permute_dlr(hessian["D"], hessian["U"], perm))
                elif hessian.dim() == 2:
                    Hg = nat.to_gpu(hessian).float()
                    if rot_h:
                        Hg = rotate_hessian_gpu(Hg, rot_h)
                        rot_h = 0
                    hessian = _pq.permute_hessian(Hg, perm)
                else:
                    # a block-diagonal Hessian cannot be permuted: undo W_work's permutation
                    of = min(tensor.shape[1], perm.numel())
                    inv = torch.empty_like(perm)
                    inv[perm] = torch.arange(perm.numel(), device=perm.device)
                    W_work[:, :of] = _pq.permute_columns(W_work[:, :of], inv[:of])
                    perm = None   # no <name>_perm; the layer stays counted as permuted, like the reference
                    logger.debug("PermuQuant: un-permuted W_work for block-diagonal Hessian for %s (%dD, shape %s)",
                                 name, hessian.dim(), tuple(hessian.shape))
    if config.quant_method == "gptq":
        if hessian is not None:
            codes, s16, z8 = _layer.gptq_codes(
                W_work, hessian, rotate_h=rot_h, block_size=config.gptq_block_size, damping=config.damping,
                int_bits=config.int_bits, asymmetric=config.asymmetric, hessian_method=config.hessian_method,
                fallbacks=fallbacks, piso=piso)
            method = "gptq_hip"
            state["gptq"] += 1
        else:
            r = None
            if piso is not None:
                from .piso import rtn_piso_codes
                r = rtn_piso_codes(W_work, piso[0], piso[1], config.int_bits, config.asymmetric,
                                   config.clipping_ratios)
            if r is not None:
                codes, s16, z8, packed = r
                method = "rtn_piso"
            else:
                codes, s16, z8, packed = _layer.rtn_codes(W_work, config.int_bits, config.asymmetric,
                                                          config.clipping_ratios)
                method = "rtn"
            state["rtn_fallback"] += 1
            logger.debug("No calibration data, using RTN fallback")
    elif config.quant_method == "ldlq":
        from .ldlq import ldlq_quantize_layer
        H = None
        if is_dlr(hessian):
            H = hessian
        elif hessian is not None:
            from .rotation import rotate_hessian_gpu
            H = nat.to_gpu(hessian).float()
            if rot_h:
                H = rotate_hessian_gpu(H, rot_h)
        r = ldlq_quantize_layer(W_work, hessian=H, block_size=config.gptq_block_size, damping=config.damping,
                                int_bits=config.int_bits, iterations=config.ldlq_iterations,
                                greedy_passes=config.greedy_passes, rank_threshold=config.rank_threshold)
        codes, s16, z8 = r.quantized_W, r.scales, r.zero_points
        method = r.method_used
        fallbacks.extend(r.fallbacks)
        state["gptq"] += 1
    else:
        codes, s16, z8, packed = _layer.rtn_codes(W_work, config.int_bits, config.asymmetric,
                                                  config.clipping_ratios)
        method = "rtn"
    out = _layer.finish(W_work, codes, s16, z8, config.int_bits, packed=packed, method=method,
                        fallbacks=fallbacks, outliers=outliers)
    out.perm = perm
    if out.bad_scales:
        logger.warning("Replaced bad scale values in %s (Inf/NaN/zero); quality may be degraded", name)
    return out


class _MemoryIO:
    """The reference's own I/O: the whole state dict in host memory, every
    output gathered and written by one save_file at the end."""

    def __init__(self, path: str):
        self.state_dict = load_file(path)
        self.output: dict[str, torch.Tensor] = {}

    def shapes(self):
        return {n: tuple(t.shape) for n, t in self.state_dict.items()}

    def nbytes(self, name):
        t = self.state_dict[name]
        return t.numel() * t.element_size()

    def tensor(self, name):
        return self.state_dict[name]

    def passthrough(self, name):
        self.output[name] = self.state_dict[name]

    def emit(self, name, t):
        self.output[name] = t.cpu()

    def finish(self, path, metadata):
        output = {k: v.contiguous() for k, v in self.output.items()}
        save_file(output, path, metadata=metadata)
        return sum(t.numel() * t.element_size() for t in output.values())

    def abort(self):
        pass


class _StreamIO:
    """Streaming I/O: layers read from the file on a host thread and copied to
    the GPU one layer ahead; results copied back and appended to the output
    file as they are produced; other tensors copied file to file."""

    def __init__(self, path: str, quantized: list[str], device):
        from .streaming import Prefetcher, SafetensorsIndex
        self.index = SafetensorsIndex(path)
        self.device = device
        self.quantized = quantized
        self.prefetch = None
        self.writer = None

    def start(self, out_path: str, metadata: dict):
        from .streaming import Prefetcher, StreamWriter, header_reserve
        self.writer = StreamWriter(out_path, header_reserve(self.index, metadata), self.device)
        self.prefetch = Prefetcher(self.index, self.quantized, self.device)

    def shapes(self):
        return {n: e[1] for n, e in self.index.entries.items()}

    def nbytes(self, name):
        return self.index.nbytes(name)

    def tensor(self, name):
        return self.prefetch.get(name)

    def passthrough(self, name):
        self.writer.add_file_copy(name, self.index)

    def emit(self, name, t):
        if t.is_cuda:
            self.writer.add_device(name, t)
        else:
            self.writer.add_host(name, t)

    def finish(self, path, metadata):
        self.prefetch.close()
        self.writer.close(metadata)
        return self.writer.offset

    def abort(self):
        if self.prefetch is not None:
            self.prefetch.close()
        if self.writer is not None:
            self.writer.abort()


def quantize_model(config: QuantizeConfig, *, progress_callback: ProgressCallback | None = None,
                   streaming: bool = True) -> None:
    """Quantise every 2-D, non-skipped tensor of ``config.input_path`` and write
    ``<output_dir>/model.safetensors`` (reference pipeline.py:150-1179).

    ``streaming`` (default) reads and writes the file layer by layer with the
    host<->device copies overlapped with the GPU work; False keeps the
    reference's load-everything / save-once I/O (same output tensors and
    metadata)."""
    skip_patterns = config.skip_patterns if config.skip_patterns is not None else DEFAULT_SKIP_PATTERNS
    if config.exclude_patterns:
        skip_patterns = list(skip_patterns) + config.exclude_patterns
        logger.info("Excluding additional patterns: %s", config.exclude_patterns)
    config = _validate(config)
    is_int8 = config.int_bits == 8
    if config.seed >= 0:
        torch.manual_seed(config.seed)
        if torch.cuda.is_available():
            torch.cuda.manual_seed_all(config.seed)
    os.makedirs(config.output_dir, exist_ok=True)

    logger.info("Loading %s...", config.input_path)
    if streaming:
        from .streaming import SafetensorsIndex
        idx = SafetensorsIndex(config.input_path)
        shapes = {n: e[1] for n, e in idx.entries.items()}
        todo = [n for n, sh in shapes.items() if not should_skip(n, skip_patterns) and len(sh) == 2]
        io = _StreamIO(config.input_path, todo, nat.device())
    else:
        io = _MemoryIO(config.input_path)
        shapes = io.shapes()
    names = list(shapes)
    logger.info("Loaded %d tensors", len(names))

    calibration, name_map = None, {}
    if config.quant_method in ("gptq", "ldlq") and config.calibration_path:
        logger.info("Loading calibration from %s...", config.calibration_path)
        calibration = load_calibration(config.calibration_path)
        cal_keys = list(calibration["hessians"].keys())
        name_map = build_name_map(names, cal_keys)
        logger.info("Matched %d/%d calibration layers to model layers", len(name_map), len(cal_keys))

    metadata = _metadata(config, shapes, skip_patterns)
    piso_on = config.piso_scales and calibration is not None
    if piso_on:
        # the counts are known at the end; these placeholders size the
        # streaming writer's header reservation
        n2d = str(sum(1 for sh in shapes.values() if len(sh) == 2))
        metadata.update({"int_crush.piso": "true", "int_crush.piso_layers": n2d, "int_crush.piso_zero_points": n2d})
    path = os.path.join(config.output_dir, "model.safetensors")
    if streaming:
        io.start(path, metadata)
    state = {"gptq": 0, "rtn_fallback": 0, "permuted": 0, "piso": 0, "piso_zp": 0}
    skipped = quantized = 0
    reports: list[dict] = []
    total = sum(1 for n, sh in shapes.items() if not should_skip(n, skip_patterns) and len(sh) == 2)
    t0 = time.monotonic() if progress_callback is not None else None
    written: set[str] = set()

    try:
        for name in names:
            if should_skip(name, skip_patterns) or len(shapes[name]) != 2:
                if name not in written:      # a bias may have gone out with its weight already
                    io.passthrough(name)
                    written.add(name)
                skipped += 1
                continue
            logger.info("Quantizing %s (%s)...", name, tuple(shapes[name]))
            out = quantize_layer(name, io.tensor(name), config, calibration, name_map, state)
            logger.debug("MSE=%.6f  max_err=%.4f", out.mse, out.max_err)
            if config.quality_report_path is not None:
                fb = list(out.fallbacks) + (["scale_repair"] if out.bad_scales else [])
                reports.append({
                    "name": name, "method": out.method, "mse": out.mse, "max_err": out.max_err,
                    "scale_range": [out.scales.min().item(), out.scales.max().item()],
                    "fallbacks": fb, "shape": list(shapes[name]), "smoothquant": False, "smoothrot": False,
                    "smooth_source": None, "svd_rank": 0,
                })
            io.emit(name, out.stored)
            io.emit(f"{name}_scale", out.scales)
            if out.zero_points is not None:
                io.emit(f"{name}_zp", out.zero_points)
            if is_int8 and config.comfy_int8_fast:
                k, v = _comfy_tensor(name, config, fmt=False)
                io.emit(k, v)
            if is_int8 and config.comfy_compat:
                k, v = _comfy_tensor(name, config, fmt=True)
                io.emit(k, v)
            if out.perm is not None:
                io.emit(f"{name}_perm", out.perm.to(torch.int32))
            written.add(name)
            quantized += 1
            if progress_callback is not None:
                elapsed = time.monotonic() - t0
                remaining = elapsed / quantized * (total - quantized) if quantized > 1 else 0.0
                progress_callback(ProgressInfo(
                    current_layer=quantized, total_layers=total, layer_name=name, layer_shape=tuple(shapes[name]),
                    elapsed_seconds=elapsed, estimated_remaining_seconds=max(remaining, 0.0), method=out.method,
                    mse=out.mse))
            if name.endswith(".weight"):
                bias = name[: -len(".weight")] + ".bias"
                if bias in shapes and bias not in written:
                    io.passthrough(bias)
                    written.add(bias)
        if piso_on:
            # pipeline.py:462-466
            for k in ("int_crush.piso", "int_crush.piso_layers", "int_crush.piso_zero_points"):
                metadata.pop(k)
            if state["piso"]:
                metadata["int_crush.piso"] = "true"
                metadata["int_crush.piso_layers"] = str(state["piso"])
                if state["piso_zp"]:
                    metadata["int_crush.piso_zero_points"] = str(state["piso_zp"])
        logger.info("Saving to %s...", path)
        out_bytes = io.finish(path, metadata)
    except BaseException:
        io.abort()
        raise

    in_gb = sum(io.nbytes(n) for n in names) / (1024 ** 3)
    out_gb = out_bytes / (1024 ** 3)
    ratio = in_gb / out_gb if out_gb else 0.0
    logger.info("Done! Quantized %d layers, skipped %d layers", quantized, skipped)
    if config.quant_method in ("gptq", "ldlq"):
        logger.info("%s: %d layers, RTN fallback: %d layers", config.quant_method.upper(), state["gptq"],
                    state["rtn_fallback"])
    logger.info("Input size: %.2f GB", in_gb)
    logger.info("Output size: %.2f GB", out_gb)
    logger.info("Compression ratio: %.2fx", ratio)
    if progress_callback is not None:
        progress_callback(ProgressSummary(
            total_layers=quantized, skipped_layers=skipped, permuted_layers=state["permuted"], gptq_layers=state["gptq"],
            rtn_fallback_layers=state["rtn_fallback"], smoothquant_layers=0, svd_layers=0,
            elapsed_seconds=time.monotonic() - t0, input_size_gb=round(in_gb, 2), output_size_gb=round(out_gb, 2),
            compression_ratio=round(ratio, 2)))
    if config.quality_report_path is not None:
        report = {"layers": reports, "summary": {
            "total_layers": quantized + skipped, "quantized": quantized, "skipped": skipped,
            "input_gb": round(in_gb, 2), "output_gb": round(out_gb, 2), "compression_ratio": round(ratio, 2)}}
        os.makedirs(os.path.dirname(os.path.abspath(config.quality_report_path)), exist_ok=True)
        with open(config.quality_report_path, "w") as f:
            json.dump(report, f, indent=2)
        logger.info("Quality report written to %s", config.quality_report_path)
