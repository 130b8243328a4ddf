"""RTN scales, zero-points and quantisation (API of ``converter/scales.py``).

All arithmetic runs in the HIP library: ``ic_rtn_scales`` (row statistics,
closed-form scale / zero-point, zero-point clamp fix, clipping-ratio search)
and ``ic_rtn_quantize`` (round-half-away-from-zero codes).  Group-wise
variants lay each group of ``group_size`` columns out as one row.  Inputs
are computed in fp32 whatever their dtype; outputs match the reference's
dtypes (fp16 scales, int8 zero-points and codes) and are returned on the
input's device.
"""

from __future__ import annotations

import ctypes

import torch
import torch.nn.functional as F

from . import _native as nat
from .config import SCALE_DTYPE


def _ratios(clipping_ratios):
    if clipping_ratios is not None and len(clipping_ratios) == 0:
        return None
    if clipping_ratios is not None and len(clipping_ratios) > 16:
        raise ValueError("at most 16 clipping ratios are supported")
    return clipping_ratios


def _grouped(W: torch.Tensor, group_size: int) -> torch.Tensor:
    """fp32 GPU copy of W padded to a multiple of group_size, as [M*G, gs]."""
    W = nat.to_gpu(W).float()
    if W.shape[1] % group_size:
        W = F.pad(W, (0, group_size - W.shape[1] % group_size))
    return W.contiguous().reshape(-1, group_size)


def _scales_rows(Wr: torch.Tensor, bits: int, asym: bool, ratios):
    rows, cols = Wr.shape
    s16 = torch.empty(rows, dtype=torch.float16, device=Wr.device)
    zp = torch.empty(rows, dtype=torch.int8, device=Wr.device) if asym else None
    if ratios:
        arr = (ctypes.c_float * len(ratios))(*[float(r) for r in ratios])
        rp, nr = arr, len(ratios)
    else:
        rp, nr = None, 0
    nat.check(nat.lib().ic_rtn_scales(Wr, rows, cols, cols, bits, int(asym), rp, nr,
                                      s16, nat.ptr(zp), nat.stream()), "ic_rtn_scales")
    return s16, zp


def _quant_rows(Wr: torch.Tensor, bits: int, scales: torch.Tensor, zps: torch.Tensor | None,
                packed: bool = False) -> torch.Tensor:
    rows, cols = Wr.shape
    sc = scales.reshape(-1)
    if sc.dtype == torch.float16:
        kind = 0
    else:
        sc, kind = sc.float(), 1
    sc = sc.contiguous()
    z = None if zps is None else zps.reshape(-1).float().contiguous()
    if sc.numel() != rows or (z is not None and z.numel() != rows):
        raise ValueError("scales / zero_points do not match the number of rows or groups")
    if packed:
        out = torch.empty(rows, (cols + 1) // 2, dtype=torch.uint8, device=Wr.device)
        nat.check(nat.lib().ic_rtn_quantize(Wr, rows, cols, cols, bits, sc, kind,
                                            nat.ptr(z), None, cols, out, out.shape[1], nat.stream()),
                  "ic_rtn_quantize")
    else:
        out = torch.empty(rows, cols, dtype=torch.int8, device=Wr.device)
        nat.check(nat.lib().ic_rtn_quantize(Wr, rows, cols, cols, bits, sc, kind,
                                            nat.ptr(z), out, cols, None, 0, nat.stream()),
                  "ic_rtn_quantize")
    return out


def _check2d(W):
    if W.dim() != 2:
        raise ValueError(f"Expected 2D tensor, got {W.dim()}D")


def calculate_scales(W: torch.Tensor, group_size: int = 128,
                     clipping_ratios: list[float] | None = None) -> torch.Tensor:
    """Symmetric INT4 scales max|W|/7 per group (reference scales.py:62-99)."""
    _check2d(W)
    M = W.shape[0]
    Wr = _grouped(W, group_size)
    s16, _ = _scales_rows(Wr, 4, False, _ratios(clipping_ratios))
    return s16.reshape(M, -1).to(W.device)


def quantize_weights(W: torch.Tensor, scales: torch.Tensor, group_size: int = 128) -> torch.Tensor:
    """INT4 codes in [-8, 7] of shape [out, in_padded] (reference scales.py:102-123)."""
    M = W.shape[0]
    Wr = _grouped(W, group_size)
    q = _quant_rows(Wr, 4, nat.to_gpu(scales), None)
    return q.reshape(M, -1).to(W.device)


def calculate_scales_int8(W: torch.Tensor, clipping_ratios: list[float] | None = None) -> torch.Tensor:
    """Symmetric INT8 per-row scales max|W|/127 (reference scales.py:126-160)."""
    _check2d(W)
    Wr = nat.to_gpu(W).float().contiguous()
    s16, _ = _scales_rows(Wr, 8, False, _ratios(clipping_ratios))
    return s16.reshape(-1, 1).to(W.device)


def quantize_weights_int8(W: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """INT8 codes in [-128, 127] (reference scales.py:163-178)."""
    _check2d(W)
    Wr = nat.to_gpu(W).float().contiguous()
    return _quant_rows(Wr, 8, nat.to_gpu(scales), None).to(W.device)


def calculate_scales_asymmetric(W: torch.Tensor, group_size: int = 128,
                                clipping_ratios: list[float] | None = None
                                ) -> tuple[torch.Tensor, torch.Tensor]:
    """Asymmetric INT4 scales (max-min)/15 and zero-points (reference scales.py:232-282)."""
    _check2d(W)
    M = W.shape[0]
    Wr = _grouped(W, group_size)
    s16, zp = _scales_rows(Wr, 4, True, _ratios(clipping_ratios))
    return s16.reshape(M, -1).to(W.device), zp.reshape(M, -1).to(W.device)


def quantize_weights_asymmetric(W: torch.Tensor, scales: torch.Tensor, zero_points: torch.Tensor,
                                group_size: int = 128) -> torch.Tensor:
    """Asymmetric INT4 codes (reference scales.py:285-313)."""
    M = W.shape[0]
    Wr = _grouped(W, group_size)
    q = _quant_rows(Wr, 4, nat.to_gpu(scales), nat.to_gpu(zero_points))
    return q.reshape(M, -1).to(W.device)


def calculate_scales_int8_asymmetric(W: torch.Tensor, clipping_ratios: list[float] | None = None
                                     ) -> tuple[torch.Tensor, torch.Tensor]:
    """Asymmetric INT8 per-row scales (max-min)/255 and zero-points (reference scales.py:316-361)."""
    _check2d(W)
    Wr = nat.to_gpu(W).float().contiguous()
    s16, zp = _scales_rows(Wr, 8, True, _ratios(clipping_ratios))
    return s16.reshape(-1, 1).to(W.device), zp.reshape(-1, 1).to(W.device)


def quantize_weights_int8_asymmetric(W: torch.Tensor, scales: torch.Tensor,
                                     zero_points: torch.Tensor) -> torch.Tensor:
    """Asymmetric INT8 codes (reference scales.py:364-384)."""
    _check2d(W)
    Wr = nat.to_gpu(W).float().contiguous()
    return _quant_rows(Wr, 8, nat.to_gpu(scales), nat.to_gpu(zero_points)).to(W.device)


__all__ = [
    "calculate_scales", "quantize_weights", "calculate_scales_int8", "quantize_weights_int8",
    "calculate_scales_asymmetric", "quantize_weights_asymmetric",
    "calculate_scales_int8_asymmetric", "quantize_weights_int8_asymmetric", "SCALE_DTYPE",
]
