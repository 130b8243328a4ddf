"""PiSO: per-row scales that minimise the Hessian-diagonal-weighted
quantisation error (API of ``converter/piso.py``).

One HIP kernel (``ic_piso_scales``) runs the reference's coarse-to-fine grid
search for every row on the GPU, summing each candidate's error in the
order the reference's PyTorch path uses, so the scales (and zero-points)
are that path's bit for bit.  Results are returned on the device of ``W``.
"""

from __future__ import annotations

import torch

from . import _native as nat

_COARSE_SYM = (0.5, 2.0)          # piso.py:62
_COARSE_INT8_ASYM = (0.8, 1.2)    # piso.py:255-258
_COARSE_INT4_ASYM = (0.5, 2.0)    # piso.py:404-407
_FINE = (0.95, 1.05)              # piso.py:63, 137


def _factors(lo: float, hi: float, n: int, device) -> torch.Tensor:
    # the reference builds its factor tables with torch.linspace; the CPU
    # path's values are taken as they are
    return torch.linspace(lo, hi, n, dtype=torch.float32).to(device)


def _check(W: torch.Tensor, hessian_diag: torch.Tensor, num_coarse: int, num_fine: int) -> torch.Tensor:
    if W.dim() != 2:
        raise ValueError(f"Expected 2D tensor, got {W.dim()}D")
    in_features = W.shape[1]
    h = hessian_diag.float()[:in_features]
    if h.shape[0] != in_features:
        raise ValueError(f"hessian_diag length {h.shape[0]} != in_features {in_features}")
    if not (1 <= num_coarse <= 1024 and 1 <= num_fine <= 1024):
        raise ValueError(f"num_coarse and num_fine must be in [1, 1024], got {num_coarse} and {num_fine}")
    return h


def _search(W, hessian_diag, num_coarse, num_fine, bits, asym, coarse):
    h = _check(W, hessian_diag, num_coarse, num_fine)
    out_dev = W.device
    Wg = nat.to_gpu(W).float()
    if Wg.stride(1) != 1:
        Wg = Wg.contiguous()
    M, N = Wg.shape
    dev = Wg.device
    hg = nat.to_gpu(h).contiguous()
    cf = _factors(*coarse, num_coarse, dev)
    ff = _factors(*_FINE, num_fine, dev)
    scales = torch.empty(M, dtype=torch.float32, device=dev)
    zp = torch.empty(M, dtype=torch.int8, device=dev) if asym else None
    if M and N:
        nat.check(nat.lib().ic_piso_scales(Wg, M, N, Wg.stride(0), hg, bits, int(asym),
                                           cf, num_coarse, ff, num_fine, scales,
                                           nat.ptr(zp), nat.stream()), "ic_piso_scales")
    elif M:
        raise ValueError("PiSO needs at least one input feature")
    scales = scales.reshape(M, 1).to(out_dev)
    return scales if not asym else (scales, zp.reshape(M, 1).to(out_dev))


def compute_piso_scales_int8(W: torch.Tensor, hessian_diag: torch.Tensor, num_coarse: int = 128,
                             num_fine: int = 16) -> torch.Tensor:
    """Symmetric INT8 scales [M, 1] fp32 (piso.py:190-233): candidates
    0.5-2.0 x absmax / 127, then 0.95-1.05 x the coarse winner."""
    return _search(W, hessian_diag, num_coarse, num_fine, 8, False, _COARSE_SYM)


def compute_piso_scales_int8_asymmetric(W: torch.Tensor, hessian_diag: torch.Tensor, num_coarse: int = 128,
                                        num_fine: int = 16):
    """Asymmetric INT8 (scales [M, 1] fp32, zero-points [M, 1] int8)
    (piso.py:236-282): candidates 0.8-1.2 x range / 255."""
    return _search(W, hessian_diag, num_coarse, num_fine, 8, True, _COARSE_INT8_ASYM)


def compute_piso_scales_int4(W: torch.Tensor, hessian_diag: torch.Tensor, num_coarse: int = 128,
                             num_fine: int = 16) -> torch.Tensor:
    """Symmetric INT4 scales [M, 1] fp32 (piso.py:290-332): absmax / 7."""
    return _search(W, hessian_diag, num_coarse, num_fine, 4, False, _COARSE_SYM)


def compute_piso_scales_int4_asymmetric(W: torch.Tensor, hessian_diag: torch.Tensor, num_coarse: int = 128,
                                        num_fine: int = 16):
    """Asymmetric INT4 (scales, zero-points) (piso.py:335-408): candidates
    0.5-2.0 x range / 15."""
    return _search(W, hessian_diag, num_coarse, num_fine, 4, True, _COARSE_INT4_ASYM)


def piso_row_params(W: torch.Tensor, scales: torch.Tensor, zero_points: torch.Tensor | None, int_bits: int,
                    asymmetric: bool):
    """GPTQ row parameters from PiSO scales (gptq.py:210-252): fp32 scales
    clamped to [1e-5, 65500], INT4 zero-points as given (clamped) or derived
    from the scale with the asymmetric fix-up, INT8 symmetric unless
    ``asymmetric``; all-zero rows get zero-point 0.  Returns (s32 [M],
    z32 [M] or None, s16 [M] fp16, z8 [M] int8 or None), or None (with the
    reference's warning) when the scales are not [M, 1]."""
    from .config import SCALE_MAX, SCALE_MIN
    from .layer import _fix_asym, _rhaz
    from .log import logger
    M = W.shape[0]
    p = scales.float().to(W.device)
    if tuple(p.shape) != (M, 1):
        logger.warning("PiSO scales shape %s != (%d, 1); falling back to default", tuple(p.shape), M)
        return None
    s = p.clamp(min=SCALE_MIN, max=SCALE_MAX)
    wmin = W.amin(dim=1, keepdim=True)
    wmax = W.amax(dim=1, keepdim=True)
    z = None
    if int_bits == 4:
        if zero_points is not None:
            z = zero_points.float().to(W.device).clamp(-8, 7)
        else:
            s = _fix_asym(s, wmin, wmax, -8, 7)
            z = (-8 - _rhaz(wmin / s)).clamp(-8, 7)
    elif asymmetric:
        s = _fix_asym(s, wmin, wmax, -128, 127)
        z = (-128 - _rhaz(wmin / s)).clamp(-128, 127)
    if z is not None:
        z = z.masked_fill((wmin == 0) & (wmax == 0), 0)
    s32 = s.reshape(M).contiguous()
    return (s32, None if z is None else z.reshape(M).contiguous(), s32.to(torch.float16),
            None if z is None else z.reshape(M).to(torch.int8))


def rtn_piso_codes(W: torch.Tensor, scales: torch.Tensor, zero_points: torch.Tensor | None, int_bits: int,
                   asymmetric: bool, clipping_ratios=None):
    """RTN with PiSO scales (gptq.py:446-483): symmetric INT8, or INT4 with
    the PiSO zero-points (else the RTN asymmetric ones).  fp16 scales clamped
    to [1e-5, 65500].  Returns (codes, s16 [M, 1], z8 [M, 1] or None, packed)
    or None when the case does not use PiSO (INT8 asymmetric, wrong shape)."""
    from .config import SCALE_MAX, SCALE_MIN
    from . import scales as _scales
    M, N = W.shape
    p = scales.float().to(W.device)
    if (int_bits == 8 and asymmetric) or p.dim() != 2 or p.shape[0] != M or p.shape[1] != 1:
        return None
    s16 = p.clamp(min=SCALE_MIN, max=SCALE_MAX).to(torch.float16).contiguous()
    z8 = None
    if int_bits == 4:
        if zero_points is not None:
            z8 = zero_points.to(device=W.device, dtype=torch.int8).reshape(M, 1)
        else:
            _, z8 = _scales.calculate_scales_asymmetric(W, N, clipping_ratios=clipping_ratios)
    codes = torch.empty(M, N, dtype=torch.int8, device=W.device)
    packed = torch.empty(M, (N + 1) // 2, dtype=torch.uint8, device=W.device) if int_bits == 4 else None
    z = None if z8 is None else z8.float().contiguous()
    nat.check(nat.lib().ic_rtn_quantize(W, M, N, W.stride(0), int_bits, s16, 0, nat.ptr(z),
                                        codes, N, nat.ptr(packed), packed.shape[1] if packed is not None
                                        else 0, nat.stream()), "ic_rtn_quantize")
    return codes, s16.reshape(M, 1), z8, packed
