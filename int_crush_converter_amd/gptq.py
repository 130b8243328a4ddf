"""GPTQ layer quantisation (API of ``converter/gptq.py``).

``gptq_quantize_layer`` runs entirely on the GPU: row statistics and the
per-row scale / zero-point (``ic_row_stats`` + ``ic_gptq_row_params``), the
damped Hessian inverse (``ic_hessian_inverse``), the column sweep with its
fp32-MFMA lazy trailing update (``ic_gptq_quantize``) and the error metrics
(``ic_quant_error``).  Results are returned on the device of ``W``.
"""

from __future__ import annotations

import torch

from . import _native as nat
from .dlr import is_dlr, woodbury_inverse
from .hessian import inverse_batch
from .log import logger
from .types import QuantizationResult
from . import scales as _scales

_HESSIAN_METHODS = {"hinv": "hinv", "cholesky": "cholesky"}

SWEEP_MAX_BLOCK = 128


def row_params(W: torch.Tensor, int_bits: int, asymmetric: bool):
    """fp32 GPU W [M, N] -> (s32 [M], z32 [M] or None, s16 [M] fp16, z8 [M] int8 or None)
    following converter/gptq.py:254-317."""
    M, N = W.shape
    dev = W.device
    L = nat.lib()
    asym = int_bits == 4 or asymmetric
    rmin = torch.empty(M, dtype=torch.float32, device=dev)
    rmax = torch.empty(M, dtype=torch.float32, device=dev)
    ramax = torch.empty(M, dtype=torch.float32, device=dev)
    nat.check(L.ic_row_stats(W, M, N, N, rmin, rmax, ramax,
                             nat.stream()), "ic_row_stats")
    s32 = torch.empty(M, dtype=torch.float32, device=dev)
    s16 = torch.empty(M, dtype=torch.float16, device=dev)
    z32 = torch.empty(M, dtype=torch.float32, device=dev) if asym else None
    z8 = torch.empty(M, dtype=torch.int8, device=dev) if asym else None
    nat.check(L.ic_gptq_row_params(rmin, rmax, ramax, M, int_bits, int(asym),
                                   s32, nat.ptr(z32), s16, nat.ptr(z8), nat.stream()),
              "ic_gptq_row_params")
    return s32, z32, s16, z8


def scale_operand(scale: torch.Tensor) -> tuple[torch.Tensor, int]:
    """Scales as the ABI reads them: contiguous fp16 (kind 0) or fp32 (kind 1)."""
    if scale.dtype == torch.float16:
        return scale.reshape(-1).contiguous(), 0
    return scale.reshape(-1).float().contiguous(), 1


def launch_quant_error(W: torch.Tensor, Q: torch.Tensor, scale: torch.Tensor, zp8: torch.Tensor | None,
                       sumsq_ptr: int, max_ptr: int) -> None:
    """Enqueue ``ic_quant_error``: the fp64 sum of squared errors of
    (Q - zp) * scale against W goes to ``sumsq_ptr`` and the max |error| (fp32)
    to ``max_ptr`` (device addresses); nothing is synchronised."""
    M, N = W.shape
    ws = nat.workspace(nat.lib().ic_quant_error_workspace_bytes(), W.device)
    sc, kind = scale_operand(scale)
    zp = None if zp8 is None else zp8.reshape(-1).to(torch.int8).contiguous()
    nat.check(nat.lib().ic_quant_error(W, M, N, N, Q, N, sc, kind, nat.ptr(zp),
                                       sumsq_ptr, max_ptr, ws, nat.stream()),
              "ic_quant_error")


def quant_error(W: torch.Tensor, Q: torch.Tensor, scale: torch.Tensor, zp8: torch.Tensor | None):
    """(mse, max_err) of (Q - zp) * scale against W, scale fp16 or fp32 [M]."""
    if W.numel() == 0:
        return float("nan"), 0.0
    out = torch.zeros(2, dtype=torch.float64, device=W.device)
    launch_quant_error(W, Q, scale, zp8, out.data_ptr(), out.data_ptr() + 8)
    host = out.cpu()
    return host[0].item() / W.numel(), host[1:].view(torch.float32)[0].item()


def sweep(W_work: torch.Tensor, Hinv: torch.Tensor, s32: torch.Tensor, z32: torch.Tensor | None,
          int_bits: int, block_size: int, groups: int = 1) -> torch.Tensor:
    """Run the GPTQ sweep on W_work [M, groups*gw] (contiguous fp32, left
    unchanged: the working residual lives in a buffer of the same size that
    the library fills without copying W_work); Hinv [gw, gw] or
    [groups, gw, gw].  Returns int8 codes [M, groups*gw]."""
    M, N = W_work.shape
    gw = N // groups
    Q = torch.empty(M, N, dtype=torch.int8, device=W_work.device)
    R = torch.empty_like(W_work)
    blk = min(int(block_size), SWEEP_MAX_BLOCK)
    ws = nat.workspace(nat.lib().ic_gptq_workspace_bytes(M, groups, blk), W_work.device)
    nat.check(nat.lib().ic_gptq_quantize_from(W_work, R, M, gw, groups, Hinv,
                                              s32, nat.ptr(z32), int_bits, blk, Q,
                                              ws, nat.stream()),
              "ic_gptq_quantize_from")
    return Q


def block_cover(N: int, nblk: int, bs: int) -> tuple[int, int]:
    """(whole blocks swept as one batch, width of the partial block after
    them) for a 3-D Hessian [nblk, bs, bs] over N columns.  Follows the
    reference's loop over the Hessian's blocks (gptq.py:345-366): block b
    covers columns [b bs, min((b + 1) bs, N)); blocks past column N do
    nothing, and columns past the last block are not swept (their codes stay
    0, as quantized_W = zeros_like(W) leaves them)."""
    full = min(N // bs, nblk) if bs > 0 else 0
    rem = min(bs, N - full * bs) if full < nblk else 0
    return full, rem


def sweep_block_diagonal(W_work: torch.Tensor, Hg: torch.Tensor, damping: float, hessian_method: str,
                         fallbacks: list[str], s32, z32, int_bits: int, block_size: int) -> torch.Tensor:
    """GPTQ over a block-diagonal 3-D Hessian: the whole blocks inverted as a
    batch and swept as independent column groups of one launch, the partial
    last block on its own.  W_work is left unchanged;
    returns int8 codes."""
    M, N = W_work.shape
    nblk, bs, _ = Hg.shape
    full, rem = block_cover(N, nblk, bs)
    Q = torch.zeros(M, N, dtype=torch.int8, device=W_work.device)
    if full > 0:
        Hinv = inverse_batch(Hg[:full].float(), damping, hessian_method, fallbacks, upper_only=True)
        Q[:, :full * bs] = sweep(W_work[:, :full * bs].contiguous(), Hinv, s32, z32, int_bits, block_size,
                                 groups=full)
    if rem > 0:
        c0 = full * bs
        Hinv = inverse_batch(Hg[full, :rem, :rem].float(), damping, hessian_method, fallbacks, upper_only=True)
        Q[:, c0:c0 + rem] = sweep(W_work[:, c0:c0 + rem].contiguous(), Hinv, s32, z32, int_bits, block_size)
    return Q


def gptq_quantize_layer(
    W: torch.Tensor,
    hessian: torch.Tensor,
    block_size: int = 128,
    damping: float = 0.01,
    int_bits: int = 4,
    asymmetric: bool = False,
    hessian_method: str = "hinv",
    piso_scales: torch.Tensor | None = None,
    piso_zero_points: torch.Tensor | None = None,
) -> QuantizationResult:
    """GPTQ with per-row scales (INT4 always asymmetric), 2-D, 3-D or DLR
    Hessian (reference gptq.py:137-417).  ``block_size`` above 128 is run as 128-column
    sweeps, which is the same update in exact arithmetic."""
    if int_bits not in (4, 8):
        raise ValueError(f"int_bits must be 4 or 8, got {int_bits}")
    if W.dim() != 2:
        raise ValueError(f"Expected 2D weight tensor, got {W.dim()}D")
    if hessian_method not in _HESSIAN_METHODS:
        raise ValueError(f"hessian_method must be one of {list(_HESSIAN_METHODS)}, got '{hessian_method}'")
    out_dev = W.device
    Wg = nat.to_gpu(W).float().contiguous()
    M, N = Wg.shape
    fallbacks: list[str] = []
    params = None
    if piso_scales is not None:
        from .piso import piso_row_params
        params = piso_row_params(Wg, piso_scales, piso_zero_points, int_bits, asymmetric)
    s32, z32, s16, z8 = params if params is not None else row_params(Wg, int_bits, asymmetric)
    W_work = Wg.contiguous()   # the sweep leaves it unchanged
    Hg = hessian if isinstance(hessian, dict) else nat.to_gpu(hessian)

    if is_dlr(Hg):
        # Woodbury H^-1, then the 2-D sweep on it directly (gptq.py:322-342:
        # the DLR branch hands the inverse itself to the column loop, without
        # the Cholesky step of hessian_method "cholesky")
        D, U = Hg["D"], Hg["U"]
        if D.shape[0] != N:
            raise ValueError(f"DLR Hessian dim {D.shape[0]} != in_features {N}")
        Hinv = woodbury_inverse(D, U, damping, Wg.device, upper_only=True)
        Q = sweep(W_work, Hinv, s32, z32, int_bits, block_size)
    elif isinstance(Hg, dict):
        raise ValueError(f"Expected 2D tensor, 3D tensor, or DLR dict Hessian, got {type(hessian).__name__}")
    elif Hg.dim() == 3:
        Q = sweep_block_diagonal(W_work, Hg, damping, hessian_method, fallbacks, s32, z32, int_bits, block_size)
    elif Hg.dim() == 2:
        if tuple(Hg.shape) != (N, N):
            raise ValueError(f"Hessian shape {hessian.shape} != ({N}, {N})")
        Hf = Hg.float().contiguous()
        if Hf.data_ptr() != hessian.data_ptr():
            # our own copy (moved to the GPU or converted): invert it in place
            Hinv = inverse_batch(Hf, damping, hessian_method, fallbacks, inplace=True,
                                 restore=lambda: nat.to_gpu(hessian).float().contiguous(), upper_only=True)
        else:
            Hinv = inverse_batch(Hf, damping, hessian_method, fallbacks, upper_only=True)
        Q = sweep(W_work, Hinv, s32, z32, int_bits, block_size)
    else:
        raise ValueError(
            f"Expected 2D tensor, 3D tensor, or DLR dict Hessian, got {type(hessian).__name__}")

    logger.debug("GPTQ: HIP path, %dx%d, block_size=%d", M, N, block_size)
    mse, max_err = quant_error(Wg, Q, s32, z8)
    return QuantizationResult(
        quantized_W=Q.to(out_dev),
        scales=s16.reshape(M, 1).to(out_dev),
        zero_points=None if z8 is None else z8.reshape(M, 1).to(out_dev),
        mse=mse,
        max_err=max_err,
        method_used="gptq_hip",
        fallbacks=fallbacks,
    )


def gptq_quantize_layer_rtn(
    W: torch.Tensor,
    int_bits: int = 4,
    asymmetric: bool = False,
    clipping_ratios: list[float] | None = None,
    piso_scales: torch.Tensor | None = None,
    piso_zero_points: torch.Tensor | None = None,
) -> QuantizationResult:
    """Round-to-nearest fallback used when no Hessian is available
    (reference gptq.py:420-533)."""
    if int_bits not in (4, 8):
        raise ValueError(f"int_bits must be 4 or 8, got {int_bits}")
    out_dev = W.device
    Wg = nat.to_gpu(W).float().contiguous()
    N = Wg.shape[1]
    if piso_scales is not None:
        from .piso import rtn_piso_codes
        r = rtn_piso_codes(Wg, piso_scales, piso_zero_points, int_bits, asymmetric, clipping_ratios)
        if r is not None:
            q, s, z, _ = r
            mse, max_err = quant_error(Wg, q, s, z)
            return QuantizationResult(
                quantized_W=q.to(out_dev), scales=s.to(out_dev), zero_points=None if z is None else z.to(out_dev),
                mse=mse, max_err=max_err, method_used="rtn_piso", fallbacks=[])
    zps = None
    if asymmetric:
        if int_bits == 8:
            scales, zps = _scales.calculate_scales_int8_asymmetric(Wg, clipping_ratios=clipping_ratios)
            q = _scales.quantize_weights_int8_asymmetric(Wg, scales, zps)
        else:
            scales, zps = _scales.calculate_scales_asymmetric(Wg, N, clipping_ratios=clipping_ratios)
            q = _scales.quantize_weights_asymmetric(Wg, scales, zps, N)
    elif int_bits == 8:
        scales = _scales.calculate_scales_int8(Wg, clipping_ratios=clipping_ratios)
        q = _scales.quantize_weights_int8(Wg, scales)
    else:
        scales = _scales.calculate_scales(Wg, N, clipping_ratios=clipping_ratios)
        q = _scales.quantize_weights(Wg, scales, N)
    mse, max_err = quant_error(Wg, q, scales, zps)
    return QuantizationResult(
        quantized_W=q.to(out_dev), scales=scales.to(out_dev),
        zero_points=None if zps is None else zps.to(out_dev),
        mse=mse, max_err=max_err, method_used="rtn", fallbacks=[])
