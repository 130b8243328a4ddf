"""LDLQ layer quantisation with optional iterative scale refinement and greedy
coordinate descent (API of ``converter/ldlq.py`` and ``converter/greedy.py``).

All array work runs in the HIP library: ``WᵀW`` and the trailing updates on
the fp32 matrix cores, the damped inverse (``ic_hessian_inverse``), the
per-element-scale sweep (``ic_ldlq_quantize``), iteration MSE / scale update
kernels, least-squares row scales and the greedy search (``greedy.py``:
full-rank ``ic_greedy`` or the eigen-truncated ``ic_greedy_lowrank``).
Host code only makes the scalar control decisions of the reference
(convergence, divergence revert, the greedy backend choice).
"""

from __future__ import annotations

import math
import warnings

import torch

from . import _native as nat
from . import greedy as _greedy
from .config import LDLQ_MSE_DIVERGENCE, LDLQ_SCALE_MOMENTUM, CONVERGENCE_EPS, CONVERGENCE_IMPROVEMENT_THRESHOLD
from .dlr import is_dlr, woodbury_inverse
from .gptq import quant_error, SWEEP_MAX_BLOCK
from .hessian import inverse_batch
from .log import logger
from .types import QuantizationResult

_HAS_TRITON = False


def _lib():
    return nat.lib()


def _row_absmax(W):
    M, N = W.shape
    ramax = torch.empty(M, dtype=torch.float32, device=W.device)
    nat.check(_lib().ic_row_stats(W, M, N, N, None, None, ramax, nat.stream()), "ic_row_stats")
    return ramax


def _gemm_tn(W: torch.Tensor, alpha: float) -> torch.Tensor:
    """alpha * W^T W on the matrix cores (fp32; one triangle computed, mirrored)."""
    M, N = W.shape
    C = torch.empty(N, N, dtype=torch.float32, device=W.device)
    nat.check(_lib().ic_gram_tn(W, M, N, N, alpha, C, nat.stream()), "ic_gram_tn")
    return C


def _damp_only(H: torch.Tensor, damping: float) -> torch.Tensor:
    """H + damping * max(mean(diag), 1e-6) * I as a new tensor, by the
    library's damping kernel (ldlq.py:207-209: the damped weight-only H
    that the greedy search uses)."""
    out = H.float().contiguous().clone()
    nat.check(_lib().ic_damp_hessian(out, 1, out.shape[0], float(damping), nat.stream()),
              "ic_damp_hessian")
    return out


def _single_pass(W: torch.Tensor, Hinv: torch.Tensor, S: torch.Tensor, block: int, bits: int) -> torch.Tensor:
    M, N = W.shape
    S = S.contiguous()
    if not bool(torch.isfinite(S).all().item()):
        S = S.clone()
        nat.check(_lib().ic_sanitize_scales(S, S.numel(), nat.stream()), "ic_sanitize_scales")
    W_work = W.clone()
    Q = torch.empty(M, N, dtype=torch.int8, device=W.device)
    blk = min(int(block), SWEEP_MAX_BLOCK)
    ws = nat.workspace(_lib().ic_gptq_workspace_bytes(M, 1, blk), W.device)
    nat.check(_lib().ic_ldlq_quantize(W_work, M, N, Hinv, S, bits, blk,
                                      Q, ws, nat.stream()), "ic_ldlq_quantize")
    return Q


def _mse(W, Q, S) -> float:
    out = torch.zeros(1, dtype=torch.float64, device=W.device)
    ws = nat.workspace(1024 * 8, W.device)
    nat.check(_lib().ic_ldlq_mse(W, Q, S, W.numel(), out,
                                 ws, nat.stream()), "ic_ldlq_mse")
    return out.item() / max(W.numel(), 1)


def _update_scales(W, Q, cur, flat, smin: float, smax: float) -> torch.Tensor:
    lo = max(smin * 0.1, 1e-8)
    hi = smax * 10.0
    out = torch.empty_like(cur)
    nat.check(_lib().ic_ldlq_update_scales(W, Q, cur, flat, W.numel(),
                                           LDLQ_SCALE_MOMENTUM, lo, hi, out, nat.stream()),
              "ic_ldlq_update_scales")
    return out


def _iterative(W, Hinv, flat, iters, block, bits):
    """converter/ldlq.py:479-550."""
    cur = flat.clone()
    if not bool(torch.isfinite(cur).all().item()):
        nat.check(_lib().ic_sanitize_scales(cur, cur.numel(), nat.stream()), "ic_sanitize_scales")
    smin, smax = (v.item() for v in flat.aminmax())
    Qr = None
    prev = float("inf")
    prev_scales = None
    for it in range(iters):
        Qi = _single_pass(W, Hinv, cur, block, bits)
        Qr = Qi
        mse = _mse(W, Qi, cur)
        logger.debug("LDLQ iteration %d/%d: MSE=%.6f", it + 1, iters, mse)
        if not math.isfinite(mse):
            logger.warning("LDLQ: non-finite MSE at iteration %d, reverting", it + 1)
            if prev_scales is not None:
                cur = prev_scales
            break
        if it > 0 and mse > prev * LDLQ_MSE_DIVERGENCE:
            logger.warning("LDLQ: diverged at iteration %d (MSE increased), reverting", it + 1)
            if prev_scales is not None:
                cur = prev_scales
            break
        imp = (prev - mse) / (prev + CONVERGENCE_EPS)
        if it > 0 and imp < CONVERGENCE_IMPROVEMENT_THRESHOLD:
            break
        prev = mse
        if it < iters - 1:
            prev_scales = cur.clone()
            cur = _update_scales(W, Qi, cur, flat, smin, smax)
    return Qr, cur


def _ls_scales(Q, W) -> torch.Tensor:
    M, N = W.shape
    out = torch.empty(M, dtype=torch.float32, device=W.device)
    nat.check(_lib().ic_ls_scales(Q, W, M, N, out, nat.stream()), "ic_ls_scales")
    return out


def greedy_local_search(W: torch.Tensor, Q: torch.Tensor, srow: torch.Tensor, H: torch.Tensor, passes: int,
                        bits: int) -> torch.Tensor:
    """Full-rank greedy coordinate descent on int8 codes (returns new int8 codes)."""
    qmin, qmax = (-128, 127) if bits == 8 else (-8, 7)
    return _greedy.greedy_local_search(W, Q, srow, H, passes, qmin, qmax)


def ldlq_quantize_layer(
    W: torch.Tensor,
    hessian: torch.Tensor | None = None,
    block_size: int = 128,
    damping: float = 0.01,
    int_bits: int = 4,
    iterations: int = 1,
    greedy_passes: int = 0,
    rank_threshold: float = 0.01,
    *,
    greedy_backend: str = "auto",
) -> QuantizationResult:
    """LDLQ with per-element scales (reference ldlq.py:95-279).  Without a
    Hessian, H = WᵀW / M (weight-only).  The greedy search follows the
    reference's GPU backend choice (ldlq.py:602-647): the low-rank search
    when the Hessian's effective rank at ``rank_threshold`` is at most
    min(512, 0.3 N), else the full-rank one; ``greedy_backend="full"``
    always takes the exact full-rank search (the reference's CPU path)."""
    if int_bits not in (4, 8):
        raise ValueError(f"int_bits must be 4 or 8, got {int_bits}")
    if W.dim() != 2:
        raise ValueError(f"Expected 2D weight tensor, got {W.dim()}D")
    out_dev = W.device
    Wg = nat.to_gpu(W).float().contiguous()
    M, N = Wg.shape
    div = 127.0 if int_bits == 8 else 7.0
    fallbacks: list[str] = []

    H_greedy = None
    if is_dlr(hessian):
        # Woodbury H^-1 (ldlq.py:149-158).  The reference keeps no dense H for
        # the greedy search on this branch (it fails there), so greedy passes
        # with a DLR Hessian are refused up front.
        D, U = hessian["D"], hessian["U"]
        if D.shape[0] != N:
            raise ValueError(f"DLR Hessian dim {D.shape[0]} != in_features {N}")
        if greedy_passes > 0:
            raise ValueError("greedy search needs a dense Hessian (DLR given)")
        Hinv = woodbury_inverse(D, U, damping, Wg.device, upper_only=True)
    elif isinstance(hessian, dict):
        raise ValueError("Expected 2D tensor, 3D tensor, or DLR dict Hessian, got dict")
    elif hessian is not None:
        Hg = nat.to_gpu(hessian).float().contiguous()
        if Hg.dim() == 3:
            nblk, bs, _ = Hg.shape
            Hinv = torch.zeros(N, N, dtype=torch.float32, device=Wg.device)
            full = min(N // bs, nblk)
            if full:
                inv = inverse_batch(Hg[:full], damping, "hinv", fallbacks, upper_only=True)
                for b in range(full):
                    Hinv[b * bs:(b + 1) * bs, b * bs:(b + 1) * bs] = inv[b]
            if full * bs < N and full < nblk:
                rem = N - full * bs
                Hinv[full * bs:, full * bs:] = inverse_batch(Hg[full, :rem, :rem], damping, "hinv", fallbacks,
                                                            upper_only=True)
            if greedy_passes > 0:
                raise ValueError("greedy search needs a 2-D Hessian (block-diagonal 3-D given)")
        elif Hg.dim() == 2:
            if tuple(Hg.shape) != (N, N):
                raise ValueError(f"Hessian shape {tuple(hessian.shape)} != ({N}, {N})")
            Hinv = inverse_batch(Hg, damping, "hinv", fallbacks, upper_only=True)
            H_greedy = Hg
        else:
            raise ValueError(f"Expected 2D tensor, 3D tensor, or DLR dict Hessian, got {hessian.dim()}D")
    else:
        warnings.warn(
            "LDLQ: no calibration Hessian provided; using H = W^T W / M. "
            "This can perform worse than RTN. Pass a calibration Hessian "
            "from GPTQ calibration data for best results.", stacklevel=2)
        H = _gemm_tn(Wg, 1.0 / M)
        if not bool(torch.isfinite(H).all().item()):
            logger.warning("LDLQ: Hessian has inf/nan, falling back to RTN")
            return _hessian_nan_rtn(Wg, int_bits, out_dev)
        Hinv = inverse_batch(H, damping, "hinv", fallbacks, upper_only=True)
        H_greedy = _damp_only(H, damping)

    ramax = _row_absmax(Wg)
    srow = torch.empty(M, dtype=torch.float32, device=Wg.device)
    flat = torch.empty(M, N, dtype=torch.float32, device=Wg.device)
    nat.check(_lib().ic_ldlq_init_scales(ramax, M, N, int_bits, srow, flat,
                                         nat.stream()), "ic_ldlq_init_scales")
    if iterations > 1:
        Q, _ = _iterative(Wg, Hinv, flat, iterations, block_size, int_bits)
    else:
        Q = _single_pass(Wg, Hinv, flat, block_size, int_bits)
    method = "ldlq_hip"
    if greedy_passes > 0:
        gs = _ls_scales(Q, Wg)
        qmin, qmax = (-128, 127) if int_bits == 8 else (-8, 7)
        Q = _greedy.greedy_search(Wg, Q, gs, H_greedy, greedy_passes, qmin, qmax, rank_threshold=rank_threshold,
                                  backend=greedy_backend)
    fs = _ls_scales(Q, Wg)
    mse, max_err = quant_error(Wg, Q, fs, None)
    return QuantizationResult(quantized_W=Q.to(out_dev), scales=fs.to(torch.float16).reshape(M, 1).to(out_dev),
                              zero_points=None, mse=mse, max_err=max_err, method_used=method, fallbacks=fallbacks)


def _hessian_nan_rtn(Wg: torch.Tensor, int_bits: int, out_dev) -> QuantizationResult:
    """RTN with round-half-even (ldlq.py:189-205): tensor divisors keep IEEE division."""
    from .layer import _div
    M = Wg.shape[0]
    qmin, qmax = (-128, 127) if int_bits == 8 else (-8, 7)
    div = 127.0 if int_bits == 8 else 7.0
    s = _div(Wg.abs().amax(dim=1, keepdim=True), div).clamp(min=1e-5, max=65500.0)
    q = (Wg / s).round().clamp(qmin, qmax).to(torch.int8)
    mse, max_err = quant_error(Wg, q, s.reshape(-1), None)
    return QuantizationResult(quantized_W=q.to(out_dev), scales=s.to(torch.float16).to(out_dev), zero_points=None,
                              mse=mse, max_err=max_err, method_used="rtn", fallbacks=["hessian_nan_rtn"])
