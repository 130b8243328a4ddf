"""Diagonal + low-rank (DLR) Hessians, H = diag(D) + U Uᵀ (API of
``converter/dlr.py``).

The damped inverse (Woodbury identity) and the dense form run in the HIP
library (``ic_woodbury_inverse``, ``ic_dlr_to_dense``); the rest is
bookkeeping on the factors.  Results are computed on the GPU.
"""

from __future__ import annotations

import torch

from . import _native as nat
from .config import DIAG_MEAN_FLOOR
from .log import logger

_DLR_DIAG_FLOOR = 1e-12   # dlr.py:22


def is_dlr(hessian) -> bool:
    """True for a dict ``{"format": "dlr", "D": ..., "U": ...}`` (dlr.py:25-33)."""
    return (isinstance(hessian, dict) and hessian.get("format") == "dlr"
            and "D" in hessian and "U" in hessian)


def validate_dlr(hessian, in_features: int | None = None) -> bool:
    """Shapes, finiteness and a non-negative diagonal (dlr.py:36-67); logs a
    warning and returns False on the first failed check, never raises."""
    if not is_dlr(hessian):
        return False
    D, U = hessian["D"], hessian["U"]
    if not isinstance(D, torch.Tensor) or not isinstance(U, torch.Tensor):
        logger.warning("DLR: D or U is not a tensor")
        return False
    if D.dim() != 1 or U.dim() != 2:
        logger.warning("DLR: expected D (n,) and U (n, r), got %sD, %sD", D.dim(), U.dim())
        return False
    if D.shape[0] != U.shape[0]:
        logger.warning("DLR: D rows (%d) != U rows (%d)", D.shape[0], U.shape[0])
        return False
    if in_features is not None and D.shape[0] != in_features:
        logger.warning("DLR: feature dim %d != expected %d", D.shape[0], in_features)
        return False
    if not bool(torch.isfinite(D).all()) or not bool(torch.isfinite(U).all()):
        logger.warning("DLR: non-finite values in D or U")
        return False
    if D.numel() and D.min().item() < 0:
        logger.warning("DLR: negative diagonal entry (min=%.6e)", D.min().item())
        return False
    return True


def make_dlr_dict(D: torch.Tensor, U: torch.Tensor) -> dict:
    """The DLR dict of ``D`` and ``U`` (dlr.py:178-186)."""
    return {"format": "dlr", "D": D, "U": U, "rank": int(U.shape[1]), "n": int(D.shape[0])}


def damped_diag_mean(D: torch.Tensor, U: torch.Tensor) -> torch.Tensor:
    """mean(D + rowsum(U²)) floored at 1e-6, the damping base (dlr.py:70-73)."""
    diag_full = D.float() + (U.float() * U.float()).sum(dim=1)
    return diag_full.mean().clamp(min=DIAG_MEAN_FLOOR)


def _factors(D: torch.Tensor, U: torch.Tensor):
    if D.dim() != 1 or U.dim() != 2 or U.shape[0] != D.shape[0]:
        raise ValueError(f"DLR factors must be D (n,) and U (n, r), got {tuple(D.shape)} and {tuple(U.shape)}")
    Dg = nat.to_gpu(D).float().contiguous()
    Ug = nat.to_gpu(U).float()
    if Ug.stride(1) != 1:
        Ug = Ug.contiguous()
    return Dg, Ug


def woodbury_inverse(D: torch.Tensor, U: torch.Tensor, damping: float = 0.0,
                     device: torch.device | None = None, *, upper_only: bool = False) -> torch.Tensor:
    """``(diag(D) + U Uᵀ + damping · mean(diag(H)) · I)⁻¹`` (dlr.py:76-119),
    fp32 [n, n] on ``device`` (default: the device of ``D``).  ``upper_only``:
    only the entries on and above the diagonal are the inverse's (the sweeps
    read nothing else).  When the Cholesky factorisation of the r x r capacitance
    matrix fails the reference's fallbacks follow: ``torch.linalg.inv``, then
    ``pinv``."""
    out_dev = D.device if device is None else torch.device(device)
    Dg, Ug = _factors(D, U)
    n, r = Ug.shape
    dev = Dg.device
    Hinv = torch.empty(n, n, dtype=torch.float32, device=dev)
    M = torch.empty(r, r, dtype=torch.float32, device=dev)
    info = torch.zeros(2, dtype=torch.int32, device=dev)
    ws = nat.workspace(nat.lib().ic_woodbury_workspace_bytes(n, r), dev)

    def call(minv):
        nat.check(nat.lib().ic_woodbury_inverse(Dg, Ug.data_ptr() if r else None, n, r, Ug.stride(0),
                                                float(damping), nat.ptr(minv), int(upper_only), Hinv, n,
                                                M.data_ptr() if r else None, info, ws,
                                                nat.stream()), "ic_woodbury_inverse")

    call(None)
    if r and int(info[0].item()) != 0:
        logger.debug("DLR: Cholesky of the capacitance matrix failed at column %d; using inv", int(info[0].item()))
        try:
            Minv = torch.linalg.inv(M)
        except torch.linalg.LinAlgError:
            Minv = torch.linalg.pinv(M)
        call(Minv.contiguous())
    return Hinv.to(out_dev)


def dlr_to_dense(D: torch.Tensor, U: torch.Tensor) -> torch.Tensor:
    """``diag(D) + U Uᵀ`` as fp32 [n, n] (dlr.py:122-127), on the GPU."""
    Dg, Ug = _factors(D, U)
    n, r = Ug.shape
    H = torch.empty(n, n, dtype=torch.float32, device=Dg.device)
    nat.check(nat.lib().ic_dlr_to_dense(Dg, Ug.data_ptr() if r else None, n, r, Ug.stride(0),
                                        H, n, nat.stream()), "ic_dlr_to_dense")
    return H


def transform_dlr_for_smoothquant(D: torch.Tensor, U: torch.Tensor, smoothing_factors: torch.Tensor):
    """SmoothQuant column scaling of the factors, D/s² and U/s with s clamped
    at 1e-8 (dlr.py:130-146)."""
    s = smoothing_factors.float().clamp(min=1e-8)
    return D.float() * (1.0 / (s * s)), U.float() / s.unsqueeze(1)


def permute_dlr(D: torch.Tensor, U: torch.Tensor, perm: torch.Tensor):
    """``D[perm], U[perm]`` (dlr.py:149-156); ``perm`` may be a prefix."""
    perm = perm.to(device=D.device, dtype=torch.int64)
    return D[perm].clone(), U[perm.to(U.device)].clone()


def rotate_dlr_to_dense(D: torch.Tensor, U: torch.Tensor, rot_size: int) -> torch.Tensor:
    """Dense form rotated as a 2-D Hessian, Rᵀ H R (dlr.py:159-175)."""
    from .rotation import rotate_hessian
    return rotate_hessian(dlr_to_dense(D, U), rot_size)


def dlr_hessian_diag(D: torch.Tensor, U: torch.Tensor) -> torch.Tensor:
    """The true diagonal D + rowsum(U²) (calibration_io.py:207-210)."""
    return D.float() + (U.float() ** 2).sum(dim=1)
