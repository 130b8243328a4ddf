"""Damped Hessian inverse on the GPU (``ic_hessian_inverse``).

Mirrors ``converter/gptq.py:91-121`` (``_prepare_hessian`` / ``_prepare_hinv``),
``converter/rounding.py:19-34`` (``_invert_hessian``) and the block loop of
``converter/ldlq.py:64-92``.  The Cholesky branch runs in the HIP library;
when a pivot is not positive the reference falls back to ``torch.linalg.inv``
and then ``pinv`` (with a ``UserWarning``): that rare branch is kept, on the
GPU, for the affected matrices only.
"""

from __future__ import annotations

import warnings

import torch

from . import _native as nat
from .log import logger

METHODS = {"hinv": 0, "cholesky": 1}


def _damped(H: torch.Tensor, damping: float) -> torch.Tensor:
    """H + damping * max(mean(diag H), 1e-6) * I as a new tensor (the
    library's damping kernel, the reference's CPU summation order)."""
    out = H.float().contiguous().clone()
    nat.check(nat.lib().ic_damp_hessian(out, 1, out.shape[0], float(damping), nat.stream()),
              "ic_damp_hessian")
    return out


def _fallback_inverse(H_damped: torch.Tensor) -> torch.Tensor:
    try:
        return torch.linalg.inv(H_damped)
    except torch.linalg.LinAlgError:
        warnings.warn(
            "Hessian is singular/ill-conditioned; falling back to pseudoinverse. "
            "This may produce inaccurate quantization scales.",
            stacklevel=4,
        )
        return torch.linalg.pinv(H_damped)


def inverse_batch(H: torch.Tensor, damping: float, method: str = "hinv",
                  fallbacks: list[str] | None = None, *, inplace: bool = False, restore=None,
                  upper_only: bool = False) -> torch.Tensor:
    """``H``: fp32 GPU tensor [n, n] or [batch, n, n].  Returns the damped
    inverse (method "hinv") or the upper Cholesky factor of the damped
    inverse (method "cholesky") of every matrix, same shape.

    ``H`` is not modified unless ``inplace`` (a contiguous fp32 tensor the
    caller owns, which then holds the result); an in-place call needs
    ``restore()``, which returns the original ``H`` again for the fallback
    chain when a Cholesky factorisation fails.  ``upper_only`` (method
    "hinv"): only the entries on and above the diagonal are the inverse's,
    the rest are finite scratch values - for callers that read rows j from
    column j on, as the GPTQ / LDLQ sweeps do."""
    squeeze = H.dim() == 2
    Hb = H.unsqueeze(0) if squeeze else H
    batch, n, _ = Hb.shape
    if inplace:
        if restore is None or Hb.dtype != torch.float32 or not Hb.is_contiguous():
            raise ValueError("inverse_batch: inplace needs a contiguous fp32 tensor and restore()")
        out = Hb
    else:
        out = Hb.float().contiguous().clone()
    if n == 0 or batch == 0:
        return out[0] if squeeze else out
    code = METHODS[method]
    if upper_only and code == 0:
        code = 2
    info = torch.zeros(2 * batch, dtype=torch.int32, device=out.device)
    ws = nat.workspace(nat.lib().ic_hessian_inverse_workspace_bytes(batch, n), out.device)
    nat.check(nat.lib().ic_hessian_inverse(out, batch, n, float(damping), code, info,
                                           ws, nat.stream()), "ic_hessian_inverse")
    del ws
    inf = info.tolist()
    orig = None
    for b in range(batch):
        chol_failed = inf[b] != 0
        inv_chol_failed = code == 1 and inf[batch + b] != 0
        if not (chol_failed or inv_chol_failed):
            continue
        if inplace and orig is None:
            orig = restore()
            orig = orig.unsqueeze(0) if squeeze else orig
        Hd = _damped((orig if inplace else Hb)[b].float(), damping)
        if chol_failed:
            logger.debug("Cholesky of the damped Hessian failed at column %d; using inv", inf[b])
            if fallbacks is not None:
                fallbacks.append("hessian_inv_fallback")
            Hi = _fallback_inverse(Hd)
        else:
            Hi = None
        src = (orig if inplace else Hb)[b]
        out[b] = fallback_output(code, Hi, lambda: inverse_batch(src, damping, "hinv"))
    return out[0] if squeeze else out


def fallback_output(code: int, Hi: torch.Tensor | None, hinv_of_input) -> torch.Tensor:
    """The matrix the reference hands to the column loop when a GPU Cholesky
    failed.  ``code``: 0 = method "hinv", 2 = "hinv" with only the upper
    triangle read (both: converter/gptq.py:113-121, the inverse itself),
    1 = method "cholesky" (converter/gptq.py:91-110: the upper Cholesky factor
    of the inverse, or the inverse when that factorisation fails).  ``Hi``:
    the inv / pinv fallback of the damped H when chol(H) failed, None when
    chol(H) worked and only chol(H^-1) failed (then ``hinv_of_input()`` gives
    H^-1)."""
    if code in (0, 2):
        if Hi is None:
            raise ValueError("fallback_output: method hinv needs the fallback inverse")
        return Hi
    if Hi is None:
        return hinv_of_input()
    try:
        return torch.linalg.cholesky(Hi).T
    except torch.linalg.LinAlgError:
        return Hi
