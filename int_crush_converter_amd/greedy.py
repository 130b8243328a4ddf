"""Greedy local search on the quantisation grid (API of ``converter/greedy.py``).

Coordinate descent that, column by column, gives every row the grid value
minimising tr((Q s - W) H (Q s - W)^T).  Everything runs in libicq.so:

* ``greedy_local_search``: the full-rank search, exact cross terms
  (reference ``greedy_local_search_pytorch`` greedy.py:487-541 and its GPU
  twin ``greedy_local_search_triton`` greedy.py:207-285).
* ``lowrank_decompose``: the top eigenpairs of H (greedy.py:293-366).
* ``greedy_lowrank``: cross terms from the eigen-truncated Hessian
  U_k diag(s_k) U_k^T with the exact diagonal and the stall test
  (greedy.py:369-479); falls back to the full-rank search when the rank is
  too high, like the reference.
* ``greedy_search``: the backend choice of ``converter/ldlq.py:602-647`` on
  a GPU - low-rank when the Hessian allows it, else full rank.

The scale is per element, as the reference's ``scale_2d[:, j]``
(greedy.py:487-541): the pipeline passes the least-squares row scale
broadcast over the row (ldlq.py:222-231), which the library takes as one
value per row; any other [M, N] scale runs the per-element kernels.
"""

from __future__ import annotations

import torch

from . import _native as nat
from .config import EIGENVALUE_FLOOR, LOWRANK_MAX_K, LOWRANK_MAX_RANK_FRAC
from .log import logger

# Subspace-iteration settings of the eigen-truncation: the subspace holds the
# largest admissible rank plus this many extra directions; LOWRANK_ITERS
# steps of (H + mu I) Q; the Gaussian start is seeded so runs repeat.
LOWRANK_OVERSAMPLE = 64
LOWRANK_ITERS = 8
LOWRANK_SEED = 0x1C9C0DE


def _lib():
    return nat.lib()


def _bits(clamp_min: int, clamp_max: int) -> int:
    if (clamp_min, clamp_max) == (-8, 7):
        return 4
    if (clamp_min, clamp_max) == (-128, 127):
        return 8
    raise ValueError(f"unsupported grid [{clamp_min}, {clamp_max}]: INT4 (-8, 7) or INT8 (-128, 127)")


def _scale_arg(scale: torch.Tensor, M: int, N: int) -> tuple[torch.Tensor, int]:
    """(fp32 scales, kind) for the library: [M] per row (kind 0) from an [M],
    [M, 1] or row-constant [M, N] scale, else [M, N] per element (kind 1)."""
    s = nat.to_gpu(scale).float()
    if s.dim() == 2 and tuple(s.shape) == (M, N):
        if s.stride(1) == 0 or torch.equal(s, s[:, :1].expand(M, N)):
            return s[:, 0].contiguous(), 0
        return s.contiguous(), 1
    if s.numel() != M:
        raise ValueError(f"greedy search: scale of shape {tuple(scale.shape)} for weights [{M}, {N}]")
    return s.reshape(M).contiguous(), 0


def _prep(W, Q, scale, H):
    Wg = nat.to_gpu(W).float().contiguous()
    if Wg.dim() != 2:
        raise ValueError(f"Expected 2D weight tensor, got {Wg.dim()}D")
    M, N = Wg.shape
    Hg = nat.to_gpu(H).float().contiguous()
    if Hg.dim() != 2 or tuple(Hg.shape) != (N, N):
        raise ValueError(f"greedy search needs a 2-D Hessian [{N}, {N}], got {tuple(H.shape)}")
    Qg = nat.to_gpu(Q)
    Qg = (Qg.round().clamp(-128, 127) if Qg.is_floating_point() else Qg).to(torch.int8).contiguous()
    s, kind = _scale_arg(scale, M, N)
    return Wg, Qg, s, kind, Hg


def greedy_local_search(W, Q, scale, H, num_passes: int, clamp_min: int, clamp_max: int) -> torch.Tensor:
    """Full-rank greedy search; returns the new int8 codes (Q is not modified)."""
    bits = _bits(clamp_min, clamp_max)
    Wg, Qg, s, kind, Hg = _prep(W, Q, scale, H)
    M, N = Wg.shape
    Qo = Qg.clone()
    ws = nat.workspace(_lib().ic_greedy_workspace_bytes(M, N), Wg.device)
    nat.check(_lib().ic_greedy(Wg, Qo, s, kind, Hg, M, N, int(num_passes), bits, ws, nat.stream()), "ic_greedy")
    return Qo.to(W.device)


def lowrank_decompose(H, rank_threshold: float = 0.01, max_rank_frac: float = LOWRANK_MAX_RANK_FRAC):
    """(s_k, U_k, k, used) like the reference's ``_lowrank_decompose``:
    eigenvalues above ``rank_threshold`` x the largest, refused (used =
    False) when the largest is below EIGENVALUE_FLOOR or k > max_rank_frac x N
    or k > LOWRANK_MAX_K (greedy.py:330-341)."""
    Hg = nat.to_gpu(H).float().contiguous()
    N = Hg.shape[0]
    kcap = min(LOWRANK_MAX_K, int(max_rank_frac * N))
    n_even = N - N % 2
    if n_even < 2:
        mx = float(Hg.reshape(-1)[0].item()) if N == 1 else 0.0
        if not mx >= EIGENVALUE_FLOOR:
            return None, None, 0, False
        if 1 > max_rank_frac * N:
            return None, None, 1, False
        return Hg.reshape(1).clone(), torch.ones(1, 1, device=Hg.device), 1, True
    p = min(n_even, kcap + LOWRANK_OVERSAMPLE + (kcap + LOWRANK_OVERSAMPLE) % 2)
    iters = 0 if p == N else LOWRANK_ITERS
    evals = torch.empty(p, dtype=torch.float32, device=Hg.device)
    evecs = torch.empty(N, p, dtype=torch.float32, device=Hg.device)
    ws = nat.workspace(_lib().ic_lowrank_workspace_bytes(N, p), Hg.device)
    sweeps = nat._c.c_int(0)
    # p > k_cap: a certificate that p eigenvalues exceed the cut settles the refusal early
    rc = _lib().ic_lowrank_eigs(Hg, N, p, iters, LOWRANK_SEED, float(rank_threshold), evals,
                                evecs, nat._c.byref(sweeps), ws, nat.stream())
    if rc == 1:    # IC_LOWRANK_REFUSED: at least p > k_cap eigenvalues above the cut
        return None, None, p, False
    if rc == -3:   # orthonormalisation failed: no low-rank basis (the reference's eigh failure path)
        logger.warning("Greedy: low-rank decomposition failed (%s); full-rank search",
                       _lib().ic_last_error().decode(errors="replace"))
        return None, None, 0, False
    nat.check(rc, "ic_lowrank_eigs")
    ev = evals.cpu()
    mx = float(ev[0])
    if not mx >= EIGENVALUE_FLOOR:
        return None, None, 0, False
    k = int((ev > mx * rank_threshold).sum())
    logger.debug("Greedy: eigen-truncation k=%d of p=%d (Jacobi sweeps %d)", k, p, sweeps.value)
    if k > max_rank_frac * N or k > LOWRANK_MAX_K:
        return None, None, k, False
    return evals[:k].contiguous(), evecs[:, :k].contiguous(), k, True


def greedy_lowrank(W, Q, scale, H, num_passes: int, clamp_min: int, clamp_max: int, rank_threshold: float = 0.01,
                   max_rank_frac: float = LOWRANK_MAX_RANK_FRAC):
    """Low-rank greedy search; (codes, k, used_lowrank).  Falls back to the
    full-rank search when the Hessian's effective rank is too high."""
    bits = _bits(clamp_min, clamp_max)
    Wg, Qg, s, kind, Hg = _prep(W, Q, scale, H)
    M, N = Wg.shape
    s_k, U_k, k, used = lowrank_decompose(Hg, rank_threshold, max_rank_frac)
    if not used:
        sc = s if kind == 1 else s.reshape(M, 1)
        return greedy_local_search(Wg, Qg, sc, Hg, num_passes, clamp_min, clamp_max).to(W.device), k, False
    Qo = Qg.clone()
    ws = nat.workspace(_lib().ic_greedy_lowrank_workspace_bytes(M, N, k), Wg.device)
    done = nat._c.c_int(0)
    nat.check(_lib().ic_greedy_lowrank(Wg, Qo, s, kind, Hg, U_k, k, s_k, k, M, N, int(num_passes), bits,
                                       nat._c.byref(done), ws, nat.stream()), "ic_greedy_lowrank")
    if done.value < num_passes:
        logger.warning("Greedy[lowrank] stalled at pass %d", done.value + 1)
    return Qo.to(W.device), k, True


def greedy_search(W, Q, scale, H, num_passes: int, clamp_min: int, clamp_max: int, rank_threshold: float = 0.01,
                  backend: str = "auto") -> torch.Tensor:
    """Backend choice of ``converter/ldlq.py:602-647`` on a GPU.  ``backend``:
    "auto" (low-rank when admissible, else full rank - the reference's GPU
    behaviour) or "full" (always exact cross terms - the reference's CPU
    behaviour)."""
    if backend == "full":
        return greedy_local_search(W, Q, scale, H, num_passes, clamp_min, clamp_max)
    if backend != "auto":
        raise ValueError(f"greedy backend must be 'auto' or 'full', got {backend!r}")
    q, k, used = greedy_lowrank(W, Q, scale, H, num_passes, clamp_min, clamp_max, rank_threshold)
    logger.debug("Greedy: GPU path (%s), k=%d", "lowrank" if used else "full rank", k)
    return q
