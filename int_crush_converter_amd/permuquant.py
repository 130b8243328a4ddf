"""PermuQuant channel reordering (API of ``converter/permuquant.py``).

The statistics, the sort, the acceptance error and the gathers run in
libicq.so on the GPU:

* ``channel_second_moments``: ``ic_col_moments``, bit-exact with the
  reference's ``(W ** 2).mean(dim=0)`` on the CPU (same summation order).
* ``find_permutation_weight``: ``ic_argsort_desc``, a stable descending sort.
  It equals torch's ``argsort(descending=True)`` whenever no two moments are
  exactly equal; on exact ties torch's CPU sort (not stable from 100
  elements on) may order them differently.
* ``compute_group_quant_error``: ``ic_group_quant_error``, bit-exact with the
  reference run with ``threads`` CPU threads (default: this process's
  ``torch.get_num_threads()``).  For per-row scales (every call the
  pipeline makes) the reordered error sums the same values in another
  order, so the reference's accept / reject decision is decided by fp32
  rounding; reproducing its summation order reproduces that decision.
* ``find_permutation_joint``: the joint criterion ``act^a * w^(1-a)`` is
  computed with torch on the GPU (its ``pow`` is not bit-exact with the CPU's;
  the pipeline never uses this path).
"""

from __future__ import annotations

import torch

from . import _native as nat

# Vector width of torch's CPU float reductions (AVX-512 builds: 16 floats);
# columns past the last whole vector are summed by a scalar loop.
CPU_VEC = 16


def _cpu_vec() -> int:
    cap = ""
    try:
        cap = torch.backends.cpu.get_cpu_capability()
    except Exception:  # pragma: no cover - older torch
        pass
    return 8 if cap in ("AVX2", "DEFAULT", "NO AVX") else CPU_VEC


def _lib():
    return nat.lib()


def _as_matrix(W: torch.Tensor) -> torch.Tensor:
    Wg = nat.to_gpu(W)
    if Wg.dim() != 2:
        raise ValueError(f"Expected 2D weight tensor, got {Wg.dim()}D")
    Wg = Wg.float()
    if Wg.stride(1) != 1:
        Wg = Wg.contiguous()
    return Wg


def channel_second_moments(W: torch.Tensor) -> torch.Tensor:
    """mu2 [in_features] fp32 on the GPU (permuquant.py:13-23)."""
    Wg = _as_matrix(W)
    M, N = Wg.shape
    mu2 = torch.empty(N, dtype=torch.float32, device=Wg.device)
    if M == 0:
        return mu2.fill_(float("nan"))
    ws = nat.workspace(_lib().ic_col_moments_workspace_bytes(M, N), Wg.device)
    nat.check(_lib().ic_col_moments(Wg, M, N, Wg.stride(0), _cpu_vec(), mu2, ws,
                                    nat.stream()), "ic_col_moments")
    return mu2


def argsort_descending(v: torch.Tensor) -> torch.Tensor:
    """Stable descending argsort of a 1-D fp32 vector (int64, GPU)."""
    vg = nat.to_gpu(v).float().contiguous().reshape(-1)
    n = vg.numel()
    perm = torch.empty(n, dtype=torch.int64, device=vg.device)
    if n == 0:
        return perm
    ws = nat.workspace(_lib().ic_argsort_workspace_bytes(n), vg.device)
    nat.check(_lib().ic_argsort_desc(vg, n, perm, ws, nat.stream()),
              "ic_argsort_desc")
    return perm


def find_permutation_weight(W: torch.Tensor, group_size: int = 128) -> torch.Tensor:
    """Channels by descending second moment (permuquant.py:26-41)."""
    return argsort_descending(channel_second_moments(W))


def find_permutation_joint(W: torch.Tensor, act_mu2: torch.Tensor, alpha: float = 0.5,
                           group_size: int = 128) -> torch.Tensor:
    """Channels by descending act_mu2^alpha * mu2^(1-alpha) (permuquant.py:44-69)."""
    weight_mu2 = channel_second_moments(W)
    a = nat.to_gpu(act_mu2).float()
    v = (a.clamp(min=1e-12) ** alpha) * (weight_mu2.clamp(min=1e-12) ** (1.0 - alpha))
    return argsort_descending(v)


def _quant_error(Wg: torch.Tensor, perm: torch.Tensor | None, group_size: int, int_bits: int,
                 threads: int | None) -> float:
    M, N = Wg.shape
    if int_bits not in (4, 8):
        raise ValueError(f"int_bits must be 4 or 8, got {int_bits}")
    if int_bits == 4 and group_size < 1:
        raise ValueError(f"group_size must be >= 1, got {group_size}")
    T = int(threads) if threads is not None else torch.get_num_threads()
    out = torch.empty(1, dtype=torch.float32, device=Wg.device)
    ws = nat.workspace(_lib().ic_group_quant_error_workspace_bytes(M, N, group_size, int_bits, T), Wg.device)
    pp = None
    if perm is not None:
        pp = nat.to_gpu(perm).to(torch.int64).contiguous()
        if pp.numel() != N:
            raise ValueError(f"permutation of length {pp.numel()} for {N} columns")
    nat.check(_lib().ic_group_quant_error(Wg, M, N, Wg.stride(0), nat.ptr(pp), int(group_size), int_bits,
                                          T, out, ws, nat.stream()), "ic_group_quant_error")
    return float(out.item())


def compute_group_quant_error(W: torch.Tensor, group_size: int = 128, int_bits: int = 4, *,
                              threads: int | None = None) -> float:
    """Total squared RTN error, symmetric, fp16 scales per group (INT4) or
    per row (INT8) (permuquant.py:72-111)."""
    return _quant_error(_as_matrix(W), None, group_size, int_bits, threads)


def _acceptance(Wg: torch.Tensor, perm: torch.Tensor, group_size: int, tau: float, int_bits: int,
                threads: int | None):
    """(accepted, W[:, perm], error of W[:, perm]): the reordered matrix is
    gathered once (coalesced) and reused by callers that keep it."""
    error_orig = _quant_error(Wg, None, group_size, int_bits, threads)
    Wp = permute_columns(Wg, perm)
    error_reorder = _quant_error(Wp, None, group_size, int_bits, threads)
    relative_improvement = (error_orig - error_reorder) / error_orig if error_orig > 0 else 0.0
    return bool(relative_improvement > tau), Wp, error_reorder


def find_permutation_with_acceptance(W: torch.Tensor, act_mu2: torch.Tensor | None = None, alpha: float = 0.5,
                                     group_size: int = 128, tau: float = 0.0, int_bits: int = 4, *,
                                     threads: int | None = None) -> tuple[torch.Tensor, bool]:
    """Candidate permutation and whether its relative error reduction
    exceeds tau (permuquant.py:114-156)."""
    Wg = _as_matrix(W)
    perm = find_permutation_joint(Wg, act_mu2, alpha, group_size) if act_mu2 is not None \
        else find_permutation_weight(Wg, group_size)
    accepted, _, _ = _acceptance(Wg, perm, group_size, tau, int_bits, threads)
    return perm, accepted


def weight_only_permutation(W: torch.Tensor, group_size: int, tau: float, int_bits: int, *,
                            threads: int | None = None):
    """sweep_alpha(W, act_mu2=None, ...) as the pipeline calls it, plus the
    reordered matrix: (perm, accepted, W[:, perm])."""
    Wg = _as_matrix(W)
    perm = find_permutation_weight(Wg, group_size)
    accepted, Wp, _ = _acceptance(Wg, perm, group_size, tau, int_bits, threads)
    return perm, accepted, Wp


def sweep_alpha(W: torch.Tensor, act_mu2: torch.Tensor | None = None, group_size: int = 128, tau: float = 0.0,
                num_alpha: int = 11, int_bits: int = 4, *,
                threads: int | None = None) -> tuple[torch.Tensor, float, bool]:
    """Best accepted permutation over alpha in [0, 1] (permuquant.py:159-213)."""
    if num_alpha < 1:
        raise ValueError(f"num_alpha must be >= 1, got {num_alpha}")
    Wg = _as_matrix(W)
    if act_mu2 is None or num_alpha == 1:
        perm, accepted = find_permutation_with_acceptance(Wg, act_mu2, 0.0, group_size, tau, int_bits,
                                                          threads=threads)
        return perm, 0.0, accepted
    best_perm, best_alpha, best_error, best_accepted = None, 0.0, float("inf"), False
    for i in range(num_alpha):
        alpha = i / (num_alpha - 1)
        perm = find_permutation_joint(Wg, act_mu2, alpha, group_size)
        accepted, _, error = _acceptance(Wg, perm, group_size, tau, int_bits, threads)
        if accepted:
            # the reference recomputes this error of W[:, perm]: the same value
            if error < best_error:
                best_error, best_perm, best_alpha, best_accepted = error, perm, alpha, True
    if best_perm is None:
        best_perm = torch.arange(Wg.shape[1], device=Wg.device)
        best_accepted = False
    return best_perm, best_alpha, best_accepted


def permute_columns(W: torch.Tensor, perm: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """W[:, perm] for an fp32 GPU matrix (``ic_permute_cols``); ``out`` may
    be a column slice of another matrix (not W itself)."""
    Wg = _as_matrix(W)
    pp = nat.to_gpu(perm).to(torch.int64).contiguous()
    M = Wg.shape[0]
    n = pp.numel()
    if out is None:
        out = torch.empty(M, n, dtype=torch.float32, device=Wg.device)
    if out.shape != (M, n) or out.dtype != torch.float32 or out.stride(1) != 1:
        raise ValueError("permute_columns: out must be fp32 [rows, len(perm)] with unit column stride")
    nat.check(_lib().ic_permute_cols(Wg, M, Wg.shape[1], Wg.stride(0), pp, n, out,
                                     out.stride(0), nat.stream()), "ic_permute_cols")
    return out


def permute_hessian(H: torch.Tensor, perm: torch.Tensor) -> torch.Tensor:
    """H[perm][:, perm] for a 2-D fp32 GPU Hessian (``ic_permute_sym``)."""
    Hg = nat.to_gpu(H).float()
    if Hg.dim() != 2 or Hg.shape[0] != Hg.shape[1]:
        raise ValueError(f"permute_hessian needs a square 2-D Hessian, got {tuple(Hg.shape)}")
    if Hg.stride(1) != 1:
        Hg = Hg.contiguous()
    pp = nat.to_gpu(perm).to(torch.int64).contiguous()
    n = pp.numel()
    out = torch.empty(n, n, dtype=torch.float32, device=Hg.device)
    nat.check(_lib().ic_permute_sym(Hg, Hg.shape[0], Hg.stride(0), pp, n, out, n,
                                    nat.stream()), "ic_permute_sym")
    return out


# State-dict helpers (permuquant.py:216-332): plain indexing of tensors of
# any dtype and device, like the reference.

def apply_permutation_to_weight(W: torch.Tensor, perm: torch.Tensor) -> torch.Tensor:
    return W[:, perm]


def apply_permutation_to_norm(norm_weight: torch.Tensor, perm: torch.Tensor) -> torch.Tensor:
    return norm_weight[perm]


def apply_permutation_to_norm_bias(norm_bias: torch.Tensor, perm: torch.Tensor) -> torch.Tensor:
    return norm_bias[perm]


def apply_permutation_to_linear_output(W: torch.Tensor, perm: torch.Tensor) -> torch.Tensor:
    return W[perm, :]


def permute_state_dict(state_dict: dict[str, torch.Tensor], layer_perms: dict[str, torch.Tensor],
                       norm_map: dict[str, str] | None = None,
                       linear_map: dict[str, str] | None = None) -> dict[str, torch.Tensor]:
    """Permute each layer's input channels and absorb the permutation into
    the preceding norm (weight / bias) or linear layer (output rows)."""
    norm_map = norm_map or {}
    linear_map = linear_map or {}
    for layer_name, perm in layer_perms.items():
        weight_key = f"{layer_name}.weight"
        if weight_key not in state_dict:
            continue
        state_dict[weight_key] = apply_permutation_to_weight(state_dict[weight_key], perm)
        if layer_name in norm_map:
            norm_name = norm_map[layer_name]
            if f"{norm_name}.weight" in state_dict:
                state_dict[f"{norm_name}.weight"] = apply_permutation_to_norm(state_dict[f"{norm_name}.weight"], perm)
            if f"{norm_name}.bias" in state_dict:
                state_dict[f"{norm_name}.bias"] = apply_permutation_to_norm_bias(state_dict[f"{norm_name}.bias"],
                                                                                 perm)
        elif layer_name in linear_map:
            prev = f"{linear_map[layer_name]}.weight"
            if prev in state_dict:
                state_dict[prev] = apply_permutation_to_linear_output(state_dict[prev], perm)
    return state_dict
