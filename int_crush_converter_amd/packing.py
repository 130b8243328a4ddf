"""INT4 packing (API of ``converter/packing.py``): two's complement nibbles,
low nibble = even index, uint8 storage.  Validation and (un)packing run in
the HIP library (``ic_pack_int4``, ``ic_unpack_int4``)."""

from __future__ import annotations

import torch

from . import _native as nat

INT4_MIN = -8
INT4_MAX = 7
INT4_PACK_FACTOR = 2


class INT4PackingError(ValueError):
    """Raised when values are out of INT4 range during packing."""


def _as_rows(t: torch.Tensor):
    g = nat.to_gpu(t)
    if g.dtype not in (torch.int8, torch.float32):
        g = g.to(torch.float32)
    k = g.shape[-1] if g.dim() else 1
    g = g.contiguous().reshape(-1, k)
    return g, (0 if g.dtype == torch.int8 else 1)


def _validate_rows(g: torch.Tensor, kind: int, dst: torch.Tensor | None) -> None:
    flags = torch.zeros(3, dtype=torch.int32, device=g.device)
    rows, cols = g.shape
    nat.check(nat.lib().ic_pack_int4(g, kind, rows, cols, cols, nat.ptr(dst),
                                     dst.shape[1] if dst is not None else 0, flags, nat.stream()),
              "ic_pack_int4")
    nf, lo, hi = flags.tolist()
    if nf:
        raise INT4PackingError("Tensor contains NaN or Inf values")
    if lo or hi:
        raise INT4PackingError(
            f"Values must be in [{INT4_MIN}, {INT4_MAX}], got [{g.min().item()}, {g.max().item()}]")


def validate_int4_range(tensor: torch.Tensor) -> None:
    """Raise INT4PackingError if any value is non-finite or outside [-8, 7]."""
    if tensor.numel() == 0:
        return
    g, kind = _as_rows(tensor)
    _validate_rows(g, kind, None)


def pack_int4(values: torch.Tensor) -> torch.Tensor:
    """[..., K] INT4 values -> [..., ceil(K/2)] uint8 (reference packing.py:30-46)."""
    lead = values.shape[:-1]
    K = values.shape[-1]
    if values.numel() == 0:
        return torch.zeros(*lead, (K + 1) // 2, dtype=torch.uint8, device=values.device)
    g, kind = _as_rows(values)
    out = torch.empty(g.shape[0], (K + 1) // 2, dtype=torch.uint8, device=g.device)
    _validate_rows(g, kind, out)
    return out.reshape(*lead, (K + 1) // 2).to(values.device)


def unpack_int4(packed: torch.Tensor, K: int) -> torch.Tensor:
    """[..., ceil(K/2)] uint8 -> [..., K] int8 (reference packing.py:49-66)."""
    lead = packed.shape[:-1]
    if packed.numel() == 0 or K == 0:
        return torch.zeros(*lead, K, dtype=torch.int8, device=packed.device)
    g = nat.to_gpu(packed).contiguous().reshape(-1, packed.shape[-1])
    out = torch.empty(g.shape[0], K, dtype=torch.int8, device=g.device)
    nat.check(nat.lib().ic_unpack_int4(g, g.shape[0], K, g.shape[1], out, K, nat.stream()),
              "ic_unpack_int4")
    return out.reshape(*lead, K).to(packed.device)
