"""Calibration file access (API of ``converter/calibration_io.py``).

Host-side only: reading the ``.pt`` file (``torch.load(weights_only=True)``),
matching layer names, and normalising the Hessian formats (full 2-D,
stacked 3-D blocks, a list of blocks zero-padded to the largest block, or a
diagonal + low-rank dict ``{"format": "dlr", "D": [n], "U": [n, r]}``).
"""

from __future__ import annotations

import torch

from .dlr import is_dlr, validate_dlr
from .log import logger


def load_calibration(path: str) -> dict:
    """Load and validate a calibration file (reference calibration_io.py:9-37)."""
    try:
        data = torch.load(path, map_location="cpu", weights_only=True)
    except FileNotFoundError:
        raise ValueError(f"Calibration file not found: {path}")
    except Exception as e:
        raise ValueError(f"Calibration file at {path} is corrupted or not a valid .pt file: {e}") from e
    required = {"hessians", "shapes", "layer_types"}
    missing = required - set(data.keys())
    if missing:
        raise KeyError(f"Calibration file missing required keys: {missing}")
    return data


def build_name_map(state_dict_keys: list[str], calibration_keys: list[str]) -> dict[str, str]:
    """``<module>.weight`` -> ``<module>`` when the module has calibration data."""
    cal = set(calibration_keys)
    out = {}
    for key in state_dict_keys:
        if key.endswith(".weight"):
            mod = key[: -len(".weight")]
            if mod in cal:
                out[key] = mod
    return out


def get_hessian(calibration: dict, layer_name: str, weight_shape, *,
                device: torch.device | None = None) -> torch.Tensor | dict | None:
    """2-D, 3-D or DLR Hessian of a layer, or None when missing / mismatched /
    non-finite (reference calibration_io.py:65-123).  With ``device`` a dense
    Hessian is moved there first and checked and returned there (the host's
    cores stay free for the file I/O threads)."""
    hessians = calibration["hessians"]
    if layer_name not in hessians:
        return None
    raw = hessians[layer_name]
    in_features = weight_shape[1]
    if is_dlr(raw):
        if not validate_dlr(raw, in_features=in_features):
            logger.warning("DLR Hessian for %s is invalid; skipping (RTN fallback)", layer_name)
            return None
        return dict(raw)   # a shallow copy: callers may replace D and U
    if isinstance(raw, list):
        if not raw or not isinstance(raw[0], torch.Tensor):
            return None
        bs = max(t.shape[0] for t in raw)
        blocks = []
        for t in raw:
            if t.shape[0] == bs and t.shape[1] == bs:
                blocks.append(t)
            else:
                b = torch.zeros(bs, bs, dtype=t.dtype)
                b[: t.shape[0], : t.shape[1]] = t
                blocks.append(b)
        H = torch.stack(blocks)
    elif isinstance(raw, torch.Tensor):
        H = raw
    else:
        return None
    if H.dim() == 2:
        if H.shape[0] != in_features or H.shape[1] != in_features:
            return None
    elif H.dim() == 3:
        nb, bs, bs2 = H.shape
        if nb != (in_features + bs - 1) // bs or bs != bs2:
            return None
    else:
        return None
    if device is not None:
        H = H.to(device, non_blocking=False)
    if not torch.isfinite(H).all():
        logger.warning("Hessian for %s contains non-finite values; skipping (RTN fallback)", layer_name)
        return None
    return H


def get_hessian_diag(calibration: dict, layer_name: str, in_features: int) -> torch.Tensor | None:
    """fp32 Hessian diagonal [in_features] of a layer (calibration_io.py:
    158-240): the ``hessian_diag`` store when present (returned whole when it
    is shorter), else the diagonal of the 2-D / 3-D / list Hessian (None when
    shorter than in_features), or D + rowsum(U^2) of a DLR Hessian."""
    store = calibration.get("hessian_diag")
    if store and layer_name in store:
        d = store[layer_name].float()
        return d[:in_features] if d.shape[0] >= in_features else d
    hessians = calibration.get("hessians", {})
    if layer_name not in hessians:
        return None
    raw = hessians[layer_name]
    if is_dlr(raw):
        d = raw["D"].float() + (raw["U"].float() * raw["U"].float()).sum(dim=1)
        return d[:in_features] if d.shape[0] >= in_features else d
    if isinstance(raw, list):
        parts = [b.diagonal() for b in raw if isinstance(b, torch.Tensor) and b.dim() == 2]
        if not parts:
            return None
        d = torch.cat(parts).float()
    elif isinstance(raw, torch.Tensor) and raw.dim() == 2:
        d = raw.diagonal().float()
    elif isinstance(raw, torch.Tensor) and raw.dim() == 3:
        d = torch.cat([raw[i].diagonal() for i in range(raw.shape[0])]).float()
    else:
        return None
    return d[:in_features] if d.shape[0] >= in_features else None


def get_permutation(calibration: dict, layer_name: str) -> torch.Tensor | None:
    perm = calibration.get("permuquant")
    if not perm or layer_name not in perm:
        return None
    return perm[layer_name].to(torch.int64)


def get_per_channel_amax(calibration: dict, layer_name: str, in_features: int) -> torch.Tensor | None:
    store = calibration.get("amax_per_channel")
    if not store or layer_name not in store:
        return None
    a = store[layer_name].float()
    return a[:in_features] if a.shape[0] >= in_features else a
