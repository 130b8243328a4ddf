"""ConvRot group-wise Hadamard rotation (API of ``converter/rotation.py``).

``make_hadamard_*`` / ``get_hadamard`` build the dense matrices (used for
reference and inverse transforms by callers).  The rotations run in the HIP
library with one of two kernels:

* ``"exact"`` (the default): the dense product in the reference's own fp32
  summation order - every output one fused multiply-add chain over the
  group in increasing order, as the reference's CPU ``x @ H.T`` and its
  Hessian einsum round (``ic_rotate_rows_exact``,
  ``ic_rotate_hessian_exact``, K = 1 MFMA chains on the matrix cores).
  Results are bit-identical to the reference's for rot <= 512 (weights) and
  rot <= 256 (Hessians); 2·R flops per element.
* ``"fwht"``: a fast Walsh-Hadamard transform (``ic_rotate_rows``,
  ``ic_rotate_hessian``): 2·log4(R) flops per element, HBM-bound; equal to
  the reference's within a few fp32 ulps, not bit for bit.

Sizes the exact kernels do not cover (rot >= 1024, where the reference's
CPU GEMM splits the sum in a way of its own) use the FWHT.  The choice is
process-wide: ``set_rotation_kernel()``, or the environment variable
``IC_ROTATION_KERNEL`` read at import.
"""

from __future__ import annotations

import math
import os

import torch
import torch.nn.functional as F

from . import _native as nat

_hadamard_cache: dict[tuple[int, str, str], torch.Tensor] = {}


def _is_power_of_four(n: int) -> bool:
    return n >= 4 and (n & (n - 1)) == 0 and (n & 0x55555555) == n


def _is_power_of_two(n: int) -> bool:
    return n > 0 and (n & (n - 1)) == 0


def make_hadamard_sylvester(n: int, dtype: torch.dtype = torch.float16, device: str = "cpu") -> torch.Tensor:
    """Normalised Sylvester Hadamard matrix (reference rotation.py:26-36)."""
    if not _is_power_of_two(n):
        raise ValueError(f"n must be a power of 2, got {n}")
    h = torch.ones(1, 1, dtype=dtype, device=device)
    base = torch.tensor([[1.0, 1.0], [1.0, -1.0]], dtype=dtype, device=device)
    while h.shape[0] < n:
        h = torch.kron(base, h)
    return h * (1.0 / math.sqrt(n))


def make_hadamard_regular(n: int, dtype: torch.dtype = torch.float16, device: str = "cpu") -> torch.Tensor:
    """Regular Hadamard (H4/2)^{kron k} for n = 4^k (reference rotation.py:39-62)."""
    if not _is_power_of_four(n):
        raise ValueError(f"Regular Hadamard requires power of 4, got {n}. Use rot_size=16/64/256.")
    h4 = torch.tensor([[1.0, 1.0, 1.0, -1.0],
                       [1.0, 1.0, -1.0, 1.0],
                       [1.0, -1.0, 1.0, 1.0],
                       [-1.0, 1.0, 1.0, 1.0]], dtype=dtype, device=device) / 2.0
    h = h4
    while h.shape[0] < n:
        h = torch.kron(h, h4)
    return h


def get_hadamard(size: int, dtype: torch.dtype = torch.float16, device: str = "cpu") -> torch.Tensor:
    key = (size, str(dtype), str(device))
    if key not in _hadamard_cache:
        _hadamard_cache[key] = make_hadamard_regular(size, dtype=dtype, device=device)
    return _hadamard_cache[key]


def clear_hadamard_cache() -> None:
    _hadamard_cache.clear()


_KERNELS = ("exact", "fwht")
_kernel = os.environ.get("IC_ROTATION_KERNEL", "exact")
if _kernel not in _KERNELS:
    raise ValueError(f"IC_ROTATION_KERNEL must be one of {_KERNELS}, got {_kernel!r}")


def set_rotation_kernel(kind: str) -> str:
    """Select the rotation kernel ("exact" or "fwht") for every later call;
    returns the previous choice."""
    global _kernel
    if kind not in _KERNELS:
        raise ValueError(f"rotation kernel must be one of {_KERNELS}, got {kind!r}")
    prev, _kernel = _kernel, kind
    return prev


def rotation_kernel() -> str:
    return _kernel


def _check_rot(rot_size: int) -> None:
    if not _is_power_of_two(rot_size):
        raise ValueError(f"rot_size must be a power of 2, got {rot_size}")
    if rot_size > 4096:
        raise ValueError(f"rot_size {rot_size} exceeds the supported maximum 4096")


def rotate_rows_gpu(W: torch.Tensor, rot_size: int, zero_above: float = 0.0,
                    n_zeroed: torch.Tensor | None = None) -> torch.Tensor:
    """Rotate the rows of a 2-D GPU tensor (f32/bf16/f16) into a fresh fp32
    [rows, cols_pad] GPU tensor (rot_size 1 = convert only).  With
    zero_above > 0, |w| > zero_above is zeroed first and counted into the
    int64 GPU tensor ``n_zeroed``.  Internal fast path used by the pipeline."""
    W = W.contiguous()
    rows, cols = W.shape
    cols_pad = -(-cols // rot_size) * rot_size
    out = torch.empty(rows, cols_pad, dtype=torch.float32, device=W.device)
    L = nat.lib()
    exact = _kernel == "exact" and rot_size <= 512
    fn, name = (L.ic_rotate_rows_exact, "ic_rotate_rows_exact") if exact else (L.ic_rotate_rows, "ic_rotate_rows")
    nat.check(fn(W, nat.dtype_code(W), rows, cols, cols, out, cols_pad, cols_pad, rot_size,
                 float(zero_above), nat.ptr(n_zeroed), nat.stream()), name)
    return out


def rotate_weights(W: torch.Tensor, rot_size: int) -> torch.Tensor:
    """[out, in] -> [out, in_padded]: zero-pad to a multiple of ``rot_size`` and
    rotate every group of ``rot_size`` columns (reference rotation.py:95-125).
    The result has W's dtype and device; arithmetic is fp32."""
    if W.dim() != 2:
        raise ValueError(f"Expected 2D tensor, got {W.dim()}D")
    _check_rot(rot_size)
    if W.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        W = W.float()
    out = rotate_rows_gpu(nat.to_gpu(W), rot_size)
    if W.dtype != torch.float32:
        out = out.to(W.dtype)
    return out.to(W.device)


def rotate_activations(x: torch.Tensor, rot_size: int) -> torch.Tensor:
    """Same rotation on the last dimension of any-rank activations
    (reference rotation.py:128-153)."""
    _check_rot(rot_size)
    lead = x.shape[:-1]
    flat = x.reshape(-1, x.shape[-1])
    out = rotate_weights(flat, rot_size) if flat.shape[0] > 0 else F.pad(flat, (0, (-flat.shape[1]) % rot_size))
    return out.reshape(*lead, out.shape[-1])


def _check_hessian_rot(rot_size: int) -> None:
    # rotate_hessian takes the regular (power-of-4) matrix only
    # (converter/rotation.py:247 -> get_hadamard -> make_hadamard_regular)
    if not _is_power_of_four(rot_size):
        raise ValueError(f"Regular Hadamard requires power of 4, got {rot_size}. Use rot_size=16/64/256.")


def rotate_hessian_gpu(H: torch.Tensor, rot_size: int, lower_only: bool = False,
                       inplace: bool = False) -> torch.Tensor:
    """R^T H R of a 2-D or 3-D fp32 GPU Hessian (padded first for 2-D).
    Internal fast path used by the GPTQ/LDLQ drivers.  ``inplace``: H (a
    contiguous fp32 tensor the caller owns) is overwritten when no padding
    is needed.  ``lower_only`` (2-D, exact kernel): only the rot x rot blocks
    on and below the block diagonal are rotated - all that the lower Cholesky
    factorisation and the damping read; the other entries are unspecified
    (in place: input values or partial results, out of place: unset)."""
    _check_hessian_rot(rot_size)
    H = H.float().contiguous()
    if H.dim() == 2 and H.shape[0] % rot_size:
        p = rot_size - H.shape[0] % rot_size
        src = out = F.pad(H, (0, p, 0, p))          # a new tensor: rotated in place
    elif inplace:
        src = out = H
    else:
        src, out = H, torch.empty_like(H)          # the first pass reads H and writes out
    batch, n = (1, out.shape[0]) if out.dim() == 2 else (out.shape[0], out.shape[1])
    if out.numel():
        L = nat.lib()
        if _kernel == "exact" and rot_size <= 256:
            nat.check(L.ic_rotate_hessian_exact(src, out, batch, n, n, rot_size,
                                                int(bool(lower_only) and batch == 1), nat.stream()),
                      "ic_rotate_hessian_exact")
        else:
            nat.check(L.ic_rotate_hessian(src, out, batch, n, n, rot_size, nat.stream()),
                      "ic_rotate_hessian")
    return out


def rotate_hessian(H, rot_size: int):
    """Hessian in the rotated weight space: H_rot = R^T H R (reference
    rotation.py:156-248).  2-D input is zero-padded to a multiple of
    ``rot_size``; 3-D [blocks, bs, bs] input needs bs % rot_size == 0; a DLR
    dict becomes the rotated dense 2-D Hessian (on the GPU).  Like the
    reference, only powers of 4 are accepted (its get_hadamard)."""
    if not _is_power_of_two(rot_size):
        raise ValueError(f"rot_size must be a power of 2, got {rot_size}")
    if isinstance(H, dict):
        # a DLR Hessian is densified first: rotation does not keep its structure
        from .dlr import dlr_to_dense, is_dlr
        if not is_dlr(H):
            raise ValueError("Expected a 2-D / 3-D tensor or a DLR dict Hessian")
        H = dlr_to_dense(H["D"], H["U"])
    if H.dim() == 2:
        if H.shape[0] != H.shape[1]:
            raise ValueError(f"Expected square Hessian, got {H.shape}")
    elif H.dim() == 3:
        if H.shape[1] != H.shape[2]:
            raise ValueError(f"Expected square blocks, got block shape ({H.shape[1]}, {H.shape[2]})")
        if H.shape[1] % rot_size != 0:
            raise ValueError(f"Block size {H.shape[1]} is not divisible by rot_size {rot_size}")
    else:
        raise ValueError(f"Expected 2D or 3D Hessian, got {H.dim()}D")
    _check_rot(rot_size)
    return rotate_hessian_gpu(nat.to_gpu(H), rot_size).to(H.device)
