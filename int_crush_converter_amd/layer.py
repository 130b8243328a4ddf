"""Per-layer GPU step of the pipeline (``converter/pipeline.py:511-1013``).

One call takes a weight tensor (any float dtype, CPU or GPU) and produces
the stored tensors on the GPU: outlier zeroing and ConvRot rotation in one
pass (``ic_rotate_rows``), RTN / GPTQ quantisation, the fp64 verification
(``ic_quant_error``), the bad-scale repair and INT4 packing.  ``bench.py``
times exactly this function.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from . import _native as nat
from .dlr import dlr_to_dense, is_dlr, woodbury_inverse
from .config import INT4_SCALE_DIVISOR, INT8_SCALE_DIVISOR, SCALE_MAX, SCALE_MIN, WEIGHT_OUTLIER_CLAMP
from .gptq import launch_quant_error, row_params, scale_operand, sweep, sweep_block_diagonal
from .hessian import inverse_batch
from .rotation import rotate_rows_gpu, rotate_hessian_gpu
from . import scales as _scales


@dataclass
class LayerOutput:
    stored: torch.Tensor                 # uint8 packed [M, ceil(N/2)] (INT4) or int8 [M, N] (INT8)
    scales: torch.Tensor                 # fp16 [M, 1] (fp32 after some repairs, like the reference)
    zero_points: torch.Tensor | None     # int8 [M, 1]
    codes: torch.Tensor                  # int8 [M, N]
    W_work: torch.Tensor                 # fp32 rotated weights [M, N]
    mse: float = 0.0
    max_err: float = 0.0
    method: str = "rtn"
    fallbacks: list[str] = field(default_factory=list)
    outliers: int = 0
    bad_scales: bool = False
    perm: torch.Tensor | None = None     # PermuQuant column permutation (int64), if applied


def prepare_weights(tensor: torch.Tensor, rot_size: int) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 GPU W_work (outliers zeroed, rotated when rot_size > 0) and the
    outlier count (int64 GPU scalar)."""
    Wg = nat.to_gpu(tensor)
    if Wg.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        Wg = Wg.float()
    nz = torch.zeros(1, dtype=torch.int64, device=Wg.device)
    W_work = rotate_rows_gpu(Wg, rot_size if rot_size > 0 else 1, WEIGHT_OUTLIER_CLAMP, nz)
    return W_work, nz


def rtn_codes(W_work: torch.Tensor, int_bits: int, asymmetric: bool, clipping_ratios):
    """RTN (converter/pipeline.py:890-917): fp16 scales, int8 zp, codes and
    (INT4) packed bytes in one quantisation pass."""
    M, N = W_work.shape
    ratios = _scales._ratios(clipping_ratios)
    s16, zp = _scales._scales_rows(W_work, int_bits, asymmetric, ratios)
    codes = torch.empty(M, N, dtype=torch.int8, device=W_work.device)
    packed = torch.empty(M, (N + 1) // 2, dtype=torch.uint8, device=W_work.device) if int_bits == 4 else None
    z = None if zp is None else zp.float()
    nat.check(nat.lib().ic_rtn_quantize(W_work, M, N, N, int_bits, s16, 0, nat.ptr(z),
                                        codes, N, nat.ptr(packed), packed.shape[1] if packed is not None
                                        else 0, nat.stream()), "ic_rtn_quantize")
    return codes, s16.reshape(M, 1), None if zp is None else zp.reshape(M, 1), packed


def _gptq_params(W_work, int_bits, asymmetric, piso):
    if piso is not None:
        from .piso import piso_row_params
        p = piso_row_params(W_work, piso[0], piso[1], int_bits, asymmetric)
        if p is not None:
            return p
    return row_params(W_work, int_bits, asymmetric)


def gptq_codes(W_work: torch.Tensor, H: torch.Tensor, *, rotate_h: int, block_size: int, damping: float,
               int_bits: int, asymmetric: bool, hessian_method: str, fallbacks: list[str], piso=None):
    """GPTQ on a rotated W_work with a (raw or rotated) 2-D / 3-D Hessian, or
    a DLR Hessian (densified when it is to be rotated, as rotation.py:181-184
    does; else inverted by the Woodbury identity, gptq.py:322-342).  ``piso``:
    (scales [M, 1], zero-points [M, 1] or None) from the PiSO search, which
    replace the row scales (gptq.py:210-252)."""
    M, N = W_work.shape
    if is_dlr(H):
        if rotate_h <= 0:
            D, U = H["D"], H["U"]
            if D.shape[0] != N:
                raise ValueError(f"DLR Hessian dim {D.shape[0]} != in_features {N}")
            s32, z32, s16, z8 = _gptq_params(W_work, int_bits, asymmetric, piso)
            Hinv = woodbury_inverse(D, U, damping, W_work.device, upper_only=True)
            Q = sweep(W_work, Hinv, s32, z32, int_bits, block_size)
            return Q, s16.reshape(M, 1), None if z8 is None else z8.reshape(M, 1)
        H = dlr_to_dense(H["D"], H["U"])
    Hsrc = nat.to_gpu(H).float()
    # a 2-D Hessian is factored from its lower triangle only, so only the
    # blocks on and below the diagonal are rotated (the fallback chain's
    # restore() below rotates the whole matrix); a copy made here is rotated
    # in place
    Hg = (rotate_hessian_gpu(Hsrc, rotate_h, lower_only=Hsrc.dim() == 2, inplace=Hsrc.data_ptr() != H.data_ptr())
          if rotate_h > 0 else Hsrc)
    # a Hessian this function created (rotated, or copied to the GPU / fp32)
    # is inverted in place; the fallback chain rebuilds it from the caller's
    # untouched one
    own = Hg.data_ptr() != H.data_ptr() and Hg.is_contiguous()

    def restore():
        src = nat.to_gpu(H).float()
        return rotate_hessian_gpu(src, rotate_h) if rotate_h > 0 else src

    inv_kw = dict(inplace=True, restore=restore, upper_only=True) if own else dict(upper_only=True)
    s32, z32, s16, z8 = _gptq_params(W_work, int_bits, asymmetric, piso)
    # the sweep reads W_work and keeps its working residual elsewhere
    if Hg.dim() == 3:
        Q = sweep_block_diagonal(W_work, Hg, damping, hessian_method, fallbacks, s32, z32, int_bits, block_size)
    else:
        if tuple(Hg.shape) != (N, N):
            raise ValueError(f"Hessian shape {tuple(Hg.shape)} != ({N}, {N})")
        Hinv = inverse_batch(Hg, damping, hessian_method, fallbacks, **inv_kw)
        Q = sweep(W_work, Hinv, s32, z32, int_bits, block_size)
    return Q, s16.reshape(M, 1), None if z8 is None else z8.reshape(M, 1)


def pack_codes(codes: torch.Tensor) -> torch.Tensor:
    from .packing import _validate_rows
    M, N = codes.shape
    out = torch.empty(M, (N + 1) // 2, dtype=torch.uint8, device=codes.device)
    _validate_rows(codes, 0, out)
    return out


def _div(x: torch.Tensor, d: float) -> torch.Tensor:
    """IEEE x / d (a 0-dim device tensor divisor keeps the true division)."""
    return x / torch.tensor(d, dtype=x.dtype, device=x.device)


def _rhaz(x):
    return torch.where(x >= 0, torch.floor(x + 0.5), torch.ceil(x - 0.5))


def _fix_asym(s, wmin, wmax, qmin, qmax):
    spread = float(qmax - qmin)
    zraw = qmin - _rhaz(wmin / s)
    lo, hi = zraw < qmin, zraw > qmax
    if lo.any():
        f = _div(wmax.float(), spread).clamp(min=SCALE_MIN, max=SCALE_MAX)
        s = torch.maximum(s, torch.where(lo, f, s))
    if hi.any():
        f = _div(-wmin.float(), spread).clamp(min=SCALE_MIN, max=SCALE_MAX)
        s = torch.maximum(s, torch.where(hi, f, s))
    return s


def repair_bad_scales(W_work, codes, scales, zero_points, is_int8):
    """Replace Inf/NaN/0 scales and re-quantise their rows, statement for
    statement like converter/pipeline.py:938-1007 (a rare error path; runs as
    torch GPU ops with tensor divisors so every division stays IEEE)."""
    bad = scales.isinf() | scales.isnan() | (scales == 0)
    div = INT8_SCALE_DIVISOR if is_int8 else INT4_SCALE_DIVISOR
    sym = _div(W_work.float().abs().amax(dim=1, keepdim=True), div).clamp(min=SCALE_MIN, max=SCALE_MAX).to(torch.float16)
    qmin, qmax = (-128, 127) if is_int8 else (-8, 7)
    wmin = W_work.amin(dim=1, keepdim=True)
    wmax = W_work.amax(dim=1, keepdim=True)
    rows = bad.squeeze(1).nonzero(as_tuple=True)[0].tolist()
    if zero_points is not None:
        spread = 255.0 if is_int8 else 15.0
        asym = _div((wmax - wmin).float(), spread).clamp(min=SCALE_MIN, max=SCALE_MAX).to(torch.float16)
        asym = _fix_asym(asym, wmin, wmax, qmin, qmax)
        ok = bad & torch.isfinite(asym) & (asym > 0)
        scales = torch.where(bad, torch.where(ok, asym, sym), scales)
        for r in rows:
            rs = scales[r].to(W_work.dtype)
            rz = (qmin - _rhaz(W_work[r].amin() / rs)).clamp(qmin, qmax)
            zero_points[r] = rz.to(zero_points.dtype)
            codes[r] = _rhaz(W_work[r] / rs + rz.to(W_work.dtype)).clamp(qmin, qmax).to(torch.int8)
    else:
        scales = torch.where(bad, sym, scales)
        if not is_int8:
            asym = _div((wmax - wmin).float(), 15.0).clamp(min=SCALE_MIN, max=SCALE_MAX).to(torch.float16)
            asym = _fix_asym(asym, wmin, wmax, -8, 7)
            ok = bad & torch.isfinite(asym) & (asym > 0)
            scales = torch.where(bad, torch.where(ok, asym, sym), scales)
            zero_points = torch.zeros(W_work.shape[0], 1, dtype=torch.int8, device=W_work.device)
        for r in rows:
            rs = scales[r].to(W_work.dtype)
            if not is_int8:
                rz = (-8 - _rhaz(W_work[r].amin() / rs)).clamp(-8, 7)
                codes[r] = _rhaz(W_work[r] / rs + rz.to(W_work.dtype)).clamp(-8, 7).to(torch.int8)
                zero_points[r] = rz.to(zero_points.dtype)
            else:
                codes[r] = _rhaz(W_work[r] / rs).clamp(qmin, qmax).to(torch.int8)
    return codes, scales, zero_points, int(bad.sum().item())


def finish(W_work, codes, s16, z8, int_bits, packed=None, **kw) -> LayerOutput:
    """Verification, bad-scale repair and packing (pipeline.py:919-1013).

    The verification sums, the bad-scale test and (INT4) the packing with its
    range check are enqueued together and read back in one transfer; rows
    with bad scales are repaired and re-packed afterwards (a rare path)."""
    M, N = codes.shape
    dev = codes.device
    # one status block: [0] fp64 sum of squares, bytes 8..11 fp32 max |error|,
    # int32 [3] bad-scale flag, int32 [4:7] packing flags (non-finite, < -8, > 7)
    status = torch.zeros(4, dtype=torch.float64, device=dev)
    base = status.data_ptr()
    if W_work.numel():
        launch_quant_error(W_work, codes, s16, z8, base, base + 8)
    sc, kind = scale_operand(s16)
    nat.check(nat.lib().ic_scale_status(sc, kind, sc.numel(), base + 12, nat.stream()), "ic_scale_status")
    if int_bits == 4 and packed is None:
        packed = torch.empty(M, (N + 1) // 2, dtype=torch.uint8, device=dev)
        if codes.numel():
            nat.check(nat.lib().ic_pack_int4(codes, 0, M, N, N, packed, packed.shape[1],
                                             base + 16, nat.stream()), "ic_pack_int4")
    host = status.cpu()
    words = host.view(torch.int32)
    mse = host[0].item() / W_work.numel() if W_work.numel() else float("nan")
    max_err = host[1:2].view(torch.float32)[0].item() if W_work.numel() else 0.0
    bad = bool(words[3].item())
    if bad:
        codes, s16, z8, _ = repair_bad_scales(W_work, codes, s16, z8, int_bits == 8)
        packed = pack_codes(codes) if int_bits == 4 else None
    elif int_bits == 4:
        nf, lo, hi = (int(v) for v in words[4:7].tolist())
        if nf or lo or hi:
            pack_codes(codes)   # raises the reference's INT4PackingError
    stored = codes if int_bits == 8 else packed
    return LayerOutput(stored=stored, scales=s16, zero_points=z8, codes=codes, W_work=W_work, mse=mse,
                       max_err=max_err, bad_scales=bad, **kw)
