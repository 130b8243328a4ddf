"""CPU oracle for the per-layer quantization path.  TEST INFRASTRUCTURE ONLY.

This module restates, op for op in PyTorch on the CPU, the arithmetic of the
reference's CPU backends (``converter/rotation.py``, ``scales.py``,
``rounding.py``, ``packing.py``, ``gptq.py``, ``ldlq.py``, ``greedy.py`` and
the per-layer step of ``pipeline.py``).  The same torch calls in the same
order give the same fp32 roundings, so results here are what the reference's
CPU path produces on the same inputs.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker or as the timed CPU
baseline.  The product package never imports it.

Parity pinning (how each function is checked against something other than
itself; see tests/test_oracle.py):
  * hadamard_regular / hadamard_sylvester: closed form (involution, entries
    +-2^-k, Kronecker structure), reference KATs of tests/test_rotation.py.
  * rotate_weights / rotate_hessian: the reference's own outputs, bit for
    bit (tests/golden/golden_rotation.safetensors: every rot to 512, 2-D /
    3-D Hessians); an independent numpy restatement of the sequential fp32
    chains; brute-force dense R, norm and trace preservation, (XR)^T(XR)
    identity.  The products run in rotation_seq.c (C, no BLAS) so the
    oracle rounds like the reference on any host.
  * rhaz: reference KATs (tests/unit/test_ldlq_hessian.py:34-49), numpy.
  * rtn_* scale/quantize functions: reference KAT (tests/test_scales.py:48-55),
    numpy float32 restatement of every formula, brute-force clip search.
  * pack_int4 / unpack_int4: KAT bytes + round trip (tests/test_packing.py).
  * invert_hessian / prepare_hinv: H @ Hinv ~ I, fp64 inverse.
  * gptq_block / ldlq_loop: brute-force column-by-column float32 numpy loop
    on tiny shapes; golden vectors from the reference (tests/golden/).
  * greedy_pytorch: coordinate-wise optimality by brute force; golden vectors.
  * lowrank_decompose: planted spectra (H = V diag(l) V^T with known l) for
    the rank count and both gates; eigen-equation residual.
  * greedy_lowrank_loop: with the full eigendecomposition (k = N) it is the
    exact greedy_pytorch; golden vectors of the reference's own low-rank
    kernel and its full-rank v2 path (Triton interpreter, tests/golden/).
  * iterative LDLQ / final least-squares scales: golden vectors.
  * PermuQuant (channel_second_moments .. permuquant_layer): the same torch
    CPU calls as permuquant.py, so torch's own reductions fix the results;
    pinned by the reference's KATs (tests/unit/test_permuquant_channel.py:
    formula [[2,-1],[0,3]] -> [2, 5], descending moments, a scaled channel
    first, alpha 0 = weight-only, alpha 1 = activation order, zero matrix
    rejected), by brute force (sorted order, valid permutation), and by the
    identity that per-row errors of W and W[:, perm] are the same multiset
    (equal in exact arithmetic, so fp64 sums agree).
  * piso_scales_sym / piso_scales_asym: brute force in fp64 on small rows
    (every candidate's error; the chosen one is within fp32 rounding of the
    smallest and is a table entry times the stage's base), the reference's
    behaviour tests (tests/gpu/test_piso_triton.py:86-170, 470-516: shapes,
    positive scales, all-zero rows, large weights, zero-point range), and a
    planted case whose optimum is known in closed form.
  * woodbury_inverse / dlr_to_dense: the fp64 dense inverse of the damped
    diag(D) + U U^T and the reference's KATs (tests/unit/
    test_dlr_hessian.py:142-235: damping definition, H H^-1 = I, U = 0 gives
    diag(1/D), rank one equals Sherman-Morrison's closed form, zero diagonal
    entries stay finite, symmetry); a factor permutation equals
    H[perm][:, perm] of the dense form.
"""

from __future__ import annotations

import math
import warnings

import torch
import torch.nn.functional as F

SCALE_MIN = 1e-5
SCALE_MAX = 65500.0
DIAG_MEAN_FLOOR = 1e-6
ERR_CLAMP = 100.0
HINV_DIAG_FLOOR = 1e-8
SCALE_FLOOR = 1e-8
EIGENVALUE_FLOOR = 1e-12      # config.py:124
STALL_THRESHOLD = 0.99        # config.py:128
LOWRANK_MAX_RANK_FRAC = 0.3   # config.py:133
LOWRANK_MAX_K = 512           # config.py:137
GREEDY_COL_BLOCK = 64         # config.py:177


# --------------------------------------------------------------------------
# Hadamard rotation  (converter/rotation.py:26-125, 156-248)
# --------------------------------------------------------------------------

def is_pow2(n: int) -> bool:
    return n > 0 and (n & (n - 1)) == 0


def is_pow4(n: int) -> bool:
    # rotation.py:16-19
    return n >= 4 and is_pow2(n) and (n & 0x55555555) == n


def hadamard_regular(n: int, dtype=torch.float32) -> torch.Tensor:
    """(H4/2)^{kron k}; rotation.py:39-62."""
    h4 = torch.tensor([[1.0, 1.0, 1.0, -1.0],
                       [1.0, 1.0, -1.0, 1.0],
                       [1.0, -1.0, 1.0, 1.0],
                       [-1.0, 1.0, 1.0, 1.0]], dtype=dtype) / 2.0
    out = h4
    while out.shape[0] < n:
        out = torch.kron(out, h4)
    return out


def hadamard_sylvester(n: int, dtype=torch.float32) -> torch.Tensor:
    """kron([[1,1],[1,-1]], .) * fp(1/sqrt(n)); rotation.py:26-36."""
    out = torch.tensor([[1.0]], dtype=dtype)
    base = torch.tensor([[1.0, 1.0], [1.0, -1.0]], dtype=dtype)
    while out.shape[0] < n:
        out = torch.kron(base, out)
    return out * (1.0 / math.sqrt(n))


def _hadamard_for(n: int, dtype) -> torch.Tensor:
    return hadamard_regular(n, dtype) if is_pow4(n) else hadamard_sylvester(n, dtype)


_ROT_LIB = None


def _rot_lib():
    """ctypes handle of rotation_seq.c (built by oracle/build.py, on demand
    where gcc exists)."""
    global _ROT_LIB
    if _ROT_LIB is None:
        import ctypes
        import os
        from oracle import build as _b
        if not os.path.exists(_b.LIB):
            _b.build()
        lib = ctypes.CDLL(_b.LIB)
        for fn in (lib.oracle_rotate_rows, lib.oracle_rotate_blocks):
            fn.restype = ctypes.c_int
        lib.oracle_rotate_rows.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
                                           ctypes.c_int, ctypes.c_int]
        lib.oracle_rotate_blocks.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int,
                                             ctypes.c_int]
        _ROT_LIB = lib
    return _ROT_LIB


def rotate_weights(W: torch.Tensor, rot: int) -> torch.Tensor:
    """Pad the last dim to a multiple of ``rot``, then ``x @ H.T`` per group
    (rotation.py:95-125).  For fp32 and rot 2 .. 512 the product is the C
    restatement of the reference's rounding (rotation_seq.c: sequential fma
    chains, as the reference's CPU sgemm rounds); otherwise torch's matmul."""
    M, N = W.shape
    if N % rot:
        W = F.pad(W, (0, rot - N % rot))
    g = W.shape[1] // rot
    if W.dtype == torch.float32 and 2 <= rot <= 512 and W.numel():
        x = W.contiguous()
        out = torch.empty_like(x)
        if _rot_lib().oracle_rotate_rows(x.data_ptr(), M, x.shape[1], out.data_ptr(), rot,
                                         torch.get_num_threads()) != 0:
            raise RuntimeError("oracle_rotate_rows failed")
        return out
    Hm = _hadamard_for(rot, W.dtype)
    return (W.reshape(M, g, rot) @ Hm.T).reshape(M, -1)


def rotate_hessian(H: torch.Tensor, rot: int) -> torch.Tensor:
    """R^T H R on 2-D or 3-D Hessians (rotation.py:156-248).  Only the
    regular matrix: rotation.py:247 takes it from get_hadamard, which raises
    for sizes that are not powers of 4 (rotation.py:45-47)."""
    if not is_pow4(rot):
        raise ValueError(f"Regular Hadamard requires power of 4, got {rot}. Use rot_size=16/64/256.")
    H = H.float()
    R = hadamard_regular(rot, H.dtype)

    def blocks(h3):
        # the einsum's two products, each as sequential fma chains
        # (rotation_seq.c), for the sizes whose order is pinned
        if rot <= 256 and h3.numel():
            h3 = h3.contiguous()
            out = torch.empty_like(h3)
            if _rot_lib().oracle_rotate_blocks(h3.data_ptr(), h3.shape[0], out.data_ptr(), rot,
                                               torch.get_num_threads()) != 0:
                raise RuntimeError("oracle_rotate_blocks failed")
            return out
        return torch.einsum("kp, nkl, le -> npe", R, h3, R)

    if H.dim() == 2:
        n = H.shape[0]
        if n % rot:
            p = rot - n % rot
            H = F.pad(H, (0, p, 0, p))
            n = H.shape[0]
        nb = n // rot
        flat = H.reshape(nb, rot, nb, rot).permute(0, 2, 1, 3).reshape(nb * nb, rot, rot)
        flat = blocks(flat)
        return flat.reshape(nb, nb, rot, rot).permute(0, 2, 1, 3).reshape(n, n)
    nblk, bs, _ = H.shape
    if bs == rot:
        return blocks(H)
    ns = bs // rot
    flat = H.reshape(nblk, ns, rot, ns, rot).permute(0, 1, 3, 2, 4).reshape(nblk * ns * ns, rot, rot)
    flat = blocks(flat)
    return flat.reshape(nblk, ns, ns, rot, rot).permute(0, 1, 3, 2, 4).reshape(nblk, bs, bs)


# --------------------------------------------------------------------------
# Rounding, scales, RTN  (converter/rounding.py:106-112, scales.py:25-384)
# --------------------------------------------------------------------------

def rhaz(x: torch.Tensor) -> torch.Tensor:
    """Round half away from zero with the literal ``x + 0.5`` (rounding.py:106-112)."""
    return torch.where(x >= 0, torch.floor(x + 0.5), torch.ceil(x - 0.5))


def _clip_search(ratios, fn):
    # scales.py:25-59: strict '<', first ratio wins ties
    best_s = best_z = best_m = None
    for r in ratios:
        s, z, m = fn(r)
        if best_s is None:
            best_s, best_z, best_m = s, z, m
            continue
        better = m < best_m
        best_s = torch.where(better, s, best_s)
        if z is not None:
            best_z = torch.where(better, z, best_z)
        best_m = torch.where(better, m, best_m)
    return best_s, best_z


def fix_asym_scale(s, wmin, wmax, qmin, qmax):
    """scales.py:184-229."""
    spread = float(qmax - qmin)
    zraw = qmin - rhaz(wmin / s)
    lo = zraw < qmin
    hi = zraw > qmax
    if lo.any():
        f = (wmax.float() / spread).clamp(min=SCALE_MIN, max=SCALE_MAX)
        s = torch.maximum(s, torch.where(lo, f, s))
    if hi.any():
        f = (-wmin.float() / spread).clamp(min=SCALE_MIN, max=SCALE_MAX)
        s = torch.maximum(s, torch.where(hi, f, s))
    return s


def _norm_ratios(ratios):
    if ratios is not None and len(ratios) == 0:
        return None
    return ratios


def _pad_groups(W, gs):
    if W.shape[1] % gs:
        W = F.pad(W, (0, gs - W.shape[1] % gs))
    return W


def scales_int4_sym(W, group_size=None, ratios=None):
    """calculate_scales (scales.py:62-99).  group_size None = per row."""
    ratios = _norm_ratios(ratios)
    gs = W.shape[1] if group_size is None else group_size
    Wp = _pad_groups(W, gs)
    M, Np = Wp.shape
    Wg = Wp.reshape(M, Np // gs, gs)
    amax = Wg.abs().amax(dim=2)
    if ratios is None:
        return (amax.float() / 7.0).clamp(min=SCALE_MIN, max=SCALE_MAX).to(torch.float16)

    def cand(r):
        s = (amax.float() * r / 7.0).clamp(min=SCALE_MIN, max=SCALE_MAX)
        q = (Wg / s.unsqueeze(2)).round().clamp(-8, 7)
        return s, None, (Wg - q * s.unsqueeze(2)).pow(2).mean(dim=2)

    return _clip_search(ratios, cand)[0].to(torch.float16)


def quant_int4_sym(W, scales, group_size=None):
    """quantize_weights (scales.py:102-123)."""
    gs = W.shape[1] if group_size is None else group_size
    Wp = _pad_groups(W, gs)
    M, Np = Wp.shape
    Wg = Wp.reshape(M, Np // gs, gs)
    q = rhaz(Wg / scales.unsqueeze(2).to(Wp.dtype)).clamp(-8, 7)
    return q.reshape(M, Np).to(torch.int8)


def scales_int8_sym(W, ratios=None):
    """calculate_scales_int8 (scales.py:126-160)."""
    ratios = _norm_ratios(ratios)
    amax = W.abs().amax(dim=1, keepdim=True)
    if ratios is None:
        return (amax.float() / 127.0).clamp(min=SCALE_MIN, max=SCALE_MAX).to(torch.float16)
    W3 = W.unsqueeze(1)

    def cand(r):
        s = (amax.float() * r / 127.0).clamp(min=SCALE_MIN, max=SCALE_MAX)
        q = (W3 / s.unsqueeze(2)).round().clamp(-128, 127)
        return s, None, (W3 - q * s.unsqueeze(2)).pow(2).mean(dim=2)

    return _clip_search(ratios, cand)[0].to(torch.float16)


def quant_int8_sym(W, scales):
    """quantize_weights_int8 (scales.py:163-178)."""
    return rhaz(W / scales.to(W.dtype)).clamp(-128, 127).to(torch.int8)


def scales_int4_asym(W, group_size=None, ratios=None):
    """calculate_scales_asymmetric (scales.py:232-282)."""
    ratios = _norm_ratios(ratios)
    gs = W.shape[1] if group_size is None else group_size
    Wp = _pad_groups(W, gs)
    M, Np = Wp.shape
    Wg = Wp.reshape(M, Np // gs, gs)
    wmin = Wg.amin(dim=2)
    wmax = Wg.amax(dim=2)
    if ratios is None:
        s = ((wmax - wmin).float() / 15.0).clamp(min=SCALE_MIN, max=SCALE_MAX)
        s = fix_asym_scale(s, wmin, wmax, -8, 7)
        z = (-8 - rhaz(wmin / s)).clamp(-8, 7)
        z = z.masked_fill((wmin == 0) & (wmax == 0), 0)
        return s.to(torch.float16), z.to(torch.int8)

    def cand(r):
        s = ((wmax - wmin).float() * r / 15.0).clamp(min=SCALE_MIN, max=SCALE_MAX)
        s = fix_asym_scale(s, wmin, wmax, -8, 7)
        z = (-8 - rhaz(wmin / s)).clamp(-8, 7)
        q = (Wg / s.unsqueeze(2) + z.unsqueeze(2)).round().clamp(-8, 7)
        d = (q - z.unsqueeze(2)) * s.unsqueeze(2)
        return s, z, (Wg - d).pow(2).mean(dim=2)

    s, z = _clip_search(ratios, cand)
    return s.to(torch.float16), z.to(torch.int8)


def quant_int4_asym(W, scales, zps, group_size=None):
    """quantize_weights_asymmetric (scales.py:285-313)."""
    gs = W.shape[1] if group_size is None else group_size
    Wp = _pad_groups(W, gs)
    M, Np = Wp.shape
    Wg = Wp.reshape(M, Np // gs, gs)
    x = Wg / scales.unsqueeze(2).to(Wp.dtype) + zps.unsqueeze(2).to(Wp.dtype)
    return rhaz(x).clamp(-8, 7).reshape(M, Np).to(torch.int8)


def scales_int8_asym(W, ratios=None):
    """calculate_scales_int8_asymmetric (scales.py:316-361)."""
    ratios = _norm_ratios(ratios)
    wmin = W.amin(dim=1, keepdim=True)
    wmax = W.amax(dim=1, keepdim=True)
    if ratios is None:
        s = ((wmax - wmin).float() / 255.0).clamp(min=SCALE_MIN, max=SCALE_MAX)
        s = fix_asym_scale(s, wmin, wmax, -128, 127)
        z = (-128 - rhaz(wmin / s)).clamp(-128, 127)
        return s.to(torch.float16), z.to(torch.int8)
    W3 = W.unsqueeze(1)

    def cand(r):
        s = ((wmax - wmin).float() * r / 255.0).clamp(min=SCALE_MIN, max=SCALE_MAX)
        s = fix_asym_scale(s, wmin, wmax, -128, 127)
        z = (-128 - rhaz(wmin / s)).clamp(-128, 127)
        q = (W3 / s.unsqueeze(2) + z.unsqueeze(2)).round().clamp(-128, 127)
        d = (q - z.unsqueeze(2)) * s.unsqueeze(2)
        return s, z, (W3 - d).pow(2).mean(dim=2)

    s, z = _clip_search(ratios, cand)
    return s.to(torch.float16), z.to(torch.int8)


def quant_int8_asym(W, scales, zps):
    """quantize_weights_int8_asymmetric (scales.py:364-384)."""
    return rhaz(W / scales.to(W.dtype) + zps.to(W.dtype)).clamp(-128, 127).to(torch.int8)


# --------------------------------------------------------------------------
# INT4 packing  (converter/packing.py:17-66)
# --------------------------------------------------------------------------

def pack_int4(v: torch.Tensor) -> torch.Tensor:
    """Low nibble = even index, two's complement (packing.py:30-46)."""
    v = v.to(torch.int8)
    if v.shape[-1] % 2:
        v = torch.cat([v, torch.zeros(*v.shape[:-1], 1, dtype=torch.int8)], dim=-1)
    u = torch.where(v < 0, 16 + v, v).to(torch.uint8)
    return u[..., 0::2] | (u[..., 1::2] << 4)


def unpack_int4(p: torch.Tensor, K: int) -> torch.Tensor:
    lo = (p & 0x0F).to(torch.int8)
    hi = ((p >> 4) & 0x0F).to(torch.int8)
    lo = torch.where(lo >= 8, lo - 16, lo)
    hi = torch.where(hi >= 8, hi - 16, hi)
    out = torch.zeros(*p.shape[:-1], p.shape[-1] * 2, dtype=torch.int8)
    out[..., 0::2] = lo
    out[..., 1::2] = hi
    return out[..., :K]


# --------------------------------------------------------------------------
# Hessian inverse  (converter/rounding.py:19-34, gptq.py:91-121)
# --------------------------------------------------------------------------

def invert_hessian(H: torch.Tensor) -> torch.Tensor:
    try:
        return torch.cholesky_inverse(torch.linalg.cholesky(H))
    except torch.linalg.LinAlgError:
        pass
    try:
        return torch.linalg.inv(H)
    except torch.linalg.LinAlgError:
        warnings.warn("Hessian is singular; using pseudoinverse", stacklevel=2)
        return torch.linalg.pinv(H)


def damp(H: torch.Tensor, damping: float) -> torch.Tensor:
    dm = H.diagonal().mean().clamp(min=DIAG_MEAN_FLOOR)
    return H + damping * dm * torch.eye(H.shape[0], dtype=torch.float32)


def prepare_hinv(H, damping):
    """Full damped inverse (gptq.py:113-121)."""
    return invert_hessian(damp(H, damping))


def prepare_chol(H, damping):
    """Upper Cholesky factor of the damped inverse (gptq.py:91-110)."""
    Hi = invert_hessian(damp(H, damping))
    try:
        return torch.linalg.cholesky(Hi).T
    except torch.linalg.LinAlgError:
        return Hi


# --------------------------------------------------------------------------
# GPTQ  (converter/rounding.py:37-103, gptq.py:137-533)
# --------------------------------------------------------------------------

def gptq_block(Ww, Q, s, Hinv, c0, c1, B, qmin, qmax, zp=None):
    """Column sweep with eager in-block and lazy cross-block updates
    (rounding.py:37-103).  Mutates ``Ww`` and ``Q``."""
    M = Ww.shape[0]
    n = c1 - c0
    sv = s.squeeze(1)
    zv = zp.squeeze(1) if zp is not None else None
    for b0 in range(0, n, B):
        b1 = min(b0 + B, n)
        E = torch.zeros(M, b1 - b0, dtype=torch.float32)
        for jo in range(b1 - b0):
            jl = b0 + jo
            jg = c0 + jl
            col = Ww[:, jg]
            if zv is not None:
                q = rhaz(col / sv + zv).clamp(qmin, qmax)
                deq = (q - zv) * sv
            else:
                q = rhaz(col / sv).clamp(qmin, qmax)
                deq = q * sv
            Q[:, jg] = q.to(torch.int8)
            e = (col - deq) / Hinv[jl, jl]
            e = e.clamp(-ERR_CLAMP, ERR_CLAMP)
            e = torch.nan_to_num(e, nan=0.0, posinf=ERR_CLAMP, neginf=-ERR_CLAMP)
            E[:, jo] = e
            if jo < b1 - b0 - 1:
                Ww[:, jg + 1:c0 + b1] -= e.unsqueeze(1) * Hinv[jl, jl + 1:b1].unsqueeze(0)
        if b1 < n:
            Ww[:, c0 + b1:c1] -= E @ Hinv[b0:b1, b1:n]


def gptq_row_params(W, int_bits, asymmetric):
    """Per-row fp32 scales and zero-points used by the sweep (gptq.py:254-317).
    Returns (scales fp32 [M,1], zp int8 [M,1] or None)."""
    if int_bits == 4 or asymmetric:
        qmin, qmax, spread = (-8, 7, 15.0) if int_bits == 4 else (-128, 127, 255.0)
        wmin = W.amin(dim=1, keepdim=True)
        wmax = W.amax(dim=1, keepdim=True)
        s = ((wmax - wmin).float() / spread).clamp(min=SCALE_MIN, max=SCALE_MAX)
        zraw = qmin - rhaz(wmin / s)
        lo = zraw < qmin
        hi = zraw > qmax
        if lo.any():
            f = (wmax.float() / spread).clamp(min=SCALE_MIN, max=SCALE_MAX)
            s = torch.maximum(s, torch.where(lo, f, s))
        if hi.any():
            f = (-wmin.float() / spread).clamp(min=SCALE_MIN, max=SCALE_MAX)
            s = torch.maximum(s, torch.where(hi, f, s))
        z = (qmin - rhaz(wmin / s)).clamp(qmin, qmax)
        z = z.masked_fill((wmin == 0) & (wmax == 0), 0)
        return s, z.to(torch.int8)
    s = (W.abs().amax(dim=1, keepdim=True) / 127.0).clamp(min=SCALE_MIN, max=SCALE_MAX)
    return s, None


def gptq_quantize_layer(W, H, block_size=128, damping=0.01, int_bits=4,
                        asymmetric=False, hessian_method="hinv"):
    """gptq.py:137-417 without the PiSO branch.  A DLR dict H takes the
    Woodbury inverse straight into the column loop (gptq.py:322-342)."""
    W = W.float()
    M, N = W.shape
    qmin, qmax = (-128, 127) if int_bits == 8 else (-8, 7)
    prep = prepare_hinv if hessian_method == "hinv" else prepare_chol
    s, z = gptq_row_params(W, int_bits, asymmetric)
    Q = torch.zeros_like(W, dtype=torch.int8)
    Ww = W.clone()
    if isinstance(H, dict):
        if H["D"].shape[0] != N:
            raise ValueError(f"DLR Hessian dim {H['D'].shape[0]} != in_features {N}")
        gptq_block(Ww, Q, s, woodbury_inverse(H["D"], H["U"], damping), 0, N, block_size, qmin, qmax, z)
    elif H.dim() == 3:
        nb, bs, _ = H.shape
        for bi in range(nb):
            c0 = bi * bs
            c1 = min(c0 + bs, N)
            Hb = H[bi, :c1 - c0, :c1 - c0].float()
            gptq_block(Ww, Q, s, prep(Hb, damping), c0, c1, block_size, qmin, qmax, z)
    else:
        gptq_block(Ww, Q, s, prep(H.float(), damping), 0, N, block_size, qmin, qmax, z)
    deq = Q.float() * s.float()
    if z is not None:
        deq = (Q.float() - z.float()) * s.float()
    from types import SimpleNamespace
    return SimpleNamespace(
        quantized_W=Q, scales=s.to(torch.float16), zero_points=z,
        scales_fp32=s,
        mse=(W - deq).double().pow(2).mean().item(),
        max_err=(W - deq).abs().max().item(),
        method_used="gptq_pytorch")


def rtn_layer(W, int_bits=4, asymmetric=False, ratios=None):
    """gptq_quantize_layer_rtn without PiSO (gptq.py:420-533): returns
    (q int8, scales fp16, zp int8 or None)."""
    if asymmetric:
        if int_bits == 8:
            s, z = scales_int8_asym(W, ratios)
            return quant_int8_asym(W, s, z), s, z
        s, z = scales_int4_asym(W, W.shape[1], ratios)
        return quant_int4_asym(W, s, z, W.shape[1]), s, z
    if int_bits == 8:
        s = scales_int8_sym(W, ratios)
        return quant_int8_sym(W, s), s, None
    s = scales_int4_sym(W, W.shape[1], ratios)
    return quant_int4_sym(W, s, W.shape[1]), s, None


# --------------------------------------------------------------------------
# LDLQ  (converter/ldlq.py:95-599, rounding.py:115-155)
# --------------------------------------------------------------------------

def ldlq_round_column(col, sc, qmin, qmax):
    """rounding.py:115-155 (sign flip is inert for positive scales)."""
    ss = sc.clamp(min=SCALE_FLOOR)
    q = rhaz(col / ss).clamp(float(qmin), float(qmax))
    wsgn = torch.where(col.abs() > 1e-8, col.sign(), q.sign())
    flip = (wsgn * q.sign()) < 0
    can = flip & (q > float(qmin))
    q = torch.where(flip & (q == float(qmin)), torch.full_like(q, float(qmax)), q)
    q = torch.where(can, -q, q).clamp(float(qmin), float(qmax))
    return q, col - q * ss


def ldlq_loop_cpu(Ww, Hinv, S, Q, N, M, B, qmin, qmax):
    """ldlq.py:369-417: reciprocal-multiply normalisation, no +-100 clamp."""
    for i1 in range(0, N, B):
        i2 = min(i1 + B, N)
        nb = i2 - i1
        Hb = Hinv[i1:i2, i1:i2]
        dinv = (1.0 / torch.diag(Hb).clamp(min=HINV_DIAG_FLOOR)).to(torch.float32)
        E = torch.zeros(M, nb, dtype=torch.float32)
        for jl in range(nb):
            j = i1 + jl
            q, e = ldlq_round_column(Ww[:, j], S[:, j], qmin, qmax)
            Q[:, j] = q.to(torch.int8)
            en = e * dinv[jl]
            E[:, jl] = en
            if jl + 1 < nb:
                Ww[:, j + 1:i2] -= en.unsqueeze(1) * Hb[jl, jl + 1:nb].unsqueeze(0)
        if i2 < N:
            Ww[:, i2:] -= E @ Hinv[i1:i2, i2:]
    return Q


def ldlq_single_pass(W, Hinv, flat_scales, B, qmin, qmax):
    M, N = W.shape
    Q = torch.zeros(M, N, dtype=torch.int8)
    Ww = W.clone()
    S = flat_scales.reshape(M, N)
    if not torch.isfinite(S).all():
        S = torch.nan_to_num(S, nan=1e-8, posinf=1e30, neginf=1e-8).clamp(min=1e-8)
    return ldlq_loop_cpu(Ww, Hinv, S, Q, N, M, B, qmin, qmax).clamp(qmin, qmax)


def ldlq_update_scales(W, Q, cur, flat, momentum=0.3, nz=1e-8):
    """ldlq.py:553-599."""
    Wf = W.reshape(-1)
    Qf = Q.reshape(-1).float()
    nonzero = Qf != 0
    wnz = Wf.abs() > nz
    consistent = wnz & ((Wf * Qf) > 0)
    valid = nonzero & consistent
    bad = nonzero & ~consistent
    new = cur.clone()
    smin, smax = flat.aminmax()
    lo = max(smin.item() * 0.1, 1e-8)
    hi = smax.item() * 10.0
    if valid.any():
        comp = (Wf[valid].abs() / Qf[valid].abs()).clamp(lo, hi)
        new[valid] = momentum * cur[valid] + (1 - momentum) * comp
    if bad.any():
        new[bad] = flat[bad].clamp(lo, hi)
    return new


def ldlq_iterative(W, Hinv, flat, iters, B, qmin, qmax):
    """ldlq.py:479-550."""
    M, N = W.shape
    cur = flat.clone()
    if not torch.isfinite(cur).all():
        cur = torch.nan_to_num(cur, nan=1e-8, posinf=1e30, neginf=1e-8).clamp(min=1e-8)
    Qr = None
    prev = float("inf")
    prev_scales = None
    for it in range(iters):
        Qi = ldlq_single_pass(W, Hinv, cur, B, qmin, qmax)
        Qr = Qi
        mse = (W - Qi.float() * cur.reshape(M, N)).double().abs().pow(2).mean().item()
        if not math.isfinite(mse):
            if prev_scales is not None:
                cur = prev_scales
            break
        if it > 0 and mse > prev * 1.05:
            if prev_scales is not None:
                cur = prev_scales
            break
        imp = (prev - mse) / (prev + 1e-10)
        if it > 0 and imp < 1e-4:
            break
        prev = mse
        if it < iters - 1:
            prev_scales = cur.clone()
            cur = ldlq_update_scales(W, Qi, cur, flat)
    return Qr, cur


def greedy_pytorch(W, Q, S, H, passes, qmin, qmax):
    """greedy.py:487-541.  ``Q`` is float32 and mutated."""
    M, N = W.shape
    grid = torch.arange(qmin, qmax + 1, dtype=torch.float32)
    hd = torch.diag(H)
    err = Q * S - W
    for _ in range(passes):
        for j in range(N):
            qo = Q[:, j]
            sj = S[:, j]
            cross = err @ H[j, :] - err[:, j] * H[j, j]
            ne = err[:, j].unsqueeze(1) + (grid.unsqueeze(0) - qo.unsqueeze(1)) * sj.unsqueeze(1)
            cost = ne.pow(2) * hd[j] + 2 * ne * cross.unsqueeze(1)
            qn = grid[cost.argmin(dim=1)]
            da = (qn - qo) * sj
            Q[:, j] = qn
            err[:, j] += da
    return Q.clamp(qmin, qmax).to(torch.int8)


def lowrank_decompose(H, rank_threshold=0.01, max_rank_frac=0.3):
    """greedy.py:293-366, the eigh branch (_lowrank_decompose_eigh, 344-366):
    eigenvalues in descending order, keep those > threshold * max; refuse
    (used = False) when max < EIGENVALUE_FLOOR or k > max_rank_frac * N or
    k > LOWRANK_MAX_K.  The reference tries torch.svd_lowrank first, whose
    randomised result equals this one up to its approximation error."""
    N = H.shape[0]
    ev, V = torch.linalg.eigh(H)
    ev = ev.flip(0)
    V = V.flip(1)
    mx = ev[0].item()
    if mx < EIGENVALUE_FLOOR:
        return None, None, 0, False
    mask = ev > mx * rank_threshold
    k = int(mask.sum().item())
    if k > max_rank_frac * N or k > LOWRANK_MAX_K:
        # the svd branch (greedy.py:323-341) counts among its q = min(max(N // 2,
        # 64), N) singular values only, so a refused k it reports is <= q
        return None, None, min(k, min(max(N // 2, 64), N)), False
    return ev[mask], V[:, mask], k, True


def greedy_lowrank_loop(W, Q, S, H, s_k, U_k, passes, qmin, qmax, col_block=GREEDY_COL_BLOCK):
    """greedy.py:400-479 with the kernel of greedy.py:99-199, vectorised over
    rows.  err_lr = err @ U_k is kept up to date by rank-1 updates; the cross
    term of column j is err_lr @ (s_k * U_k[j]) - err_j * H_jj; candidates
    are scanned in grid order with a strict < from 1e30 (first minimum wins,
    q_old kept if no cost is below 1e30).  After every pass the proxy
    sum((err @ H) * err) stops the search once it is >= 0.99 x the previous
    pass's (from the second pass on).  ``Q`` is float32 and mutated."""
    M, N = W.shape
    hd = torch.diag(H)
    err = Q * S - W
    err_lr = err @ U_k
    su = U_k * s_k.unsqueeze(0)
    prev = float("inf")
    for p in range(passes):
        for j0 in range(0, N, col_block):
            for j in range(j0, min(j0 + col_block, N)):
                cross = err_lr @ su[j] - err[:, j] * hd[j]
                e = err[:, j]
                sj = S[:, j].clamp(min=1e-8)
                qo = Q[:, j]
                best = torch.full((M,), 1e30)
                bq = qo.clone()
                for g in range(qmin, qmax + 1):
                    ne = e + (g - qo) * sj
                    cost = ne * ne * hd[j] + 2.0 * ne * cross
                    better = cost < best
                    best = torch.where(better, cost, best)
                    bq = torch.where(better, torch.full_like(bq, float(g)), bq)
                bq = bq.clamp(qmin, qmax)
                d = (bq - qo) * sj
                Q[:, j] = bq
                err[:, j] = e + d
                err_lr += d.unsqueeze(1) * U_k[j].unsqueeze(0)
        proxy = (err @ H * err).sum().item()
        if p > 0 and proxy >= prev * STALL_THRESHOLD:
            break
        prev = proxy
    return Q.clamp(qmin, qmax).to(torch.int8)


def greedy_gpu(W, Q, S, H, passes, qmin, qmax, rank_threshold=0.01):
    """ldlq.py:602-647 on a GPU: the low-rank search when the Hessian's
    effective rank is small enough (greedy.py:369-479), else the full-rank
    search (greedy.py:207-285, whose cross terms equal greedy_pytorch's in
    exact arithmetic).  Returns (codes, k, used_lowrank)."""
    s_k, U_k, k, used = lowrank_decompose(H, rank_threshold, LOWRANK_MAX_RANK_FRAC)
    Qf = Q.clone().float().contiguous()
    if not used:
        return greedy_pytorch(W, Qf, S, H, passes, qmin, qmax), k, False
    return greedy_lowrank_loop(W, Qf, S, H, s_k, U_k, passes, qmin, qmax), k, True


def ls_scales(Q, W):
    """Per-row least-squares scale (ldlq.py:227-231, 262-265)."""
    Qf = Q.float()
    num = (Qf * W).sum(dim=1, keepdim=True)
    den = (Qf * Qf).sum(dim=1, keepdim=True).clamp(min=1e-8)
    return (num / den).clamp(min=SCALE_MIN)


def ldlq_quantize_layer(W, hessian=None, block_size=128, damping=0.01, int_bits=4,
                        iterations=1, greedy_passes=0, rank_threshold=0.01, greedy_device="cpu",
                        weight_only_gram=None):
    """ldlq.py:95-279 (2-D / 3-D / weight-only Hessians).  The greedy search
    is the one ldlq.py:602-647 picks for tensors on ``greedy_device``: "cpu"
    the PyTorch search, "gpu" the low-rank / full-rank choice.
    ``weight_only_gram`` (noise studies only): W^T W / M computed in another
    summation order, used in place of the matmul of the weight-only branch;
    None is the reference."""
    from types import SimpleNamespace
    W = W.float()
    M, N = W.shape
    div = 127.0 if int_bits == 8 else 7.0
    qmin, qmax = (-128, 127) if int_bits == 8 else (-8, 7)
    if isinstance(hessian, dict):
        # ldlq.py:149-158; the greedy search needs the dense H this branch
        # never builds (the reference fails there)
        if hessian["D"].shape[0] != N:
            raise ValueError(f"DLR Hessian dim {hessian['D'].shape[0]} != in_features {N}")
        if greedy_passes > 0:
            raise ValueError("greedy search needs a dense Hessian (DLR given)")
        Hinv = woodbury_inverse(hessian["D"], hessian["U"], damping)
    elif hessian is not None:
        H = hessian.float()
        if H.dim() == 3:
            nb, bs, _ = H.shape
            Hinv = torch.zeros(N, N, dtype=torch.float32)
            for bi in range(nb):
                c0 = bi * bs
                c1 = min(c0 + bs, N)
                Hinv[c0:c1, c0:c1] = invert_hessian(damp(H[bi, :c1 - c0, :c1 - c0].float(), damping))
        else:
            Hinv = invert_hessian(damp(H, damping))
    else:
        H = W.T @ W / M if weight_only_gram is None else weight_only_gram.float()
        if not torch.isfinite(H).all():
            s = (W.abs().amax(dim=1, keepdim=True) / div).clamp(min=SCALE_MIN, max=SCALE_MAX)
            q = (W / s).round().clamp(qmin, qmax).to(torch.int8)
            d = q.float() * s.float()
            return SimpleNamespace(quantized_W=q, scales=s.to(torch.float16), zero_points=None,
                                   mse=(W - d).double().pow(2).mean().item(),
                                   max_err=(W - d).abs().max().item(),
                                   method_used="rtn", fallbacks=["hessian_nan_rtn"])
        H = damp(H, damping)
        Hinv = invert_hessian(H)
    rs = (W.abs().amax(dim=1, keepdim=True) / div).clamp(min=SCALE_MIN)
    flat = rs.expand(M, N).reshape(-1).clone()
    if iterations > 1:
        Q, _ = ldlq_iterative(W, Hinv, flat, iterations, block_size, qmin, qmax)
    else:
        Q = ldlq_single_pass(W, Hinv, flat, block_size, qmin, qmax)
    if greedy_passes > 0:
        gs = ls_scales(Q, W)
        if greedy_device == "gpu":
            Q, _, _ = greedy_gpu(W, Q, gs.expand(M, N), H, greedy_passes, qmin, qmax, rank_threshold)
        else:
            Q = greedy_pytorch(W, Q.clone().float().contiguous(), gs.expand(M, N), H,
                               greedy_passes, qmin, qmax)
    fs = ls_scales(Q, W)
    d = Q.float() * fs.float()
    return SimpleNamespace(quantized_W=Q, scales=fs.to(torch.float16), zero_points=None,
                           mse=(W - d).double().pow(2).mean().item(),
                           max_err=(W - d).abs().max().item(),
                           method_used="ldlq_cpu", fallbacks=[])


# ---------------------------------------------------------------- DLR Hessians

DLR_DIAG_FLOOR = 1e-12        # dlr.py:22


def woodbury_inverse(D, U, damping=0.0):
    """(diag(D) + U U^T + damping * mean(diag H) I)^-1 by the Woodbury
    identity, dlr.py:76-119: D' = D + damping * max(mean(D + rowsum(U^2)),
    1e-6), Dinv = 1 / max(D', 1e-12), Z = Dinv U, M = I + U^T Z,
    H^-1 = diag(Dinv) - (Z M^-1) Z^T, M^-1 by Cholesky (inv, then pinv, when
    that fails)."""
    D = D.float()
    U = U.float()
    r = U.shape[1]
    if damping > 0.0:
        dm = (D + (U * U).sum(dim=1)).mean().clamp(min=DIAG_MEAN_FLOOR)
        D = D + damping * dm
    Dinv = 1.0 / D.clamp(min=DLR_DIAG_FLOOR)
    Z = Dinv.unsqueeze(1) * U
    M = torch.eye(r, dtype=torch.float32) + U.T @ Z
    try:
        Minv = torch.cholesky_inverse(torch.linalg.cholesky(M))
    except torch.linalg.LinAlgError:
        try:
            Minv = torch.linalg.inv(M)
        except torch.linalg.LinAlgError:
            Minv = torch.linalg.pinv(M)
    return torch.diag(Dinv) - Z @ Minv @ Z.T


def dlr_to_dense(D, U):
    """diag(D) + U U^T (dlr.py:122-127)."""
    return torch.diag(D.float()) + U.float() @ U.float().T


# ---------------------------------------------------------------- PiSO

def _piso_batch(W, bytes_per_row):
    return max(1, min(W.shape[0], (512 * 1024 * 1024) // max(1, bytes_per_row)))


def piso_scales_sym(W, h_diag, num_coarse, num_fine, qmin, qmax, divisor):
    """piso.py:28-94 (_compute_piso_scales_pytorch): per-row symmetric scale
    grid search, the first minimum of each stage."""
    M, D = W.shape
    out = torch.empty(M, 1, dtype=torch.float32)
    cf = torch.linspace(0.5, 2.0, num_coarse, dtype=torch.float32)
    ff = torch.linspace(0.95, 1.05, num_fine, dtype=torch.float32)
    bs = _piso_batch(W, (num_coarse + num_fine) * D * 4)
    for r0 in range(0, M, bs):
        Wb = W[r0:r0 + bs]
        B = Wb.shape[0]
        sa = (Wb.abs().amax(dim=1, keepdim=True) / divisor).clamp(min=1e-10)
        sc = sa * cf.unsqueeze(0)
        W3 = Wb.unsqueeze(1)
        s3 = sc.unsqueeze(2)
        q = rhaz(W3 / s3).clamp(qmin, qmax)
        cost = ((W3 - q * s3) ** 2 * h_diag).sum(dim=2)
        best = sc[torch.arange(B), cost.argmin(dim=1)]
        sf = best.unsqueeze(1) * ff.unsqueeze(0)
        s3 = sf.unsqueeze(2)
        q = rhaz(W3 / s3).clamp(qmin, qmax)
        cost = ((W3 - q * s3) ** 2 * h_diag).sum(dim=2)
        out[r0:r0 + B, 0] = sf[torch.arange(B), cost.argmin(dim=1)]
    return out


def piso_scales_asym(W, h_diag, num_coarse, num_fine, qmin, qmax, lo, hi):
    """piso.py:97-183 (_compute_piso_scales_asymmetric_pytorch): scales and
    zero-points, every candidate clamped at 1e-10."""
    M, D = W.shape
    out = torch.empty(M, 1, dtype=torch.float32)
    zps = torch.empty(M, 1, dtype=torch.int8)
    cf = torch.linspace(lo, hi, num_coarse, dtype=torch.float32)
    ff = torch.linspace(0.95, 1.05, num_fine, dtype=torch.float32)
    divisor = float(qmax - qmin)
    bs = _piso_batch(W, (num_coarse + num_fine) * D * 4)
    for r0 in range(0, M, bs):
        Wb = W[r0:r0 + bs].float()
        B = Wb.shape[0]
        wmin = Wb.amin(dim=1, keepdim=True)
        wmax = Wb.amax(dim=1, keepdim=True)
        sref = ((wmax - wmin) / divisor).clamp(min=1e-10)
        W3 = Wb.unsqueeze(1)
        best = None
        for factors, base in ((cf, sref), (ff, None)):
            s = ((base if best is None else best.unsqueeze(1)) * factors.unsqueeze(0)).clamp(min=1e-10)
            s3 = s.unsqueeze(2)
            z3 = rhaz(qmin - wmin.unsqueeze(2) / s3).clamp(qmin, qmax)
            q = rhaz(W3 / s3 + z3).clamp(qmin, qmax)
            cost = ((W3 - (q - z3) * s3) ** 2 * h_diag).sum(dim=2)
            idx = cost.argmin(dim=1)
            best = s[torch.arange(B), idx]
            bz = z3.squeeze(2)[torch.arange(B), idx]
        out[r0:r0 + B, 0] = best
        zps[r0:r0 + B, 0] = bz.to(torch.int8)
    return out, zps


# ---------------------------------------------------------------- PermuQuant

def channel_second_moments(W):
    """permuquant.py:13-23: per-column mean of squares (torch CPU order)."""
    return (W ** 2).mean(dim=0)


def permutation_weight(W):
    """permuquant.py:26-41: torch's argsort(descending=True) of the moments
    (not stable on exact ties from 100 elements on)."""
    return channel_second_moments(W).argsort(descending=True)


def permutation_joint(W, act_mu2, alpha):
    """permuquant.py:44-69."""
    v = (act_mu2.clamp(min=1e-12) ** alpha) * (channel_second_moments(W).clamp(min=1e-12) ** (1.0 - alpha))
    return v.argsort(descending=True)


def group_quant_error(W, group_size=128, int_bits=4):
    """permuquant.py:72-111: sum of squared symmetric-RTN errors, as torch's
    CPU sum computes it with the current torch.get_num_threads()."""
    M, N = W.shape
    if int_bits == 8:
        s = scales_int8_sym(W)
        dq = (quant_int8_sym(W, s).float() * s.float())[:, :N]
    else:
        s = scales_int4_sym(W, group_size)
        q = quant_int4_sym(W, s, group_size)
        G = q.shape[1] // group_size
        dq = (q.reshape(M, G, group_size).float() * s.unsqueeze(2).float()).reshape(M, G * group_size)[:, :N]
    return ((W - dq) ** 2).sum().item()


def permutation_with_acceptance(W, act_mu2=None, alpha=0.5, group_size=128, tau=0.0, int_bits=4):
    """permuquant.py:114-156: (perm, accepted)."""
    perm = permutation_joint(W, act_mu2, alpha) if act_mu2 is not None else permutation_weight(W)
    e0 = group_quant_error(W, group_size, int_bits)
    e1 = group_quant_error(W[:, perm], group_size, int_bits)
    rel = (e0 - e1) / e0 if e0 > 0 else 0.0
    return perm, rel > tau


def sweep_alpha(W, act_mu2=None, group_size=128, tau=0.0, num_alpha=11, int_bits=4):
    """permuquant.py:159-213: (perm, alpha, accepted)."""
    if num_alpha < 1:
        raise ValueError(f"num_alpha must be >= 1, got {num_alpha}")
    if act_mu2 is None or num_alpha == 1:
        perm, acc = permutation_with_acceptance(W, act_mu2, 0.0, group_size, tau, int_bits)
        return perm, 0.0, acc
    best = (None, 0.0, float("inf"))
    for i in range(num_alpha):
        a = i / (num_alpha - 1)
        perm, acc = permutation_with_acceptance(W, act_mu2, a, group_size, tau, int_bits)
        if acc:
            err = group_quant_error(W[:, perm], group_size, int_bits)
            if err < best[2]:
                best = (perm, a, err)
    if best[0] is None:
        return torch.arange(W.shape[1]), 0.0, False
    return best[0], best[1], True


def permuquant_layer(W_work, orig_in, int_bits, tau, perm_group_size=128, cal_perm=None):
    """The PermuQuant step of the per-layer pipeline (pipeline.py:572-615):
    returns (W_work permuted in its first orig_in columns, perm or None,
    came_from_calibration)."""
    W_work = W_work.clone()
    if cal_perm is not None:
        of = min(orig_in, cal_perm.shape[0])
        ps = cal_perm[:of]
        if ps.max() < of and ps.min() >= 0 and ps.unique().numel() == ps.numel():
            W_orig = W_work[:, :of]
            W_work[:, :of] = W_orig[:, ps]
            return W_work, ps, True
    W_orig = W_work[:, :orig_in]
    gs = W_orig.shape[1] if int_bits == 4 else perm_group_size
    perm, _, acc = sweep_alpha(W_orig, None, gs, tau, int_bits=int_bits)
    if acc:
        W_work[:, :orig_in] = W_orig[:, perm]
        return W_work, perm, False
    return W_work, None, False
