"""Loader and thin typed wrappers for the HIP library ``libicq.so``.

There is no fallback: if the library is missing or no GPU is visible, every
compute entry point raises ``RuntimeError``.  Tensors live on the GPU; CPU
tensors handed to the public API are copied to ``cuda:0`` and results are
copied back by the calling module.
"""

from __future__ import annotations

import ctypes
import os
import re
import threading

import torch

_PKG = os.path.dirname(os.path.abspath(__file__))
# IC_LIBICQ_PATH names another build of the same library (the host-sanitizer
# build of build.py --asan-check); by default the in-tree libicq.so
LIB_PATH = os.environ.get("IC_LIBICQ_PATH") or os.path.join(_PKG, "libicq.so")
HEADER_PATH = os.path.join(os.path.dirname(_PKG), "include", "ic_abi.h")

DT_F32, DT_BF16, DT_F16 = 0, 1, 2

_lib = None
_lock = threading.Lock()

_c = ctypes
_vp = _c.c_void_p
_i64 = _c.c_int64
_i32 = _c.c_int
_f32 = _c.c_float

# name -> (restype, argtypes)
_SIGS = {
    "ic_abi_version": (_i32, []),
    "ic_last_error": (_c.c_char_p, []),
    "ic_rotate_rows": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _i64, _i64, _i32, _f32, _vp, _vp]),
    "ic_rotate_hessian": (_i32, [_vp, _vp, _i64, _i64, _i64, _i32, _vp]),
    "ic_rotate_rows_exact": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _i64, _i64, _i32, _f32, _vp, _vp]),
    "ic_rotate_hessian_exact": (_i32, [_vp, _vp, _i64, _i64, _i64, _i32, _i32, _vp]),
    "ic_row_stats": (_i32, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp]),
    "ic_rtn_scales": (_i32, [_vp, _i64, _i64, _i64, _i32, _i32, _c.POINTER(_f32), _i32, _vp, _vp, _vp]),
    "ic_rtn_quantize": (_i32, [_vp, _i64, _i64, _i64, _i32, _vp, _i32, _vp, _vp, _i64, _vp, _i64, _vp]),
    "ic_pack_int4": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _i64, _vp, _vp]),
    "ic_unpack_int4": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _vp]),
    "ic_quant_error_workspace_bytes": (_i64, []),
    "ic_quant_error": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _vp, _i32, _vp, _vp, _vp, _vp, _vp]),
    "ic_scale_status": (_i32, [_vp, _i32, _i64, _vp, _vp]),
    "ic_sgemm": (_i32, [_i32, _i32, _i64, _i64, _i64, _f32, _vp, _i64, _vp, _i64, _f32, _vp, _i64, _i32, _i32, _vp]),
    "ic_hessian_inverse_workspace_bytes": (_i64, [_i64, _i64]),
    "ic_hessian_inverse": (_i32, [_vp, _i64, _i64, _f32, _i32, _vp, _vp, _vp]),
    "ic_cholesky": (_i32, [_vp, _i64, _i64, _vp, _vp, _vp]),
    "ic_damp_hessian": (_i32, [_vp, _i64, _i64, _f32, _vp]),
    "ic_gram_tn": (_i32, [_vp, _i64, _i64, _i64, _f32, _vp, _vp]),
    "ic_gptq_row_params": (_i32, [_vp, _vp, _vp, _i64, _i32, _i32, _vp, _vp, _vp, _vp, _vp]),
    "ic_gptq_workspace_bytes": (_i64, [_i64, _i64, _i32]),
    "ic_gptq_quantize": (_i32, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _i32, _i32, _vp, _vp, _vp]),
    "ic_gptq_quantize_from": (_i32, [_vp, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _i32, _i32, _vp, _vp, _vp]),
    "ic_gptq_noalloc_scratch_bytes": (_i64, []),
    "ic_gptq_quantize_noalloc": (_i32, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _i32, _i32, _vp, _vp]),
    "ic_ldlq_quantize": (_i32, [_vp, _i64, _i64, _vp, _vp, _i32, _i32, _vp, _vp, _vp]),
    "ic_ldlq_init_scales": (_i32, [_vp, _i64, _i64, _i32, _vp, _vp, _vp]),
    "ic_sanitize_scales": (_i32, [_vp, _i64, _vp]),
    "ic_ldlq_mse": (_i32, [_vp, _vp, _vp, _i64, _vp, _vp, _vp]),
    "ic_ldlq_update_scales": (_i32, [_vp, _vp, _vp, _vp, _i64, _f32, _f32, _f32, _vp, _vp]),
    "ic_ls_scales": (_i32, [_vp, _vp, _i64, _i64, _vp, _vp]),
    "ic_greedy_workspace_bytes": (_i64, [_i64, _i64]),
    "ic_greedy": (_i32, [_vp, _vp, _vp, _i32, _vp, _i64, _i64, _i32, _i32, _vp, _vp]),
    "ic_lowrank_workspace_bytes": (_i64, [_i64, _i64]),
    "ic_lowrank_eigs": (_i32, [_vp, _i64, _i64, _i32, _c.c_ulonglong, _f32, _vp, _vp, _c.POINTER(_i32), _vp,
                               _vp]),
    "ic_greedy_lowrank_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "ic_greedy_lowrank": (_i32, [_vp, _vp, _vp, _i32, _vp, _vp, _i64, _vp, _i64, _i64, _i64, _i32, _i32,
                                 _c.POINTER(_i32), _vp, _vp]),
    "ic_hbm_stream": (_i32, [_i32, _vp, _vp, _i64, _vp]),
    "ic_profile_enable": (_i32, [_i32]),
    "ic_profile_read": (_i32, [_vp, _vp, _vp, _vp, _i32]),
    "ic_col_moments_workspace_bytes": (_i64, [_i64, _i64]),
    "ic_col_moments": (_i32, [_vp, _i64, _i64, _i64, _i32, _vp, _vp, _vp]),
    "ic_argsort_workspace_bytes": (_i64, [_i64]),
    "ic_argsort_desc": (_i32, [_vp, _i64, _vp, _vp, _vp]),
    "ic_group_quant_error_workspace_bytes": (_i64, [_i64, _i64, _i64, _i32, _i32]),
    "ic_group_quant_error": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _i32, _i32, _vp, _vp, _vp]),
    "ic_torch_sum_workspace_bytes": (_i64, [_i64, _i32]),
    "ic_torch_sum": (_i32, [_vp, _i64, _i32, _vp, _vp, _vp]),
    "ic_permute_cols": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _vp]),
    "ic_permute_sym": (_i32, [_vp, _i64, _i64, _vp, _i64, _vp, _i64, _vp]),
    "ic_woodbury_workspace_bytes": (_i64, [_i64, _i64]),
    "ic_woodbury_inverse": (_i32, [_vp, _vp, _i64, _i64, _i64, _f32, _vp, _i32, _vp, _i64, _vp, _vp, _vp, _vp]),
    "ic_dlr_to_dense": (_i32, [_vp, _vp, _i64, _i64, _i64, _vp, _i64, _vp]),
    "ic_piso_scales": (_i32, [_vp, _i64, _i64, _i64, _vp, _i32, _i32, _vp, _i32, _vp, _i32, _vp, _vp, _vp]),
}

PROFILE_TAGS = ["gemm_trailing", "gemm_cholesky", "gemm_inverse", "diag_factor", "sweep", "rotate_w",
                "rotate_h", "rtn_quant_pack", "greedy", "other", "gemm_greedy", "chol_panel", "rtn_scales",
                "verify", "permute", "permute_sum", "dlr", "dlr_gemm", "piso"]

# kernel family -> (the profiler phases its launches are tagged with, the
# bound it is graded against: "mfma", "hbm", or "latency" for kernels whose
# time is a dependency chain / instruction issue, reported as a share of the
# step).  The rotation phases are MFMA-bound with the exact kernels (the
# default) and HBM-bound with the fast Walsh-Hadamard transform.
PROFILE_KERNELS = {
    "gemm_f32_kernel": (["gemm_trailing", "gemm_cholesky", "gemm_inverse", "gemm_greedy", "dlr", "dlr_gemm"], "mfma"),
    "potrf_diag_kernel": (["diag_factor"], "latency"),
    "panel64_kernel": (["chol_panel"], "latency"),
    "sweep16_kernel / sweep4_kernel": (["sweep"], "latency"),
    "greedy_sb_kernel": (["greedy"], "latency"),
    "rot_rows_wave_kernel / rot_rows_exact_kernel": (["rotate_w"], "mfma"),
    "rot_cols_exact_kernel + rot_rows_exact_kernel": (["rotate_h"], "mfma"),
    "rtn_clip_reg_kernel / rtn_clip_kernel": (["rtn_scales"], "latency"),   # VALU-bound: a share of the step
    "rtn_quant_kernel": (["rtn_quant_pack"], "hbm"),
    "quant_error_partial": (["verify"], "hbm"),
    "fsum_group_kernel": (["permute_sum"], "hbm"),   # (fsum_block_kernel: its fallback for cascade groups above 32)
    "piso_kernel": (["piso"], "latency"),
}
FWHT_KERNELS = {"rot_rows_wave_kernel / rot_rows_exact_kernel": ("rotate256_coal / rotate_rows_reg", "hbm"),
                "rot_cols_exact_kernel + rot_rows_exact_kernel": ("rotate_cols256_kernel + rotate256_coal", "hbm")}


def profile_enable(on: bool) -> None:
    check(lib().ic_profile_enable(int(on)), "ic_profile_enable")


def profile_read() -> dict[str, dict]:
    n = len(PROFILE_TAGS)
    ms, fl, by = ((ctypes.c_double * n)() for _ in range(3))
    la = (ctypes.c_int64 * n)()
    check(lib().ic_profile_read(ms, fl, by, la, n), "ic_profile_read")
    return {t: {"ms": ms[i], "flops": fl[i], "bytes": by[i], "launches": la[i]} for i, t in enumerate(PROFILE_TAGS)}


def header_functions() -> list[str]:
    """Names of the functions declared in include/ic_abi.h."""
    with open(HEADER_PATH) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ic_[a-z0-9_]+)\s*\(", text)))


class _Checked:
    """A library function that takes tensors where the C ABI takes device
    pointers: a GPU tensor becomes its data pointer; a tensor in host memory
    is refused with ValueError before the call, so no kernel is ever handed
    a host address.  None (a NULL pointer) and plain integers pass through;
    the library itself rejects a NULL where one is not allowed."""

    __slots__ = ("fn", "name")

    def __init__(self, fn, name: str):
        self.fn, self.name = fn, name

    def __call__(self, *args):
        conv = list(args)
        for i, a in enumerate(conv):
            if isinstance(a, torch.Tensor):
                if a.device.type != "cuda":
                    raise ValueError(f"{self.name}: argument {i} is a {a.device.type} tensor; "
                                     "the library takes GPU memory")
                conv[i] = a.data_ptr()
        return self.fn(*conv)


class _Lib:
    """The loaded library: one _Checked per function of _SIGS."""

    def __init__(self, cdll):
        self.cdll = cdll


def load(require_gpu: bool = True):
    """Load the library once; raise RuntimeError if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
                "(hipcc --offload-arch=gfx950).  There is no CPU fallback.")
        cdll = ctypes.CDLL(LIB_PATH)
        lib = _Lib(cdll)
        for name, (res, args) in _SIGS.items():
            fn = getattr(cdll, name)
            fn.restype = res
            fn.argtypes = args
            setattr(lib, name, _Checked(fn, name))
        _lib = lib
    return _lib


def lib():
    if not torch.cuda.is_available():
        raise RuntimeError("int_crush_converter_amd needs a ROCm GPU (gfx950); none is visible")
    return load()


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = _lib.ic_last_error().decode(errors="replace") if _lib is not None else ""
        if rc == -1:
            raise ValueError(f"{what}: {msg}")
        raise RuntimeError(f"{what} failed ({rc}): {msg}")


def ptr(t: torch.Tensor | None) -> torch.Tensor | None:
    """An optional tensor argument (None = NULL); the library wrapper checks it."""
    return t


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def device() -> torch.device:
    return torch.device("cuda", torch.cuda.current_device())


def to_gpu(t: torch.Tensor) -> torch.Tensor:
    """Move a tensor to the current GPU (no copy if already there)."""
    lib()
    if t.device.type == "cuda":
        return t
    return t.to(device(), non_blocking=False)


def dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return DT_F32
    if t.dtype == torch.bfloat16:
        return DT_BF16
    if t.dtype == torch.float16:
        return DT_F16
    raise TypeError(f"unsupported dtype {t.dtype}")


def workspace(nbytes: int, dev: torch.device) -> torch.Tensor:
    """Caller-owned scratch for an ABI call (uint8, through torch's allocator)."""
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=dev)


def row_ld(t: torch.Tensor) -> int:
    """Leading dimension of a 2-D tensor whose rows are contiguous."""
    if t.dim() != 2 or t.stride(1) != 1:
        raise ValueError("expected a 2-D tensor with contiguous rows")
    return max(t.stride(0), t.shape[1]) if t.shape[0] > 1 else t.shape[1]
