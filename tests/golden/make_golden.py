"""Write golden input/output vectors from the reference implementation.

Run in the development container only (the reference is not present on the
GPU box):

    PYTHONPATH=/root/reference python tests/golden/make_golden.py

It covers the functions whose results no closed form pins bit for bit
because they depend on fp32 LAPACK/BLAS rounding or fp32 reduction order:
GPTQ / LDLQ / greedy codes, LDLQ iteration decisions, clipping-ratio choices
and a small end-to-end pipeline file.  Every case is a small seeded input;
the outputs are stored as ``.safetensors`` next to this script.

    PYTHONPATH=/root/reference python tests/golden/make_golden.py --greedy-gpu

    PYTHONPATH=/root/reference python tests/golden/make_golden.py --rotation

writes ``golden_rotation.safetensors`` / ``.json``: inputs and outputs of
the reference's ``rotate_weights`` (every power of 2 up to 512, fp32 and
bf16 sources, padding, the pipeline's outlier zeroing first) and
``rotate_hessian`` (2-D with padding, 3-D whole blocks and sub-blocks), plus
the raw W and H of the rotated GPTQ golden cases with their rotations.
These pin the fp32 rounding of the rotation itself.

    PYTHONPATH=/root/reference python tests/golden/make_golden.py --greedy-gpu

writes ``golden_greedy_gpu.safetensors`` / ``.json`` instead: the
reference's GPU greedy backends (the low-rank kernel of
converter/greedy.py:99-199, 369-479 and the full-rank v2 path of
greedy.py:207-285), run on CPU tensors under Triton's interpreter
(TRITON_INTERPRET=1), with torch's global RNG seeded before each call
because ``torch.svd_lowrank`` draws its test matrix from it.
"""

from __future__ import annotations

import json
import os
import sys
import tempfile

GREEDY_GPU = "--greedy-gpu" in sys.argv
ROTATION = "--rotation" in sys.argv
if GREEDY_GPU:
    os.environ["TRITON_INTERPRET"] = "1"   # must precede the first triton import

import torch
from safetensors.torch import save_file, load_file

HERE = os.path.dirname(os.path.abspath(__file__))
REF = os.environ.get("IC_REFERENCE", "/root/reference")
sys.path.insert(0, REF)

from converter.gptq import gptq_quantize_layer, gptq_quantize_layer_rtn  # noqa: E402
from converter.ldlq import ldlq_quantize_layer  # noqa: E402
from converter.scales import (  # noqa: E402
    calculate_scales, calculate_scales_asymmetric,
    calculate_scales_int8, calculate_scales_int8_asymmetric,
)
from converter.rotation import rotate_weights, rotate_hessian  # noqa: E402
from converter.pipeline import quantize_model  # noqa: E402
from converter.config import WEIGHT_OUTLIER_CLAMP  # noqa: E402
from converter.types import QuantizeConfig  # noqa: E402


def lognormal_hessian(n: int, samples: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    s = torch.exp(torch.randn(n, generator=g))
    X = torch.randn(samples, n, generator=g) * s
    return X.T @ X / samples


def weights(m: int, n: int, seed: int, std: float = 0.02) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return torch.randn(m, n, generator=g) * std


def gptq_cases(out: dict, meta: dict) -> None:
    cases = [
        # name, M, N, samples, bits, asym, method, block, rot
        ("gptq_a", 32, 256, 512, 4, False, "hinv", 128, 0),
        ("gptq_b", 48, 256, 128, 4, False, "hinv", 64, 256),
        ("gptq_c", 64, 512, 256, 4, False, "hinv", 128, 256),
        ("gptq_d", 32, 192, 400, 8, False, "hinv", 128, 64),
        ("gptq_e", 32, 256, 400, 8, True, "hinv", 128, 16),
        ("gptq_f", 32, 256, 300, 4, False, "cholesky", 128, 0),
    ]
    for i, (name, M, N, S, bits, asym, hm, B, rot) in enumerate(cases):
        W = weights(M, N, 100 + i)
        H = lognormal_hessian(N, S, 200 + i)
        if rot:
            W = rotate_weights(W, rot)
            H = rotate_hessian(H, rot)
        r = gptq_quantize_layer(W, H, block_size=B, damping=0.01, int_bits=bits,
                                asymmetric=asym, hessian_method=hm)
        out[f"{name}.W"] = W.contiguous()
        out[f"{name}.H"] = H.contiguous()
        out[f"{name}.q"] = r.quantized_W
        out[f"{name}.scales"] = r.scales
        if r.zero_points is not None:
            out[f"{name}.zp"] = r.zero_points
        meta[name] = dict(kind="gptq", bits=bits, asym=asym, method=hm, block=B,
                          mse=r.mse, max_err=r.max_err)
    # 3-D block-diagonal Hessian
    M, N, bs = 32, 512, 256
    W = weights(M, N, 150)
    g = torch.Generator().manual_seed(250)
    blocks = []
    for _ in range(N // bs):
        s = torch.exp(torch.randn(bs, generator=g))
        X = torch.randn(300, bs, generator=g) * s
        blocks.append(X.T @ X / 300)
    H3 = torch.stack(blocks)
    r = gptq_quantize_layer(W, H3, block_size=128, damping=0.01, int_bits=4)
    out["gptq3d.W"] = W
    out["gptq3d.H"] = H3
    out["gptq3d.q"] = r.quantized_W
    out["gptq3d.scales"] = r.scales
    out["gptq3d.zp"] = r.zero_points
    meta["gptq3d"] = dict(kind="gptq", bits=4, asym=False, method="hinv", block=128,
                          mse=r.mse, max_err=r.max_err)


def ldlq_cases(out: dict, meta: dict) -> None:
    cases = [
        # name, M, N, bits, iters, greedy, block, with_H
        ("ldlq_a", 32, 128, 4, 1, 0, 64, False),
        ("ldlq_b", 32, 128, 4, 2, 0, 128, False),
        ("ldlq_c", 24, 96, 4, 2, 3, 32, False),
        ("ldlq_d", 32, 128, 8, 1, 2, 64, False),
        ("ldlq_e", 32, 128, 4, 1, 2, 64, True),
    ]
    for i, (name, M, N, bits, iters, gp, B, with_h) in enumerate(cases):
        g = torch.Generator().manual_seed(300 + i)
        W = torch.randn(M, N, generator=g) * 0.02
        H = lognormal_hessian(N, 256, 400 + i) if with_h else None
        import warnings
        with warnings.catch_warnings():
            warnings.simplefilter("ignore")
            r = ldlq_quantize_layer(W, hessian=H, block_size=B, damping=0.01, int_bits=bits,
                                    iterations=iters, greedy_passes=gp)
        out[f"{name}.W"] = W
        if H is not None:
            out[f"{name}.H"] = H
        out[f"{name}.q"] = r.quantized_W
        out[f"{name}.scales"] = r.scales
        meta[name] = dict(kind="ldlq", bits=bits, iters=iters, greedy=gp, block=B,
                          mse=r.mse, max_err=r.max_err, method_used=r.method_used)


def clip_cases(out: dict, meta: dict) -> None:
    g = torch.Generator().manual_seed(500)
    W = torch.randn(64, 512, generator=g) * 0.02
    cols = torch.randperm(512, generator=g)[:5]
    W[:, cols] *= 20
    ratios = [0.8, 0.85, 0.9, 0.95, 1.0]
    out["clip.W"] = W
    out["clip.s4"] = calculate_scales(W, W.shape[1], clipping_ratios=ratios)
    s, z = calculate_scales_asymmetric(W, W.shape[1], clipping_ratios=ratios)
    out["clip.s4a"], out["clip.z4a"] = s, z
    out["clip.s8"] = calculate_scales_int8(W, clipping_ratios=ratios)
    s, z = calculate_scales_int8_asymmetric(W, clipping_ratios=ratios)
    out["clip.s8a"], out["clip.z8a"] = s, z
    meta["clip"] = dict(kind="clip", ratios=ratios)


def pipeline_cases(out: dict, meta: dict) -> None:
    # C1-shaped RTN run (8 layers [64,256] fp32, rot 256, INT4)
    g = torch.Generator().manual_seed(42)
    state = {f"layers.{i}.q_proj.weight": torch.randn(64, 256, generator=g) * 0.02
             for i in range(8)}
    state["layers.0.q_proj.bias"] = torch.randn(64, generator=g)
    state["model.norm.weight"] = torch.randn(256, generator=g)
    # a layer whose in_features is not a multiple of 256 (padding path)
    state["layers.9.up.weight"] = torch.randn(16, 200, generator=g) * 0.02
    with tempfile.TemporaryDirectory() as td:
        src = os.path.join(td, "in.safetensors")
        save_file(state, src)
        for tag, kw in [("pipe_rtn4", dict(rot_size=256, int_bits=4)),
                        ("pipe_rtn8a", dict(rot_size=64, int_bits=8, asymmetric=True,
                                            clipping_ratios=[0.8, 0.85, 0.9, 0.95, 1.0]))]:
            od = os.path.join(td, tag)
            quantize_model(QuantizeConfig(input_path=src, output_dir=od, **kw))
            res = load_file(os.path.join(od, "model.safetensors"))
            from safetensors import safe_open
            with safe_open(os.path.join(od, "model.safetensors"), framework="pt") as f:
                md = f.metadata()
            for k, v in res.items():
                out[f"{tag}/{k}"] = v
            meta[tag] = dict(kind="pipeline", config=kw, metadata=md)
        for k, v in state.items():
            out[f"pipe_in/{k}"] = v


def rotation_cases(out: dict, meta: dict) -> None:
    # weights: every power of 2 up to 512 (regular for powers of 4, else
    # Sylvester), fp32 source with padding (300 columns)
    for rot in (2, 4, 8, 16, 32, 64, 128, 256, 512):
        W = weights(33, 300, 600 + rot, std=1.0)
        out[f"rw{rot}.W"] = W
        out[f"rw{rot}.out"] = rotate_weights(W, rot)
        meta[f"rw{rot}"] = dict(kind="rotate_weights", rot=rot)
    # bf16 source (cast to fp32 first, converter/pipeline.py:524) at R = 256 and 64
    for rot in (64, 256):
        Wb = weights(20, 512, 700 + rot).to(torch.bfloat16)
        out[f"rwb{rot}.W"] = Wb
        out[f"rwb{rot}.out"] = rotate_weights(Wb.float(), rot)
        meta[f"rwb{rot}"] = dict(kind="rotate_weights", rot=rot, source="bf16")
    # the pipeline's outlier zeroing before rotation (converter/pipeline.py:527-555)
    W = weights(16, 256, 800)
    W[0, 3], W[5, 100], W[15, 255] = 5000.0, -1500.0, 1000.5
    Wz = W.masked_fill(W.abs() > WEIGHT_OUTLIER_CLAMP, 0.0)
    out["rwz.W"] = W
    out["rwz.out"] = rotate_weights(Wz, 256)
    meta["rwz"] = dict(kind="rotate_weights", rot=256, zero_above=WEIGHT_OUTLIER_CLAMP, zeroed=3)
    # Hessians: 2-D (padded when n % rot), 3-D whole blocks and sub-blocks
    for name, rot, n in (("rh16", 16, 64), ("rh64", 64, 200), ("rh256", 256, 300)):
        H = lognormal_hessian(n, 2 * n, 900 + n + rot)
        out[f"{name}.H"] = H
        out[f"{name}.out"] = rotate_hessian(H, rot)
        meta[name] = dict(kind="rotate_hessian", rot=rot, n=n)
    for name, rot, nb, bs in (("rh3_256", 256, 1, 256), ("rh3_64", 64, 2, 128), ("rh3_16", 16, 3, 64)):
        H3 = torch.stack([lognormal_hessian(bs, 2 * bs, 950 + b) for b in range(nb)])
        out[f"{name}.H"] = H3
        out[f"{name}.out"] = rotate_hessian(H3, rot)
        meta[name] = dict(kind="rotate_hessian", rot=rot, blocks=nb, bs=bs)
    # the raw inputs of rotated GPTQ golden cases (gptq_cases above); their
    # rotations are that file's <name>.W / <name>.H, checked equal here
    gold = load_file(os.path.join(HERE, "golden.safetensors"))
    for name, k, M, N, S, rot in (("gptq_b", 1, 48, 256, 128, 256), ("gptq_d", 3, 32, 192, 400, 64),
                                  ("gptq_e", 4, 32, 256, 400, 16)):
        W = weights(M, N, 100 + k)
        H = lognormal_hessian(N, S, 200 + k)
        if not (torch.equal(rotate_weights(W, rot), gold[f"{name}.W"])
                and torch.equal(rotate_hessian(H, rot), gold[f"{name}.H"])):
            raise SystemExit(f"{name}: regenerated inputs do not rotate to the stored golden case")
        out[f"{name}_raw.W"] = W
        out[f"{name}_raw.H"] = H
        meta[f"{name}_raw"] = dict(kind="gptq_raw", rot=rot)


def greedy_gpu_cases(out: dict, meta: dict) -> None:
    """Reference GPU greedy backends on seeded inputs.  Each case starts from
    RTN codes of W and the per-row least-squares scales of those codes (what
    ldlq.py:222-231 hands to the greedy search)."""
    from converter.greedy import (greedy_lowrank_triton, greedy_local_search_triton,
                                  _lowrank_decompose)

    def lowrank_h(n, r, seed, damp):
        g = torch.Generator().manual_seed(seed)
        s = torch.exp(torch.randn(n, generator=g))
        X = torch.randn(r, n, generator=g) * s
        H = X.T @ X / r
        if damp:
            H = H + damp * H.diagonal().mean() * torch.eye(n)
        return H

    cases = [
        # name, M, N, bits, passes, H recipe (rank, damping) or None = full rank
        ("lr_a", 32, 256, 4, 3, (20, 0.0)),
        ("lr_b", 48, 192, 4, 5, (48, 0.01)),
        ("lr_c", 16, 128, 8, 2, (16, 0.0)),
        ("lr_d", 64, 320, 4, 4, (60, 0.01)),
        ("fr_a", 32, 128, 4, 2, None),
    ]
    for i, (name, M, N, bits, passes, hr) in enumerate(cases):
        qmin, qmax = (-128, 127) if bits == 8 else (-8, 7)
        W = weights(M, N, 600 + i)
        H = lognormal_hessian(N, 4 * N, 700 + i) if hr is None else lowrank_h(N, hr[0], 700 + i, hr[1])
        s0 = (W.abs().amax(dim=1, keepdim=True) / (qmax)).clamp(min=1e-5)
        Q0 = (W / s0).round().clamp(qmin, qmax)
        num = (Q0 * W).sum(dim=1, keepdim=True)
        den = (Q0 * Q0).sum(dim=1, keepdim=True).clamp(min=1e-8)
        sls = (num / den).clamp(min=1e-5)
        S2 = sls.expand(M, N).contiguous()
        torch.manual_seed(800 + i)
        s_k, U_k, k, used = _lowrank_decompose(H, rank_threshold=0.01, max_rank_frac=0.3)
        torch.manual_seed(800 + i)
        if hr is None:
            q = greedy_local_search_triton(W, Q0.clone(), S2, H, passes, qmin, qmax)
            used_lr = False
        else:
            q, k2, used_lr = greedy_lowrank_triton(W, Q0.clone(), S2, H, passes, qmin, qmax,
                                                   rank_threshold=0.01)
            assert k2 == k
        out[f"{name}.W"] = W
        out[f"{name}.H"] = H.contiguous()
        out[f"{name}.q0"] = Q0.to(torch.int8)
        out[f"{name}.s"] = sls
        out[f"{name}.q"] = q
        if used:
            out[f"{name}.s_k"] = s_k.contiguous()
            out[f"{name}.U_k"] = U_k.contiguous()
        meta[name] = dict(kind="greedy_gpu", bits=bits, passes=passes, k=int(k),
                          lowrank=bool(used_lr), rank_threshold=0.01)


def main() -> None:
    torch.set_num_threads(1)
    if GREEDY_GPU:
        out: dict[str, torch.Tensor] = {}
        meta: dict = {}
        greedy_gpu_cases(out, meta)
        out = {k: v.contiguous() for k, v in out.items()}
        save_file(out, os.path.join(HERE, "golden_greedy_gpu.safetensors"))
        with open(os.path.join(HERE, "golden_greedy_gpu.json"), "w") as f:
            json.dump(meta, f, indent=1, sort_keys=True)
        print(f"wrote {len(out)} tensors, {len(meta)} cases: {meta}")
        return
    if ROTATION:
        out: dict[str, torch.Tensor] = {}
        meta: dict = {}
        rotation_cases(out, meta)
        out = {k: v.contiguous() for k, v in out.items()}
        save_file(out, os.path.join(HERE, "golden_rotation.safetensors"))
        with open(os.path.join(HERE, "golden_rotation.json"), "w") as f:
            json.dump(meta, f, indent=1, sort_keys=True)
        print(f"wrote {len(out)} tensors, {len(meta)} cases")
        return
    out: dict[str, torch.Tensor] = {}
    meta: dict = {}
    gptq_cases(out, meta)
    ldlq_cases(out, meta)
    clip_cases(out, meta)
    pipeline_cases(out, meta)
    out = {k: v.contiguous() for k, v in out.items()}
    save_file(out, os.path.join(HERE, "golden.safetensors"))
    with open(os.path.join(HERE, "golden.json"), "w") as f:
        json.dump(meta, f, indent=1, sort_keys=True)
    print(f"wrote {len(out)} tensors, {len(meta)} cases")


if __name__ == "__main__":
    main()
