"""Benchmark of the per-layer quantisation path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--workload NAME] [--no-cpu-baseline]

A step is one pass of the per-layer path over one synthetic layer whose
inputs are already resident in HBM: bf16 weights and the fp32 calibration
Hessian in, packed INT4 codes + fp16 scales + int8 zero-points out
(rotation of W, two-sided rotation of H, damping, Cholesky, inverse, GPTQ
sweep with the fp32-MFMA lazy update, fp64 verification, packing).  Building
H = X^T X / n from X is calibration and is outside the timed region.

Prints one JSON line (the last line of stdout).  ``value`` is Mweights/s
(out x in weights per second of wall time); ``roofline`` reports the
dominant kernel phase measured with HIP events inside the timed region;
``cpu_baseline`` times the CPU oracle (torch on the host cores, the
reference's own algorithm) on one layer of the same workload.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "GPTQ-INT4 Mweights/s at 4096x12288 rot256; % of HBM / fp32-MFMA peak"
PEAK_HBM_GBS = 8000.0
PEAK_FP32_MFMA_TFLOPS = 157.3

WORKLOADS = {
    # name: (kind, out, in, extra)
    "gptq_int4_rot256_4096x12288": ("gptq", 4096, 12288, {"samples": 8192}),
    "gptq_int4_rot256_3072x12288": ("gptq", 3072, 12288, {"samples": 8192}),
    "gptq_int4_rot256_12288x3072": ("gptq", 12288, 3072, {"samples": 8192}),
    "rtn_int8_asym_clip5_rot64_4096x4096": ("rtn8", 4096, 4096, {}),
    "rtn_int4_rot256_64x256": ("rtn4", 64, 256, {}),
    "ldlq_int4_it2_greedy5_rot256_4096x4096": ("ldlq", 4096, 4096, {}),
    # PermuQuant (weight-only, tau 0) + RTN INT4 on the headline layer shape
    "rtn_int4_permuquant_rot256_4096x12288": ("pq4", 4096, 12288, {}),
    # GPTQ INT4 on the headline layer shape with a rank-128 DLR Hessian
    # collected in the rotated space (Woodbury inverse, no densification)
    "gptq_int4_dlr128_rot256_4096x12288": ("dlr", 4096, 12288, {"rank": 128}),
    # GPTQ INT4 with PiSO scales (128 coarse + 16 fine candidates per row) on the headline layer
    "gptq_int4_piso_rot256_4096x12288": ("piso", 4096, 12288, {"samples": 8192, "cpu_rows": 512}),
    # configs[4] end to end, file to file (quantize_model with streaming I/O):
    # the first 4 of its 40 DiT blocks, bf16 safetensors + 3-D calibration
    "e2e_dit_gptq_int4_rot256_4blocks": ("e2e", 0, 0, {"blocks": 4, "samples": 4096,
                                                       "layers": [("attn.qkv", 12288, 4096), ("attn.proj", 4096, 4096),
                                                                  ("mlp.up", 16384, 4096),
                                                                  ("mlp.down", 4096, 16384)]}),
    # configs[4] end to end at its stated size: all 40 DiT blocks (16 GB of bf16
    # weights in, 4 GB of packed codes out), file to file
    "e2e_dit_gptq_int4_rot256_40blocks": ("e2e", 0, 0, {"blocks": 40, "samples": 4096,
                                                        "layers": [("attn.qkv", 12288, 4096), ("attn.proj", 4096, 4096),
                                                                   ("mlp.up", 16384, 4096),
                                                                   ("mlp.down", 4096, 16384)]}),
    # one block of configs[4]'s 40-block DiT sweep: four layers, block-diagonal Hessians
    "gptq_int4_rot256_dit_block": ("dit", 0, 0, {"layers": [("qkv", 12288, 4096), ("proj", 4096, 4096),
                                                            ("mlp_up", 16384, 4096), ("mlp_down", 4096, 16384)],
                                                 "samples": 4096}),
}
DEFAULT = "gptq_int4_rot256_4096x12288"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def block_hessian(X):
    """[in/256, 256, 256] block-diagonal Hessian X_b^T X_b / n of X [n, in]."""
    import torch
    n, d = X.shape
    Xb = X.reshape(n, d // 256, 256).permute(1, 0, 2).contiguous()       # [g, n, 256]
    return torch.bmm(Xb.transpose(1, 2).contiguous(), Xb) / n


def make_e2e_files(extra, seed=0):
    """A model file with configs[4]'s layer shapes (bf16, N(0, 0.02^2)) and a
    calibration file of 3-D block-diagonal Hessians, in a temporary folder."""
    import tempfile
    import torch
    from safetensors.torch import save_file
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(seed)
    d = tempfile.mkdtemp(prefix="icq_e2e_")
    state, hess = {}, {}
    for b in range(extra["blocks"]):
        for name, out_f, in_f in extra["layers"]:
            key = f"blocks.{b}.{name}"
            state[f"{key}.weight"] = (torch.randn(out_f, in_f, generator=g, device=dev) * 0.02).to(torch.bfloat16).cpu()
            s = torch.exp(torch.randn(in_f, generator=g, device=dev))
            X = torch.randn(extra["samples"], in_f, generator=g, device=dev) * s
            hess[key] = block_hessian(X).cpu()
            del X
        if (b + 1) % 4 == 0:
            log(f"[bench] generated {b + 1} of {extra['blocks']} blocks")
    src = os.path.join(d, "model.safetensors")
    save_file(state, src)
    cal = os.path.join(d, "calibration.pt")
    torch.save({"hessians": hess, "shapes": {k: list(v.shape) for k, v in hess.items()},
                "layer_types": {k: "linear" for k in hess},
                "metadata": {"num_samples": extra["samples"], "hessian_rotated": False}}, cal)
    weights = sum(t.numel() for t in state.values())
    return d, src, cal, weights


def e2e_run(d, src, cal, streaming):
    from int_crush_converter_amd.pipeline import quantize_model
    from int_crush_converter_amd.types import QuantizeConfig
    quantize_model(QuantizeConfig(input_path=src, output_dir=os.path.join(d, "out"), rot_size=256,
                                  quant_method="gptq", calibration_path=cal), streaming=streaming)


def make_inputs(kind, M, N, extra, seed=0):
    import torch
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(seed)
    if kind == "dit":
        Ws, Hs = [], []
        for _, out_f, in_f in extra["layers"]:
            Ws.append((torch.randn(out_f, in_f, generator=g, device=dev) * 0.02).to(torch.bfloat16))
            s = torch.exp(torch.randn(in_f, generator=g, device=dev))
            X = torch.randn(extra["samples"], in_f, generator=g, device=dev) * s
            Hs.append(block_hessian(X))
            del X
        torch.cuda.synchronize()
        return Ws, Hs
    W = (torch.randn(M, N, generator=g, device=dev) * 0.02)
    H = None
    if kind == "rtn8":
        cols = torch.randperm(N, generator=g, device=dev)[: max(1, N // 100)]
        W[:, cols] *= 20
    if kind == "ldlq":
        # Student-t(4) scaled to std 0.02; t = z / sqrt(chi2_4 / 4)
        z = torch.randn(M, N, generator=g, device=dev)
        chi = (torch.randn(M, N, 4, generator=g, device=dev) ** 2).sum(-1)
        W = z / torch.sqrt(chi / 4) * (0.02 / math.sqrt(2))
    W = W.to(torch.bfloat16 if kind not in ("rtn4",) else torch.float32)
    if kind == "dlr":
        # U: r orthogonal-ish directions with decaying energy; D: positive residual diagonal
        r = extra["rank"]
        lam = torch.exp(-torch.arange(r, device=dev, dtype=torch.float32) / 32.0) * 4.0
        U = torch.randn(N, r, generator=g, device=dev) / math.sqrt(N) * lam.sqrt() * math.sqrt(N / 64)
        D = torch.exp(torch.randn(N, generator=g, device=dev)) ** 2 * 0.25
        H = {"format": "dlr", "D": D, "U": U.contiguous(), "rank": r, "n": N}
    if kind in ("gptq", "piso"):
        S = extra["samples"]
        s = torch.exp(torch.randn(N, generator=g, device=dev))
        H = torch.zeros(N, N, dtype=torch.float32, device=dev)
        for r0 in range(0, S, 2048):     # X^T X / S in chunks of X rows
            X = torch.randn(min(2048, S - r0), N, generator=g, device=dev) * s
            H.addmm_(X.T, X)
            del X
        H /= S
    torch.cuda.synchronize()
    return W, H


def gpu_step(kind, W, H):
    from int_crush_converter_amd import layer as L
    if kind == "dit":
        outs = [gpu_step("gptq", Wl, Hl) for Wl, Hl in zip(W, H)]
        return outs[-1]
    if kind == "gptq":
        W_work, _ = L.prepare_weights(W, 256)
        codes, s16, z8 = L.gptq_codes(W_work, H, rotate_h=256, block_size=128, damping=0.01, int_bits=4,
                                      asymmetric=False, hessian_method="hinv", fallbacks=[])
        return L.finish(W_work, codes, s16, z8, 4)
    if kind == "piso":
        from int_crush_converter_amd import piso
        W_work, _ = L.prepare_weights(W, 256)
        ps = piso.compute_piso_scales_int4_asymmetric(W_work, H.diagonal())
        codes, s16, z8 = L.gptq_codes(W_work, H, rotate_h=256, block_size=128, damping=0.01, int_bits=4,
                                      asymmetric=False, hessian_method="hinv", fallbacks=[], piso=ps)
        return L.finish(W_work, codes, s16, z8, 4)
    if kind == "dlr":
        W_work, _ = L.prepare_weights(W, 256)
        codes, s16, z8 = L.gptq_codes(W_work, H, rotate_h=0, block_size=128, damping=0.01, int_bits=4,
                                      asymmetric=False, hessian_method="hinv", fallbacks=[])
        return L.finish(W_work, codes, s16, z8, 4)
    if kind == "rtn8":
        W_work, _ = L.prepare_weights(W, 64)
        codes, s16, z8, packed = L.rtn_codes(W_work, 8, True, [0.8, 0.85, 0.9, 0.95, 1.0])
        return L.finish(W_work, codes, s16, z8, 8, packed=packed)
    if kind == "rtn4":
        W_work, _ = L.prepare_weights(W, 256)
        codes, s16, z8, packed = L.rtn_codes(W_work, 4, False, None)
        return L.finish(W_work, codes, s16, z8, 4, packed=packed)
    if kind == "pq4":
        from int_crush_converter_amd import permuquant as pq
        W_work, _ = L.prepare_weights(W, 256)
        perm, accepted, Wp = pq.weight_only_permutation(W_work, W_work.shape[1], 0.0, 4)
        if accepted:
            W_work = Wp
        codes, s16, z8, packed = L.rtn_codes(W_work, 4, False, None)
        return L.finish(W_work, codes, s16, z8, 4, packed=packed)
    if kind == "ldlq":
        import warnings
        from int_crush_converter_amd.ldlq import ldlq_quantize_layer
        W_work, _ = L.prepare_weights(W, 256)
        with warnings.catch_warnings():
            warnings.simplefilter("ignore")
            r = ldlq_quantize_layer(W_work, None, 128, 0.01, 4, iterations=2, greedy_passes=5)
        return L.finish(W_work, r.quantized_W, r.scales, None, 4)
    raise ValueError(kind)


WORKLOADS_CPU_ROWS = 512


def cpu_step(kind, W, H):
    """The reference's CPU algorithm (oracle restatement) on the same layer.
    Returns what the parity check needs: codes, stored scales, zero-points,
    the oracle-rotated W (rows of the sample) and, for a dense Hessian, the
    rotated H."""
    import torch
    from oracle import torch_ref as ref
    if kind == "dit":   # bounded sample: the block's first layer (qkv)
        return cpu_step("gptq", W[0], H[0])
    Wf = W.float()
    Wf = Wf.masked_fill(Wf.abs() > 1000.0, 0.0)
    Hr = None
    if kind == "gptq":
        Wr = ref.rotate_weights(Wf, 256)
        Hr = ref.rotate_hessian(H, 256)
        r = ref.gptq_quantize_layer(Wr, Hr, 128, 0.01, 4)
        q, s, z = r.quantized_W, r.scales, r.zero_points
    elif kind == "piso":   # bounded sample: the first rows of the layer
        Wr = ref.rotate_weights(Wf[:WORKLOADS_CPU_ROWS], 256)
        s, z = ref.piso_scales_asym(Wr, H.diagonal().contiguous(), 128, 16, -8, 7, 0.5, 2.0)
        s = s.clamp(min=1e-5, max=65500.0)
        Q = torch.zeros(Wr.shape, dtype=torch.int8)
        ref.gptq_block(Wr.clone(), Q, s, ref.prepare_hinv(ref.rotate_hessian(H, 256), 0.01), 0, Wr.shape[1], 128,
                       -8, 7, z)
        q, s, z = Q, s.to(torch.float16), z
    elif kind == "dlr":
        Wr = ref.rotate_weights(Wf, 256)
        r = ref.gptq_quantize_layer(Wr, H, 128, 0.01, 4)
        q, s, z = r.quantized_W, r.scales, r.zero_points
    elif kind == "rtn8":
        Wr = ref.rotate_weights(Wf, 64)
        q, s, z = ref.rtn_layer(Wr, 8, True, [0.8, 0.85, 0.9, 0.95, 1.0])
    elif kind == "rtn4":
        Wr = ref.rotate_weights(Wf, 256)
        q, s, z = ref.rtn_layer(Wr, 4, False, None)
    elif kind == "pq4":
        Wr = ref.rotate_weights(Wf, 256)
        Wr, _, _ = ref.permuquant_layer(Wr, Wr.shape[1], 4, 0.0)
        q, s, z = ref.rtn_layer(Wr, 4, False, None)
    else:
        import warnings
        Wr = ref.rotate_weights(Wf, 256)
        with warnings.catch_warnings():
            warnings.simplefilter("ignore")
            r = ref.ldlq_quantize_layer(Wr, None, 128, 0.01, 4, iterations=2, greedy_passes=5)
        q, s, z = r.quantized_W, r.scales, None
    d = (q.float() - (z.float() if z is not None else 0)) * s.float()
    (Wr - d).double().pow(2).mean().item()
    if kind != "rtn8":
        ref.pack_int4(q)
    return {"q": q, "s": s, "z": z, "Wr": Wr, "Hr": Hr}


def oracle_self_codes(cpu):
    """The oracle's GPTQ codes again with half the CPU threads: LAPACK's
    Cholesky / inverse change their fp32 summation order with the thread
    count, which measures the reference's own run-to-run noise."""
    import torch
    from oracle import torch_ref as ref
    threads = torch.get_num_threads()
    torch.set_num_threads(max(1, threads // 2))
    try:
        Hinv = ref.prepare_hinv(cpu["Hr"], 0.01)
    finally:
        torch.set_num_threads(threads)
    s32, z = ref.gptq_row_params(cpu["Wr"], 4, False)
    Q = torch.zeros(cpu["Wr"].shape, dtype=torch.int8)
    ref.gptq_block(cpu["Wr"].clone(), Q, s32, Hinv, 0, cpu["Wr"].shape[1], 128, -8, 7, z)
    return Q


def oracle_on_gpu_rotation(out, H):
    """The oracle's GPTQ layer on the GPU-rotated W and H of the timed step
    (the same quantiser inputs; the rotations round differently)."""
    from oracle import torch_ref as ref
    from int_crush_converter_amd.rotation import rotate_hessian_gpu
    Hg = rotate_hessian_gpu(H, 256).cpu()
    return ref.gptq_quantize_layer(out.W_work.cpu(), Hg, 128, 0.01, 4).quantized_W


def parity(kind, out, cpu, self_codes=None, same_codes=None):
    """Codes of the timed GPU step against the oracle's: share of equal codes
    (against the oracle from the same raw inputs, and against the oracle on
    the GPU-rotated inputs), relative tr(dW H dW^T) difference (dense-Hessian
    GPTQ), stored-scale equality and the largest fp16-ulp scale difference;
    for GPTQ also the oracle's own noise (half the CPU threads, and its
    layer on the GPU's rotation)."""
    import torch
    dev = torch.device("cuda:0")
    rows = cpu["q"].shape[0]
    q = out.codes[:rows].cpu()
    s = out.scales.reshape(-1)[:rows].cpu()
    s_ref = cpu["s"].reshape(-1)
    res = {"vs": "oracle (the reference's CPU algorithm) on the same inputs", "rows": rows,
           "agreement": round((q == cpu["q"]).float().mean().item(), 6),
           "scales_equal": bool(torch.equal(s.to(s_ref.dtype), s_ref))}
    if s_ref.dtype == torch.float16:
        ulps = (s.view(torch.int16).int() - s_ref.view(torch.int16).int()).abs().max().item()
        res["scale_max_fp16_ulps"] = int(ulps)
    if cpu["Hr"] is not None:
        Hr = cpu["Hr"] if cpu["Hr"].dim() == 2 else torch.block_diag(*cpu["Hr"])
        Hd = Hr.to(dev).double()
        Wd = cpu["Wr"].to(dev).double()

        def proxy(Q, sc, zp):
            d = (Q.to(dev).double() - (zp.to(dev).double().reshape(-1, 1) if zp is not None else 0)) \
                * sc.to(dev).double().reshape(-1, 1) - Wd
            return ((d @ Hd) * d).sum().item()

        p_ref = proxy(cpu["q"], cpu["s"].float(), cpu["z"])
        zg = None if out.zero_points is None else out.zero_points.reshape(-1)[:rows].cpu()
        res["proxy_rel"] = round(proxy(q, s.float(), zg) / p_ref - 1, 7)
        if self_codes is not None:
            res["oracle_self_agreement"] = round((self_codes == cpu["q"]).float().mean().item(), 6)
            res["oracle_self_proxy_rel"] = round(proxy(self_codes, cpu["s"].float(), cpu["z"]) / p_ref - 1, 7)
        if same_codes is not None:
            res["agreement_same_inputs"] = round((q == same_codes).float().mean().item(), 6)
            res["oracle_rotation_agreement"] = round((same_codes == cpu["q"]).float().mean().item(), 6)
        del Hd, Wd
    return res


def host_cpu():
    """Model name, sockets, cores and SMT of the host (lscpu), and the CPU
    share this process may use."""
    import subprocess
    info = {}
    try:
        txt = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        for line in txt.splitlines():
            k, _, v = line.partition(":")
            info[k.strip()] = v.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    out = {"model": info.get("Model name"), "sockets": info.get("Socket(s)"),
           "cores_per_socket": info.get("Core(s) per socket"), "threads_per_core": info.get("Thread(s) per core"),
           "logical_cpus": os.cpu_count()}
    try:
        out["affinity_cpus"] = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        pass
    return out


def measured_traffic(workload, kernel):
    """HBM bytes per launch of `kernel` on `workload`, from the committed
    FETCH_SIZE / WRITE_SIZE counter runs (profiles/gemm_traffic.json), already
    scaled by what the same counters read for a plain copy; None if absent."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "gemm_traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None
    if rec.get("workload") != workload or rec.get("kernel") != kernel:
        return None
    return rec.get("traffic_bytes_per_launch")


def roofline_from(prof, workload):
    """The roofline of the dominant MFMA- or HBM-bound kernel (most summed
    time over the timed steps): achieved = algorithmic work per launch /
    average launch duration.  Kernels bound by a dependency chain or by
    instruction issue (the column sweep, the greedy block kernel, the
    diagonal-block factorisation) have no roofline; they are reported as
    shares of the profiled time instead (`latency_shares`)."""
    from int_crush_converter_amd._native import FWHT_KERNELS, PROFILE_KERNELS
    from int_crush_converter_amd.rotation import rotation_kernel
    kernels, total = {}, sum(v["ms"] for v in prof.values())
    for kname, (phases, bound) in PROFILE_KERNELS.items():
        if rotation_kernel() == "fwht" and kname in FWHT_KERNELS:
            kname, bound = FWHT_KERNELS[kname]
        kernels[kname] = {k: sum(prof[p][k] for p in phases) for k in ("ms", "flops", "bytes", "launches")}
        kernels[kname]["bound"] = bound
    shares = {k: round(v["ms"] / total, 4) for k, v in kernels.items()
              if v["bound"] == "latency" and v["ms"] > 0 and total > 0}
    bounded = {k: v for k, v in kernels.items() if v["bound"] != "latency"}
    name, ph = max(bounded.items(), key=lambda kv: kv[1]["ms"])
    n = max(ph["launches"], 1)
    avg_ms = ph["ms"] / n
    if ph["bound"] == "mfma":
        achieved = (ph["flops"] / n) / (avg_ms * 1e-3) / 1e12 if avg_ms > 0 else 0.0
        bound, peak, unit = "mfma", PEAK_FP32_MFMA_TFLOPS, "TFLOP/s"
    else:
        achieved = (ph["bytes"] / n) / (avg_ms * 1e-3) / 1e9 if avg_ms > 0 else 0.0
        bound, peak, unit = "hbm", PEAK_HBM_GBS, "GB/s"
    return name, {"bound": bound, "achieved": round(achieved, 3), "peak": peak, "unit": unit,
                  "frac": round(achieved / peak, 4), "traffic": measured_traffic(workload, name),
                  "share_of_profiled_time": round(ph["ms"] / total, 4) if total > 0 else None,
                  "latency_shares": shares}


def hbm_ceiling(nbytes=1 << 30, reps=10):
    """GB/s of the library's streaming probes (ic_hbm_stream) on 1 GiB: the
    practical HBM ceiling of the box for each read/write mix.  Bytes counted:
    copy read + written, read, write, convert 2 read + 4 written per element."""
    import torch
    from int_crush_converter_amd import _native as nat
    L = nat.lib()
    src = torch.ones(nbytes // 4, device="cuda:0")
    dst = torch.empty(nbytes // 2, device="cuda:0")     # room for kind 3's 2 x nbytes
    out = {}
    for kind, name, moved in ((0, "copy", 2 * nbytes), (1, "read", nbytes), (2, "write", nbytes),
                              (3, "bf16_to_fp32", 3 * nbytes)):
        call = lambda: nat.check(L.ic_hbm_stream(kind, src.data_ptr(), dst.data_ptr(), nbytes, nat.stream()),
                                 "ic_hbm_stream")
        call()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            call()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        out[name] = {"GB/s": round(moved / ms / 1e6, 1), "us": round(ms * 1e3, 1), "bytes": moved}
    return {"hbm_ceiling": out, "peak_GB/s": PEAK_HBM_GBS}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default=DEFAULT, choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-profile", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 256 MiB fp32 device copy (3 times), the reference for HBM counters")
    ap.add_argument("--hbm-ceiling", action="store_true",
                    help="only time the library's streaming probes (copy, read, write, bf16->fp32 convert)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build runs the per-layer path on a single MI355X "
              "(layers shard across GPUs without communication; see the sharding notes).", file=sys.stderr)
        sys.exit(2)

    import torch
    from int_crush_converter_amd import _native as nat
    if args.copy_calibration:
        a = torch.ones(64 << 20, device="cuda:0")
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration": True, "bytes_read": a.numel() * 4, "bytes_written": b.numel() * 4,
                          "launches": 3}), flush=True)
        return
    if args.hbm_ceiling:
        print(json.dumps(hbm_ceiling()), flush=True)
        return
    kind, M, N, extra = WORKLOADS[args.workload]
    if kind == "e2e":
        return main_e2e(args, extra)
    log(f"[bench] workload {args.workload}: generating inputs")
    W, H = make_inputs(kind, M, N, extra)
    nat.lib()
    log(f"[bench] warmup {args.warmup}")
    for _ in range(args.warmup):
        gpu_step(kind, W, H)
    torch.cuda.synchronize()
    log(f"[bench] timing {args.steps} steps")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        out = gpu_step(kind, W, H)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms = (t1 - t0) * 1e3 / args.steps
    # Per-kernel HIP-event timing brackets every library launch with two
    # events, which costs a few percent of wall time; it runs on separate
    # steps of the same workload so that ms_per_step is the plain rate.
    prof = None
    prof_steps = 0
    if not args.no_profile:
        prof_steps = min(args.steps, 3)
        nat.profile_enable(True)
        for _ in range(prof_steps):
            gpu_step(kind, W, H)
        torch.cuda.synchronize()
        prof = nat.profile_read()
        nat.profile_enable(False)
    weights = M * N if kind != "dit" else sum(o * i for _, o, i in extra["layers"])
    value = weights / (ms * 1e-3) / 1e6
    log(f"[bench] {ms:.3f} ms/step, {value:.1f} Mweights/s, mse {out.mse:.3e}")

    result = {
        "metric": METRIC if args.workload == DEFAULT else f"{args.workload} Mweights/s",
        "value": round(value, 3),
        "unit": "Mweights/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded N(0,0.02^2) bf16 weights; H = X^T X / n, X rows N(0, diag(s^2)), "
                "s ~ LogNormal(0,1)); random-init, no checkpoint",
        "config": {"workload": args.workload, "out_features": M, "in_features": N,
                   **({"layers": [f"{n} {o}x{i}" for n, o, i in extra["layers"]], "hessian": "block-diagonal 256"}
                      if kind == "dit" else {}),
                   **({"hessian": f"DLR rank {extra['rank']}, collected rotated (Woodbury inverse)"}
                      if kind == "dlr" else {}),
                   "layers_per_s": round(1e3 / ms, 4), "rot_size": 256 if kind != "rtn8" else 64,
                   "block": 128, "damping": 0.01},
    }
    if prof is not None:
        dom, roof = roofline_from(prof, args.workload)
        result["roofline"] = roof
        result["roofline"]["kernel"] = dom
        steps = prof_steps
        result["phases"] = {k: {"ms_per_step": round(v["ms"] / steps, 4), "launches_per_step": v["launches"] // steps,
                                "TFLOP/s": round(v["flops"] / max(v["ms"], 1e-9) / 1e9, 3),
                                "GB/s": round(v["bytes"] / max(v["ms"], 1e-9) / 1e6, 1)}
                            for k, v in prof.items() if v["launches"]}
    if not args.no_cpu_baseline:
        # torch's intra-op threads: OMP_NUM_THREADS, the CPU share of one GPU
        # on the box (os.cpu_count() counts the whole host)
        threads = torch.get_num_threads()
        log(f"[bench] CPU baseline (oracle, {threads} threads): 1 layer")
        if kind == "dit":
            Wc, Hc = [w.cpu() for w in W], [h.cpu() for h in H]
            sample_w, sample = extra["layers"][0][1] * extra["layers"][0][2], "the qkv layer of one DiT block"
        elif kind == "piso":
            Wc, Hc = W.cpu(), H.cpu()
            sample_w = extra["cpu_rows"] * N
            sample = f"the first {extra['cpu_rows']} rows of 1 layer of {args.workload}"
        else:
            Wc = W.cpu()
            Hc = ({k: (v.cpu() if torch.is_tensor(v) else v) for k, v in H.items()} if isinstance(H, dict)
                  else H.cpu() if H is not None else None)
            sample_w, sample = weights, f"1 layer of {args.workload}"
        c0 = time.perf_counter()
        cpu = cpu_step(kind, Wc, Hc)
        c1 = time.perf_counter()
        result["cpu_baseline"] = {"value": round(sample_w / (c1 - c0) / 1e6, 3), "unit": "Mweights/s",
                                  "cores": threads, "kind": "port",
                                  "sample": f"{sample} ({c1 - c0:.1f} s), torch CPU oracle "
                                            "restating the reference's CPU path",
                                  "host": host_cpu()}
        log(f"[bench] CPU {c1 - c0:.2f} s; parity of the timed step's output")
        # untimed: the codes of the timed step against the oracle's
        ref_out = gpu_step("gptq", W[0], H[0]) if kind == "dit" else out
        self_codes = oracle_self_codes(cpu) if kind == "gptq" else None
        same_codes = oracle_on_gpu_rotation(out, H) if kind == "gptq" else None
        result["parity"] = parity(kind, ref_out, cpu, self_codes, same_codes)
        log(f"[bench] parity {result['parity']}")
    print(json.dumps(result), flush=True)


def main_e2e(args, extra):
    """File to file: quantize_model on a synthetic slice of configs[4]; a step
    is one whole conversion.  Also times the reference's load-all /
    save-once I/O on the same files (in_memory_ms)."""
    import shutil
    import torch
    from int_crush_converter_amd import _native as nat
    log(f"[bench] workload {args.workload}: writing the model and calibration files")
    d, src, cal, weights = make_e2e_files(extra)
    try:
        nat.lib()
        for _ in range(args.warmup):
            e2e_run(d, src, cal, True)
        torch.cuda.synchronize()
        times = {}
        for streaming in (True, False):
            t0 = time.perf_counter()
            for _ in range(args.steps):
                e2e_run(d, src, cal, streaming)
            torch.cuda.synchronize()
            times[streaming] = (time.perf_counter() - t0) * 1e3 / args.steps
        ms = times[True]
        prof = None
        if not args.no_profile:
            nat.profile_enable(True)
            e2e_run(d, src, cal, True)
            torch.cuda.synchronize()
            prof = nat.profile_read()
            nat.profile_enable(False)
        in_bytes = os.path.getsize(src)
        out_bytes = os.path.getsize(os.path.join(d, "out", "model.safetensors"))
        value = weights / (ms * 1e-3) / 1e6
        log(f"[bench] {ms:.1f} ms per conversion ({value:.0f} Mweights/s); in-memory I/O {times[False]:.1f} ms")
        result = {
            "metric": f"{args.workload} Mweights/s (file to file)",
            "value": round(value, 3), "unit": "Mweights/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(ms, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "fp32",
            "data": "synthetic safetensors file (seeded N(0,0.02^2) bf16 weights) + 3-D calibration Hessians "
                    "X_b^T X_b / 4096 with LogNormal channel scales; random-init, no checkpoint",
            "config": {"workload": args.workload, "blocks": extra["blocks"],
                       "layers": [f"{n} {o}x{i}" for n, o, i in extra["layers"]], "weights": weights,
                       "input_bytes": in_bytes, "output_bytes": out_bytes, "rot_size": 256, "block": 128,
                       "damping": 0.01, "in_memory_ms": round(times[False], 3),
                       "in_memory_mweights_per_s": round(weights / (times[False] * 1e-3) / 1e6, 3),
                       "streaming_speedup": round(times[False] / ms, 3)},
        }
        if prof is not None:
            dom, roof = roofline_from(prof, args.workload)
            result["roofline"] = roof
            result["roofline"]["kernel"] = dom
            result["phases"] = {k: {"ms_per_step": round(v["ms"], 4), "launches_per_step": v["launches"],
                                    "TFLOP/s": round(v["flops"] / max(v["ms"], 1e-9) / 1e9, 3),
                                    "GB/s": round(v["bytes"] / max(v["ms"], 1e-9) / 1e6, 1)}
                                for k, v in prof.items() if v["launches"]}
        if not args.no_cpu_baseline:
            from safetensors import safe_open
            threads = torch.get_num_threads()
            name0 = f"blocks.0.{extra['layers'][0][0]}"
            with safe_open(src, framework="pt") as f:
                W0 = f.get_tensor(name0 + ".weight")
            H0 = torch.load(cal, weights_only=True)["hessians"][name0]
            c0 = time.perf_counter()
            cpu_step("gptq", W0, H0)
            c1 = time.perf_counter()
            result["cpu_baseline"] = {"value": round(W0.numel() / (c1 - c0) / 1e6, 3), "unit": "Mweights/s",
                                      "cores": threads, "kind": "port",
                                      "sample": f"layer {name0} ({c1 - c0:.1f} s), torch CPU oracle restating "
                                                "the reference's CPU path (compute only, no file I/O)",
                                      "host": host_cpu()}
        print(json.dumps(result), flush=True)
    finally:
        shutil.rmtree(d, ignore_errors=True)


if __name__ == "__main__":
    main()
