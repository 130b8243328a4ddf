"""End-to-end ``quantize_model`` on the GPU: output names, dtypes, shapes and
metadata against the reference's golden pipeline files, stored bytes and
scales against the oracle, GPTQ / LDLQ runs with calibration files,
progress events and the quality report."""

from __future__ import annotations

import json
import os
import warnings

import pytest
import torch
from safetensors import safe_open
from safetensors.torch import load_file, save_file

from oracle import torch_ref as ref
from tests.conftest import lognormal_hessian

pytestmark = pytest.mark.gpu


def _run(tmp_path, state, **kw):
    from int_crush_converter_amd.pipeline import quantize_model
    from int_crush_converter_amd.types import QuantizeConfig
    src = str(tmp_path / "in.safetensors")
    save_file(state, src)
    out = str(tmp_path / "out")
    events = []
    quantize_model(QuantizeConfig(input_path=src, output_dir=out, **kw), progress_callback=events.append)
    path = os.path.join(out, "model.safetensors")
    with safe_open(path, framework="pt") as f:
        md = f.metadata()
    return load_file(path), md, events


@pytest.mark.parametrize("tag", ["pipe_rtn4", "pipe_rtn8a"])
def test_pipeline_matches_reference_golden(gpu_dev, golden, tmp_path, tag):
    t, meta = golden
    state = {k[len("pipe_in/"):]: v for k, v in t.items() if k.startswith("pipe_in/")}
    res, md, _ = _run(tmp_path, state, **meta[tag]["config"])
    want = {k[len(tag) + 1:]: v for k, v in t.items() if k.startswith(tag + "/")}
    assert md == meta[tag]["metadata"]
    assert set(res) == set(want)
    for k, v in want.items():
        assert res[k].dtype == v.dtype and res[k].shape == v.shape, k
        # the default (exact) rotation rounds like the reference's matmul, so
        # every stored byte, scale and zero-point equals the reference's
        nd = int((res[k] != v).sum())
        print(f"[parity] pipeline_golden {tag} {k} differing={nd} of {v.numel()}", flush=True)
        assert torch.equal(res[k], v), (k, nd)


def test_pipeline_rtn_bytes_vs_oracle(gpu_dev, tmp_path):
    g = torch.Generator().manual_seed(3)
    state = {"blk.0.fc.weight": (torch.randn(96, 512, generator=g) * 0.02).to(torch.bfloat16),
             "blk.0.fc2.weight": torch.randn(32, 300, generator=g) * 0.05}
    res, md, ev = _run(tmp_path, state, rot_size=256, int_bits=4)
    for name, W in state.items():
        Wr = ref.rotate_weights(W.float(), 256)
        # bytes follow from the rotated weights: compare against codes of the GPU rotation
        from int_crush_converter_amd.rotation import rotate_weights
        Wg = rotate_weights(W.float().to(gpu_dev), 256).cpu()
        assert torch.allclose(Wg, Wr, atol=1e-6)
        # the oracle's CPU matmul on this host and the exact GPU kernel round alike
        print(f"[parity] pipeline_rtn_bytes {name} rotation_equal={torch.equal(Wg, Wr)}", flush=True)
        s = ref.scales_int4_sym(Wg, Wg.shape[1])
        q = ref.quant_int4_sym(Wg, s, Wg.shape[1])
        assert torch.equal(res[f"{name}_scale"], s)
        assert torch.equal(res[name], ref.pack_int4(q))
    assert [type(e).__name__ for e in ev] == ["ProgressInfo", "ProgressInfo", "ProgressSummary"]
    assert ev[0].current_layer == 1 and ev[1].total_layers == 2


def test_pipeline_outlier_zeroing(gpu_dev, tmp_path):
    W = torch.randn(16, 64) * 0.02
    W[3, 5] = 5000.0
    W[7, 9] = float("inf")
    res, _, _ = _run(tmp_path, {"a.weight": W}, rot_size=0, int_bits=8)
    Wz = W.masked_fill(W.abs() > 1000, 0.0)
    s = ref.scales_int8_sym(Wz)
    assert torch.equal(res["a.weight_scale"], s)
    assert torch.equal(res["a.weight"], ref.quant_int8_sym(Wz, s))


def _calib(tmp_path, hessians, rotated=False, rot=0):
    path = str(tmp_path / "cal.pt")
    torch.save({"hessians": hessians, "shapes": {k: list(v.shape) for k, v in hessians.items()},
                "layer_types": {k: "linear" for k in hessians},
                "metadata": {"num_samples": 256, "hessian_rotated": rotated, "rot_size": rot}}, path)
    return path


def test_pipeline_gptq_with_calibration(gpu_dev, tmp_path):
    g = torch.Generator().manual_seed(5)
    state = {"layers.0.attn.qkv.weight": torch.randn(64, 512, generator=g) * 0.02,
             "layers.0.mlp.up.weight": torch.randn(48, 256, generator=g) * 0.02,
             "layers.0.nocal.weight": torch.randn(16, 256, generator=g) * 0.02}
    hs = {"layers.0.attn.qkv": lognormal_hessian(512, 700, 1),
          "layers.0.mlp.up": torch.stack([lognormal_hessian(256, 400, 2)])}
    cal = _calib(tmp_path, hs)
    res, md, ev = _run(tmp_path, state, rot_size=256, quant_method="gptq", calibration_path=cal,
                       quality_report_path=str(tmp_path / "rep.json"))
    assert md["int_crush.method"] == "int_crush_gptq" and md["int_crush.scale_type"] == "per_row_asymmetric"
    for name, W in state.items():
        assert res[name].dtype == torch.uint8 and res[name].shape == (W.shape[0], W.shape[1] // 2)
        assert res[f"{name}_scale"].dtype == torch.float16
    # GPTQ INT4 is always asymmetric; the uncalibrated layer falls back to symmetric RTN (no _zp)
    assert res["layers.0.attn.qkv.weight_zp"].dtype == torch.int8 and "layers.0.nocal.weight_zp" not in res
    # the calibrated layers against the oracle
    for name, key in [("layers.0.attn.qkv.weight", "layers.0.attn.qkv"), ("layers.0.mlp.up.weight", "layers.0.mlp.up")]:
        Wr = ref.rotate_weights(state[name], 256)
        Hr = ref.rotate_hessian(hs[key], 256)
        r = ref.gptq_quantize_layer(Wr, Hr, 128, 0.01, 4)
        assert torch.equal(res[f"{name}_scale"], r.scales)
        q = ref.unpack_int4(res[name], Wr.shape[1])
        assert (q == r.quantized_W).float().mean().item() >= 0.999
    assert [e.method for e in ev[:-1]] == ["gptq_hip", "gptq_hip", "rtn"]
    assert ev[-1].gptq_layers == 2 and ev[-1].rtn_fallback_layers == 1
    rep = json.load(open(tmp_path / "rep.json"))
    assert len(rep["layers"]) == 3 and rep["summary"]["quantized"] == 3


def test_pipeline_ldlq_weight_only(gpu_dev, tmp_path):
    g = torch.Generator().manual_seed(6)
    state = {"l.0.w.weight": torch.randn(64, 256, generator=g) * 0.02}
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        res, md, ev = _run(tmp_path, state, rot_size=256, quant_method="ldlq", ldlq_iterations=2, greedy_passes=2)
    assert md["int_crush.method"] == "int_crush_ldlq" and md["int_crush.greedy_passes"] == "2"
    assert "l.0.w.weight_zp" not in res and res["l.0.w.weight"].shape == (64, 128)
    Wr = ref.rotate_weights(state["l.0.w.weight"], 256)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        # H = W^T W / 64 has rank 64 <= 0.3 x 256: the reference on a GPU takes the low-rank greedy
        r = ref.ldlq_quantize_layer(Wr, None, 128, 0.01, 4, iterations=2, greedy_passes=2, greedy_device="gpu")
    q = ref.unpack_int4(res["l.0.w.weight"], 256)
    agree = (q == r.quantized_W).float().mean().item()
    print(f"[parity] pipeline_ldlq_weight_only agreement={agree:.6f} "
          f"scales_equal={torch.equal(res['l.0.w.weight_scale'], r.scales)}", flush=True)
    assert agree >= 0.999


def test_pipeline_callback_abort_leaves_no_output(gpu_dev, tmp_path):
    from int_crush_converter_amd.pipeline import quantize_model
    from int_crush_converter_amd.types import QuantizeConfig
    src = str(tmp_path / "in.safetensors")
    save_file({"a.weight": torch.randn(8, 32)}, src)

    def boom(info):
        raise RuntimeError("stop")

    with pytest.raises(RuntimeError, match="stop"):
        quantize_model(QuantizeConfig(input_path=src, output_dir=str(tmp_path / "o"), rot_size=0),
                       progress_callback=boom)
    assert not os.path.exists(tmp_path / "o" / "model.safetensors")


def test_cli_end_to_end(gpu_dev, tmp_path):
    from int_crush_converter_amd.cli import main
    src = str(tmp_path / "in.safetensors")
    save_file({"b.0.q.weight": torch.randn(16, 256) * 0.02, "b.0.q.bias": torch.randn(16)}, src)
    main(["-i", src, "-o", str(tmp_path / "cli"), "--rot-size", "64", "--int-bits", "8", "--asymmetric",
          "--clipping-ratios", "0.9,1.0", "--comfy-compat", "--no-progress", "-q"])
    res = load_file(str(tmp_path / "cli" / "model.safetensors"))
    assert set(res) == {"b.0.q.weight", "b.0.q.weight_scale", "b.0.q.weight_zp", "b.0.q.bias", "b.0.q.comfy_quant"}
    assert json.loads(bytes(res["b.0.q.comfy_quant"].tolist()).decode()) == {
        "format": "int8_tensorwise", "convrot": True, "convrot_groupsize": 64}


@pytest.mark.parametrize("tau", [0.0, -1.0])
def test_pipeline_permuquant_rtn_vs_oracle(gpu_dev, tmp_path, tau):
    # tau = -1 accepts every permutation; tau = 0 follows the reference's
    # (rounding-decided) decision for per-row INT4
    g = torch.Generator().manual_seed(12)
    state = {"blk.0.fc.weight": torch.randn(96, 512, generator=g) * 0.02,
             "blk.0.fc2.weight": torch.randn(40, 256, generator=g) * 0.05}
    res, md, ev = _run(tmp_path, state, rot_size=256, int_bits=4, use_permuquant=True, tau=tau)
    assert md["int_crush.method"] == "int_crush_permuq" and md["int_crush.permuquant"] == "true"
    assert md["int_crush.permuquant_tau"] == str(tau)
    permuted = 0
    from int_crush_converter_amd.rotation import rotate_weights
    for name, W in state.items():
        # the reference rotates with an MKL sgemm (fp32 order not reproducible):
        # the permutation and the decision are bit-exact given the rotated weights
        Wr = rotate_weights(W.float().to(gpu_dev), 256).cpu()
        assert torch.allclose(Wr, ref.rotate_weights(W.float(), 256), atol=1e-6)
        Wp, perm, _ = ref.permuquant_layer(Wr, W.shape[1], 4, tau)
        if tau < 0:
            assert perm is not None
        if perm is None:
            assert f"{name}_perm" not in res
        else:
            permuted += 1
            assert res[f"{name}_perm"].dtype == torch.int32 and torch.equal(res[f"{name}_perm"].long(), perm)
        s = ref.scales_int4_sym(Wp, Wp.shape[1])
        assert torch.equal(res[f"{name}_scale"], s)
        assert torch.equal(res[name], ref.pack_int4(ref.quant_int4_sym(Wp, s, Wp.shape[1])))
    assert ev[-1].permuted_layers == permuted


def test_pipeline_permuquant_gptq_hessians(gpu_dev, tmp_path):
    # 2-D H: rotated then re-permuted with the weights; 3-D H: the weights
    # are un-permuted and no permutation is stored; a calibration
    # permutation is applied as given
    g = torch.Generator().manual_seed(13)
    state = {"layers.0.a.weight": torch.randn(64, 512, generator=g) * 0.02,
             "layers.0.b.weight": torch.randn(48, 256, generator=g) * 0.02,
             "layers.0.c.weight": torch.randn(32, 256, generator=g) * 0.02}
    hs = {"layers.0.a": lognormal_hessian(512, 700, 3),
          "layers.0.b": torch.stack([lognormal_hessian(256, 400, 4)]),
          "layers.0.c": lognormal_hessian(256, 400, 5)}
    cal_perm = torch.randperm(256, generator=g)
    path = str(tmp_path / "cal.pt")
    torch.save({"hessians": hs, "shapes": {k: list(v.shape) for k, v in hs.items()},
                "layer_types": {k: "linear" for k in hs}, "permuquant": {"layers.0.c": cal_perm},
                "metadata": {"num_samples": 256, "hessian_rotated": False, "rot_size": 0}}, path)
    res, md, ev = _run(tmp_path, state, rot_size=256, quant_method="gptq", calibration_path=path,
                       use_permuquant=True, tau=-1.0)
    assert md["int_crush.method"] == "int_crush_permuq_gptq"
    from int_crush_converter_amd.rotation import rotate_weights
    # 2-D (the permutation from the GPU-rotated weights, see above)
    Wr = rotate_weights(state["layers.0.a.weight"].to(gpu_dev), 256).cpu()
    Wp, perm, _ = ref.permuquant_layer(Wr, 512, 4, -1.0)
    assert torch.equal(res["layers.0.a.weight_perm"].long(), perm)
    Hr = ref.rotate_hessian(hs["layers.0.a"], 256)[perm][:, perm]
    r = ref.gptq_quantize_layer(Wp, Hr, 128, 0.01, 4)
    assert torch.equal(res["layers.0.a.weight_scale"], r.scales)
    assert (ref.unpack_int4(res["layers.0.a.weight"], 512) == r.quantized_W).float().mean().item() >= 0.999
    # 3-D: back to the unpermuted weights, no <name>_perm
    assert "layers.0.b.weight_perm" not in res
    Wb = ref.rotate_weights(state["layers.0.b.weight"], 256)
    rb = ref.gptq_quantize_layer(Wb, ref.rotate_hessian(hs["layers.0.b"], 256), 128, 0.01, 4)
    assert torch.equal(res["layers.0.b.weight_scale"], rb.scales)
    assert (ref.unpack_int4(res["layers.0.b.weight"], 256) == rb.quantized_W).float().mean().item() >= 0.999
    # calibration permutation: weights permuted, the Hessian taken as it is
    assert torch.equal(res["layers.0.c.weight_perm"].long(), cal_perm)
    Wc = ref.rotate_weights(state["layers.0.c.weight"], 256)[:, cal_perm]
    rc = ref.gptq_quantize_layer(Wc, ref.rotate_hessian(hs["layers.0.c"], 256), 128, 0.01, 4)
    assert torch.equal(res["layers.0.c.weight_scale"], rc.scales)
    assert (ref.unpack_int4(res["layers.0.c.weight"], 256) == rc.quantized_W).float().mean().item() >= 0.999
    assert ev[-1].permuted_layers == 3


def test_streaming_matches_in_memory_io(gpu_dev, tmp_path):
    # the streaming loop (prefetch, D2H stream, incremental file) writes the
    # same tensors and metadata as the reference's load-all / save-once I/O
    from int_crush_converter_amd.pipeline import quantize_model
    from int_crush_converter_amd.types import QuantizeConfig
    g = torch.Generator().manual_seed(21)
    state = {"blocks.0.attn.qkv.weight": (torch.randn(64, 512, generator=g) * 0.02).to(torch.bfloat16),
             "blocks.0.attn.qkv.bias": torch.randn(64, generator=g),
             "blocks.0.norm.weight": torch.ones(512),
             "blocks.0.mlp.up.weight": torch.randn(96, 300, generator=g) * 0.02,
             "blocks.0.embed.weight": torch.randn(10, 20, generator=g),
             "blocks.1.attn.qkv.weight": torch.randn(32, 256, generator=g) * 0.02,
             "blocks.1.attn.qkv.bias": torch.zeros(32)}
    hs = {"blocks.0.attn.qkv": lognormal_hessian(512, 600, 7), "blocks.1.attn.qkv": lognormal_hessian(256, 400, 8)}
    cal = _calib(tmp_path, hs)
    src = str(tmp_path / "in.safetensors")
    save_file(state, src)
    outs = []
    for streaming in (True, False):
        d = str(tmp_path / f"o{int(streaming)}")
        ev = []
        quantize_model(QuantizeConfig(input_path=src, output_dir=d, rot_size=256, quant_method="gptq",
                                      calibration_path=cal), progress_callback=ev.append, streaming=streaming)
        with safe_open(os.path.join(d, "model.safetensors"), framework="pt") as f:
            md = f.metadata()
        outs.append((load_file(os.path.join(d, "model.safetensors")), md, ev[-1]))
    (a, ma, sa), (b, mb, sb) = outs
    assert ma == mb and set(a) == set(b)
    for k in a:
        assert a[k].dtype == b[k].dtype and torch.equal(a[k], b[k]), k
    assert (sa.total_layers, sa.skipped_layers, sa.gptq_layers, sa.rtn_fallback_layers) == \
        (sb.total_layers, sb.skipped_layers, sb.gptq_layers, sb.rtn_fallback_layers)
    assert sa.input_size_gb == sb.input_size_gb and sa.output_size_gb == sb.output_size_gb
    assert torch.equal(a["blocks.0.attn.qkv.bias"], state["blocks.0.attn.qkv.bias"])
    assert torch.equal(a["blocks.0.embed.weight"], state["blocks.0.embed.weight"])
