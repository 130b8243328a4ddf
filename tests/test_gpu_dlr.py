"""Diagonal + low-rank Hessians on the GPU against the oracle.

Bars:
  * Woodbury inverse: error against the fp64 inverse of the damped dense H
    at most 4x the oracle's own fp32 error (same formula, MFMA products and
    a blocked Cholesky instead of MKL / LAPACK), plus 2e-7 of its largest
    entry for the cases where the oracle happens to be nearly exact.
  * Dense form and rotation: within fp32 accumulation error of fp64.
  * GPTQ / LDLQ layers: scales / zero-points bit-exact (they do not depend on
    H), codes agree on >= 99.9 % with the oracle's, the proxy loss
    tr(dW H dW^T) within 1e-2 (the small-case fp32 noise band).
  * Pipeline: a DLR calibration file gives the same outputs as the dense
    Hessian it stands for wherever the path densifies (rotation); the
    Woodbury path agrees with the oracle to the layer bar.
"""

from __future__ import annotations

import os

import pytest
import torch
from safetensors.torch import load_file, save_file

from oracle import torch_ref as ref

pytestmark = pytest.mark.gpu


def _factors(n, r, seed, scale=0.3):
    g = torch.Generator().manual_seed(seed)
    return torch.rand(n, generator=g) + 0.1, torch.randn(n, r, generator=g) * scale


def _calib_factors(n, r, seed, samples=None):
    """D, U as calibration writes them: top-r eigenpairs of X^T X / s and the
    residual diagonal (tests/unit/test_dlr_hessian.py:45-60)."""
    g = torch.Generator().manual_seed(seed)
    s = torch.exp(torch.randn(n, generator=g))
    X = torch.randn(samples or 2 * n, n, generator=g) * s
    H = (X.T @ X / X.shape[0]).double()
    ev, V = torch.linalg.eigh(H)
    U = V[:, -r:] * ev[-r:].clamp(min=0).sqrt()
    D = (H.diagonal() - (U ** 2).sum(dim=1)).clamp(min=0)
    return D.float(), U.float().contiguous()


def _dense64(D, U, damping):
    H = torch.diag(D.double()) + U.double() @ U.double().T
    if damping > 0:
        dm = max((D.double() + (U.double() ** 2).sum(dim=1)).mean().item(), 1e-6)
        H = H + damping * dm * torch.eye(D.shape[0], dtype=torch.float64)
    return H


@pytest.mark.parametrize("n,r", [(1, 1), (16, 4), (300, 0), (300, 1), (1000, 64), (2048, 300), (4096, 128),
                                 (777, 77)])
@pytest.mark.parametrize("damping", [0.0, 0.01])
def test_woodbury_vs_fp64(gpu_dev, n, r, damping):
    from int_crush_converter_amd.dlr import woodbury_inverse
    D, U = _factors(n, r, n + r)
    want = torch.linalg.inv(_dense64(D, U, damping))
    got = woodbury_inverse(D.to(gpu_dev), U.to(gpu_dev), damping).cpu().double()
    mine = (got - want).abs().max().item()
    theirs = (ref.woodbury_inverse(D, U, damping).double() - want).abs().max().item()
    assert mine <= 4 * theirs + 2e-7 * want.abs().max().item(), (mine, theirs)
    # upper_only: the same upper triangle, zeros just below the diagonal
    up = woodbury_inverse(D.to(gpu_dev), U.to(gpu_dev), damping, upper_only=True).cpu()
    iu = torch.triu_indices(n, n)
    assert torch.equal(up[iu[0], iu[1]], got.float()[iu[0], iu[1]])
    band = torch.tril(torch.ones(n, n, dtype=torch.bool), -1) & ~torch.tril(torch.ones(n, n, dtype=torch.bool), -128)
    assert (up[band] == 0).all()


def test_woodbury_device_and_special_cases(gpu_dev):
    from int_crush_converter_amd.dlr import woodbury_inverse
    D, U = _factors(16, 4, 7)
    # CPU factors are computed on the GPU and returned where D lives
    assert woodbury_inverse(D, U).device.type == "cpu"
    assert woodbury_inverse(D, U, device=gpu_dev).device.type == "cuda"
    # U = 0: diag(1/D)
    got = woodbury_inverse(D.to(gpu_dev), torch.zeros(16, 1, device=gpu_dev)).cpu()
    assert torch.allclose(got, torch.diag(1.0 / D), atol=1e-6)
    # zero diagonal entries (padding columns) stay finite under damping
    D0 = D.clone()
    D0[:3] = 0.0
    assert torch.isfinite(woodbury_inverse(D0.to(gpu_dev), U.to(gpu_dev), 0.01)).all()
    # a strided U (a column slice of a wider factor)
    Uw = torch.randn(16, 9)
    a = woodbury_inverse(D.to(gpu_dev), Uw.to(gpu_dev)[:, 2:6], 0.01).cpu()
    b = woodbury_inverse(D.to(gpu_dev), Uw[:, 2:6].contiguous().to(gpu_dev), 0.01).cpu()
    assert torch.equal(a, b)


def test_woodbury_given_capacitance_inverse(gpu_dev):
    # the second call of the Cholesky-failure path: M^-1 given, M not refactored
    from int_crush_converter_amd import _native as nat
    n, r = 500, 40
    D, U = _factors(n, r, 11)
    Dg, Ug = D.to(gpu_dev), U.to(gpu_dev)
    H1 = torch.empty(n, n, device=gpu_dev)
    H2 = torch.empty(n, n, device=gpu_dev)
    M = torch.empty(r, r, device=gpu_dev)
    info = torch.zeros(2, dtype=torch.int32, device=gpu_dev)
    ws = nat.workspace(nat.lib().ic_woodbury_workspace_bytes(n, r), gpu_dev)
    L = nat.lib()
    nat.check(L.ic_woodbury_inverse(Dg.data_ptr(), Ug.data_ptr(), n, r, r, 0.01, None, 0, H1.data_ptr(), n,
                                    M.data_ptr(), info.data_ptr(), ws.data_ptr(), nat.stream()), "woodbury")
    assert info.tolist() == [0, 0]
    Mi = torch.linalg.inv(M.double()).float().contiguous()
    nat.check(L.ic_woodbury_inverse(Dg.data_ptr(), Ug.data_ptr(), n, r, r, 0.01, Mi.data_ptr(), 0, H2.data_ptr(), n,
                                    None, info.data_ptr(), ws.data_ptr(), nat.stream()), "woodbury")
    want = torch.linalg.inv(_dense64(D, U, 0.01))
    for H in (H1, H2):
        assert (H.cpu().double() - want).abs().max().item() <= 1e-5 * want.abs().max().item()
    # M itself: I + U^T diag(1/D') U
    dm = (D.double() + (U.double() ** 2).sum(dim=1)).mean()
    Dd = D.double() + 0.01 * dm
    Mw = torch.eye(r, dtype=torch.float64) + U.double().T @ (U.double() / Dd[:, None])
    assert (M.cpu().double() - Mw).abs().max().item() <= 1e-5 * Mw.abs().max().item()


@pytest.mark.parametrize("n,r", [(64, 8), (300, 17), (1024, 0)])
def test_dense_form_and_rotation(gpu_dev, n, r):
    from int_crush_converter_amd.dlr import dlr_to_dense, make_dlr_dict, rotate_dlr_to_dense
    from int_crush_converter_amd.rotation import rotate_hessian
    D, U = _factors(n, r, n)
    H = dlr_to_dense(D.to(gpu_dev), U.to(gpu_dev)).cpu()
    want = torch.diag(D.double()) + U.double() @ U.double().T
    assert (H.double() - want).abs().max().item() <= 1e-6 * (want.abs().max().item() + 1)
    if n % 64 == 0 or n == 300:
        rot = 64
        Hr = rotate_hessian(make_dlr_dict(D.to(gpu_dev), U.to(gpu_dev)), rot).cpu()
        assert torch.equal(Hr, rotate_dlr_to_dense(D.to(gpu_dev), U.to(gpu_dev), rot).cpu())
        Rr = ref.rotate_hessian(want.float(), rot).double()
        assert Hr.shape == Rr.shape
        assert (Hr.double() - Rr).abs().max().item() <= 1e-5 * (Rr.abs().max().item() + 1)


def _proxy(W, Q, s16, z8, H):
    d = ((Q.float() - (z8.float() if z8 is not None else 0)) * s16.float() - W).double()
    return (d @ H.double() * d).sum().item()


@pytest.mark.parametrize("M,n,r,bits,asym,block", [(64, 512, 16, 4, False, 128), (96, 300, 8, 8, False, 64),
                                                   (32, 1024, 64, 8, True, 128), (48, 256, 32, 4, False, 32)])
def test_gptq_dlr_layer_vs_oracle(gpu_dev, M, n, r, bits, asym, block):
    from int_crush_converter_amd.dlr import make_dlr_dict
    from int_crush_converter_amd.gptq import gptq_quantize_layer
    D, U = _calib_factors(n, r, M + n)
    W = torch.randn(M, n, generator=torch.Generator().manual_seed(n)) * 0.02
    want = ref.gptq_quantize_layer(W, make_dlr_dict(D, U), block, 0.01, bits, asym)
    got = gptq_quantize_layer(W.to(gpu_dev), make_dlr_dict(D.to(gpu_dev), U.to(gpu_dev)), block_size=block,
                              damping=0.01, int_bits=bits, asymmetric=asym)
    assert torch.equal(got.scales.cpu(), want.scales)
    if want.zero_points is not None:
        assert torch.equal(got.zero_points.cpu(), want.zero_points)
    q = got.quantized_W.cpu()
    assert (q == want.quantized_W).float().mean().item() >= 0.999
    H = _dense64(D, U, 0.0)
    z = want.zero_points
    p_ref = _proxy(W, want.quantized_W, want.scales, z, H)
    assert abs(_proxy(W, q, got.scales.cpu(), z, H) / p_ref - 1) <= 1e-2


def test_gptq_dlr_reference_behaviour(gpu_dev):
    # tests/unit/test_dlr_hessian.py:480-680 on this build
    from int_crush_converter_amd.dlr import make_dlr_dict
    from int_crush_converter_amd.gptq import gptq_quantize_layer
    D, U = _calib_factors(64, 8, 1)
    dlr = make_dlr_dict(D, U)
    W = torch.randn(16, 64, generator=torch.Generator().manual_seed(2))
    r4 = gptq_quantize_layer(W, dlr, int_bits=4)
    assert r4.quantized_W.dtype == torch.int8 and r4.scales.shape == (16, 1) and r4.zero_points is not None
    assert r4.quantized_W.min() >= -8 and r4.quantized_W.max() <= 7 and (r4.scales > 0).all()
    r8 = gptq_quantize_layer(W, dlr, int_bits=8)
    assert r8.zero_points is None and torch.isfinite(r8.scales.float()).all()
    assert gptq_quantize_layer(W, dlr, int_bits=8, asymmetric=True).zero_points is not None
    assert (gptq_quantize_layer(torch.zeros(8, 64), dlr).quantized_W == 0).all()
    # damping keeps a nearly singular DLR Hessian usable
    Ds = torch.zeros(32)
    Ds[0] = 1.0
    rs = gptq_quantize_layer(torch.randn(8, 32), make_dlr_dict(Ds, torch.zeros(32, 4)), damping=0.1)
    assert torch.isfinite(rs.quantized_W.float()).all()
    for bs in (32, 64, 128):
        assert gptq_quantize_layer(W, dlr, block_size=bs).quantized_W.shape == (16, 64)
    with pytest.raises(ValueError, match="dim.*in_features"):
        gptq_quantize_layer(torch.randn(8, 128), dlr)
    # DLR against the dense Hessian it approximates: within 2x its MSE (the reference's bar)
    X = torch.randn(256, 64, generator=torch.Generator().manual_seed(3))
    Hf = X.T @ X
    ev, V = torch.linalg.eigh(Hf.double())
    Uf = (V[:, -16:] * ev[-16:].clamp(min=0).sqrt()).float()
    Df = (Hf.diagonal().double() - (Uf.double() ** 2).sum(dim=1)).clamp(min=0).float()
    qf = gptq_quantize_layer(W, Hf, int_bits=8)
    qd = gptq_quantize_layer(W, make_dlr_dict(Df, Uf), int_bits=8)
    assert qd.mse <= qf.mse * 2.0 + 1e-8


@pytest.mark.parametrize("iters", [1, 3])
def test_ldlq_dlr_vs_oracle(gpu_dev, iters):
    from int_crush_converter_amd.dlr import make_dlr_dict
    from int_crush_converter_amd.ldlq import ldlq_quantize_layer
    D, U = _calib_factors(512, 32, 9)
    W = torch.randn(64, 512, generator=torch.Generator().manual_seed(10)) * 0.02
    want = ref.ldlq_quantize_layer(W, make_dlr_dict(D, U), 128, 0.01, 4, iterations=iters)
    got = ldlq_quantize_layer(W.to(gpu_dev), make_dlr_dict(D.to(gpu_dev), U.to(gpu_dev)), 128, 0.01, 4,
                              iterations=iters)
    assert (got.quantized_W.cpu() == want.quantized_W).float().mean().item() >= 0.999
    assert got.zero_points is None and (got.scales > 0).all()
    with pytest.raises(ValueError):
        ldlq_quantize_layer(W.to(gpu_dev), make_dlr_dict(D, U), greedy_passes=1)
    with pytest.raises(ValueError, match="dim.*in_features"):
        ldlq_quantize_layer(W[:, :256].to(gpu_dev), make_dlr_dict(D, U))


def _run(tmp_path, state, cal, sub, **kw):
    from int_crush_converter_amd.pipeline import quantize_model
    from int_crush_converter_amd.types import QuantizeConfig
    src = str(tmp_path / "in.safetensors")
    save_file(state, src)
    cpath = str(tmp_path / f"{sub}.pt")
    torch.save(cal, cpath)
    out = str(tmp_path / sub)
    quantize_model(QuantizeConfig(input_path=src, output_dir=out, calibration_path=cpath, **kw))
    return load_file(os.path.join(out, "model.safetensors"))


def _cal(hs):
    return {"hessians": hs, "shapes": {}, "layer_types": {k: "linear" for k in hs},
            "metadata": {"num_samples": 256, "hessian_rotated": False, "rot_size": 0}}


@pytest.mark.parametrize("method", ["gptq", "ldlq"])
def test_pipeline_dlr_rotated_equals_dense(gpu_dev, tmp_path, method):
    # rotation densifies the DLR Hessian: same outputs as its dense form
    from int_crush_converter_amd.dlr import dlr_to_dense, make_dlr_dict
    g = torch.Generator().manual_seed(21)
    state = {"blocks.0.attn.qkv.weight": torch.randn(64, 512, generator=g) * 0.02,
             "blocks.0.mlp.fc.weight": torch.randn(32, 300, generator=g) * 0.02}
    f = {"blocks.0.attn.qkv": _calib_factors(512, 32, 1), "blocks.0.mlp.fc": _calib_factors(300, 16, 2)}
    dlr = {k: make_dlr_dict(*v) for k, v in f.items()}
    dense = {k: dlr_to_dense(v[0].to(gpu_dev), v[1].to(gpu_dev)).cpu() for k, v in f.items()}
    a = _run(tmp_path, state, _cal(dlr), "dlr", rot_size=256, quant_method=method)
    b = _run(tmp_path, state, _cal(dense), "dense", rot_size=256, quant_method=method)
    assert a.keys() == b.keys()
    for k in a:
        assert torch.equal(a[k], b[k]), k


def test_pipeline_dlr_woodbury_and_permutation(gpu_dev, tmp_path):
    # no rotation: the Woodbury path; with PermuQuant the factors are permuted
    from int_crush_converter_amd.dlr import make_dlr_dict
    g = torch.Generator().manual_seed(23)
    W = torch.randn(64, 512, generator=g) * 0.02
    W = W * torch.exp(torch.randn(512, generator=g))
    state = {"blocks.0.attn.proj.weight": W}
    D, U = _calib_factors(512, 24, 3)
    cal = _cal({"blocks.0.attn.proj": make_dlr_dict(D, U)})
    res = _run(tmp_path, state, cal, "plain", rot_size=0, quant_method="gptq")
    want = ref.gptq_quantize_layer(W, make_dlr_dict(D, U), 128, 0.01, 4)
    assert torch.equal(res["blocks.0.attn.proj.weight_scale"], want.scales)
    q = ref.unpack_int4(res["blocks.0.attn.proj.weight"], 512)
    assert (q == want.quantized_W).float().mean().item() >= 0.999
    res = _run(tmp_path, state, cal, "perm", rot_size=0, quant_method="gptq", use_permuquant=True, tau=-1.0)
    perm = res["blocks.0.attn.proj.weight_perm"].long()
    assert sorted(perm.tolist()) == list(range(512))
    want = ref.gptq_quantize_layer(W[:, perm], make_dlr_dict(D[perm], U[perm]), 128, 0.01, 4)
    assert torch.equal(res["blocks.0.attn.proj.weight_scale"], want.scales)
    q = ref.unpack_int4(res["blocks.0.attn.proj.weight"], 512)
    assert (q == want.quantized_W).float().mean().item() >= 0.999
