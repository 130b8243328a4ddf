"""Host-side logic on the CPU (no GPU calls): validation and error
conventions, the metadata contract, calibration parsing, skip rules and the
CLI flag surface."""

from __future__ import annotations

import pytest
import torch

from int_crush_converter_amd import calibration_io as cio
from int_crush_converter_amd.config import DEFAULT_SKIP_PATTERNS
from int_crush_converter_amd.pipeline import _metadata, _validate, should_skip
from int_crush_converter_amd.types import QuantizeConfig


def cfg(**kw):
    return QuantizeConfig(input_path="x", output_dir="y", **kw)


def test_config_defaults_match_reference():
    c = cfg()
    assert (c.rot_size, c.int_bits, c.quant_method, c.gptq_block_size, c.damping, c.hessian_method) == \
        (256, 4, "rtn", 128, 0.01, "hinv")
    assert (c.ldlq_iterations, c.greedy_passes, c.rank_threshold, c.seed) == (1, 0, 0.01, 42)


@pytest.mark.parametrize("kw,msg", [
    (dict(quant_method="awq"), "quant_method must be"),
    (dict(quant_method="gptq"), "GPTQ requires --calibration"),
    (dict(rot_size=12), "rot_size must be 0"),
    (dict(perm_group_size=16), "perm_group_size must be"),
    (dict(quant_group_size=100), "quant_group_size must be"),
    (dict(int_bits=3), "int_bits must be 4 or 8"),
    (dict(svd_rank=-1), "svd_rank must be"),
    (dict(smoothrot=True, rot_size=0, int_bits=8), "SmoothRot requires rot_size"),
])
def test_validation_errors(kw, msg):
    with pytest.raises(ValueError, match=msg):
        _validate(cfg(**kw))


@pytest.mark.parametrize("kw", [dict(smoothquant=True, int_bits=8), dict(svd_rank=16)])
def test_unsupported_features_raise(kw):
    with pytest.raises(NotImplementedError):
        _validate(cfg(**kw))


def test_permuquant_config_accepted_and_in_metadata():
    from int_crush_converter_amd.pipeline import _metadata
    c = _validate(cfg(use_permuquant=True, tau=0.05, quant_method="rtn"))
    md = _metadata(c, {}, [])
    assert md["int_crush.method"] == "int_crush_permuq"
    assert md["int_crush.permuquant"] == "true" and md["int_crush.permuquant_tau"] == "0.05"


def test_should_skip_default_patterns():
    assert should_skip("model.embed_tokens.weight", DEFAULT_SKIP_PATTERNS)
    assert should_skip("blocks.3.NORM1.weight", DEFAULT_SKIP_PATTERNS)
    assert should_skip("final.proj_out.weight", DEFAULT_SKIP_PATTERNS)
    assert not should_skip("blocks.3.attn.qkv.weight", DEFAULT_SKIP_PATTERNS)


def _sd():   # name -> shape
    return {"blocks.0.attn.qkv.weight": (4, 300), "blocks.0.norm.weight": (300,), "blocks.0.mlp.up.weight": (4, 512)}


def test_metadata_configs():
    """The output contract of the five benchmark configurations."""
    sd = {"a.weight": (2, 256)}   # name -> shape
    assert _metadata(cfg(rot_size=256, int_bits=4), sd, DEFAULT_SKIP_PATTERNS) == {
        "int_crush.format_version": "3", "int_crush.method": "int_crush", "int_crush.rot_size": "256",
        "int_crush.scale_type": "per_row", "int_crush.hadamard_type": "regular", "int_crush.packing_order": "little"}
    assert _metadata(cfg(rot_size=64, int_bits=8, asymmetric=True, clipping_ratios=[0.9]), sd,
                     DEFAULT_SKIP_PATTERNS) == {
        "int_crush.format_version": "1", "int_crush.method": "int_crush", "int_crush.rot_size": "64",
        "int_crush.scale_type": "per_row_asymmetric", "int_crush.hadamard_type": "regular",
        "int_crush.packing_order": "native"}
    assert _metadata(cfg(rot_size=256, quant_method="gptq", calibration_path="c"), sd, DEFAULT_SKIP_PATTERNS) == {
        "int_crush.format_version": "3", "int_crush.method": "int_crush_gptq", "int_crush.rot_size": "256",
        "int_crush.scale_type": "per_row_asymmetric", "int_crush.hadamard_type": "regular",
        "int_crush.packing_order": "little", "int_crush.gptq_block_size": "128", "int_crush.damping_ratio": "0.01"}
    assert _metadata(cfg(rot_size=256, quant_method="ldlq", ldlq_iterations=2, greedy_passes=5), sd,
                     DEFAULT_SKIP_PATTERNS) == {
        "int_crush.format_version": "3", "int_crush.method": "int_crush_ldlq", "int_crush.rot_size": "256",
        "int_crush.scale_type": "per_row", "int_crush.hadamard_type": "regular", "int_crush.packing_order": "little",
        "int_crush.ldlq_block_size": "128", "int_crush.damping_ratio": "0.01", "int_crush.ldlq_iterations": "2",
        "int_crush.greedy_passes": "5", "int_crush.rank_threshold": "0.01"}


def test_metadata_padded_and_excluded():
    md = _metadata(cfg(rot_size=256, exclude_patterns=["mlp"]), _sd(), DEFAULT_SKIP_PATTERNS + ["mlp"])
    assert md["int_crush.padded_layers"] == "blocks.0.attn.qkv.weight=300"
    assert md["int_crush.exclude_patterns"] == "mlp"


def test_calibration_formats(tmp_path):
    full = torch.eye(6)
    blocks = torch.stack([torch.eye(4), torch.eye(4)])
    lst = [torch.eye(4), torch.eye(2)]
    bad = torch.eye(6)
    bad[0, 0] = float("nan")
    cal = {"hessians": {"a": full, "b": blocks, "c": lst, "d": bad, "e": torch.eye(5)},
           "shapes": {}, "layer_types": {}}
    assert torch.equal(cio.get_hessian(cal, "a", (3, 6)), full)
    assert cio.get_hessian(cal, "b", (3, 8)).shape == (2, 4, 4)
    assert cio.get_hessian(cal, "b", (3, 9)) is None             # wrong block count
    h = cio.get_hessian(cal, "c", (3, 6))
    assert h.shape == (2, 4, 4) and h[1, 2:, 2:].abs().sum() == 0
    assert cio.get_hessian(cal, "d", (3, 6)) is None             # non-finite
    assert cio.get_hessian(cal, "e", (3, 6)) is None             # shape mismatch
    assert cio.get_hessian(cal, "zz", (3, 6)) is None
    path = tmp_path / "c.pt"
    torch.save(cal, path)
    assert set(cio.load_calibration(str(path))["hessians"]) == set(cal["hessians"])
    torch.save({"hessians": {}}, tmp_path / "bad.pt")
    with pytest.raises(KeyError):
        cio.load_calibration(str(tmp_path / "bad.pt"))
    with pytest.raises(ValueError):
        cio.load_calibration(str(tmp_path / "missing.pt"))


def test_build_name_map():
    m = cio.build_name_map(["a.b.weight", "a.c.weight", "a.b.bias", "x"], ["a.b", "q"])
    assert m == {"a.b.weight": "a.b"}


def test_cli_flags_parse():
    from int_crush_converter_amd.cli import build_parser
    a = build_parser().parse_args(["-i", "in", "-o", "out", "--rot-size", "256", "--quant-method", "gptq", "-c",
                                   "cal.pt", "--gptq-block-size", "64", "--damping", "0.02", "--hessian-method",
                                   "cholesky", "--ldlq-iterations", "2", "--greedy-passes", "5",
                                   "--clipping-ratios", "0.9,1.0", "--int-bits", "8", "--asymmetric"])
    assert (a.rot_size, a.quant_method, a.calibration, a.gptq_block_size, a.damping, a.hessian_method) == \
        (256, "gptq", "cal.pt", 64, 0.02, "cholesky")
    assert (a.ldlq_iterations, a.greedy_passes, a.clipping_ratios, a.int_bits, a.asymmetric) == \
        (2, 5, "0.9,1.0", 8, True)


def test_cli_rejects_bad_rot(capsys):
    from int_crush_converter_amd.cli import main
    with pytest.raises(SystemExit):
        main(["-i", "a", "-o", "b", "--rot-size", "12", "-q"])


def test_dlr_detection_and_validation():
    from int_crush_converter_amd import dlr
    d = dlr.make_dlr_dict(torch.rand(8) + 0.1, torch.randn(8, 4))
    assert d["rank"] == 4 and d["n"] == 8 and dlr.is_dlr(d)
    assert not dlr.is_dlr(torch.eye(3)) and not dlr.is_dlr({"D": d["D"], "U": d["U"]})
    assert not dlr.is_dlr({"format": "block", "D": d["D"], "U": d["U"]})
    assert dlr.validate_dlr(d, in_features=8) and not dlr.validate_dlr(d, in_features=16)
    bad = dict(d, D=d["D"].clone())
    bad["D"][0] = -1.0
    assert not dlr.validate_dlr(bad)
    bad["D"][0] = float("nan")
    assert not dlr.validate_dlr(bad)
    assert not dlr.validate_dlr(dlr.make_dlr_dict(torch.rand(8), torch.randn(16, 4)))
    assert not dlr.validate_dlr({"format": "dlr", "D": [1, 2, 3], "U": torch.randn(3, 2)})


def test_dlr_factor_transforms():
    from int_crush_converter_amd import dlr
    g = torch.Generator().manual_seed(3)
    D, U, s = torch.rand(16, generator=g) + 0.1, torch.randn(16, 4, generator=g) * 0.3, torch.rand(16, generator=g) + .5
    Dn, Un = dlr.transform_dlr_for_smoothquant(D, U, s)
    H = torch.diag(D) + U @ U.T
    assert torch.allclose(torch.diag(Dn) + Un @ Un.T, H / (s[:, None] * s[None, :]), atol=1e-5)
    s0 = s.clone()
    s0[0] = 0.0
    assert all(torch.isfinite(t).all() for t in dlr.transform_dlr_for_smoothquant(D, U, s0))
    perm = torch.randperm(16, generator=g)
    Dp, Up = dlr.permute_dlr(D, U, perm)
    assert torch.equal(Dp, D[perm]) and torch.equal(Up, U[perm])
    Dp, Up = dlr.permute_dlr(D, U, perm[:8])
    assert Dp.shape == (8,) and Up.shape == (8, 4)
    assert abs(dlr.damped_diag_mean(D, U).item() - H.diagonal().mean().item()) <= 1e-5 * H.diagonal().mean().item()
    assert dlr.damped_diag_mean(torch.zeros(8), torch.zeros(8, 4)).item() == pytest.approx(1e-6)


def test_calibration_dlr(tmp_path):
    from int_crush_converter_amd import dlr
    g = torch.Generator().manual_seed(5)
    D, U = torch.rand(64, generator=g) + 0.1, torch.randn(64, 8, generator=g)
    cal = {"hessians": {"layer.0": dlr.make_dlr_dict(D, U), "full": torch.eye(64)},
           "shapes": {}, "layer_types": {}}
    h = cio.get_hessian(cal, "layer.0", (32, 64))
    assert dlr.is_dlr(h) and h["D"].shape == (64,) and h["U"].shape == (64, 8)
    assert cio.get_hessian(cal, "layer.0", (32, 128)) is None
    neg = dict(cal["hessians"]["layer.0"], D=D.clone())
    neg["D"][3] = -0.5
    assert cio.get_hessian({"hessians": {"x": neg}}, "x", (32, 64)) is None
    diag = cio.get_hessian_diag(cal, "layer.0", 64)
    assert torch.allclose(diag, D + (U ** 2).sum(dim=1), atol=1e-5)
    assert cio.get_hessian_diag(cal, "layer.0", 32).shape == (32,)
    assert cio.get_hessian_diag(cal, "missing", 64) is None
    assert torch.equal(cio.get_hessian_diag(cal, "full", 64), torch.ones(64))
    assert cio.get_hessian_diag(cal, "full", 65) is None
    cal["hessian_diag"] = {"full": torch.arange(10.0)}
    assert torch.equal(cio.get_hessian_diag(cal, "full", 64), torch.arange(10.0))
    path = tmp_path / "dlr.pt"
    torch.save(cal, path)
    h = cio.get_hessian(cio.load_calibration(str(path)), "layer.0", (32, 64))
    assert torch.equal(h["D"], D) and torch.equal(h["U"], U)


def test_piso_config_accepted():
    c = _validate(cfg(piso_scales=True, quant_method="gptq", calibration_path="c"))
    assert c.piso_scales


def test_piso_api_validation():
    from int_crush_converter_amd import piso
    with pytest.raises(ValueError, match="2D"):
        piso.compute_piso_scales_int8(torch.randn(8), torch.ones(64))
    with pytest.raises(ValueError, match="in_features"):
        piso.compute_piso_scales_int8(torch.randn(8, 64), torch.ones(32))
    with pytest.raises(ValueError, match="num_coarse"):
        piso.compute_piso_scales_int4(torch.randn(8, 64), torch.ones(64), num_coarse=0)


@pytest.mark.parametrize("code", [0, 2])
def test_fallback_output_hinv_returns_inverse(code):
    """Method "hinv" (full or upper-triangle reads) hands the inv / pinv
    result itself to the column loop (converter/gptq.py:113-121), even when
    that inverse is positive definite."""
    from int_crush_converter_amd.hessian import fallback_output
    g = torch.Generator().manual_seed(3)
    A = torch.randn(12, 12, generator=g)
    Hi = A @ A.T + 12 * torch.eye(12)
    got = fallback_output(code, Hi, lambda: pytest.fail("no second inverse for method hinv"))
    assert got is Hi


def test_fallback_output_cholesky_method():
    """Method "cholesky" (converter/gptq.py:91-110): the upper Cholesky factor
    of the fallback inverse; the inverse itself when it does not factor; H^-1
    when only the factorisation of H^-1 failed."""
    from int_crush_converter_amd.hessian import fallback_output
    g = torch.Generator().manual_seed(4)
    A = torch.randn(10, 10, generator=g)
    Hi = A @ A.T + 10 * torch.eye(10)
    U = fallback_output(1, Hi, lambda: pytest.fail("unused"))
    assert torch.allclose(U.T @ U, Hi, rtol=1e-5, atol=1e-4)
    assert torch.equal(U, torch.triu(U))
    indef = torch.diag(torch.tensor([1.0, -2.0, 3.0]))
    assert fallback_output(1, indef, lambda: pytest.fail("unused")) is indef
    marker = torch.ones(3, 3)
    assert fallback_output(1, None, lambda: marker) is marker
    with pytest.raises(ValueError):
        fallback_output(2, None, lambda: marker)


@pytest.mark.parametrize("N,nblk,bs,want", [
    (1024, 4, 256, (4, 0)),      # exact cover
    (1024, 2, 256, (2, 0)),      # fewer blocks than columns need: the rest stays unswept
    (1000, 4, 256, (3, 232)),    # partial last block
    (1000, 3, 256, (3, 0)),      # partial tail not covered by any block
    (512, 6, 256, (2, 0)),       # blocks past the last column do nothing
    (100, 1, 256, (0, 100)),     # one block wider than the layer
])
def test_block_cover(N, nblk, bs, want):
    from int_crush_converter_amd.gptq import block_cover
    assert block_cover(N, nblk, bs) == want
