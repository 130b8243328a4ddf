"""GPU parity: rotation, RTN scales/codes, clipping search, INT4 packing and
the verification error, HIP library vs the CPU oracle.

Bars: codes, packed bytes and fp16 scales bit-exact given the same fp32
input (RTN is integer-valued arithmetic on identical fp32 operands); the
exact rotation kernels bit-exact against the reference's own rotated tensors
(tests/golden/golden_rotation.safetensors); the FWHT kernels within 2e-6
relative to the row norm (they associate the sums differently); fp64 MSE
within 1e-9 relative.
"""

from __future__ import annotations

import pytest
import torch

from oracle import torch_ref as ref
from tests.conftest import lognormal_hessian

pytestmark = pytest.mark.gpu

RATIOS = [0.8, 0.85, 0.9, 0.95, 1.0]


def _w(m, n, seed, std=0.02, outliers=0):
    g = torch.Generator().manual_seed(seed)
    W = torch.randn(m, n, generator=g) * std
    if outliers:
        cols = torch.randperm(n, generator=g)[:outliers]
        W[:, cols] *= 20
    return W


@pytest.fixture(params=["exact", "fwht"])
def rot_kernel(request):
    from int_crush_converter_amd.rotation import set_rotation_kernel
    prev = set_rotation_kernel(request.param)
    yield request.param
    set_rotation_kernel(prev)


@pytest.mark.parametrize("rot", [1, 2, 4, 8, 16, 32, 64, 128, 256, 512, 1024])
@pytest.mark.parametrize("n", [256, 300])
def test_rotate_weights_matches_oracle(gpu_dev, rot_kernel, rot, n):
    from int_crush_converter_amd.rotation import rotate_weights
    W = _w(33, n, rot + n, std=1.0)
    want = ref.rotate_weights(W, rot)
    got = rotate_weights(W.to(gpu_dev), rot).cpu()
    assert got.shape == want.shape and got.dtype == torch.float32
    tol = 2e-6 * W.norm(dim=1, keepdim=True).clamp(min=1)
    assert torch.all((got - want).abs() <= tol), (got - want).abs().max()


def test_rotate_weights_bf16_source(gpu_dev, rot_kernel):
    from int_crush_converter_amd.rotation import rotate_rows_gpu
    W = _w(64, 4096, 3).to(torch.bfloat16)
    want = ref.rotate_weights(W.float(), 256)
    got = rotate_rows_gpu(W.to(gpu_dev), 256).cpu()
    assert torch.allclose(got, want, atol=1e-7, rtol=0)


def test_rotate_weights_deterministic(gpu_dev, rot_kernel):
    from int_crush_converter_amd.rotation import rotate_rows_gpu
    W = _w(128, 1024, 4).to(gpu_dev)
    a = rotate_rows_gpu(W, 256)
    b = rotate_rows_gpu(W, 256)
    assert torch.equal(a, b)


def _rotate_raw(src, dtype_code, rows, cols, ld_src, zero_above=0.0, nz=None):
    from int_crush_converter_amd import _native as nat
    out = torch.empty(rows, cols, dtype=torch.float32, device=src.device)
    nat.check(nat.lib().ic_rotate_rows(src.data_ptr(), dtype_code, rows, cols, ld_src, out.data_ptr(), cols, cols,
                                       256, float(zero_above), nat.ptr(nz), nat.stream()), "ic_rotate_rows")
    return out


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,cols", [(33, 512), (7, 256), (1, 1024), (129, 768)])
def test_rotate256_coalesced_equals_register_kernel(gpu_dev, dtype, rows, cols):
    """The coalesced 256-group kernel (aligned whole-group rows) gives the
    same bits as the per-lane register kernel, which an unaligned source
    (one element in) forces, with outlier zeroing and its count (item counts
    not a multiple of the four per wave)."""
    from int_crush_converter_amd import _native as nat
    g = torch.Generator().manual_seed(rows * cols)
    W = torch.randn(rows, cols + 8, generator=g) * 0.02
    W[0, 5] = 5000.0
    W[-1, cols - 1] = -2000.0
    buf = W.to(dtype).to(gpu_dev)
    code = nat.dtype_code(buf)
    aligned = buf[:, :cols].contiguous()
    nz_a = torch.zeros(1, dtype=torch.int64, device=gpu_dev)
    nz_b = torch.zeros(1, dtype=torch.int64, device=gpu_dev)
    a = _rotate_raw(aligned, code, rows, cols, cols, 1000.0, nz_a)
    # the same rows read one element in (pitch cols + 8): no 16-byte alignment
    shifted = torch.cat([torch.zeros(rows, 1, dtype=dtype), W.to(dtype)[:, :cols + 7]], 1).to(gpu_dev)
    b = torch.empty(rows, cols, dtype=torch.float32, device=gpu_dev)
    nat.check(nat.lib().ic_rotate_rows(shifted.data_ptr() + shifted.element_size(), code, rows, cols, cols + 8,
                                       b.data_ptr(), cols, cols, 256, 1000.0, nz_b.data_ptr(), nat.stream()),
              "ic_rotate_rows")
    assert torch.equal(a, b)
    assert int(nz_a.item()) == int(nz_b.item()) == 2


@pytest.mark.parametrize("rot,n", [(16, 64), (64, 192), (256, 512), (256, 300), (4, 40)])
def test_rotate_hessian_2d(gpu_dev, rot_kernel, rot, n):
    from int_crush_converter_amd.rotation import rotate_hessian
    H = lognormal_hessian(n, 2 * n, 5)
    want = ref.rotate_hessian(H, rot)
    got = rotate_hessian(H.to(gpu_dev), rot).cpu()
    assert got.shape == want.shape
    assert torch.allclose(got, want, atol=2e-6 * want.abs().max().item(), rtol=0)


def test_rotate_hessian_3d(gpu_dev, rot_kernel):
    from int_crush_converter_amd.rotation import rotate_hessian
    H = torch.stack([lognormal_hessian(256, 300, s) for s in range(3)])
    want = ref.rotate_hessian(H, 64)
    got = rotate_hessian(H.to(gpu_dev), 64).cpu()
    assert torch.allclose(got, want, atol=2e-6 * want.abs().max().item(), rtol=0)


# ------------------------------------------- exact rotation vs the reference

def test_exact_rotate_weights_equals_reference(gpu_dev, golden_rotation):
    """ic_rotate_rows_exact gives the reference's rotate_weights bits for
    every rot up to 512 (regular and Sylvester), fp32 and bf16 sources and
    padded groups."""
    from int_crush_converter_amd.rotation import rotate_rows_gpu, set_rotation_kernel
    t, meta = golden_rotation
    prev = set_rotation_kernel("exact")
    try:
        for name, m in meta.items():
            if m["kind"] != "rotate_weights" or "zero_above" in m:
                continue
            got = rotate_rows_gpu(t[f"{name}.W"].to(gpu_dev), m["rot"]).cpu()
            assert torch.equal(got, t[f"{name}.out"]), (name, (got != t[f"{name}.out"]).sum().item())
    finally:
        set_rotation_kernel(prev)


def test_exact_rotate_weights_outlier_zeroing(gpu_dev, golden_rotation):
    """The pipeline's |w| > 1000 zeroing fused into the exact rotation
    (converter/pipeline.py:527-555): the reference's bits and its count."""
    from int_crush_converter_amd.layer import prepare_weights
    from int_crush_converter_amd.rotation import set_rotation_kernel
    t, meta = golden_rotation
    prev = set_rotation_kernel("exact")
    try:
        for dtype in (torch.float32, torch.bfloat16):
            W = t["rwz.W"].to(dtype)
            W_work, nz = prepare_weights(W.to(gpu_dev), 256)
            Wf = W.float()
            want = t["rwz.out"] if dtype == torch.float32 else ref.rotate_weights(Wf.masked_fill(Wf.abs() > 1000.0, 0.0),
                                                                                 256)
            assert torch.equal(W_work.cpu(), want), dtype
            # bf16 rounds 1000.5 to 1000, which is not above the threshold
            assert int(nz.item()) == int((Wf.abs() > 1000.0).sum()), dtype
        assert meta["rwz"]["zeroed"] == 3
    finally:
        set_rotation_kernel(prev)


def test_exact_rotate_hessian_equals_reference(gpu_dev, golden_rotation):
    """ic_rotate_hessian_exact gives the reference's rotate_hessian bits
    (2-D with padding, 3-D whole blocks and sub-blocks)."""
    from int_crush_converter_amd.rotation import rotate_hessian, set_rotation_kernel
    t, meta = golden_rotation
    prev = set_rotation_kernel("exact")
    try:
        for name, m in meta.items():
            if m["kind"] != "rotate_hessian":
                continue
            got = rotate_hessian(t[f"{name}.H"].to(gpu_dev), m["rot"]).cpu()
            assert torch.equal(got, t[f"{name}.out"]), (name, (got != t[f"{name}.out"]).sum().item())
    finally:
        set_rotation_kernel(prev)


def test_exact_rotation_of_golden_gptq_inputs(gpu_dev, golden, golden_rotation):
    """The raw W / H of the rotated GPTQ golden cases rotate on the GPU to
    exactly the tensors the reference quantised."""
    from int_crush_converter_amd.rotation import rotate_hessian_gpu, rotate_rows_gpu, set_rotation_kernel
    g, _ = golden
    t, meta = golden_rotation
    prev = set_rotation_kernel("exact")
    try:
        for name, m in meta.items():
            if m["kind"] != "gptq_raw":
                continue
            case = name[:-len("_raw")]
            assert torch.equal(rotate_rows_gpu(t[f"{name}.W"].to(gpu_dev), m["rot"]).cpu(), g[f"{case}.W"]), name
            assert torch.equal(rotate_hessian_gpu(t[f"{name}.H"].to(gpu_dev), m["rot"]).cpu(), g[f"{case}.H"]), name
    finally:
        set_rotation_kernel(prev)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rot,rows,cols", [(256, 33, 512), (64, 70, 300), (16, 5, 40), (512, 9, 1000)])
def test_exact_rotation_unaligned_source(gpu_dev, dtype, rot, rows, cols):
    """ic_rotate_rows_exact from a source one element in (no vector loads)
    gives the bits of the aligned source, outlier zeroing and count included."""
    from int_crush_converter_amd import _native as nat
    g = torch.Generator().manual_seed(rot + rows)
    W = torch.randn(rows, cols + 8, generator=g) * 0.02
    W[0, 5] = 5000.0
    W[-1, cols - 1] = -2000.0
    code = nat.dtype_code(W.to(dtype))
    cols_pad = -(-cols // rot) * rot

    def run(ptr, ld):
        out = torch.empty(rows, cols_pad, dtype=torch.float32, device=gpu_dev)
        nz = torch.zeros(1, dtype=torch.int64, device=gpu_dev)
        nat.check(nat.lib().ic_rotate_rows_exact(ptr, code, rows, cols, ld, out.data_ptr(), cols_pad, cols_pad, rot,
                                                 1000.0, nz.data_ptr(), nat.stream()), "ic_rotate_rows_exact")
        return out.cpu(), int(nz.item())

    aligned = W[:, :cols].to(dtype).contiguous().to(gpu_dev)
    a, na = run(aligned.data_ptr(), cols)
    shifted = torch.cat([torch.zeros(rows, 1), W[:, :cols + 7]], 1).to(dtype).to(gpu_dev)
    b, nb = run(shifted.data_ptr() + shifted.element_size(), cols + 8)
    assert torch.equal(a, b) and na == nb == 2
    Wz = W[:, :cols].to(dtype).float()
    want = ref.rotate_weights(Wz.masked_fill(Wz.abs() > 1000.0, 0.0), rot)
    assert torch.allclose(a, want, atol=1e-6, rtol=0)


@pytest.mark.parametrize("rot,n", [(256, 768), (64, 320), (16, 128)])
def test_exact_rotate_hessian_lower_blocks(gpu_dev, rot, n):
    """lower_only writes the blocks on and below the block diagonal with the
    full rotation's bits (in place, the rest stays finite: input values or
    partial results)."""
    from int_crush_converter_amd.rotation import rotate_hessian_gpu, set_rotation_kernel
    prev = set_rotation_kernel("exact")
    try:
        H = lognormal_hessian(n, 2 * n, 40 + rot).to(gpu_dev)
        full = rotate_hessian_gpu(H, rot)
        part = rotate_hessian_gpu(H.clone(), rot, lower_only=True, inplace=True)
        blk = torch.arange(n, device=gpu_dev) // rot
        lower = blk[:, None] >= blk[None, :]
        assert torch.equal(part[lower], full[lower])
        assert torch.isfinite(part).all()
        assert torch.equal(full.cpu(), ref.rotate_hessian(H.cpu(), rot))
    finally:
        set_rotation_kernel(prev)


@pytest.mark.parametrize("rot", [2, 8, 32, 128])
def test_rotate_hessian_rejects_non_power_of_four(gpu_dev, rot):
    from int_crush_converter_amd.rotation import rotate_hessian
    with pytest.raises(ValueError, match="power of 4"):
        rotate_hessian(torch.eye(2 * rot, device=gpu_dev), rot)


@pytest.mark.parametrize("bits,asym", [(4, False), (4, True), (8, False), (8, True)])
@pytest.mark.parametrize("ratios", [None, RATIOS])
def test_rtn_bit_exact(gpu_dev, bits, asym, ratios):
    from int_crush_converter_amd import scales as S
    W = ref.rotate_weights(_w(97, 320, bits * 10 + asym, outliers=3), 64)
    W[5] = 0.0                # zero row
    W[6] = W[6] + 3.0         # far from zero: zero-point clamp fix
    W[7] = W[7] - 4.0
    Wg = W.to(gpu_dev)
    s_want, z_want, q_want = None, None, None
    if bits == 4 and not asym:
        s_want = ref.scales_int4_sym(W, W.shape[1], ratios)
        q_want = ref.quant_int4_sym(W, s_want, W.shape[1])
        s_got = S.calculate_scales(Wg, W.shape[1], clipping_ratios=ratios)
        q_got = S.quantize_weights(Wg, s_got, W.shape[1])
    elif bits == 4:
        s_want, z_want = ref.scales_int4_asym(W, W.shape[1], ratios)
        q_want = ref.quant_int4_asym(W, s_want, z_want, W.shape[1])
        s_got, z_got = S.calculate_scales_asymmetric(Wg, W.shape[1], clipping_ratios=ratios)
        q_got = S.quantize_weights_asymmetric(Wg, s_got, z_got, W.shape[1])
    elif not asym:
        s_want = ref.scales_int8_sym(W, ratios)
        q_want = ref.quant_int8_sym(W, s_want)
        s_got = S.calculate_scales_int8(Wg, clipping_ratios=ratios)
        q_got = S.quantize_weights_int8(Wg, s_got)
    else:
        s_want, z_want = ref.scales_int8_asym(W, ratios)
        q_want = ref.quant_int8_asym(W, s_want, z_want)
        s_got, z_got = S.calculate_scales_int8_asymmetric(Wg, clipping_ratios=ratios)
        q_got = S.quantize_weights_int8_asymmetric(Wg, s_got, z_got)
    assert torch.equal(s_got.cpu(), s_want)
    if z_want is not None:
        assert torch.equal(z_got.cpu(), z_want)
    assert torch.equal(q_got.cpu(), q_want)


@pytest.mark.parametrize("rows,cols", [(4096, 4096), (64, 7), (9, 15872), (5, 16000), (33, 1000)])
@pytest.mark.parametrize("bits,asym", [(8, True), (4, False)])
def test_clip_search_bit_exact_widths(gpu_dev, rows, cols, bits, asym):
    """The clip search at C2's shape (INT8 asymmetric, five ratios, 1 % of
    the input columns x 20) and at widths around the LDS-staged limit
    (15872 columns; 16000 takes the fp64-sum kernel): scales and zero-points
    equal the oracle's, whose MSE is the reference's fp32 mean."""
    from int_crush_converter_amd import scales as S
    W = _w(rows, cols, rows + cols + bits, outliers=max(1, cols // 100))
    Wg = W.to(gpu_dev)
    if asym:
        fn_w, fn_g = ((lambda: ref.scales_int8_asym(W, RATIOS)),
                      (lambda: S.calculate_scales_int8_asymmetric(Wg, clipping_ratios=RATIOS)))
    else:
        fn_w, fn_g = ((lambda: (ref.scales_int4_sym(W, cols, RATIOS), None)),
                      (lambda: (S.calculate_scales(Wg, cols, clipping_ratios=RATIOS), None)))
    s_want, z_want = fn_w()
    s_got, z_got = fn_g()
    assert torch.equal(s_got.cpu(), s_want)
    if z_want is not None:
        assert torch.equal(z_got.cpu(), z_want)


@pytest.mark.parametrize("cols", [512, 1031, 2079, 4096, 4127])
@pytest.mark.parametrize("nr", [1, 3, 5, 8])
@pytest.mark.parametrize("bits,asym", [(8, True), (4, False), (4, True), (8, False)])
def test_clip_search_register_rows(gpu_dev, cols, nr, bits, asym):
    """Rows whose 32 inner-sum sequences are whole groups of 16 (512 ..
    4127 columns) take the register-resident clip search with every
    candidate in one pass: 1 to 8 ratios, leftover columns past the
    sequences, a row count that leaves work-group slots empty, a zero row,
    rows far from zero, and rows outside the fast division's domain (huge
    and tiny magnitudes) - scales and zero-points equal the oracle's."""
    from int_crush_converter_amd import scales as S
    ratios = [1.0 - 0.05 * i for i in range(nr)][::-1] if nr > 1 else [0.9]
    W = _w(37, cols, cols + nr + bits, outliers=3)
    W[2] = 0.0
    W[3] = W[3] + 3.0
    W[4] = W[4] - 5.0
    W[5, 7] = 3.0e19          # beyond 2^61: the IEEE division for the whole row
    W[6] = W[6] * 1e-18       # values below 2^-60
    Wg = W.to(gpu_dev)
    if bits == 4 and not asym:
        s_want, z_want = ref.scales_int4_sym(W, cols, ratios), None
        s_got, z_got = S.calculate_scales(Wg, cols, clipping_ratios=ratios), None
    elif bits == 4:
        s_want, z_want = ref.scales_int4_asym(W, cols, ratios)
        s_got, z_got = S.calculate_scales_asymmetric(Wg, cols, clipping_ratios=ratios)
    elif not asym:
        s_want, z_want = ref.scales_int8_sym(W, ratios), None
        s_got, z_got = S.calculate_scales_int8(Wg, clipping_ratios=ratios), None
    else:
        s_want, z_want = ref.scales_int8_asym(W, ratios)
        s_got, z_got = S.calculate_scales_int8_asymmetric(Wg, clipping_ratios=ratios)
    assert torch.equal(s_got.cpu(), s_want)
    if z_want is not None:
        assert torch.equal(z_got.cpu(), z_want)


def test_rtn_group_wise(gpu_dev):
    from int_crush_converter_amd import scales as S
    W = _w(16, 200, 9, std=1.0)
    for gs in (32, 64, 128):
        s_want = ref.scales_int4_sym(W, gs, RATIOS)
        got = S.calculate_scales(W.to(gpu_dev), group_size=gs, clipping_ratios=RATIOS).cpu()
        assert torch.equal(got, s_want)
        assert torch.equal(S.quantize_weights(W.to(gpu_dev), got.to(gpu_dev), gs).cpu(),
                           ref.quant_int4_sym(W, s_want, gs))


def test_clip_golden_gpu(gpu_dev, golden):
    from int_crush_converter_amd import scales as S
    t, _ = golden
    W = t["clip.W"].to(gpu_dev)
    assert torch.equal(S.calculate_scales(W, W.shape[1], clipping_ratios=RATIOS).cpu(), t["clip.s4"])
    s, z = S.calculate_scales_asymmetric(W, W.shape[1], clipping_ratios=RATIOS)
    assert torch.equal(s.cpu(), t["clip.s4a"]) and torch.equal(z.cpu(), t["clip.z4a"])
    assert torch.equal(S.calculate_scales_int8(W, clipping_ratios=RATIOS).cpu(), t["clip.s8"])
    s, z = S.calculate_scales_int8_asymmetric(W, clipping_ratios=RATIOS)
    assert torch.equal(s.cpu(), t["clip.s8a"]) and torch.equal(z.cpu(), t["clip.z8a"])


def test_rtn_extreme_values(gpu_dev):
    """fp16 scale clamp limits (reference tests/test_scales.py:369-496)."""
    from int_crush_converter_amd import scales as S
    W = torch.cat([torch.full((2, 64), 1e8), torch.full((2, 64), 1e-9), torch.zeros(2, 64)])
    for fn in (S.calculate_scales, S.calculate_scales_int8):
        s = fn(W.to(gpu_dev)).cpu()
        assert s.dtype == torch.float16 and torch.isfinite(s).all() and (s > 0).all()
    assert torch.equal(S.calculate_scales(W.to(gpu_dev)).cpu(), ref.scales_int4_sym(W, 128))


@pytest.mark.parametrize("shape", [(7,), (4, 33), (3, 5, 16), (1, 1), (64, 256), (33, 12288), (2, 3, 64)])
def test_pack_unpack_bit_exact(gpu_dev, shape):
    from int_crush_converter_amd.packing import pack_int4, unpack_int4
    g = torch.Generator().manual_seed(1)
    v = torch.randint(-8, 8, shape, generator=g, dtype=torch.int8)
    p = pack_int4(v.to(gpu_dev)).cpu()
    assert torch.equal(p, ref.pack_int4(v))
    assert torch.equal(unpack_int4(p.to(gpu_dev), shape[-1]).cpu(), v)


def test_pack_validation(gpu_dev):
    from int_crush_converter_amd.packing import pack_int4, validate_int4_range, INT4PackingError
    with pytest.raises(INT4PackingError):
        validate_int4_range(torch.tensor([8], dtype=torch.int8, device=gpu_dev))
    with pytest.raises(INT4PackingError):
        validate_int4_range(torch.tensor([-9], dtype=torch.int8, device=gpu_dev))
    with pytest.raises(INT4PackingError):
        pack_int4(torch.tensor([1.0, float("nan")], device=gpu_dev))
    validate_int4_range(torch.tensor([-8, -1, 0, 7], device=gpu_dev))
    # float input is truncated like .to(torch.int8)
    f = torch.tensor([-7.5, 3.7, 0.2, -0.9], device=gpu_dev)
    assert torch.equal(pack_int4(f).cpu(), ref.pack_int4(f.cpu().to(torch.int8)))


@pytest.mark.parametrize("bad,err", [(8, "above"), (-9, "below"), (127, "above"), (-128, "below")])
def test_pack_validation_vector_path(gpu_dev, bad, err):
    """Whole 32-code rows take the vectorised packer; its range flags must
    match the scalar rules for every position of a bad code."""
    from int_crush_converter_amd.packing import pack_int4, INT4PackingError
    g = torch.Generator().manual_seed(2)
    v = torch.randint(-8, 8, (16, 64), generator=g, dtype=torch.int8)
    for pos in [(0, 0), (5, 31), (15, 63), (7, 33)]:
        w = v.clone()
        w[pos] = bad
        with pytest.raises(INT4PackingError):
            pack_int4(w.to(gpu_dev))
    assert torch.equal(pack_int4(v.to(gpu_dev)).cpu(), ref.pack_int4(v))


@pytest.mark.parametrize("M,N", [(64, 512), (37, 201)])
def test_quant_error_matches_oracle(gpu_dev, M, N):
    """16-byte row path (N % 4 == 0) and the element path (ragged N)."""
    from int_crush_converter_amd import _native as nat
    W = _w(M, N, 2)
    s, z = ref.scales_int4_asym(W, W.shape[1])
    q = ref.quant_int4_asym(W, s, z, W.shape[1])
    d = (q.float() - z.float()) * s.float()
    want_mse = (W - d).double().pow(2).mean().item()
    want_max = (W - d).abs().max().item()
    Wg, qg, sg, zg = (x.to(gpu_dev).contiguous() for x in (W, q, s, z))
    out_s = torch.zeros(1, dtype=torch.float64, device=gpu_dev)
    out_m = torch.zeros(1, dtype=torch.float32, device=gpu_dev)
    ws = torch.empty(nat.lib().ic_quant_error_workspace_bytes(), dtype=torch.uint8, device=gpu_dev)
    nat.check(nat.lib().ic_quant_error(Wg.data_ptr(), M, N, N, qg.data_ptr(), N, sg.data_ptr(), 0,
                                       zg.data_ptr(), out_s.data_ptr(), out_m.data_ptr(), ws.data_ptr(),
                                       nat.stream()), "ic_quant_error")
    assert out_s.item() / W.numel() == pytest.approx(want_mse, rel=1e-9)
    assert out_m.item() == want_max
