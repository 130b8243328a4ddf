"""GPU parity of the GPTQ path: fp32-MFMA GEMM, damped Hessian inverse,
column sweep and the full layer, against the CPU oracle and the reference's
golden vectors.

Bars (see the module docstrings of oracle/torch_ref.py):
  * GEMM: within 2e-6 relative (fp32 accumulation, different order).
  * Hessian inverse: error vs the fp64 inverse at most 4x the reference's own
    fp32 error (same algorithm family, different rounding order).
  * Sweep of one block given the same Hinv: codes bit-exact.
  * Whole layer: scales / zero-points bit-exact; codes agree on >= 99.9 %
    at these sizes; tr(dW H dW^T) within the 1e-2 fp32 noise band of these
    small cases (the 1e-3 bar is asserted at N = 2048, where it is above
    the noise).  (At N >= 6144 the
    reference disagrees with itself by ~0.7 % between MKL thread counts; the
    large-size bars live in tests/test_gpu_gptq_large.py.)
"""

from __future__ import annotations

import pytest
import torch

from oracle import torch_ref as ref
from tests.conftest import lognormal_hessian

pytestmark = pytest.mark.gpu


def _sgemm(A, B, C, transA=0, transB=0, alpha=1.0, beta=0.0, cmask=0, krange=0):
    from int_crush_converter_amd import _native as nat
    M = A.shape[1] if transA else A.shape[0]
    K = A.shape[0] if transA else A.shape[1]
    N = B.shape[0] if transB else B.shape[1]
    nat.check(nat.lib().ic_sgemm(transA, transB, M, N, K, alpha, A.data_ptr(), A.shape[1], B.data_ptr(),
                                 B.shape[1], beta, C.data_ptr(), C.shape[1], cmask, krange, nat.stream()),
              "ic_sgemm")
    return C


@pytest.mark.parametrize("M,N,K", [(128, 128, 16), (200, 72, 33), (1, 5, 300), (513, 257, 129), (64, 1000, 128)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_sgemm_matches_fp64(gpu_dev, M, N, K, ta, tb):
    g = torch.Generator().manual_seed(M * 7 + N + K)
    A = torch.randn(K, M, generator=g) if ta else torch.randn(M, K, generator=g)
    B = torch.randn(N, K, generator=g) if tb else torch.randn(K, N, generator=g)
    C0 = torch.randn(M, N, generator=g)
    want = 0.5 * ((A.T if ta else A).double() @ (B.T if tb else B).double()) - 2.0 * C0.double()
    got = _sgemm(A.to(gpu_dev), B.to(gpu_dev), C0.clone().to(gpu_dev), ta, tb, 0.5, -2.0).cpu()
    scale = ((A.T if ta else A).abs().double() @ (B.T if tb else B).abs().double()).max().item() + 1
    assert (got.double() - want).abs().max().item() <= 2e-6 * scale * max(1, K ** 0.5)


@pytest.mark.parametrize("M,N,K", [(2304, 2304, 64), (2100, 2200, 70)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_sgemm_large_tiles_match_fp64(gpu_dev, M, N, K, ta, tb):
    # >= 256 tiles of 128: the 128-tile kernel (the cases above take the 64-tile one)
    g = torch.Generator().manual_seed(M + N * 3 + K + 10 * ta + tb)
    A = torch.randn(K, M, generator=g) if ta else torch.randn(M, K, generator=g)
    B = torch.randn(N, K, generator=g) if tb else torch.randn(K, N, generator=g)
    C0 = torch.randn(M, N, generator=g)
    want = 0.5 * ((A.T if ta else A).double() @ (B.T if tb else B).double()) - 2.0 * C0.double()
    got = _sgemm(A.to(gpu_dev), B.to(gpu_dev), C0.clone().to(gpu_dev), ta, tb, 0.5, -2.0).cpu()
    scale = ((A.T if ta else A).abs().double() @ (B.T if tb else B).abs().double()).max().item() + 1
    assert (got.double() - want).abs().max().item() <= 2e-6 * scale * max(1, K ** 0.5)


@pytest.mark.parametrize("n", [300, 2900])
def test_sgemm_masks_both_tiles(gpu_dev, n):
    # n = 2900: 276 upper tiles of 128; with K from max(i0, j0) the (0, 0)
    # tile's full K bounds the launch and it runs 64-tiles, with the whole K
    # range the 128-tile kernel.  n = 300: 64-tile kernel.  The two results
    # are the same sums in the same order.
    g = torch.Generator().manual_seed(n)
    X = torch.tril(torch.randn(n, n, generator=g)) / n ** 0.5
    want = X.double().T @ X.double()
    iu = torch.triu_indices(n, n)
    il = torch.tril_indices(n, n, -1)
    outs = []
    for krange in (1, 0):
        C = torch.full((n, n), float("nan"))
        got = _sgemm(X.to(gpu_dev), X.to(gpu_dev), C.to(gpu_dev), 1, 0, 1.0, 0.0, cmask=2, krange=krange).cpu()
        assert torch.allclose(got[iu[0], iu[1]].double(), want[iu[0], iu[1]], atol=3e-5)
        assert torch.isnan(got[il[0], il[1]]).all()
        outs.append(got[iu[0], iu[1]])
    assert torch.equal(outs[0], outs[1])
    A = torch.randn(n, 160, generator=g)
    C = torch.randn(n, n, generator=g)
    got = _sgemm(A.to(gpu_dev), A.to(gpu_dev), C.clone().to(gpu_dev), 0, 1, -1.0, 1.0, cmask=1).cpu()
    want = C.double() - A.double() @ A.double().T
    il = torch.tril_indices(n, n)
    assert torch.allclose(got[il[0], il[1]].double(), want[il[0], il[1]], atol=1e-4)
    iu = torch.triu_indices(n, n, 1)
    assert torch.equal(got[iu[0], iu[1]], C[iu[0], iu[1]])


@pytest.mark.parametrize("M,N", [(300, 200), (1000, 2900), (257, 4096)])
def test_gram_tn_is_the_full_product(gpu_dev, M, N):
    """ic_gram_tn (one triangle, mirrored) equals ic_sgemm's full W^T W bit
    for bit, and the fp64 product to fp32 accuracy."""
    from int_crush_converter_amd import _native as nat
    g = torch.Generator().manual_seed(M + N)
    W = (torch.randn(M, N, generator=g) * torch.exp(torch.randn(1, N, generator=g))).to(gpu_dev)
    full = _sgemm(W, W, torch.empty(N, N, device=gpu_dev), 1, 0, 1.0 / M, 0.0)
    C = torch.full((N, N), float("nan"), device=gpu_dev)
    nat.check(nat.lib().ic_gram_tn(W.data_ptr(), M, N, N, 1.0 / M, C.data_ptr(), nat.stream()), "ic_gram_tn")
    assert torch.equal(C, full)
    want = W.double().T @ W.double() / M
    scale = (W.abs().double().T @ W.abs().double() / M).max().item()
    assert (C.double() - want).abs().max().item() <= 2e-6 * scale * max(1, M ** 0.5)


def test_sgemm_masks(gpu_dev):
    g = torch.Generator().manual_seed(1)
    n = 300
    X = torch.tril(torch.randn(n, n, generator=g))
    # upper tiles of X^T X with k >= max(i0, j0)
    C = torch.full((n, n), float("nan"))
    got = _sgemm(X.to(gpu_dev), X.to(gpu_dev), C.to(gpu_dev), 1, 0, 1.0, 0.0, cmask=2, krange=1).cpu()
    want = (X.double().T @ X.double())
    iu = torch.triu_indices(n, n)
    assert torch.allclose(got[iu[0], iu[1]].double(), want[iu[0], iu[1]], atol=1e-4)
    il = torch.tril_indices(n, n, -1)
    assert torch.isnan(got[il[0], il[1]]).all()          # lower part never written
    # lower SYRK update
    A = torch.randn(n, 128, generator=g)
    C = torch.randn(n, n, generator=g)
    got = _sgemm(A.to(gpu_dev), A.to(gpu_dev), C.clone().to(gpu_dev), 0, 1, -1.0, 1.0, cmask=1).cpu()
    want = C.double() - A.double() @ A.double().T
    il = torch.tril_indices(n, n)
    assert torch.allclose(got[il[0], il[1]].double(), want[il[0], il[1]], atol=1e-4)
    iu = torch.triu_indices(n, n, 1)
    assert torch.equal(got[iu[0], iu[1]], C[iu[0], iu[1]])


@pytest.mark.parametrize("n,samples", [(64, 200), (200, 150), (256, 512), (1024, 700), (2048, 1536)])
def test_hessian_inverse_accuracy(gpu_dev, n, samples):
    from int_crush_converter_amd.hessian import inverse_batch
    H = lognormal_hessian(n, samples, n)
    Hd = ref.damp(H, 0.01)
    truth = torch.cholesky_inverse(torch.linalg.cholesky(Hd.double()))
    ref32 = ref.prepare_hinv(H, 0.01)
    got = inverse_batch(H.to(gpu_dev), 0.01, "hinv").cpu()
    e_ref = ((ref32.double() - truth).norm() / truth.norm()).item()
    e_got = ((got.double() - truth).norm() / truth.norm()).item()
    assert torch.equal(got, got.T)
    assert e_got <= 4 * e_ref + 1e-6, (e_got, e_ref)


def test_hessian_inverse_batched_3d(gpu_dev):
    from int_crush_converter_amd.hessian import inverse_batch
    H3 = torch.stack([lognormal_hessian(256, 300, s) for s in range(5)])
    got = inverse_batch(H3.to(gpu_dev), 0.01, "hinv").cpu()
    for b in range(5):
        want = ref.prepare_hinv(H3[b], 0.01)
        assert torch.allclose(got[b], want, rtol=1e-3, atol=1e-3 * want.abs().max().item())


@pytest.mark.parametrize("n", [1100, 2300])
def test_hessian_inverse_batch_equals_single(gpu_dev, n):
    """Every matrix of a 3-D batch is factored and inverted exactly as it is
    alone (the diagonal-block launches also run the batch's update tiles,
    indexed by matrix), across super-blocks and a partial last block, and
    the inverse stays as accurate as the reference's own fp32 path."""
    from int_crush_converter_amd.hessian import inverse_batch
    Hs = torch.stack([lognormal_hessian(n, n + 200, 40 + s) for s in range(3)])
    for method in ("hinv", "cholesky"):
        got = inverse_batch(Hs.to(gpu_dev), 0.01, method).cpu()
        for b in range(3):
            one = inverse_batch(Hs[b].to(gpu_dev), 0.01, method).cpu()
            assert torch.equal(got[b], one), (method, b)
        if method == "hinv":
            Hd = ref.damp(Hs[2], 0.01)
            truth = torch.cholesky_inverse(torch.linalg.cholesky(Hd.double()))
            e_ref = ((ref.prepare_hinv(Hs[2], 0.01).double() - truth).norm() / truth.norm()).item()
            e_got = ((got[2].double() - truth).norm() / truth.norm()).item()
            assert e_got <= 4 * e_ref + 1e-6, (e_got, e_ref)


def test_hessian_cholesky_method(gpu_dev):
    from int_crush_converter_amd.hessian import inverse_batch
    H = lognormal_hessian(300, 400, 3)
    want = ref.prepare_chol(H, 0.01)
    got = inverse_batch(H.to(gpu_dev), 0.01, "cholesky").cpu()
    assert torch.equal(torch.tril(got, -1), torch.zeros_like(got))
    assert torch.allclose(got, want, atol=2e-3 * want.abs().max().item())


@pytest.mark.parametrize("n", [200, 1024])
def test_hessian_inverse_upper_only_in_place(gpu_dev, n):
    # method 2 / inplace: the same upper triangle, bit for bit, as the full
    # out-of-place inverse; the lower part finite; the input consumed
    from int_crush_converter_amd.hessian import inverse_batch
    H = lognormal_hessian(n, n + 100, 7).to(gpu_dev)
    full = inverse_batch(H, 0.01, "hinv")
    work = H.clone()
    calls = []
    got = inverse_batch(work, 0.01, "hinv", inplace=True, restore=lambda: calls.append(1) or H.clone(),
                        upper_only=True)
    assert got.data_ptr() == work.data_ptr() and not calls
    iu = torch.triu_indices(n, n, device=gpu_dev)
    assert torch.equal(got[iu[0], iu[1]], full[iu[0], iu[1]])
    assert torch.isfinite(got).all()


def test_hessian_in_place_fallback_uses_restore(gpu_dev):
    from int_crush_converter_amd.hessian import inverse_batch
    H = torch.zeros(8, 8)
    H[0, 0] = -1.0
    work = H.to(gpu_dev)
    fb = []
    got = inverse_batch(work, 0.01, "hinv", fb, inplace=True, restore=lambda: H.to(gpu_dev)).cpu()
    assert fb == ["hessian_inv_fallback"]
    assert torch.allclose(got, torch.linalg.inv(ref.damp(H, 0.01)), atol=1e-5)


@pytest.mark.parametrize("kernel", ["exact", "fwht"])
def test_rotate_hessian_out_of_place(gpu_dev, kernel):
    from int_crush_converter_amd.rotation import rotate_hessian_gpu, set_rotation_kernel
    H = lognormal_hessian(512, 600, 5).to(gpu_dev)
    H0 = H.clone()
    prev = set_rotation_kernel(kernel)
    try:
        got = rotate_hessian_gpu(H, 256)
    finally:
        set_rotation_kernel(prev)
    assert torch.equal(H, H0) and got.data_ptr() != H.data_ptr()
    want = ref.rotate_hessian(H0.cpu(), 256)
    assert torch.allclose(got.cpu(), want, atol=2e-6 * want.abs().max().item(), rtol=0)
    # src == dst through the C ABI (what the padded path does): the same bits
    from int_crush_converter_amd import _native as nat
    inplace = H0.clone()
    if kernel == "exact":
        nat.check(nat.lib().ic_rotate_hessian_exact(inplace.data_ptr(), inplace.data_ptr(), 1, 512, 512, 256, 0,
                                                    nat.stream()), "ic_rotate_hessian_exact")
    else:
        nat.check(nat.lib().ic_rotate_hessian(inplace.data_ptr(), inplace.data_ptr(), 1, 512, 512, 256,
                                              nat.stream()), "ic_rotate_hessian")
    assert torch.equal(inplace, got)


def test_hessian_singular_falls_back(gpu_dev):
    from int_crush_converter_amd.hessian import inverse_batch
    H = torch.zeros(8, 8)
    H[0, 0] = -1.0             # damped matrix is not positive definite
    fb = []
    got = inverse_batch(H.to(gpu_dev), 0.01, "hinv", fb).cpu()
    assert fb == ["hessian_inv_fallback"]
    want = torch.linalg.inv(ref.damp(H, 0.01))
    assert torch.allclose(got, want, atol=1e-5)


@pytest.mark.parametrize("bits,asym,B,N", [(4, False, 32, 32), (4, False, 128, 128), (8, False, 64, 64),
                                          (8, True, 100, 100), (4, False, 128, 96)])
def test_sweep_single_block_bit_exact(gpu_dev, bits, asym, B, N):
    from int_crush_converter_amd.gptq import row_params, sweep
    g = torch.Generator().manual_seed(B + N + bits)
    M = 77
    W = torch.randn(M, N, generator=g) * 0.02
    W[3] = 0.0
    Hinv = ref.prepare_hinv(lognormal_hessian(N, 3 * N, 9), 0.01)
    s, z = ref.gptq_row_params(W, bits, asym)
    Q = torch.zeros(M, N, dtype=torch.int8)
    ref.gptq_block(W.clone(), Q, s, Hinv, 0, N, B, *((-8, 7) if bits == 4 else (-128, 127)), z)
    Wg = W.to(gpu_dev)
    s32, z32, s16, z8 = row_params(Wg, bits, asym)
    assert torch.equal(s32.cpu(), s.squeeze(1))
    if z is not None:
        assert torch.equal(z8.cpu(), z.squeeze(1))
    Qg = sweep(Wg.clone(), Hinv.to(gpu_dev), s32, z32, bits, B).cpu()
    assert torch.equal(Qg, Q)


@pytest.mark.parametrize("case", ["tiny_rows", "tiny_pivots", "huge_rows"])
@pytest.mark.parametrize("rows", [77, 12300])
def test_sweep_exact_fallback_bit_exact(gpu_dev, case, rows):
    """Inputs outside the fast division's exact domain make the sweep redo
    the block with the IEEE-exact test: rows of values near 1e-25 (residuals
    below 2^-60), an inverse Hessian scaled to pivots below 2^-30, and rows
    near 1e20 (residuals from 2^61 on).  Codes equal the CPU sweep's given
    the same Hinv.  One matrix of whole blocks runs the row sweep
    (sweep16_kernel, 4 and 16 waves per work-group at these row counts)."""
    from int_crush_converter_amd.gptq import row_params, sweep
    g = torch.Generator().manual_seed(rows + len(case))
    N = 128
    W = torch.randn(rows, N, generator=g) * 0.02
    Hinv = ref.prepare_hinv(lognormal_hessian(N, 3 * N, 21), 0.01)
    if case == "tiny_rows":
        W[1] = W[1] * 1e-23
        W[rows // 2] = W[rows // 2] * 1e-30
    elif case == "tiny_pivots":
        Hinv = Hinv * 1e-12
    else:
        W[2] = W[2] * 1e22
    s, z = ref.gptq_row_params(W, 4, False)
    Q = torch.zeros(rows, N, dtype=torch.int8)
    ref.gptq_block(W.clone(), Q, s, Hinv, 0, N, 128, -8, 7, z)
    Wg = W.to(gpu_dev)
    s32, z32, _, _ = row_params(Wg, 4, False)
    Qg = sweep(Wg.clone(), Hinv.to(gpu_dev), s32, z32, 4, 128).cpu()
    assert torch.equal(Qg, Q)


@pytest.mark.parametrize("case", ["tiny_rows", "tiny_pivots", "huge_rows"])
def test_sweep_exact_fallback_batched_groups(gpu_dev, case):
    """The quad sweep of block-diagonal groups (sweep4_kernel, 4 groups of
    128 columns) redoes a row exactly, in the row's error output, when its
    values leave the fast division's domain: codes equal the CPU sweep's per
    group given the same Hinv."""
    from int_crush_converter_amd.gptq import row_params, sweep
    g = torch.Generator().manual_seed(90 + len(case))
    M, G, bs = 300, 4, 128
    W = torch.randn(M, G * bs, generator=g) * 0.02
    Hinv = torch.stack([ref.prepare_hinv(lognormal_hessian(bs, 3 * bs, 60 + k), 0.01) for k in range(G)])
    if case == "tiny_rows":
        W[3] = W[3] * 1e-23
        W[150] = W[150] * 1e-30
    elif case == "tiny_pivots":
        Hinv[2] = Hinv[2] * 1e-12
    else:
        W[7] = W[7] * 1e22
    s, z = ref.gptq_row_params(W, 4, False)
    Q = torch.zeros(M, G * bs, dtype=torch.int8)
    for k in range(G):
        Qk = torch.zeros(M, bs, dtype=torch.int8)
        ref.gptq_block(W[:, k * bs:(k + 1) * bs].clone(), Qk, s, Hinv[k], 0, bs, bs, -8, 7, z)
        Q[:, k * bs:(k + 1) * bs] = Qk
    Wg = W.to(gpu_dev)
    s32, z32, _, _ = row_params(Wg, 4, False)
    Qg = sweep(Wg.clone(), Hinv.to(gpu_dev).contiguous(), s32, z32, 4, bs, G).cpu()
    assert torch.equal(Qg, Q)


@pytest.mark.parametrize("case", ["tiny_weights", "huge_weights"])
@pytest.mark.parametrize("rows", [77, 12300])
def test_ldlq_sweep_exact_fallback_bit_exact(gpu_dev, case, rows):
    """The LDLQ row sweep's exact rerun: nonzero weights below 2^-60 (scale
    at its 1e-5 floor) or from 2^61 on (scale above 2^31) leave the fast
    division's domain; codes equal the CPU LDLQ pass given the same Hinv."""
    from int_crush_converter_amd.ldlq import _single_pass
    g = torch.Generator().manual_seed(rows + 7 * len(case))
    N = 128
    W = torch.randn(rows, N, generator=g) * 0.02
    Hinv = ref.prepare_hinv(lognormal_hessian(N, 3 * N, 23), 0.01)
    if case == "tiny_weights":
        W[1] = W[1] * 1e-18
        W[rows // 2, :5] = 1e-20
    else:
        W[2] = W[2] * 1e21
    S = (W.abs().amax(dim=1, keepdim=True) / 7.0).clamp(min=1e-5).expand(rows, N)
    S = S * (1 + 0.1 * torch.rand(rows, N, generator=g))
    want = ref.ldlq_single_pass(W, Hinv, S.reshape(-1).clone(), N, -8, 7)
    got = _single_pass(W.to(gpu_dev), Hinv.to(gpu_dev), S.contiguous().to(gpu_dev), N, 4).cpu()
    assert torch.equal(got, want)


@pytest.mark.parametrize("bits,asym", [(4, False), (8, True)])
def test_sweep_batched_groups_bit_exact(gpu_dev, bits, asym):
    """16 block-diagonal groups of one 128-column block over 2048 rows
    (rows x groups = 32768: the kernel variant with 8 lanes per row): every
    group's codes equal the CPU sweep's given the same per-group Hinv."""
    from int_crush_converter_amd.gptq import row_params, sweep
    g = torch.Generator().manual_seed(40 + bits)
    M, G, bs = 2048, 16, 128
    W = torch.randn(M, G * bs, generator=g) * 0.02
    W[5] = 0.0
    Hinv = torch.stack([ref.prepare_hinv(lognormal_hessian(bs, 3 * bs, 50 + k), 0.01) for k in range(G)])
    s, z = ref.gptq_row_params(W, bits, asym)
    qlim = (-8, 7) if bits == 4 else (-128, 127)
    Q = torch.zeros(M, G * bs, dtype=torch.int8)
    for k in range(G):
        Qk = torch.zeros(M, bs, dtype=torch.int8)
        ref.gptq_block(W[:, k * bs:(k + 1) * bs].clone(), Qk, s, Hinv[k], 0, bs, bs, *qlim, z)
        Q[:, k * bs:(k + 1) * bs] = Qk
    Wg = W.to(gpu_dev)
    s32, z32, _, _ = row_params(Wg, bits, asym)
    Qg = sweep(Wg.clone(), Hinv.to(gpu_dev).contiguous(), s32, z32, bits, bs, G).cpu()
    assert torch.equal(Qg, Q)


def test_ldlq_sweep_many_rows_bit_exact(gpu_dev):
    """LDLQ sweep with per-element scales over 32768 rows (8 lanes per row)."""
    from int_crush_converter_amd.ldlq import _single_pass
    g = torch.Generator().manual_seed(77)
    M, N = 32768, 128
    W = torch.randn(M, N, generator=g) * 0.02
    Hinv = ref.prepare_hinv(lognormal_hessian(N, 3 * N, 13), 0.01)
    S = (W.abs().amax(dim=1, keepdim=True) / 7.0).clamp(min=1e-5).expand(M, N)
    S = S * (1 + 0.1 * torch.rand(M, N, generator=g))
    want = ref.ldlq_single_pass(W, Hinv, S.reshape(-1).clone(), N, -8, 7)
    got = _single_pass(W.to(gpu_dev), Hinv.to(gpu_dev), S.contiguous().to(gpu_dev), N, 4).cpu()
    assert torch.equal(got, want)


@pytest.mark.parametrize("B", [16, 32, 64, 128])
def test_sweep_multi_block_close(gpu_dev, B):
    """Whole-layer sweep given the same Hinv.  Block sizes 32 / 64 / 128: the
    lazy updates subtract one block's product at a time, as the reference
    does, so every code is equal; other block sizes sum whole 128-chunks of
    k first (>= 99.9 %)."""
    from int_crush_converter_amd.gptq import row_params, sweep
    g = torch.Generator().manual_seed(B)
    M, N = 256, 1024
    W = ref.rotate_weights(torch.randn(M, N, generator=g) * 0.02, 256)
    H = ref.rotate_hessian(lognormal_hessian(N, 2048, 11), 256)
    Hinv = ref.prepare_hinv(H, 0.01)
    s, z = ref.gptq_row_params(W, 4, False)
    Q = torch.zeros(M, N, dtype=torch.int8)
    ref.gptq_block(W.clone(), Q, s, Hinv, 0, N, B, -8, 7, z)
    Wg = W.to(gpu_dev)
    s32, z32, _, _ = row_params(Wg, 4, False)
    Qg = sweep(Wg.clone(), Hinv.to(gpu_dev), s32, z32, 4, B).cpu()
    if B in (32, 64, 128):
        assert torch.equal(Qg, Q)
    assert (Qg == Q).float().mean().item() >= 0.999


@pytest.mark.parametrize("M,N,K,kblk", [(300, 700, 1024, 128), (4096, 1000, 1024, 128), (129, 700, 384, 128)])
def test_sgemm_update_equals_blockwise_cpu_updates(gpu_dev, M, N, K, kblk):
    """C <- C - A B on the GPU with a long K equals the CPU's rank-128 updates
    applied in order, C - A[:, :128] B[:128] - A[:, 128:256] B[128:256] - ...,
    bit for bit: the kernel subtracts each 128-chunk of k, summed from zero
    in k order (the order of MKL's sgemm at K = 128), as soon as it is
    complete.  (MKL sums a lone last column, N mod 16 = 1, in another
    order; measured equal for every other shape tried.)"""
    g = torch.Generator().manual_seed(M + N + K)
    A = torch.randn(M, K, generator=g)
    B = torch.randn(K, N, generator=g)
    C = torch.randn(M, N, generator=g)
    want = C.clone()
    for k0 in range(0, K, kblk):
        want = want - A[:, k0:k0 + kblk] @ B[k0:k0 + kblk]
    from int_crush_converter_amd import _native as nat
    Cg = C.to(gpu_dev)
    Ag, Bg = A.to(gpu_dev), B.to(gpu_dev)
    nat.check(nat.lib().ic_sgemm(0, 0, M, N, K, -1.0, Ag.data_ptr(), K, Bg.data_ptr(), N, 1.0, Cg.data_ptr(), N,
                                 0, 0, nat.stream()), "ic_sgemm")
    got = Cg.cpu()
    assert torch.equal(got, want)


def _proxy(W, Q, s16, z8, H):
    d = ((Q.float() - (z8.float() if z8 is not None else 0)) * s16.float() - W).double()
    return (d @ H.double() * d).sum().item()


@pytest.mark.parametrize("case", ["gptq_a", "gptq_b", "gptq_c", "gptq_d", "gptq_e", "gptq_f", "gptq3d"])
def test_gptq_layer_golden(gpu_dev, golden, case):
    from int_crush_converter_amd.gptq import gptq_quantize_layer
    t, meta = golden
    m = meta[case]
    W, H = t[f"{case}.W"], t[f"{case}.H"]
    r = gptq_quantize_layer(W.to(gpu_dev), H.to(gpu_dev), block_size=m["block"], damping=0.01,
                            int_bits=m["bits"], asymmetric=m["asym"], hessian_method=m["method"])
    assert r.quantized_W.dtype == torch.int8 and r.scales.dtype == torch.float16
    assert torch.equal(r.scales.cpu(), t[f"{case}.scales"])
    if f"{case}.zp" in t:
        assert torch.equal(r.zero_points.cpu(), t[f"{case}.zp"])
    q = r.quantized_W.cpu()
    agree = (q == t[f"{case}.q"]).float().mean().item()
    assert agree >= 0.999, agree
    Hd = H if H.dim() == 2 else torch.block_diag(*H)
    z = t.get(f"{case}.zp")
    p_ref = _proxy(W, t[f"{case}.q"], t[f"{case}.scales"], z, Hd)
    p_got = _proxy(W, q, r.scales.cpu(), z, Hd)
    # These cases are small (<= 64 x 512) and ill-conditioned, so a handful of
    # codes decide the proxy: random symmetric perturbations of Hinv at
    # 3e-5 / 6e-5 relative (LAPACK's own fp32 error here is 3e-5) move it by
    # up to 3.9e-3 / 5.5e-3 and flip up to 0.9 % / 2.4 % of the codes.  The
    # 1e-3 bar is asserted at N = 2048 in test_gpu_gptq_large.py.
    assert abs(p_got / p_ref - 1) <= 1e-2
    assert r.mse == pytest.approx(m["mse"], rel=1e-2)


def test_gptq_layer_cpu_tensors_roundtrip(gpu_dev):
    """CPU inputs are computed on the GPU and returned on the CPU."""
    from int_crush_converter_amd.gptq import gptq_quantize_layer
    W = torch.randn(16, 64) * 0.02
    H = lognormal_hessian(64, 128, 1)
    r = gptq_quantize_layer(W, H)
    assert r.quantized_W.device.type == "cpu" and r.scales.shape == (16, 1) and r.zero_points.shape == (16, 1)
    assert r.quantized_W.min() >= -8 and r.quantized_W.max() <= 7


def test_gptq_layer_errors(gpu_dev):
    from int_crush_converter_amd.gptq import gptq_quantize_layer
    W = torch.randn(8, 32, device=gpu_dev)
    with pytest.raises(ValueError):
        gptq_quantize_layer(W, torch.eye(16, device=gpu_dev))
    with pytest.raises(ValueError):
        gptq_quantize_layer(W, torch.eye(32, device=gpu_dev), int_bits=3)
    with pytest.raises(ValueError):
        gptq_quantize_layer(W[0], torch.eye(32, device=gpu_dev))
    with pytest.raises(ValueError):
        gptq_quantize_layer(W, torch.eye(32, device=gpu_dev), hessian_method="lu")


def test_gptq_rtn_fallback_bit_exact(gpu_dev):
    from int_crush_converter_amd.gptq import gptq_quantize_layer_rtn
    W = ref.rotate_weights(torch.randn(32, 256) * 0.02, 256)
    for bits, asym in [(4, False), (4, True), (8, False), (8, True)]:
        r = gptq_quantize_layer_rtn(W.to(gpu_dev), bits, asym, [0.9, 1.0])
        q, s, z = ref.rtn_layer(W, bits, asym, [0.9, 1.0])
        assert torch.equal(r.quantized_W.cpu(), q) and torch.equal(r.scales.cpu(), s)
        if z is not None:
            assert torch.equal(r.zero_points.cpu(), z)


@pytest.mark.parametrize("N,nblk", [(1024, 2), (1000, 3), (1000, 4)])
def test_gptq_3d_partial_cover(gpu_dev, N, nblk):
    """A 3-D Hessian that covers fewer columns than the layer has: the
    reference loops over its blocks only and leaves the other codes at 0
    (converter/gptq.py:345-366); a partial last block is swept on its own."""
    from int_crush_converter_amd.gptq import gptq_quantize_layer
    g = torch.Generator().manual_seed(N + nblk)
    M, bs = 64, 256
    W = torch.randn(M, N, generator=g) * 0.02
    H = torch.stack([lognormal_hessian(bs, 3 * bs, 70 + k) for k in range(nblk)])
    want = ref.gptq_quantize_layer(W, H, 128, 0.01, 4)
    got = gptq_quantize_layer(W.to(gpu_dev), H.to(gpu_dev), block_size=128, damping=0.01, int_bits=4)
    q = got.quantized_W.cpu()
    covered = min(N, nblk * bs)
    assert torch.count_nonzero(q[:, covered:]) == 0
    assert torch.equal(got.scales.cpu(), want.scales)
    assert (q == want.quantized_W).float().mean().item() >= 0.999
    assert got.mse == pytest.approx(want.mse, rel=1e-2)


@pytest.mark.parametrize("bits,N", [(4, 96), (4, 128), (8, 96), (8, 128)])
def test_sweep_one_group_many_rows_bit_exact(gpu_dev, bits, N):
    """One group of 12300 rows (at least 12288 rows: the sweep with 8 lanes
    per row; 12300 is not a multiple of the 64 rows of a work-group, so the
    last wave has rows past the end) and a partial block (N = 96): codes
    equal the CPU sweep's given the same Hinv, INT4 and INT8 asymmetric."""
    from int_crush_converter_amd.gptq import row_params, sweep
    g = torch.Generator().manual_seed(bits * 1000 + N)
    M = 12300
    W = torch.randn(M, N, generator=g) * 0.02
    W[11] = 0.0
    Hinv = ref.prepare_hinv(lognormal_hessian(N, 3 * N, 17), 0.01)
    s, z = ref.gptq_row_params(W, bits, True)
    Q = torch.zeros(M, N, dtype=torch.int8)
    ref.gptq_block(W.clone(), Q, s, Hinv, 0, N, 128, *((-8, 7) if bits == 4 else (-128, 127)), z)
    Wg = W.to(gpu_dev)
    s32, z32, _, _ = row_params(Wg, bits, True)
    Qg = sweep(Wg.clone(), Hinv.to(gpu_dev), s32, z32, bits, 128).cpu()
    assert torch.equal(Qg, Q)


@pytest.mark.parametrize("M", [1000, 4100, 12283])
def test_sweep_fused_next_block_update_bit_exact(gpu_dev, M):
    """Four 128-column blocks given the same Hinv, with 4, 8 and 12 waves per
    work-group of the row sweep (M = 1000, 4100, 12283; none a multiple of
    the work-group's rows): the sweeps of blocks 0 and 2 also apply the next
    block's first lazy update, and the codes equal the CPU sweep's."""
    from int_crush_converter_amd.gptq import row_params, sweep
    g = torch.Generator().manual_seed(M)
    N = 512
    W = ref.rotate_weights(torch.randn(M, N, generator=g) * 0.02, 256)
    Hinv = ref.prepare_hinv(ref.rotate_hessian(lognormal_hessian(N, 1024, 23), 256), 0.01)
    s, z = ref.gptq_row_params(W, 4, True)
    Q = torch.zeros(M, N, dtype=torch.int8)
    ref.gptq_block(W.clone(), Q, s, Hinv, 0, N, 128, -8, 7, z)
    Wg = W.to(gpu_dev)
    s32, z32, _, _ = row_params(Wg, 4, True)
    Qg = sweep(Wg.clone(), Hinv.to(gpu_dev), s32, z32, 4, 128).cpu()
    assert torch.equal(Qg, Q)


def test_sweep_many_rows_multi_block_close(gpu_dev):
    """12288 rows over 4 blocks of 128 (8 lanes per row, lazy updates on the
    matrix cores) given the same Hinv: >= 99.9 % of codes equal."""
    from int_crush_converter_amd.gptq import row_params, sweep
    g = torch.Generator().manual_seed(5)
    M, N = 12288, 512
    W = ref.rotate_weights(torch.randn(M, N, generator=g) * 0.02, 256)
    Hinv = ref.prepare_hinv(ref.rotate_hessian(lognormal_hessian(N, 1024, 19), 256), 0.01)
    s, z = ref.gptq_row_params(W, 4, False)
    Q = torch.zeros(M, N, dtype=torch.int8)
    ref.gptq_block(W.clone(), Q, s, Hinv, 0, N, 128, -8, 7, z)
    Wg = W.to(gpu_dev)
    s32, z32, _, _ = row_params(Wg, 4, False)
    Qg = sweep(Wg.clone(), Hinv.to(gpu_dev), s32, z32, 4, 128).cpu()
    assert (Qg == Q).float().mean().item() >= 0.999


@pytest.mark.parametrize("M,gw,groups,block", [(300, 100, 1, 32), (257, 2500, 1, 128), (130, 256, 3, 128),
                                               (64, 1100, 1, 64), (70, 128, 1, 128)])
def test_sweep_from_leaves_input_and_matches_in_place(gpu_dev, M, gw, groups, block):
    """ic_gptq_quantize_from reads the weights without changing them and never
    reads the residual buffer's initial contents (filled with NaN here): its
    codes equal ic_gptq_quantize's on a copy, bit for bit, and so does every
    residual column it writes (all but each group's first block, which is
    swept straight from the input).  One block, one super-block, several
    super-blocks with a partial last one, 3-D groups, block sizes 32 / 64 / 128."""
    from int_crush_converter_amd import _native as nat
    L = nat.lib()
    g = torch.Generator().manual_seed(M + gw + groups + block)
    N = gw * groups
    W = (torch.randn(M, N, generator=g) * 0.02).to(gpu_dev)
    Hs = [ref.prepare_hinv(lognormal_hessian(gw, 2 * gw, 7 + k), 0.01) for k in range(groups)]
    Hinv = (torch.stack(Hs) if groups > 1 else Hs[0]).to(gpu_dev).contiguous()
    s = (W.abs().amax(dim=1) / 7.0).clamp(min=1e-5).contiguous()
    z = torch.zeros(M, device=gpu_dev)
    ws = nat.workspace(L.ic_gptq_workspace_bytes(M, groups, block), W.device)
    Wk = W.clone()
    Q0 = torch.full((M, N), 99, dtype=torch.int8, device=gpu_dev)
    nat.check(L.ic_gptq_quantize(Wk.data_ptr(), M, gw, groups, Hinv.data_ptr(), s.data_ptr(), z.data_ptr(), 4,
                                 block, Q0.data_ptr(), ws.data_ptr(), nat.stream()), "ic_gptq_quantize")
    W_in = W.clone()
    R = torch.full((M, N), float("nan"), device=gpu_dev)
    Q1 = torch.full((M, N), 99, dtype=torch.int8, device=gpu_dev)
    nat.check(L.ic_gptq_quantize_from(W_in.data_ptr(), R.data_ptr(), M, gw, groups, Hinv.data_ptr(), s.data_ptr(),
                                      z.data_ptr(), 4, block, Q1.data_ptr(), ws.data_ptr(), nat.stream()),
              "ic_gptq_quantize_from")
    torch.cuda.synchronize()
    assert torch.equal(Q1, Q0)
    assert torch.equal(W_in, W)
    first = torch.zeros(N, dtype=torch.bool, device=gpu_dev)
    for k in range(groups):
        first[k * gw: k * gw + min(block, gw)] = True
    assert bool(R[:, first].isnan().all())
    assert torch.equal(R[:, ~first], Wk[:, ~first])
