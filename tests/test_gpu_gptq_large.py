"""GPTQ at larger sizes: the end-to-end layer (own damping, Cholesky, inverse,
sweep, lazy update) against the CPU oracle, and size-independent properties
at the headline shape [4096, 12288].

Why the bars are relative to the reference itself: GPTQ feeds every
rounding decision forward, so fp32 summation-order differences in the
inverse flip a growing share of codes.  The reference run against itself
with one MKL thread instead of the default agrees on 99.74 % - 99.98 % of
codes at N = 2048 (mean 99.90 % over 8 seeds), i.e. a single seed can miss
99.9 % with the reference's own arithmetic.  The tests therefore compare
this build's agreement with the reference's self-agreement on the same
seeds (means over seeds), with per-seed floors, and require the
H-weighted error tr(dW H dW^T) to be no worse than the reference's by more
than 1e-3 on average.  Scales and
zero-points are bit-exact throughout.
"""

from __future__ import annotations

import pytest
import torch

from oracle import torch_ref as ref
from tests.conftest import lognormal_hessian

pytestmark = pytest.mark.gpu


def _proxy(W, Q, s, z, H):
    d = ((Q.double() - z.double()) * s.double() - W.double())
    return (d @ H.double() * d).sum().item()


def _layer_case(gpu_dev, M, N, samples, seed):
    """(agreement with the reference, the reference's agreement with
    itself at one thread, relative proxy difference)."""
    from int_crush_converter_amd.gptq import gptq_quantize_layer
    g = torch.Generator().manual_seed(seed)
    W = ref.rotate_weights(torch.randn(M, N, generator=g) * 0.02, 256)
    H = ref.rotate_hessian(lognormal_hessian(N, samples, seed + 1), 256)
    want = ref.gptq_quantize_layer(W, H, 128, 0.01, 4)
    got = gptq_quantize_layer(W.to(gpu_dev), H.to(gpu_dev), block_size=128, damping=0.01, int_bits=4)
    assert torch.equal(got.scales.cpu(), want.scales)
    assert torch.equal(got.zero_points.cpu(), want.zero_points)
    q = got.quantized_W.cpu()
    agree = (q == want.quantized_W).float().mean().item()
    threads = torch.get_num_threads()
    torch.set_num_threads(1)
    try:
        alt = ref.gptq_quantize_layer(W, H, 128, 0.01, 4)
    finally:
        torch.set_num_threads(threads)
    self_agree = (alt.quantized_W == want.quantized_W).float().mean().item()
    s = want.scales.float()
    z = want.zero_points.float()
    rel = _proxy(W, q, s, z, H) / _proxy(W, want.quantized_W, s, z, H) - 1
    return agree, self_agree, rel


def test_gptq_layer_n2048(gpu_dev):
    # Measured over 16 seeds: agreement 99.92 % (reference vs itself
    # 99.90 %), proxy difference +5e-4 on average (|.| 9e-4; the reference
    # against itself: +7e-4, |.| 1.0e-3).
    res = [_layer_case(gpu_dev, 256, 2048, 4096, seed) for seed in range(21, 29)]
    n = len(res)
    agree = sum(r[0] for r in res) / n
    self_agree = sum(r[1] for r in res) / n
    assert agree >= self_agree - 5e-4, res
    assert min(r[0] for r in res) >= 0.995, res
    assert sum(r[2] for r in res) / n <= 1e-3, res          # not worse than the reference on average
    assert sum(abs(r[2]) for r in res) / n <= 2e-3, res


def test_gptq_layer_n6144(gpu_dev):
    agree, self_agree, rel = _layer_case(gpu_dev, 128, 6144, 8192, 31)
    assert agree >= self_agree - 3e-3, (agree, self_agree)
    assert agree >= 0.985, agree
    assert abs(rel) <= 3e-3, rel


def test_gptq_headline_shape_properties(gpu_dev):
    """[4096, 12288] bf16 with a LogNormal-channel H (the bench workload):
    deterministic, codes in range, pack/unpack round trip, scales bit-exact
    vs the oracle's, and a proxy loss well below RTN with the same scales."""
    from int_crush_converter_amd import layer as L
    from int_crush_converter_amd.packing import unpack_int4
    M, N = 4096, 12288
    g = torch.Generator(device=gpu_dev).manual_seed(7)
    W = (torch.randn(M, N, generator=g, device=gpu_dev) * 0.02).to(torch.bfloat16)
    s = torch.exp(torch.randn(N, generator=g, device=gpu_dev))
    X = torch.randn(4096, N, generator=g, device=gpu_dev) * s
    H = (X.T @ X) / 4096
    del X
    outs = []
    for _ in range(2):
        W_work, _ = L.prepare_weights(W, 256)
        codes, s16, z8 = L.gptq_codes(W_work, H.clone(), rotate_h=256, block_size=128, damping=0.01, int_bits=4,
                                      asymmetric=False, hessian_method="hinv", fallbacks=[])
        outs.append((codes.clone(), s16.clone(), z8.clone()))
    assert all(torch.equal(a, b) for a, b in zip(outs[0], outs[1]))
    codes, s16, z8 = outs[0]
    assert codes.min().item() >= -8 and codes.max().item() <= 7
    out = L.finish(W_work, codes, s16, z8, 4)
    assert torch.equal(unpack_int4(out.stored, N), codes)

    Wr = ref.rotate_weights(W.cpu().float(), 256)
    s_ref, z_ref = ref.gptq_row_params(Wr, 4, False)
    assert torch.equal(s16.cpu(), s_ref.to(torch.float16))
    assert torch.equal(z8.cpu(), z_ref)

    from int_crush_converter_amd.rotation import rotate_hessian
    Hr = rotate_hessian(H, 256).double()
    sf = s16.float().double()
    zf = z8.double()
    Wd = W_work.double()
    rtn = torch.clamp(torch.where(Wd / sf + zf >= 0, torch.floor(Wd / sf + zf + 0.5),
                                  torch.ceil(Wd / sf + zf - 0.5)), -8, 7)

    def proxy(Q):
        d = (Q.double() - zf) * sf - Wd
        return ((d @ Hr) * d).sum().item()

    p_gptq, p_rtn = proxy(codes), proxy(rtn)
    assert p_gptq < 0.8 * p_rtn, (p_gptq, p_rtn)
