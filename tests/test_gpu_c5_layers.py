"""GPU parity at configs[4]'s real layer shapes: GPTQ INT4 rot256 with a
block-diagonal calibration Hessian [in/256, 256, 256] (each block X^T X / 4096
of a seeded X with LogNormal(0, 1) channel scales), bf16 weights N(0, 0.02^2),
for the DiT block's widest layers: qkv [12288, 4096] (16 groups) and
mlp_down [4096, 16384] (64 groups, the batched quad sweep).

Bars:
* given the oracle's own per-block inverses (LAPACK on the CPU), every code
  equals the oracle's (converter/gptq.py:345-366 sweeps each block as an
  independent column group);
* the whole GPU path (its own fp32 Cholesky inverses) agrees on >= 99.9 % of
  the codes, scales and zero-points equal, tr(dW H dW^T) within 1e-3
  relative - and the disagreement is no larger than the oracle's own
  between its fp32 LAPACK inverse and an fp64 inverse rounded to fp32.
"""

from __future__ import annotations

import pytest
import torch

from oracle import torch_ref as ref

pytestmark = pytest.mark.gpu


def _c5_layer(M: int, N: int, seed: int):
    g = torch.Generator().manual_seed(seed)
    W = (torch.randn(M, N, generator=g) * 0.02).to(torch.bfloat16).float()
    blocks = []
    for _ in range(N // 256):
        s = torch.exp(torch.randn(256, generator=g))
        X = torch.randn(4096, 256, generator=g) * s
        blocks.append(X.T @ X / 4096)
    return W, torch.stack(blocks)


@pytest.mark.parametrize("name,M,N", [("qkv", 12288, 4096), ("mlp_down", 4096, 16384)])
def test_c5_layer_shape_vs_oracle(gpu_dev, name, M, N):
    from int_crush_converter_amd.gptq import gptq_quantize_layer, row_params, sweep
    W, H3 = _c5_layer(M, N, 500 + N)
    Wr = ref.rotate_weights(W, 256)
    Hr = ref.rotate_hessian(H3, 256)
    want = ref.gptq_quantize_layer(Wr, Hr, 128, 0.01, 4)
    G = N // 256
    Hinv = torch.stack([ref.prepare_hinv(Hr[b], 0.01) for b in range(G)])

    # the oracle's inverses: bit-exact codes
    Wg = Wr.to(gpu_dev)
    s32, z32, s16, z8 = row_params(Wg, 4, False)
    assert torch.equal(s16.reshape(M, 1).cpu(), want.scales) and torch.equal(z8.reshape(M, 1).cpu(), want.zero_points)
    Q = sweep(Wg, Hinv.to(gpu_dev).contiguous(), s32, z32, 4, 128, G).cpu()
    same = int((Q != want.quantized_W).sum())
    print(f"[parity] c5 {name} given_oracle_hinv differing_codes={same} of {Q.numel()}", flush=True)
    assert same == 0

    # the whole GPU path
    got = gptq_quantize_layer(Wg, Hr.to(gpu_dev), 128, 0.01, 4)
    q = got.quantized_W.cpu()
    agree = (q == want.quantized_W).float().mean().item()
    # the oracle's own fp32-inverse noise: fp64 inverses rounded to fp32
    Hinv64 = torch.stack([torch.cholesky_inverse(torch.linalg.cholesky(ref.damp(Hr[b], 0.01).double())).float()
                          for b in range(G)])
    Qn = sweep(Wg, Hinv64.to(gpu_dev).contiguous(), s32, z32, 4, 128, G).cpu()
    agree_self = (Qn == want.quantized_W).float().mean().item()

    Hd = Hr.double().to(gpu_dev)
    Wd = Wr.double().to(gpu_dev)
    s_d = want.scales_fp32.double().to(gpu_dev)
    z_d = want.zero_points.double().to(gpu_dev)

    def proxy(Qc):
        # tr(dW H dW^T) over the block-diagonal H, one 256-column group at a time
        d = ((Qc.to(gpu_dev).double() - z_d) * s_d - Wd).reshape(M, G, 256).transpose(0, 1).contiguous()
        return (torch.bmm(d, Hd) * d).sum().item()

    rel = proxy(q) / proxy(want.quantized_W) - 1
    print(f"[parity] c5 {name} agreement={agree:.6f} oracle_fp32_vs_fp64_inverse={agree_self:.6f} "
          f"proxy_rel={rel:.3g}", flush=True)
    assert torch.equal(got.scales.cpu(), want.scales) and torch.equal(got.zero_points.cpu(), want.zero_points)
    assert agree >= 0.999 and agree >= agree_self - 5e-4, (agree, agree_self)
    assert abs(rel) <= 1e-3
