"""PermuQuant on the GPU against the oracle (torch's own CPU arithmetic).

The moments and the acceptance errors must be bit-exact: the kernels add in
torch's CPU order, which the oracle gets from torch itself.  The permutation
equals torch's argsort when there are no exact ties; on ties the GPU sort is
stable (torch's CPU sort is not, from 100 elements on: tie order unpinned).
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle import torch_ref as ref

pytestmark = pytest.mark.gpu


@pytest.fixture
def cpu_threads():
    """Set torch's CPU thread count for the oracle; restored afterwards."""
    old = torch.get_num_threads()
    yield torch.set_num_threads
    torch.set_num_threads(old)


def _bits_equal(a: torch.Tensor, b: torch.Tensor) -> bool:
    return torch.equal(a.float().contiguous().view(torch.int32), b.float().contiguous().view(torch.int32))


@pytest.mark.parametrize("M,N", [(64, 256), (1000, 300), (17, 40), (4097, 333), (3, 5), (4096, 1030), (1, 16),
                                 (300, 4100)])
def test_channel_moments_bit_exact(gpu_dev, M, N):
    from int_crush_converter_amd import permuquant as pq
    g = torch.Generator().manual_seed(M * 31 + N)
    W = torch.randn(M, N, generator=g) * 0.02
    got = pq.channel_second_moments(W.to(gpu_dev)).cpu()
    assert _bits_equal(got, ref.channel_second_moments(W))


def test_channel_moments_strided_view(gpu_dev):
    # the pipeline takes W_work[:, :orig_in] of a padded rotation (row pitch > columns)
    from int_crush_converter_amd import permuquant as pq
    g = torch.Generator().manual_seed(2)
    Wp = torch.randn(96, 512, generator=g) * 0.02
    got = pq.channel_second_moments(Wp.to(gpu_dev)[:, :300]).cpu()
    assert _bits_equal(got, ref.channel_second_moments(Wp[:, :300]))


def test_channel_moments_headline_shape(gpu_dev):
    from int_crush_converter_amd import permuquant as pq
    g = torch.Generator().manual_seed(11)
    W = torch.randn(4096, 12288, generator=g) * 0.02
    got = pq.channel_second_moments(W.to(gpu_dev)).cpu()
    assert _bits_equal(got, ref.channel_second_moments(W))
    p = pq.find_permutation_weight(W.to(gpu_dev)).cpu()
    mu = ref.channel_second_moments(W)
    if mu.unique().numel() == mu.numel():
        assert torch.equal(p, ref.permutation_weight(W))


@pytest.mark.parametrize("n", [1, 5, 99, 100, 1000, 12288, 16384, 20000, 70000])
def test_argsort_matches_torch_without_ties(gpu_dev, n):
    from int_crush_converter_amd import permuquant as pq
    g = torch.Generator().manual_seed(n)
    # distinct values (torch.rand has 24-bit resolution and repeats at these sizes)
    v = (torch.randperm(n, generator=g).float() + 0.5 * torch.rand(n, generator=g)) / n
    assert v.unique().numel() == n
    assert torch.equal(pq.argsort_descending(v.to(gpu_dev)).cpu(), v.argsort(descending=True))


@pytest.mark.parametrize("n", [50, 1000, 40000])
def test_argsort_stable_with_ties_and_nan(gpu_dev, n):
    from int_crush_converter_amd import permuquant as pq
    g = torch.Generator().manual_seed(n + 1)
    v = torch.randint(0, 7, (n,), generator=g).float() / 3.0
    v[torch.randint(0, n, (n // 10 + 1,), generator=g)] = float("nan")
    v[torch.randint(0, n, (n // 10 + 1,), generator=g)] = -0.0
    got = pq.argsort_descending(v.to(gpu_dev)).cpu().tolist()

    def key(i):
        x = v[i].item()
        return (0 if math.isnan(x) else 1, 0.0 if math.isnan(x) else -x, i)

    assert got == sorted(range(n), key=key)


@pytest.mark.parametrize("threads", [1, 3, 8, 16])
@pytest.mark.parametrize("n", [1, 7, 8, 33, 1000, 32767, 32768, 100001, 3000001])
def test_torch_sum_bit_exact(gpu_dev, cpu_threads, threads, n):
    from int_crush_converter_amd import _native as nat
    cpu_threads(threads)
    g = torch.Generator().manual_seed(n + threads)
    x = torch.randn(n, generator=g) ** 2
    xg = x.to(gpu_dev)
    out = torch.empty(1, device=gpu_dev)
    ws = nat.workspace(nat.lib().ic_torch_sum_workspace_bytes(n, threads), gpu_dev)
    nat.check(nat.lib().ic_torch_sum(xg.data_ptr(), n, threads, out.data_ptr(), ws.data_ptr(), nat.stream()),
              "ic_torch_sum")
    assert _bits_equal(out.cpu(), x.sum().reshape(1))


@pytest.mark.parametrize("threads", [1, 3, 8, 16])
@pytest.mark.parametrize("M,N,gs,bits", [(64, 256, 256, 4), (100, 300, 128, 4), (33, 77, 128, 8), (512, 2048, 2048, 4),
                                         (256, 1024, 1024, 8), (40, 130, 64, 4)])
def test_group_quant_error_bit_exact(gpu_dev, cpu_threads, threads, M, N, gs, bits):
    from int_crush_converter_amd import permuquant as pq
    cpu_threads(threads)
    g = torch.Generator().manual_seed(M + N + gs + bits)
    W = torch.randn(M, N, generator=g) * torch.exp(torch.randn(N, generator=g)) * 0.02
    perm = torch.randperm(N, generator=g)
    Wg = W.to(gpu_dev)
    want = ref.group_quant_error(W, gs, bits)
    assert pq.compute_group_quant_error(Wg, gs, bits, threads=threads) == want
    assert pq._quant_error(Wg, perm.to(gpu_dev), gs, bits, threads) == ref.group_quant_error(W[:, perm], gs, bits)


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("bits", [4, 8])
def test_acceptance_decision_matches_reference(gpu_dev, seed, bits):
    # per-row scales: the two errors differ only by fp32 summation order, and
    # the decision must follow the reference's (same torch thread count)
    from int_crush_converter_amd import permuquant as pq
    g = torch.Generator().manual_seed(100 + seed)
    W = torch.randn(128 + 7 * seed, 512, generator=g) * 0.02
    gs = 512 if bits == 4 else 128
    perm, acc = pq.find_permutation_with_acceptance(W.to(gpu_dev), None, 0.0, gs, 0.0, bits)
    rperm, racc = ref.permutation_with_acceptance(W, None, 0.0, gs, 0.0, bits)
    assert torch.equal(perm.cpu(), rperm) and acc == racc


def test_grouped_acceptance_and_sweep(gpu_dev):
    from int_crush_converter_amd import permuquant as pq
    decisions = set()
    for seed in range(6):
        g = torch.Generator().manual_seed(seed)
        W = torch.randn(16, 128, generator=g) * torch.exp(torch.randn(128, generator=g) * 1.5) * 0.01
        perm, acc = pq.find_permutation_with_acceptance(W.to(gpu_dev), None, 0.0, 16, 0.0, 4)
        rperm, racc = ref.permutation_with_acceptance(W, None, 0.0, 16, 0.0, 4)
        assert torch.equal(perm.cpu(), rperm) and acc == racc
        decisions.add(acc)
        p2, a2, acc2 = pq.sweep_alpha(W.to(gpu_dev), None, 16, 0.0, 11, 4)
        assert torch.equal(p2.cpu(), rperm) and a2 == 0.0 and acc2 == racc
    assert decisions == {True, False}
    with pytest.raises(ValueError):
        pq.sweep_alpha(torch.randn(8, 64, device=gpu_dev), num_alpha=0)
    _, acc = pq.find_permutation_with_acceptance(torch.zeros(8, 64, device=gpu_dev), None, 0.0, 64, 0.0, 4)
    assert acc is False


def test_joint_criterion_alpha_sweep(gpu_dev):
    # the joint criterion's pow runs on the GPU (not bit-exact with the CPU's):
    # check the reference's structural properties
    from int_crush_converter_amd import permuquant as pq
    g = torch.Generator().manual_seed(42)
    W = torch.randn(16, 64, generator=g)
    act = torch.rand(64, generator=g)
    Wg, ag = W.to(gpu_dev), act.to(gpu_dev)
    assert torch.equal(pq.find_permutation_joint(Wg, ag, 0.0).cpu(), pq.find_permutation_weight(Wg).cpu())
    assert torch.equal(pq.find_permutation_joint(Wg, ag, 1.0).cpu(), act.argsort(descending=True))
    perm, alpha, acc = pq.sweep_alpha(torch.randn(16, 128, generator=g).to(gpu_dev), torch.rand(128, generator=g),
                                      num_alpha=11, group_size=128)
    assert sorted(perm.cpu().tolist()) == list(range(128)) and 0.0 <= alpha <= 1.0 and isinstance(acc, bool)


def test_permute_gathers(gpu_dev):
    from int_crush_converter_amd import permuquant as pq
    g = torch.Generator().manual_seed(9)
    W = torch.randn(37, 90, generator=g)
    perm = torch.randperm(90, generator=g)
    assert torch.equal(pq.permute_columns(W.to(gpu_dev), perm).cpu(), W[:, perm])
    H = torch.randn(90, 90, generator=g)
    assert torch.equal(pq.permute_hessian(H.to(gpu_dev), perm).cpu(), H[perm][:, perm])
    # a slice of the permutation and out-of-range indices (not read, output 0)
    bad = torch.tensor([3, 95, -1, 0])
    got = pq.permute_columns(W.to(gpu_dev), bad).cpu()
    assert torch.equal(got[:, 0], W[:, 3]) and torch.equal(got[:, 3], W[:, 0])
    assert (got[:, 1:3] == 0).all()
