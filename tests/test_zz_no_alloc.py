"""ic_gptq_quantize_noalloc (the allocation-free GPTQ sweep, whose error
matrix lives in a static 128 MiB device array) against ic_gptq_quantize with
a caller-supplied workspace, through the C ABI: two calls in a row, the
second on a smaller input, with codes and working weights bit-exact (the
same kernels in the same order); sizes beyond the static array are refused
before anything runs."""

from __future__ import annotations


import pytest
import torch

from oracle import torch_ref as ref
from tests.conftest import lognormal_hessian

pytestmark = pytest.mark.gpu


def _case(M, gw, groups, seed, dev):
    g = torch.Generator().manual_seed(seed)
    W = ref.rotate_weights(torch.randn(M, gw * groups, generator=g) * 0.02, 256)
    Hs = [ref.prepare_hinv(ref.rotate_hessian(lognormal_hessian(gw, 2 * gw, seed + k), 256), 0.01)
          for k in range(groups)]
    Hinv = torch.stack(Hs) if groups > 1 else Hs[0]
    s, z = ref.gptq_row_params(W, 4, False)
    return (W.to(dev), Hinv.to(dev).contiguous(), s.squeeze(1).to(dev).contiguous(),
            z.squeeze(1).float().to(dev).contiguous())


def _run(noalloc, W, Hinv, s, z, groups):
    from int_crush_converter_amd import _native as nat
    L = nat.lib()
    M, N = W.shape
    gw = N // groups
    Wk = W.clone()
    Q = torch.full((M, N), 99, dtype=torch.int8, device=W.device)
    if noalloc:
        rc = L.ic_gptq_quantize_noalloc(Wk.data_ptr(), M, gw, groups, Hinv.data_ptr(), s.data_ptr(), z.data_ptr(),
                                        4, 128, Q.data_ptr(), nat.stream())
    else:
        ws = nat.workspace(L.ic_gptq_workspace_bytes(M, groups, 128), W.device)
        rc = L.ic_gptq_quantize(Wk.data_ptr(), M, gw, groups, Hinv.data_ptr(), s.data_ptr(), z.data_ptr(), 4, 128,
                                Q.data_ptr(), ws.data_ptr(), nat.stream())
    nat.check(rc, "gptq sweep")
    torch.cuda.synchronize()
    return Q.cpu(), Wk.cpu()


def test_noalloc_matches_workspace_entry_two_calls(gpu_dev):
    # first call: one 3072-column matrix over 4000 rows (three super-blocks,
    # lazy updates with K = 1024); second, smaller: 4 groups of 256 columns
    # over 300 rows, so stale scratch contents from the first call would show
    cases = [(_case(4000, 3072, 1, 5, gpu_dev), 1), (_case(300, 256, 4, 9, gpu_dev), 4)]
    for (W, Hinv, s, z), groups in cases:
        q0, w0 = _run(False, W, Hinv, s, z, groups)
        q1, w1 = _run(True, W, Hinv, s, z, groups)
        assert torch.equal(q1, q0)
        assert torch.equal(w1, w0)
        assert int(q1.min()) >= -8 and int(q1.max()) <= 7


def test_noalloc_refuses_oversized(gpu_dev):
    from int_crush_converter_amd import _native as nat
    L = nat.lib()
    assert L.ic_gptq_noalloc_scratch_bytes() == 128 << 20
    one = torch.zeros(1, device=gpu_dev)
    q = torch.zeros(1, dtype=torch.int8, device=gpu_dev)
    # 32769 rows x 1024 super-block columns x 4 bytes > 128 MiB: refused before any launch
    rc = L.ic_gptq_quantize_noalloc(one.data_ptr(), 32769, 2048, 1, one.data_ptr(), one.data_ptr(), None, 4, 128,
                                    q.data_ptr(), nat.stream())
    assert rc != 0
    assert b"128 MiB" in L.ic_last_error()
    # 3-D groups: 16 x 16385 rows x 128 columns x 4 bytes > 128 MiB
    rc = L.ic_gptq_quantize_noalloc(one.data_ptr(), 16385, 256, 16, one.data_ptr(), one.data_ptr(), None, 4, 128,
                                    q.data_ptr(), nat.stream())
    assert rc != 0
