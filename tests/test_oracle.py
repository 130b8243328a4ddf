"""Pins the CPU oracle (oracle/torch_ref.py) against things other than itself:
closed forms, the reference's own known-answer tests, independent numpy
float32 restatements on tiny inputs, brute force, and golden vectors written
by the reference (tests/golden/).  CPU only."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import torch_ref as ref
from tests.conftest import lognormal_hessian

f32 = np.float32


# ---------------------------------------------------------------- Hadamard

@pytest.mark.parametrize("n", [4, 16, 64, 256])
def test_hadamard_regular_closed_form(n):
    H = ref.hadamard_regular(n, torch.float64)
    k = int(round(math.log(n, 4)))
    assert torch.all(H.abs() == 2.0 ** -k)
    assert torch.equal(H, H.T)                        # symmetric
    assert torch.allclose(H @ H, torch.eye(n, dtype=torch.float64), atol=0, rtol=0)
    assert torch.all(H.sum(dim=1) == 2.0 ** k / 2.0 ** k * 1.0) or torch.allclose(
        H.sum(dim=1), torch.full((n,), 2.0 ** k / 2.0 ** k))  # regular: equal row sums
    # Kronecker structure: H_n = kron(H_{n/4}, H_4)
    if n > 4:
        assert torch.equal(H, torch.kron(ref.hadamard_regular(n // 4, torch.float64),
                                         ref.hadamard_regular(4, torch.float64)))


@pytest.mark.parametrize("n", [2, 8, 32, 128])
def test_hadamard_sylvester_orthonormal(n):
    H = ref.hadamard_sylvester(n, torch.float64)
    assert torch.allclose(H @ H.T, torch.eye(n, dtype=torch.float64), atol=1e-12)
    assert torch.allclose(H.abs(), torch.full_like(H, 1 / math.sqrt(n)), atol=1e-12)


def _dense_blockdiag(n_pad, rot):
    R = torch.zeros(n_pad, n_pad, dtype=torch.float64)
    h = ref._hadamard_for(rot, torch.float64)
    for g in range(n_pad // rot):
        R[g * rot:(g + 1) * rot, g * rot:(g + 1) * rot] = h
    return R


@pytest.mark.parametrize("rot,n", [(16, 64), (64, 192), (256, 256), (256, 300), (128, 256), (32, 40)])
def test_rotate_weights_vs_dense(rot, n):
    g = torch.Generator().manual_seed(rot + n)
    W = torch.randn(9, n, generator=g)
    out = ref.rotate_weights(W, rot)
    n_pad = -(-n // rot) * rot
    Wp = torch.zeros(9, n_pad, dtype=torch.float64)
    Wp[:, :n] = W.double()
    want = Wp @ _dense_blockdiag(n_pad, rot).T
    assert out.shape == (9, n_pad)
    assert torch.allclose(out.double(), want, atol=1e-5)
    assert torch.allclose(out.double().norm(), W.double().norm(), rtol=1e-5)


@pytest.mark.parametrize("rot,n", [(16, 64), (64, 128), (256, 256), (256, 300)])
def test_rotate_hessian_two_sided(rot, n):
    g = torch.Generator().manual_seed(7)
    X = torch.randn(40, n, generator=g, dtype=torch.float64)
    H = (X.T @ X).float()
    out = ref.rotate_hessian(H, rot)
    n_pad = -(-n // rot) * rot
    Xp = torch.zeros(40, n_pad, dtype=torch.float64)
    Xp[:, :n] = X
    XR = Xp @ _dense_blockdiag(n_pad, rot)          # R symmetric
    want = XR.T @ XR
    assert torch.allclose(out.double(), want, atol=1e-3 * want.abs().max().item())
    assert abs(out.double().trace().item() - H.double().trace().item()) < 1e-4 * H.double().trace().item()


def test_rotate_hessian_3d_subblocks():
    g = torch.Generator().manual_seed(3)
    H3 = torch.randn(2, 128, 128, generator=g)
    H3 = H3 @ H3.transpose(1, 2)
    out = ref.rotate_hessian(H3, 64)
    for b in range(2):
        want = ref.rotate_hessian(H3[b], 64)
        assert torch.allclose(out[b], want, atol=1e-3)


# ------------------------------------------------ rotation rounding (goldens)

def _seq_rows_np(x: np.ndarray, rot: int) -> np.ndarray:
    """Sequential fp32 chains y_j = (((0 + x_0 h_0j) + x_1 h_1j) + ...) per
    group of ``rot`` columns, in numpy.  The regular Hadamard's entries are
    +-2^-k, so every product is exact and an fp32 add after an fp32 multiply
    IS the fused multiply-add: this restates, without torch, the order the
    reference's CPU GEMM rounds in."""
    assert ref.is_pow4(rot)
    h = ref.hadamard_regular(rot).numpy()
    m, n = x.shape
    xg = x.reshape(m, n // rot, rot)
    acc = np.zeros_like(xg, dtype=np.float32)
    for k in range(rot):
        acc = (acc + xg[:, :, k:k + 1] * h[k][None, None, :]).astype(np.float32)
    return acc.reshape(m, n)


def _pad(x: torch.Tensor, rot: int) -> torch.Tensor:
    return torch.nn.functional.pad(x, (0, (-x.shape[1]) % rot))


def test_rotation_golden_cases_present(golden_rotation):
    t, meta = golden_rotation
    kinds = {m["kind"] for m in meta.values()}
    assert kinds == {"rotate_weights", "rotate_hessian", "gptq_raw"}
    assert {m["rot"] for m in meta.values() if m["kind"] == "rotate_weights"} >= {2, 4, 8, 16, 32, 64, 128, 256, 512}


def test_oracle_rotate_weights_equals_reference(golden_rotation):
    """The oracle's x @ H.T gives the reference's bits (every rot to 512,
    fp32 / bf16 sources, padding, the pipeline's outlier zeroing)."""
    t, meta = golden_rotation
    for name, m in meta.items():
        if m["kind"] != "rotate_weights":
            continue
        W = t[f"{name}.W"].float()
        if "zero_above" in m:
            W = W.masked_fill(W.abs() > m["zero_above"], 0.0)
        assert torch.equal(ref.rotate_weights(W, m["rot"]), t[f"{name}.out"]), name


def test_sequential_chain_restatement_equals_reference(golden_rotation):
    """Independent of torch: the sequential fp32 chain (numpy) reproduces the
    reference's rotated weights and both products of its Hessian rotation
    bit for bit - the order the exact GPU kernels implement."""
    t, meta = golden_rotation
    for name, m in meta.items():
        if m["kind"] == "rotate_weights" and ref.is_pow4(m["rot"]):
            W = t[f"{name}.W"].float()
            if "zero_above" in m:
                W = W.masked_fill(W.abs() > m["zero_above"], 0.0)
            got = _seq_rows_np(_pad(W, m["rot"]).numpy(), m["rot"])
            assert np.array_equal(got, t[f"{name}.out"].numpy()), name
        elif m["kind"] == "rotate_hessian" and t[f"{name}.H"].dim() == 2:
            rot = m["rot"]
            H = t[f"{name}.H"]
            n = H.shape[0] + (-H.shape[0]) % rot
            Hp = torch.zeros(n, n)
            Hp[:H.shape[0], :H.shape[0]] = H
            # left product: T = R^T H, a chain over the rows of each block
            # = the row chain applied to the columns (R is symmetric)
            T = _seq_rows_np(np.ascontiguousarray(Hp.numpy().T), rot).T
            O = _seq_rows_np(np.ascontiguousarray(T), rot)
            assert np.array_equal(O, t[f"{name}.out"].numpy()), name


def test_oracle_rotate_hessian_equals_reference(golden_rotation):
    t, meta = golden_rotation
    for name, m in meta.items():
        if m["kind"] == "rotate_hessian":
            assert torch.equal(ref.rotate_hessian(t[f"{name}.H"], m["rot"]), t[f"{name}.out"]), name


def test_golden_raw_inputs_rotate_to_golden_cases(golden, golden_rotation):
    """The stored raw W / H of the rotated GPTQ goldens rotate (oracle) to
    the rotated inputs those cases were quantised from."""
    g, _ = golden
    t, meta = golden_rotation
    for name, m in meta.items():
        if m["kind"] == "gptq_raw":
            case = name[:-len("_raw")]
            assert torch.equal(ref.rotate_weights(t[f"{name}.W"], m["rot"]), g[f"{case}.W"]), name
            assert torch.equal(ref.rotate_hessian(t[f"{name}.H"], m["rot"]), g[f"{case}.H"]), name


@pytest.mark.parametrize("rot", [2, 8, 32, 128])
def test_rotate_hessian_rejects_non_power_of_four(rot):
    # converter/rotation.py:247 -> get_hadamard -> make_hadamard_regular raises
    with pytest.raises(ValueError, match="power of 4"):
        ref.rotate_hessian(torch.eye(2 * rot), rot)


# ---------------------------------------------------------------- rounding

def test_rhaz_reference_kats():
    # tests/unit/test_ldlq_hessian.py:34-49 of the reference
    assert torch.equal(ref.rhaz(torch.tensor([0.5, 1.5, 2.5, 3.5])), torch.tensor([1.0, 2.0, 3.0, 4.0]))
    assert torch.equal(ref.rhaz(torch.tensor([-0.5, -1.5, -2.5, -3.5])), torch.tensor([-1.0, -2.0, -3.0, -4.0]))
    x = torch.tensor([-2.0, -1.0, 0.0, 1.0, 2.0])
    assert torch.equal(ref.rhaz(x), x)


def test_rhaz_literal_add_half():
    # 0.49999997 + 0.5 rounds to 1.0 in fp32, so rhaz gives 1 (not 0)
    x = torch.tensor([0.49999997, -0.49999997], dtype=torch.float32)
    assert torch.equal(ref.rhaz(x), torch.tensor([1.0, -1.0]))


def np_rhaz(x):
    x = f32(x)
    return f32(np.floor(f32(x + f32(0.5)))) if x >= 0 else f32(np.ceil(f32(x - f32(0.5))))


# ---------------------------------------------------------------- scales / RTN

def test_scale_kat():
    # tests/test_scales.py:48-55 of the reference
    W = torch.tensor([[1.0, -2.0, 3.0], [-7.0, 1.0, 0.5]])
    s = ref.scales_int4_sym(W)
    assert s.dtype == torch.float16 and s.shape == (2, 1)
    assert abs(s[0].item() - 3 / 7) < 1e-3 and abs(s[1].item() - 1.0) < 1e-3


def _np_row_rtn_sym(row, qmax_div, qmin, qmax):
    amax = f32(np.max(np.abs(row)))
    s = f32(np.clip(f32(amax / f32(qmax_div)), f32(1e-5), f32(65500)))
    s16 = f32(np.float16(s))
    q = [max(qmin, min(qmax, np_rhaz(f32(w / s16)))) for w in row]
    return np.float16(s), np.array(q, dtype=np.int8)


def _np_fix(s, wmin, wmax, qmin, qmax):
    spread = f32(qmax - qmin)
    zr = f32(qmin) - np_rhaz(f32(wmin / s))
    if zr < qmin:
        s = max(s, f32(np.clip(f32(wmax / spread), f32(1e-5), f32(65500))))
    if zr > qmax:
        s = max(s, f32(np.clip(f32(-wmin / spread), f32(1e-5), f32(65500))))
    return f32(s)


def _np_row_rtn_asym(row, qmin, qmax, zero_fix):
    spread = f32(qmax - qmin)
    wmin, wmax = f32(np.min(row)), f32(np.max(row))
    s = f32(np.clip(f32(f32(wmax - wmin) / spread), f32(1e-5), f32(65500)))
    s = _np_fix(s, wmin, wmax, qmin, qmax)
    z = max(qmin, min(qmax, f32(qmin) - np_rhaz(f32(wmin / s))))
    if zero_fix and wmin == 0 and wmax == 0:
        z = f32(0)
    s16 = f32(np.float16(s))
    q = [max(qmin, min(qmax, np_rhaz(f32(f32(w / s16) + f32(z))))) for w in row]
    return np.float16(s), np.int8(z), np.array(q, dtype=np.int8)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_rtn_formulas_vs_numpy(seed):
    g = torch.Generator().manual_seed(seed)
    W = torch.randn(6, 37, generator=g) * 0.05
    W[1] = 0.0
    W[2] += 3.0        # far from zero: exercises the zero-point fix
    W[3] -= 5.0
    Wn = W.numpy()
    s4 = ref.scales_int4_sym(W)
    q4 = ref.quant_int4_sym(W, s4)
    s8 = ref.scales_int8_sym(W)
    q8 = ref.quant_int8_sym(W, s8)
    s4a, z4a = ref.scales_int4_asym(W)
    q4a = ref.quant_int4_asym(W, s4a, z4a)
    s8a, z8a = ref.scales_int8_asym(W)
    q8a = ref.quant_int8_asym(W, s8a, z8a)
    for r in range(6):
        s, q = _np_row_rtn_sym(Wn[r], 7.0, -8, 7)
        assert s == s4[r, 0].numpy() and np.array_equal(q, q4[r].numpy())
        s, q = _np_row_rtn_sym(Wn[r], 127.0, -128, 127)
        assert s == s8[r, 0].numpy() and np.array_equal(q, q8[r].numpy())
        s, z, q = _np_row_rtn_asym(Wn[r], -8, 7, True)
        assert s == s4a[r, 0].numpy() and z == z4a[r, 0].numpy() and np.array_equal(q, q4a[r].numpy())
        s, z, q = _np_row_rtn_asym(Wn[r], -128, 127, False)
        assert s == s8a[r, 0].numpy() and z == z8a[r, 0].numpy() and np.array_equal(q, q8a[r].numpy())


def test_clip_search_brute_force():
    """Chosen ratio minimises the per-row fp32 MSE; ties keep the first."""
    g = torch.Generator().manual_seed(11)
    W = torch.randn(8, 64, generator=g)
    ratios = [0.8, 0.85, 0.9, 0.95, 1.0]
    s = ref.scales_int4_sym(W, ratios=ratios)
    amax = W.abs().amax(dim=1)
    for r in range(8):
        best, best_m = None, None
        for ratio in ratios:
            cs = torch.clamp(amax[r:r + 1] * ratio / 7.0, 1e-5, 65500)
            q = (W[r] / cs).round().clamp(-8, 7)
            m = (W[r] - q * cs).pow(2).mean()
            if best_m is None or m < best_m:
                best, best_m = cs, m
        assert best.half().item() == s[r, 0].item()


def test_clip_golden(golden):
    t, _ = golden
    W = t["clip.W"]
    ratios = [0.8, 0.85, 0.9, 0.95, 1.0]
    assert torch.equal(ref.scales_int4_sym(W, ratios=ratios), t["clip.s4"])
    s, z = ref.scales_int4_asym(W, ratios=ratios)
    assert torch.equal(s, t["clip.s4a"]) and torch.equal(z, t["clip.z4a"])
    assert torch.equal(ref.scales_int8_sym(W, ratios=ratios), t["clip.s8"])
    s, z = ref.scales_int8_asym(W, ratios=ratios)
    assert torch.equal(s, t["clip.s8a"]) and torch.equal(z, t["clip.z8a"])


# ---------------------------------------------------------------- packing

def test_pack_kat():
    v = torch.tensor([-8, 7, 0, -1, 1, 2, 3], dtype=torch.int8)
    p = ref.pack_int4(v)
    # low nibble = even index; -8 -> 0x8, 7 -> 0x7; -1 -> 0xF; odd tail padded with 0
    assert p.tolist() == [0x78, 0xF0, 0x21, 0x03]
    assert torch.equal(ref.unpack_int4(p, 7), v)


def test_pack_roundtrip_all_pairs():
    a = torch.arange(-8, 8, dtype=torch.int8)
    v = torch.stack(torch.meshgrid(a, a, indexing="ij"), -1).reshape(-1, 2)
    p = ref.pack_int4(v)
    assert p.shape == (256, 1) and len(set(p.flatten().tolist())) == 256
    assert torch.equal(ref.unpack_int4(p, 2), v)


# ---------------------------------------------------------------- Hessian inverse

def test_prepare_hinv_is_inverse():
    H = lognormal_hessian(64, 128, 1)
    Hi = ref.prepare_hinv(H, 0.01)
    Hd = ref.damp(H, 0.01).double()
    assert torch.allclose(Hd @ Hi.double(), torch.eye(64, dtype=torch.float64), atol=1e-3)


def test_invert_singular_uses_pinv():
    H = torch.zeros(8, 8)
    H[0, 0] = 1.0
    with pytest.warns(UserWarning):
        Hi = ref.invert_hessian(H)
    assert torch.allclose(H @ Hi @ H, H, atol=1e-5)


# ---------------------------------------------------------------- GPTQ sweep

def _np_gptq_sweep(W, Hinv, s, z, B, qmin, qmax):
    """Element-by-element float32 restatement of the sweep (independent)."""
    W = W.astype(f32).copy()
    M, N = W.shape
    Q = np.zeros((M, N), dtype=np.int8)
    for b0 in range(0, N, B):
        b1 = min(b0 + B, N)
        E = np.zeros((M, b1 - b0), dtype=f32)
        for j in range(b0, b1):
            for r in range(M):
                w = W[r, j]
                raw = f32(w / s[r])
                if z is not None:
                    raw = f32(raw + f32(z[r]))
                q = f32(max(qmin, min(qmax, np_rhaz(raw))))
                deq = f32(f32(q - f32(z[r])) * s[r]) if z is not None else f32(q * s[r])
                e = f32(f32(w - deq) / Hinv[j, j])
                e = f32(0.0) if np.isnan(e) else f32(min(100.0, max(-100.0, e)))
                Q[r, j] = int(q)
                E[r, j - b0] = e
                for k in range(j + 1, b1):
                    W[r, k] = f32(W[r, k] - f32(e * Hinv[j, k]))
        if b1 < N:
            W[:, b1:] = (W[:, b1:].astype(np.float64) - E.astype(np.float64) @ Hinv[b0:b1, b1:].astype(np.float64)).astype(f32)
    return Q


@pytest.mark.parametrize("asym", [False, True])
def test_gptq_sweep_single_block_bit_exact(asym):
    g = torch.Generator().manual_seed(5)
    M, N = 6, 24
    W = torch.randn(M, N, generator=g)
    Hinv = ref.prepare_hinv(lognormal_hessian(N, 64, 2), 0.01)
    s, z = ref.gptq_row_params(W, 4, False)
    if not asym:
        z = None
    Q = torch.zeros(M, N, dtype=torch.int8)
    ref.gptq_block(W.clone(), Q, s, Hinv, 0, N, N, -8, 7, z)
    Qn = _np_gptq_sweep(W.numpy(), Hinv.numpy(), s.squeeze(1).numpy(),
                        None if z is None else z.squeeze(1).numpy().astype(f32), N, -8, 7)
    assert np.array_equal(Q.numpy(), Qn)


def test_gptq_sweep_multi_block_close():
    g = torch.Generator().manual_seed(6)
    M, N = 8, 48
    W = torch.randn(M, N, generator=g)
    Hinv = ref.prepare_hinv(lognormal_hessian(N, 96, 3), 0.01)
    s, z = ref.gptq_row_params(W, 4, False)
    Q = torch.zeros(M, N, dtype=torch.int8)
    ref.gptq_block(W.clone(), Q, s, Hinv, 0, N, 16, -8, 7, z)
    Qn = _np_gptq_sweep(W.numpy(), Hinv.numpy(), s.squeeze(1).numpy(), z.squeeze(1).numpy().astype(f32), 16, -8, 7)
    assert (Q.numpy() != Qn).mean() < 0.02


@pytest.mark.parametrize("case", ["gptq_a", "gptq_b", "gptq_c", "gptq_d", "gptq_e", "gptq_f", "gptq3d"])
def test_gptq_golden(golden, one_thread, case):
    t, meta = golden
    m = meta[case]
    r = ref.gptq_quantize_layer(t[f"{case}.W"], t[f"{case}.H"], block_size=m["block"], damping=0.01,
                                int_bits=m["bits"], asymmetric=m["asym"], hessian_method=m["method"])
    assert torch.equal(r.quantized_W, t[f"{case}.q"])
    assert torch.equal(r.scales, t[f"{case}.scales"])
    if f"{case}.zp" in t:
        assert torch.equal(r.zero_points, t[f"{case}.zp"])
    assert r.mse == pytest.approx(m["mse"], rel=1e-12)


# ---------------------------------------------------------------- LDLQ / greedy

@pytest.mark.parametrize("case", ["ldlq_a", "ldlq_b", "ldlq_c", "ldlq_d", "ldlq_e"])
def test_ldlq_golden(golden, one_thread, case):
    t, meta = golden
    m = meta[case]
    r = ref.ldlq_quantize_layer(t[f"{case}.W"], hessian=t.get(f"{case}.H"), block_size=m["block"],
                                damping=0.01, int_bits=m["bits"], iterations=m["iters"],
                                greedy_passes=m["greedy"])
    assert torch.equal(r.quantized_W, t[f"{case}.q"])
    assert torch.equal(r.scales, t[f"{case}.scales"])
    assert r.mse == pytest.approx(m["mse"], rel=1e-12)


def test_greedy_coordinatewise_optimal():
    """After a pass, no single-coordinate change lowers tr(dW H dW^T) for the
    last column visited (brute force over the 16 INT4 values)."""
    g = torch.Generator().manual_seed(9)
    M, N = 5, 12
    W = torch.randn(M, N, generator=g, dtype=torch.float32)
    H = lognormal_hessian(N, 40, 4)
    S = torch.full((M, N), 0.3)
    Q0 = ref.rhaz(W / S).clamp(-8, 7)
    Q = ref.greedy_pytorch(W, Q0.clone(), S, H, 1, -8, 7).float()

    def proxy(Qm):
        d = (Qm * S - W).double()
        return (d @ H.double() * d).sum().item()

    base = proxy(Q)
    assert base <= proxy(Q0) + 1e-9
    j = N - 1
    for r in range(M):
        for v in range(-8, 8):
            Qt = Q.clone()
            Qt[r, j] = v
            assert proxy(Qt) >= base - 1e-6 * abs(base)


# --------------------------------------------------------------------------
# Low-rank greedy (converter/greedy.py:99-199, 293-479) and the GPU dispatch
# --------------------------------------------------------------------------

def _planted(n, evals, seed):
    g = torch.Generator().manual_seed(seed)
    V, _ = torch.linalg.qr(torch.randn(n, n, generator=g, dtype=torch.float64))
    return ((V * torch.as_tensor(evals, dtype=torch.float64)) @ V.T).float(), V


def test_lowrank_decompose_planted_spectrum():
    """Known spectrum: the count of eigenvalues above threshold x max, both
    refusal gates, and the eigen-equation for the returned pairs."""
    n = 100
    ev = torch.cat([torch.linspace(10.0, 0.2, 25), torch.full((75,), 0.05)])
    H, _ = _planted(n, ev, 1)
    s_k, U_k, k, used = ref.lowrank_decompose(H, 0.01)
    assert used and k == 25
    assert torch.allclose(s_k, ev[:25], rtol=1e-4)
    r = H @ U_k - U_k * s_k
    assert r.abs().max() < 1e-4 * 10.0
    # threshold above the 0.05 floor but k > 0.3 N once the floor counts
    _, _, k2, used2 = ref.lowrank_decompose(H, 0.004)
    assert k2 == 64 and not used2   # reported within svd_lowrank's q = 64 values
    # LOWRANK_MAX_K gate (k <= 0.3 N but > 512 needs N > 1706: check the rule directly)
    assert ref.LOWRANK_MAX_K == 512
    # near-zero matrix
    _, _, k3, used3 = ref.lowrank_decompose(torch.zeros(8, 8), 0.01)
    assert k3 == 0 and not used3


def test_greedy_lowrank_loop_full_basis_is_exact_greedy():
    """With every eigenpair (k = N) the low-rank cross term is the exact one,
    so one pass equals the reference's PyTorch greedy."""
    g = torch.Generator().manual_seed(3)
    M, N = 24, 80
    W = torch.randn(M, N, generator=g) * 0.02
    H = lognormal_hessian(N, 200, 5).double()
    ev, V = torch.linalg.eigh(H)
    H = H.float()
    S = (W.abs().amax(dim=1, keepdim=True) / 7).expand(M, N).contiguous()
    Q0 = ref.rhaz(W / S).clamp(-8, 7)
    a = ref.greedy_lowrank_loop(W, Q0.clone(), S, H, ev.float(), V.float(), 1, -8, 7)
    b = ref.greedy_pytorch(W, Q0.clone(), S, H, 1, -8, 7)
    assert (a == b).float().mean().item() >= 0.995


@pytest.mark.parametrize("case", ["lr_a", "lr_b", "lr_c", "lr_d"])
def test_greedy_lowrank_loop_golden(golden_greedy_gpu, case):
    """Given the reference's own eigenpairs, the oracle's loop reproduces the
    reference's low-rank kernel bit for bit (codes, stall decisions)."""
    t, meta = golden_greedy_gpu
    m = meta[case]
    qmin, qmax = (-128, 127) if m["bits"] == 8 else (-8, 7)
    W, H, Q0, s = t[f"{case}.W"], t[f"{case}.H"], t[f"{case}.q0"], t[f"{case}.s"]
    M, N = W.shape
    q = ref.greedy_lowrank_loop(W, Q0.float(), s.expand(M, N), H, t[f"{case}.s_k"], t[f"{case}.U_k"],
                                m["passes"], qmin, qmax)
    assert torch.equal(q, t[f"{case}.q"])


@pytest.mark.parametrize("case", ["lr_a", "lr_b", "lr_c", "lr_d", "fr_a"])
def test_greedy_gpu_golden(golden_greedy_gpu, case):
    """The oracle's GPU dispatch against the reference's low-rank kernel and
    full-rank v2 path: same rank decision and k, the same truncated Hessian
    U_k diag(s_k) U_k^T up to fp32 noise, codes agree.  The reference's
    svd_lowrank basis and eigh's differ by ~1e-6 relative, which the greedy
    feedback turns into up to ~0.2 % of flipped codes (lr_b)."""
    t, meta = golden_greedy_gpu
    m = meta[case]
    qmin, qmax = (-128, 127) if m["bits"] == 8 else (-8, 7)
    W, H, Q0, s = t[f"{case}.W"], t[f"{case}.H"], t[f"{case}.q0"], t[f"{case}.s"]
    M, N = W.shape
    q, k, used = ref.greedy_gpu(W, Q0.float(), s.expand(M, N), H, m["passes"], qmin, qmax)
    assert k == m["k"] and used == m["lowrank"]
    agree = (q == t[f"{case}.q"]).float().mean().item()
    assert agree >= 0.998, agree
    if used:
        s_k, U_k, _, _ = ref.lowrank_decompose(H)
        Hk = (U_k * s_k) @ U_k.T
        Hg = (t[f"{case}.U_k"] * t[f"{case}.s_k"]) @ t[f"{case}.U_k"].T
        assert ((Hk - Hg).norm() / Hg.norm()).item() < 1e-5


# ---------------------------------------------------------------- PermuQuant

def test_permuquant_moments_kat():
    # reference tests/unit/test_permuquant_channel.py: formula, ones, zeros
    W = torch.tensor([[2.0, -1.0], [0.0, 3.0]])
    assert torch.equal(ref.channel_second_moments(W), torch.tensor([2.0, 5.0]))
    assert torch.equal(ref.channel_second_moments(torch.ones(8, 16)), torch.ones(16))
    assert torch.equal(ref.channel_second_moments(torch.zeros(8, 16)), torch.zeros(16))


def test_permuquant_permutation_properties():
    g = torch.Generator().manual_seed(42)
    W = torch.randn(16, 64, generator=g)
    W[:, 0] *= 100.0
    p = ref.permutation_weight(W)
    assert sorted(p.tolist()) == list(range(64)) and p[0].item() == 0
    mu = ref.channel_second_moments(W)[p]
    assert (mu[:-1] >= mu[1:]).all()
    # brute force: the order of the moments, no ties in random data
    mu2 = ref.channel_second_moments(W)
    assert p.tolist() == sorted(range(64), key=lambda i: -mu2[i].item())
    act = torch.rand(64, generator=g)
    assert torch.equal(ref.permutation_joint(W, act, 0.0), p)
    assert torch.equal(ref.permutation_joint(W, act, 1.0), act.argsort(descending=True))


def test_permuquant_per_row_error_is_permutation_invariant():
    # per-row scales: the squared errors of W[:, perm] are those of W permuted,
    # so exact sums agree and only fp32 rounding separates the two totals
    g = torch.Generator().manual_seed(7)
    W = torch.randn(32, 256, generator=g) * 0.02
    perm = torch.randperm(256, generator=g)
    for bits in (4, 8):
        def errs(X):
            if bits == 8:
                s = ref.scales_int8_sym(X)
                d = ref.quant_int8_sym(X, s).float() * s.float()
            else:
                s = ref.scales_int4_sym(X, X.shape[1])
                d = ref.quant_int4_sym(X, s, X.shape[1]).float() * s.float()
            return ((X - d) ** 2)
        e0, e1 = errs(W), errs(W[:, perm])
        assert torch.equal(e0[:, perm], e1)
        assert e0.double().sum().item() == pytest.approx(e1.double().sum().item(), rel=1e-12)
        a = ref.group_quant_error(W, 256, bits)
        assert a == pytest.approx(e0.double().sum().item(), rel=1e-5)


def test_permuquant_acceptance_rules():
    # zero matrix: error 0 -> never accepted (reference test_zero_weight_matrix)
    _, acc = ref.permutation_with_acceptance(torch.zeros(8, 64), tau=0.0, group_size=64, int_bits=4)
    assert acc is False
    # group scales (group 16 < row): accepted exactly when the reordered
    # error is smaller (tau = 0), and a high tau rejects (reference
    # test_tau_high_rejects_most); channel magnitudes log-normal
    seen = set()
    for seed in range(6):
        g = torch.Generator().manual_seed(seed)
        W = torch.randn(16, 128, generator=g) * torch.exp(torch.randn(128, generator=g) * 1.5) * 0.01
        perm, acc = ref.permutation_with_acceptance(W, tau=0.0, group_size=16, int_bits=4)
        e0, e1 = ref.group_quant_error(W, 16, 4), ref.group_quant_error(W[:, perm], 16, 4)
        assert acc == (e1 < e0)
        seen.add(acc)
        assert ref.permutation_with_acceptance(W, tau=0.99, group_size=16, int_bits=4)[1] is False
    assert seen == {True, False}
    g = torch.Generator().manual_seed(4)
    W = torch.randn(16, 128, generator=g) * torch.exp(torch.randn(128, generator=g) * 1.5) * 0.01
    perm, acc = ref.permutation_with_acceptance(W, tau=0.0, group_size=16, int_bits=4)
    with pytest.raises(ValueError):
        ref.sweep_alpha(torch.randn(8, 64), num_alpha=0)
    p, a, acc = ref.sweep_alpha(W, None, 16, 0.0, 11, 4)
    assert a == 0.0 and acc is True and torch.equal(p, perm)


# ---------------------------------------------------------------- DLR Hessians

def _dlr(n, r, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.rand(n, generator=g) + 0.1, torch.randn(n, r, generator=g) * 0.3


@pytest.mark.parametrize("damping", [0.0, 0.01, 0.3])
def test_woodbury_matches_fp64_inverse(damping):
    # the definition of the damped inverse (tests/unit/test_dlr_hessian.py:142-168)
    D, U = _dlr(48, 6, 1)
    H = torch.diag(D.double()) + U.double() @ U.double().T
    dm = (D.double() + (U.double() ** 2).sum(dim=1)).mean()
    want = torch.linalg.inv(H + damping * dm * torch.eye(48, dtype=torch.float64))
    got = ref.woodbury_inverse(D, U, damping).double()
    assert (got - want).abs().max().item() <= 1e-5 * want.abs().max().item()
    assert (H @ ref.woodbury_inverse(D, U).double() - torch.eye(48, dtype=torch.float64)).abs().max() < 1e-4
    assert torch.allclose(got, got.T, atol=1e-6)


def test_woodbury_special_cases():
    D, U = _dlr(16, 1, 2)
    # U = 0: diag(1/D)
    assert torch.allclose(ref.woodbury_inverse(D, torch.zeros(16, 1)), torch.diag(1.0 / D), atol=1e-6)
    # rank one: Sherman-Morrison's closed form
    Du = U.squeeze(1) / D
    sm = torch.diag(1.0 / D) - torch.outer(Du, Du) / (1 + (U.squeeze(1) * Du).sum())
    assert torch.allclose(ref.woodbury_inverse(D, U), sm, atol=1e-6)
    # a zero diagonal entry is floored, not a division by zero
    D2 = D.clone()
    D2[0] = 0.0
    assert torch.isfinite(ref.woodbury_inverse(D2, torch.randn(16, 4) * 0.3, 0.01)).all()
    # the damping base is floored at 1e-6 (all-zero factors)
    got = ref.woodbury_inverse(torch.zeros(8), torch.zeros(8, 2), 0.5)
    assert torch.allclose(torch.diag(got), torch.full((8,), 1.0 / (0.5 * 1e-6)), rtol=1e-6)


def test_dlr_dense_and_permutation():
    D, U = _dlr(20, 3, 3)
    H = ref.dlr_to_dense(D, U)
    assert torch.allclose(H.double(), torch.diag(D.double()) + U.double() @ U.double().T, atol=1e-6)
    perm = torch.randperm(20, generator=torch.Generator().manual_seed(4))
    assert torch.allclose(ref.dlr_to_dense(D[perm], U[perm]), H[perm][:, perm], atol=1e-6)


def test_gptq_dlr_uses_woodbury_inverse(one_thread):
    # the DLR branch is the 2-D column loop on the Woodbury inverse itself
    D, U = _dlr(64, 8, 5)
    W = torch.randn(16, 64, generator=torch.Generator().manual_seed(6))
    r = ref.gptq_quantize_layer(W, {"format": "dlr", "D": D, "U": U}, damping=0.01)
    s, z = ref.gptq_row_params(W, 4, False)
    Q = torch.zeros(16, 64, dtype=torch.int8)
    ref.gptq_block(W.clone(), Q, s, ref.woodbury_inverse(D, U, 0.01), 0, 64, 128, -8, 7, z)
    assert torch.equal(r.quantized_W, Q)
    with pytest.raises(ValueError, match="dim.*in_features"):
        ref.gptq_quantize_layer(W[:, :32], {"format": "dlr", "D": D, "U": U})
    with pytest.raises(ValueError):
        ref.ldlq_quantize_layer(W, {"format": "dlr", "D": D, "U": U}, greedy_passes=1)


# ---------------------------------------------------------------- PiSO

def _piso_cost64(w, h, s, zp, qmin, qmax):
    """fp64 error of one candidate; q from the fp32 quotient (numpy)."""
    w32, s32 = w.astype(np.float32), np.float32(s)
    t = (w32 / s32).astype(np.float32)
    if zp is not None:
        t = (t + np.float32(zp)).astype(np.float32)
    q = np.where(t >= 0, np.floor(t + np.float32(0.5)), np.ceil(t - np.float32(0.5))).clip(qmin, qmax)
    dq = (q - (zp or 0.0)) * float(s32)
    return float(((w.astype(np.float64) - dq) ** 2 * h.astype(np.float64)).sum())


@pytest.mark.parametrize("asym,bits", [(False, 8), (False, 4), (True, 8), (True, 4)])
def test_piso_choices_are_fp64_optimal(asym, bits):
    # brute force: every stage's pick is within fp32 noise of that stage's fp64 minimum
    g = torch.Generator().manual_seed(bits + 10 * asym)
    W = torch.randn(12, 200, generator=g) * torch.exp(torch.randn(200, generator=g) * 0.5)
    h = torch.rand(200, generator=g) + 0.01
    qmin, qmax = (-128, 127) if bits == 8 else (-8, 7)
    nc, nf = 24, 6
    lo, hi = (0.8, 1.2) if (asym and bits == 8) else (0.5, 2.0)
    if asym:
        S, Z = ref.piso_scales_asym(W, h, nc, nf, qmin, qmax, lo, hi)
    else:
        S, Z = ref.piso_scales_sym(W, h, nc, nf, qmin, qmax, float(qmax)), None
    # the factor tables are the reference's torch.linspace constants
    cf = torch.linspace(lo, hi, nc, dtype=torch.float32).numpy()
    ff = torch.linspace(0.95, 1.05, nf, dtype=torch.float32).numpy()
    for r in range(W.shape[0]):
        w, hv = W[r].numpy(), h.numpy()
        sref = np.float32((w.max() - w.min()) / np.float32(qmax - qmin)) if asym else \
            np.float32(np.abs(w).max() / np.float32(qmax))

        def zp_of(s):
            z = np.float32(qmin) - np.float32(np.float32(w.min()) / np.float32(s))
            return float(np.clip(np.floor(z + 0.5) if z >= 0 else np.ceil(z - 0.5), qmin, qmax)) if asym else None

        cs = [np.float32(max(sref * f, 1e-10) if asym else sref * f) for f in cf]
        cc = [_piso_cost64(w, hv, s, zp_of(s), qmin, qmax) for s in cs]
        # the final scale is base * fine factor for a base whose coarse cost is near-minimal
        fs = None
        for ci in np.argsort(cc):
            if cc[ci] > min(cc) * (1 + 1e-5) + 1e-30:
                break
            cand = [np.float32(max(cs[ci] * f, 1e-10) if asym else cs[ci] * f) for f in ff]
            if np.float32(S[r, 0].item()) in cand:
                fs = cand
                break
        assert fs is not None, r
        fc = [_piso_cost64(w, hv, s, zp_of(s), qmin, qmax) for s in fs]
        k = fs.index(np.float32(S[r, 0].item()))
        assert fc[k] <= min(fc) * (1 + 1e-5) + 1e-30
        if asym:
            assert Z[r, 0].item() == zp_of(fs[k])


def test_piso_closed_forms_and_reference_behaviour():
    # all-zero rows: every cost is 0, the first candidate of each stage wins
    s = ref.piso_scales_sym(torch.zeros(2, 64), torch.ones(64), 16, 4, -128, 127, 127.0)
    assert s[0, 0].item() == np.float32(np.float32(np.float32(1e-10) * np.float32(0.5)) * np.float32(0.95))
    s, z = ref.piso_scales_asym(torch.zeros(2, 64), torch.ones(64), 16, 4, -8, 7, 0.5, 2.0)
    assert s[0, 0].item() == np.float32(1e-10) and z[0, 0].item() == -8
    # tests/gpu/test_piso_triton.py:133-148: scale ~ |w|max / 127 for large weights
    g = torch.Generator().manual_seed(99)
    W = torch.randn(16, 256, generator=g) * 100.0
    s = ref.piso_scales_sym(W, torch.ones(256), 16, 4, -128, 127, 127.0)
    assert s.shape == (16, 1) and s.min() > 0.1 and s.max() < 10.0
    s, z = ref.piso_scales_asym(W, torch.rand(256, generator=g) + 1e-6, 16, 4, -128, 127, 0.8, 1.2)
    assert (s > 0).all() and z.dtype == torch.int8 and z.min() >= -128 and z.max() <= 127
