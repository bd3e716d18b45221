"""GPU tier: the bfloat16 forward (forward_bf16) against the CPU oracle.

The oracle runs fp32 math on the bf16-rounded inputs (oracle.bf16_cast, pinned
against torch's conversion). Tolerances, written out:
* O: |O - O_ref| <= 1e-2 + half a bf16 ulp of O_ref. P is rounded to bf16
  (8 significand bits) before the PV product, so a row dominated by one key
  carries up to 2^-9 |V| of error there, and the bf16 output rounding adds
  half an ulp (2^-9 |O| at most);
* L: relative error <= 1e-4 against max(|L_ref|, 1) (L comes from the fp32
  scores and fp32 row sums, as in the fp16 path);
* O-only bitwise equal to forward's O.
"""
import numpy as np
import pytest
import torch

from oracle import bf16_cast, naive_attention, naive_attention_backward

pytestmark = pytest.mark.gpu


def bf16_half_ulp(x):
    e = np.floor(np.log2(np.maximum(np.abs(np.asarray(x, np.float64)), 2.0 ** -126)))
    return 2.0 ** (e - 8)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("B,H,Hkv,N,causal", [
    (1, 1, 1, 1, False), (1, 2, 2, 63, True), (2, 4, 4, 256, False), (1, 8, 2, 1000, True),
    (1, 8, 8, 4096, False),
])
def test_bf16_forward(fa, dev, D, B, H, Hkv, N, causal):
    rng = np.random.default_rng(N + D + H)
    Q = rng.standard_normal((B, H, N, D)).astype(np.float32)
    K = rng.standard_normal((B, Hkv, N, D)).astype(np.float32)
    V = rng.standard_normal((B, Hkv, N, D)).astype(np.float32)
    tq, tk, tv = (torch.from_numpy(x).to(dev) for x in (Q, K, V))
    O, L = fa.forward_bf16(tq, tk, tv, causal=causal)
    (O2,) = fa.forward_bf16(tq, tk, tv, causal=causal, want_L=False)
    torch.cuda.synchronize()
    assert O.dtype == torch.bfloat16 and L.dtype == torch.float32
    assert torch.equal(O, O2)
    g = H // Hkv
    Or, Lr = naive_attention(bf16_cast(Q), np.repeat(bf16_cast(K), g, axis=1),
                             np.repeat(bf16_cast(V), g, axis=1), causal=causal)
    Og = O.float().cpu().numpy()
    err = np.abs(Og - Or)
    bound = 1e-2 + bf16_half_ulp(Or)
    assert (err <= bound).all(), f"O err {err.max():.3e}"
    l_err = np.abs(L.cpu().numpy() - Lr) / np.maximum(np.abs(Lr), 1.0)
    assert l_err.max() <= 1e-4, f"L rel {l_err.max():.3e}"
    print(f"bf16 B{B} H{H} Hkv{Hkv} N{N} D{D} causal={causal}: O max err {err.max():.2e}, "
          f"L rel {l_err.max():.2e}")


def test_bf16_matches_fp16_path_closely(fa, dev):
    """Same inputs (exactly representable in both formats): the two paths agree."""
    rng = np.random.default_rng(3)
    # values with 8 significant bits are exact in bf16 and fp16
    X = [np.round(rng.standard_normal((1, 4, 512, 64)) * 16) / 16 for _ in range(3)]
    tq, tk, tv = (torch.from_numpy(x.astype(np.float32)).to(dev) for x in X)
    Ob, Lb = fa.forward_bf16(tq, tk, tv)
    Oh, Lh = fa.forward(tq, tk, tv)
    assert (Ob.float() - Oh.float()).abs().max().item() <= 2e-2
    assert ((Lb - Lh).abs() / Lh.abs().clamp(min=1)).max().item() <= 1e-5


# ---------------------------------------------------------------- backward
# backward_bf16 reads bf16 Q, K, V, O, dO and rounds P and dS to bf16 before
# their MFMA products (8 significand bits against fp16's 11), so the fp16
# path's bound |g - g_ref| <= 5e-3 + 5e-3 |g_ref| grows by 2^3:
BWD_ATOL = BWD_RTOL = 4e-2


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("B,H,Hkv,N,causal", [
    (1, 1, 1, 1, False), (1, 2, 2, 63, True), (2, 4, 4, 256, False), (1, 8, 2, 333, True),
    (1, 4, 4, 1024, False),
])
def test_bf16_backward(fa, dev, D, B, H, Hkv, N, causal):
    rng = np.random.default_rng(7 * N + D + H)
    Q = rng.standard_normal((B, H, N, D)).astype(np.float32)
    K = rng.standard_normal((B, Hkv, N, D)).astype(np.float32)
    V = rng.standard_normal((B, Hkv, N, D)).astype(np.float32)
    G = rng.standard_normal((B, H, N, D)).astype(np.float32)
    tq, tk, tv, tg = (torch.from_numpy(x).to(dev) for x in (Q, K, V, G))
    O, L = fa.forward_bf16(tq, tk, tv, causal=causal)
    dQ, dK, dV = fa.backward_bf16(tq, tk, tv, O, tg, L, causal=causal)
    torch.cuda.synchronize()
    assert dQ.shape == (B, H, N, D) and dK.shape == (B, Hkv, N, D) and dV.shape == dK.shape
    g = H // Hkv
    rQ, rK, rV = naive_attention_backward(bf16_cast(Q), np.repeat(bf16_cast(K), g, axis=1),
                                          np.repeat(bf16_cast(V), g, axis=1), bf16_cast(G),
                                          causal)
    rK = rK.reshape(B, Hkv, g, N, D).sum(axis=2)
    rV = rV.reshape(B, Hkv, g, N, D).sum(axis=2)
    errs = []
    for name, t, r in (("dQ", dQ, rQ), ("dK", dK, rK), ("dV", dV, rV)):
        x = t.cpu().numpy()
        assert np.isfinite(x).all(), name
        err = np.abs(x - r)
        # a KV head's gradient sums g query heads' terms
        atol = BWD_ATOL * (g if name != "dQ" else 1)
        assert (err <= atol + BWD_RTOL * np.abs(r)).all(), f"{name} max err {err.max():.3e}"
        errs.append(err.max())
    print(f"bf16 bwd B{B} H{H} Hkv{Hkv} N{N} D{D} causal={causal}: "
          f"dQ/dK/dV max err {errs[0]:.2e} {errs[1]:.2e} {errs[2]:.2e}")


def test_bf16_backward_identities_headline(fa, dev):
    """B1 H8 N4096 D64: sum_j dV_j = sum_i dO_i and sum_j dK_j = 0 per head."""
    B, H, N, D = 1, 8, 4096, 64
    g = torch.Generator(device=dev).manual_seed(5)
    Q, K, V, G = (torch.randn(B, H, N, D, device=dev, generator=g).bfloat16() for _ in range(4))
    O, L = fa.forward_bf16(Q, K, V)
    dQ, dK, dV = fa.backward_bf16(Q, K, V, O, G, L)
    scale = N ** 0.5
    assert (dV.sum(dim=2) - G.float().sum(dim=2)).abs().max().item() <= 2e-2 * scale
    assert dK.sum(dim=2).abs().max().item() <= 2e-2 * scale


def test_bf16_backward_matches_fp16_path_closely(fa, dev):
    """Inputs exact in both formats: the bf16 and fp16 gradients agree."""
    rng = np.random.default_rng(4)
    X = [np.round(rng.standard_normal((1, 2, 384, 64)) * 16) / 16 for _ in range(4)]
    tq, tk, tv, tg = (torch.from_numpy(x.astype(np.float32)).to(dev) for x in X)
    Ob, Lb = fa.forward_bf16(tq, tk, tv, causal=True)
    Oh, Lh = fa.forward(tq, tk, tv, causal=True)
    gb = fa.backward_bf16(tq, tk, tv, Ob, tg, Lb, causal=True)
    gh = fa.backward(tq, tk, tv, Oh, tg, Lh, causal=True)
    for a, b in zip(gb, gh):
        assert (a - b).abs().max().item() <= 4e-2
