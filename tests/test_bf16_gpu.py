"""GPU tier: the bfloat16 paths against the CPU oracle: forward (forward_bf16,
which picks its kernel from the shape as the fp16 forward does: the D = 64
cases run the 64-row kernel, the 128-row one at N = 4096 (and the 64-row one
again, causal there)),
backward (backward_bf16), paged decode and page writer (decode_paged and
kv_append with bf16 tensors).

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

from oracle import (append_pages, bf16_cast, decode_attention, naive_attention,
                    naive_attention_backward)

pytestmark = pytest.mark.gpu


def bf16_half_ulp(x):
    e = np.floor(np.log2(np.maximum(np.abs(np.asarray(x, np.float64)), 2.0 ** -126)))
    return 2.0 ** (e - 8)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("B,H,Hkv,N,causal", [
    (1, 1, 1, 1, False), (1, 2, 2, 63, True), (2, 4, 4, 256, False), (1, 8, 2, 1000, True),
    (1, 8, 8, 4096, False), (1, 8, 8, 4096, True),
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


# ---- paged decode and page writer with bf16 q and pools ----

def _pages(rng, B, ctx, Hkv, D, extra=2):
    """Page table (a permutation of the pool's pages) and fp32 pools."""
    pages = [(c + 15) // 16 for c in ctx]
    P = sum(pages) + extra
    perm = rng.permutation(P).astype(np.int32)
    table = np.zeros((B, max(max(pages), 1)), np.int32)
    off = 0
    for b in range(B):
        table[b, :pages[b]] = perm[off:off + pages[b]]
        off += pages[b]
    kp = rng.standard_normal((P, Hkv, 16, D)).astype(np.float32)
    vp = rng.standard_normal((P, Hkv, 16, D)).astype(np.float32)
    return table, kp, vp


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("Hkv", [4, 2, 1])
@pytest.mark.parametrize("S", [1, 3, 16])
def test_bf16_decode_vs_oracle(fa, dev, D, Hkv, S):
    """decode_paged with bf16 q and pools. The QK products of bf16 pairs are
    exact in fp32, and P enters the PV product as the sum of two bf16 values
    (about 16 significant bits) against exact bf16 V, so O's final rounding to
    bf16 dominates its distance from the fp32 oracle on the bf16-rounded
    inputs: |O - O_ref| <= 1e-3 + half a bf16 ulp of O_ref; L relative <= 1e-4."""
    B, H = 5, 4
    ctx = [1, 15, 16, 17, 300]
    rng = np.random.default_rng(D + 10 * Hkv + S)
    table, kp, vp = _pages(rng, B, ctx, Hkv, D)
    q = rng.standard_normal((B, H, D)).astype(np.float32)
    bf = lambda x: torch.from_numpy(x).to(dev).to(torch.bfloat16)
    tt = torch.from_numpy(table).to(dev)
    tc = torch.from_numpy(np.array(ctx, np.int32)).to(dev)
    O, L = fa.decode_paged(bf(q), bf(kp), bf(vp), tt, tc, num_splits=S)
    torch.cuda.synchronize()
    assert O.dtype == torch.bfloat16 and L.dtype == torch.float32
    g = H // Hkv
    Or, Lr = decode_attention(bf16_cast(q), np.repeat(bf16_cast(kp), g, axis=1),
                              np.repeat(bf16_cast(vp), g, axis=1), table, np.array(ctx))
    err = np.abs(O.float().cpu().numpy() - Or)
    assert (err <= 1e-3 + bf16_half_ulp(Or)).all(), f"O err {err.max():.3e}"
    l_err = np.abs(L.cpu().numpy() - Lr) / np.maximum(np.abs(Lr), 1.0)
    assert l_err.max() <= 1e-4, f"L rel {l_err.max():.3e}"


def test_bf16_decode_matches_fp16_decode(fa, dev):
    """Inputs with at most 7 significant bits are exact in both formats: the
    two decodes form the same fp32 products, so L agrees to fp32 accumulation
    rounding (relative 1e-5) and O to the bf16 output rounding."""
    B, H, D = 3, 8, 128
    ctx = [40, 513, 2000]
    rng = np.random.default_rng(21)
    table, kp, vp = _pages(rng, B, ctx, H, D)
    q = rng.standard_normal((B, H, D))
    q, kp, vp = (np.clip(np.round(x * 16), -63, 63).astype(np.float32) / 16 for x in (q, kp, vp))
    tt = torch.from_numpy(table).to(dev)
    tc = torch.from_numpy(np.array(ctx, np.int32)).to(dev)
    to = lambda x, dt: torch.from_numpy(x).to(dev).to(dt)
    Oh, Lh = fa.decode_paged(*(to(x, torch.float16) for x in (q, kp, vp)), tt, tc, num_splits=16)
    Ob, Lb = fa.decode_paged(*(to(x, torch.bfloat16) for x in (q, kp, vp)), tt, tc, num_splits=16)
    torch.cuda.synchronize()
    Lh, Lb = Lh.cpu().numpy(), Lb.cpu().numpy()
    assert (np.abs(Lh - Lb) / np.maximum(np.abs(Lh), 1.0)).max() <= 1e-5
    Oh, Ob = Oh.float().cpu().numpy(), Ob.float().cpu().numpy()
    assert (np.abs(Ob - Oh) <= 1e-3 + bf16_half_ulp(Oh)).all()


def test_bf16_kv_append_bit_exact(fa, dev):
    """bf16 rows land in bf16 pools bit for bit: the GPU pools, read as int16
    bit patterns, equal the oracle's append on the same bit patterns; then a
    decode over the appended pages matches the oracle."""
    B, H, T, D = 3, 4, 40, 128
    rng = np.random.default_rng(9)
    start = np.array([0, 5, 17], np.int32)
    max_pages = 4                                   # positions up to 56 < 64
    P = B * max_pages + 2
    table = rng.permutation(P)[:B * max_pages].astype(np.int32).reshape(B, max_pages)
    bf = lambda x: torch.from_numpy(x).to(dev).to(torch.bfloat16)
    tkp = bf(rng.standard_normal((P, H, 16, D)).astype(np.float32))
    tvp = bf(rng.standard_normal((P, H, 16, D)).astype(np.float32))
    tkn = bf(rng.standard_normal((B, H, T, D)).astype(np.float32))
    tvn = bf(rng.standard_normal((B, H, T, D)).astype(np.float32))
    bits = lambda t: t.view(torch.int16).cpu().numpy()
    want_k, want_v, want_bad = append_pages(bits(tkp), bits(tvp), table, start, bits(tkn),
                                            bits(tvn))
    tt = torch.from_numpy(table).to(dev)
    bad = fa.kv_append(tkn, tvn, tkp, tvp, tt, torch.from_numpy(start).to(dev))
    torch.cuda.synchronize()
    assert np.array_equal(bad.cpu().numpy(), want_bad)
    assert np.array_equal(bits(tkp), want_k) and np.array_equal(bits(tvp), want_v)
    ctx = start + T
    tq = bf(rng.standard_normal((B, H, D)).astype(np.float32))
    O, L = fa.decode_paged(tq, tkp, tvp, tt, torch.from_numpy(ctx).to(dev), num_splits=4)
    torch.cuda.synchronize()
    f32 = lambda t: t.float().cpu().numpy()
    Or, Lr = decode_attention(f32(tq), f32(tkp), f32(tvp), table, ctx)
    err = np.abs(f32(O) - Or)
    assert (err <= 1e-3 + bf16_half_ulp(Or)).all(), f"O err {err.max():.3e}"
    assert (np.abs(L.cpu().numpy() - Lr) / np.maximum(np.abs(Lr), 1.0)).max() <= 1e-4


def test_bf16_decode_rejects_mixed_dtypes(fa, dev):
    q = torch.zeros(1, 2, 64, device=dev, dtype=torch.bfloat16)
    kp = torch.zeros(1, 2, 16, 64, device=dev, dtype=torch.float16)
    tt = torch.zeros(1, 1, device=dev, dtype=torch.int32)
    tc = torch.ones(1, device=dev, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="all float16 or all bfloat16"):
        fa.decode_paged(q, kp, kp, tt, tc)
    with pytest.raises(RuntimeError, match="decode_partials takes float16"):
        fa.decode_partials(q, kp.bfloat16(), kp.bfloat16(), tt, tc)
    with pytest.raises(RuntimeError, match="all float16 or all bfloat16"):
        fa.kv_append(kp.bfloat16(), kp.bfloat16(), kp, kp, tt, torch.zeros(1, device=dev,
                                                                            dtype=torch.int32))
