"""GPU tier: backward parity against the CPU oracle (oracle/naive.py).

Mirrors the reference's backward test (tests/test_backward.py:48-121): the
same config list, Q/K/V/dO drawn from randn, O and L from the forward, and
the reference's tolerance torch.allclose(atol=1e-2, rtol=1e-2) on dQ, dK and
dV (:70-76) against the naive backward, with the max errors printed (:81-82).
Extras: D = 128, causal, ragged N, N = 1, determinism, the headline shape
(two heads checked against the oracle) and size-independent identities.

Two oracles are compared:
* the reference's exact check: naive backward in fp32 on the raw fp32
  inputs (tests/test_backward.py:64), at atol = rtol = 1e-2;
* the tighter one: naive backward in fp32 on the fp16-rounded inputs the
  kernels actually read, at |g - g_ref| <= 5e-3 + 5e-3 |g_ref| (the
  remaining error is the fp16 rounding of P and dS before their products
  and of the forward's O in D_i).
"""
import numpy as np
import pytest
import torch

from oracle import half_cast, make_ragged_inputs, naive_attention_backward

pytestmark = pytest.mark.gpu

REF_ATOL = REF_RTOL = 1e-2     # tests/test_backward.py:70-71
TIGHT_ATOL = TIGHT_RTOL = 5e-3


def _randn(B, H, N, D, seed):
    rng = np.random.default_rng(seed)
    return [rng.standard_normal((B, H, N, D)).astype(np.float32) for _ in range(4)]


def _grads(fa, dev, Q, K, V, G, causal):
    tq, tk, tv, tg = (torch.from_numpy(np.ascontiguousarray(x)).to(dev) for x in (Q, K, V, G))
    O, L = fa.forward(tq, tk, tv, causal=causal)
    dQ, dK, dV = fa.backward(tq, tk, tv, O, tg, L, causal=causal)
    torch.cuda.synchronize()
    for t in (dQ, dK, dV):
        assert t.dtype == torch.float32 and t.shape == tuple(Q.shape)
    return [t.cpu().numpy() for t in (dQ, dK, dV)]


def _compare(got, ref, atol, rtol, tag):
    msgs = []
    for name, g, r in zip(("dQ", "dK", "dV"), got, ref):
        assert np.isfinite(g).all(), f"{tag} {name} not finite"
        err = np.abs(g - r)
        if not (err <= atol + rtol * np.abs(r)).all():
            msgs.append(f"{name} max_diff={err.max():.3e}")
    assert not msgs, f"{tag}: " + ", ".join(msgs)
    return [float(np.abs(g - r).max()) for g, r in zip(got, ref)]


def _run(fa, dev, B, H, N, D, causal=False, seed=42, reference_check=True):
    Q, K, V, G = _randn(B, H, N, D, seed)
    got = _grads(fa, dev, Q, K, V, G, causal)
    tag = f"B{B} H{H} N{N} D{D} causal={causal}"
    tight = naive_attention_backward(half_cast(Q), half_cast(K), half_cast(V), half_cast(G),
                                     causal)
    diffs = _compare(got, tight, TIGHT_ATOL, TIGHT_RTOL, tag + " (fp16 inputs)")
    if reference_check:
        ref = naive_attention_backward(Q, K, V, G, causal)
        _compare(got, ref, REF_ATOL, REF_RTOL, tag + " (reference check)")
    print(f"{tag}  dQ_diff={diffs[0]:.3e}  dK_diff={diffs[1]:.3e}  dV_diff={diffs[2]:.3e}")
    return got


# tests/test_backward.py:92-102
REFERENCE_CONFIGS = [
    (1, 1, 32, 64), (1, 1, 64, 64), (1, 1, 128, 64), (1, 1, 63, 64), (1, 1, 127, 64),
    (2, 4, 256, 64), (2, 8, 512, 64), (1, 1, 1024, 64), (1, 1, 2048, 64),
]


@pytest.mark.parametrize("B,H,N,D", REFERENCE_CONFIGS)
def test_reference_configs(fa, dev, B, H, N, D):
    _run(fa, dev, B, H, N, D)


@pytest.mark.parametrize("B,H,N,D", [
    (1, 1, 1, 64), (1, 1, 1, 128), (1, 1, 32, 128), (1, 1, 127, 128), (2, 2, 200, 128),
    (1, 2, 513, 128), (1, 1, 1024, 128), (3, 1, 65, 64), (1, 3, 129, 64),
])
def test_noncausal_extra_shapes(fa, dev, B, H, N, D):
    _run(fa, dev, B, H, N, D)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("N", [1, 17, 64, 127, 128, 300, 1024])
def test_causal(fa, dev, N, D):
    _run(fa, dev, 1, 2, N, D, causal=True, seed=N + D)


@pytest.mark.parametrize("D", [64, 128])
def test_ragged_lengths(fa, dev, D):
    """One below, at and above the 64-query and 128-key tile edges."""
    for N in (31, 33, 63, 65, 127, 129, 191, 255, 257, 383):
        _run(fa, dev, 1, 1, N, D, causal=bool(N % 4 == 3), seed=N, reference_check=False)


@pytest.mark.parametrize("D", [64, 128])
def test_ragged_hot_rows(fa, dev, D):
    """The forward's config-4 inputs: ragged N and rows of Q/K at std 3.

    Hot rows make the softmax sharp and the gradients large (|dQ|, |dK| up to
    ~9, |dV| up to ~15 here), so the fp16 rounding of P, dS and O is larger in
    absolute terms: checked at the reference's own bound (atol = rtol = 1e-2).
    """
    N, Q, K, V = make_ragged_inputs(B=1, H=2, D=D, seed=7)
    G = np.random.default_rng(8).standard_normal(Q.shape).astype(np.float32)
    Q, K, V = (x.astype(np.float32) for x in (Q, K, V))
    for causal in (False, True):
        got = _grads(fa, dev, Q, K, V, G, causal)
        ref = naive_attention_backward(Q, K, V, half_cast(G), causal)
        d = _compare(got, ref, REF_ATOL, REF_RTOL, f"hot rows N{N} D{D} causal={causal}")
        print(f"hot rows N{N} D{D} causal={causal}  max diffs dQ/dK/dV {d}")


@pytest.mark.parametrize("D,causal", [(64, False), (64, True), (128, False), (128, True)])
def test_deterministic(fa, dev, D, causal):
    """Bitwise-repeatable gradients (no atomics, fixed reduction orders) from
    both ping-pong forms, over a ragged length and more units than CUs
    (B4 H8 N2100: 544 units per half)."""
    Q, K, V, G = _randn(4, 8, 2100, D, 5)
    a = _grads(fa, dev, Q, K, V, G, causal)
    b = _grads(fa, dev, Q, K, V, G, causal)
    for x, y in zip(a, b):
        assert np.array_equal(x, y), "backward must be bitwise reproducible (no atomics)"


def test_fp16_inputs_and_forward_outputs(fa, dev):
    """fp16 tensors in, O and L straight from forward(): no conversion happens."""
    Q, K, V, G = _randn(2, 2, 96, 64, 11)
    tq, tk, tv, tg = (torch.from_numpy(x).to(dev).half() for x in (Q, K, V, G))
    O, L = fa.forward(tq, tk, tv)
    dQ, dK, dV = fa.backward(tq, tk, tv, O, tg, L)
    ref = naive_attention_backward(half_cast(Q), half_cast(K), half_cast(V), half_cast(G))
    _compare([t.cpu().numpy() for t in (dQ, dK, dV)], ref, TIGHT_ATOL, TIGHT_RTOL, "fp16")


@pytest.mark.parametrize("D,causal", [(64, False), (64, True), (128, False), (128, True)])
def test_headline_shape(fa, dev, D, causal):
    """B1 H8 N4096: two heads against the oracle, every head through identities.

    Identities (exact in real arithmetic, size-independent):
      sum_j dV_j = sum_i dO_i        (rows of P sum to one)
      sum_j dK_j = 0                 (rows of dS sum to zero)
    """
    B, H, N = 1, 8, 4096
    Q, K, V, G = _randn(B, H, N, D, 2024 + D)
    got = _grads(fa, dev, Q, K, V, G, causal)
    for h in (0, H - 1):
        sl = slice(h, h + 1)
        ref = naive_attention_backward(half_cast(Q[:, sl]), half_cast(K[:, sl]),
                                       half_cast(V[:, sl]), half_cast(G[:, sl]), causal)
        _compare([g[:, sl] for g in got], ref, TIGHT_ATOL, TIGHT_RTOL, f"head {h}")
    dQ, dK, dV = got
    scale = np.sqrt(N)   # sums of N terms of O(1)
    np.testing.assert_allclose(dV.sum(axis=2), half_cast(G).sum(axis=2), atol=2e-3 * scale)
    np.testing.assert_allclose(dK.sum(axis=2), 0, atol=2e-3 * scale)


@pytest.mark.parametrize("causal", [True, False])
def test_d128_two_rounds(fa, dev, causal):
    """D = 128 with 512 units per half (B2 H8 N4096): the fused launch over
    more workgroups than one round of CUs, so units of both roles start as
    others finish. Two heads against the oracle, every head through the
    identities of test_headline_shape."""
    B, H, N, D = 2, 8, 4096, 128
    Q, K, V, G = _randn(B, H, N, D, 77)
    got = _grads(fa, dev, Q, K, V, G, causal)
    for b, h in ((0, 0), (B - 1, H - 1)):
        bs, hs = slice(b, b + 1), slice(h, h + 1)
        ref = naive_attention_backward(half_cast(Q[bs, hs]), half_cast(K[bs, hs]),
                                       half_cast(V[bs, hs]), half_cast(G[bs, hs]), causal)
        _compare([g[bs, hs] for g in got], ref, TIGHT_ATOL, TIGHT_RTOL, f"b{b} h{h}")
    dQ, dK, dV = got
    scale = np.sqrt(N)
    np.testing.assert_allclose(dV.sum(axis=2), half_cast(G).sum(axis=2), atol=2e-3 * scale)
    np.testing.assert_allclose(dK.sum(axis=2), 0, atol=2e-3 * scale)


def test_rejects_bad_arguments(fa, dev):
    x = torch.zeros(1, 1, 8, 64, device=dev)
    L = torch.zeros(1, 1, 8, device=dev)
    with pytest.raises(RuntimeError, match="Head dimension"):
        y = torch.zeros(1, 1, 8, 96, device=dev)
        fa.backward(y, y, y, y, y, L)
    with pytest.raises(RuntimeError, match="same shape"):
        fa.backward(x, x, x, x, torch.zeros(1, 1, 9, 64, device=dev), L)
    with pytest.raises(RuntimeError, match="B\\*H\\*N"):
        fa.backward(x, x, x, x, x, torch.zeros(1, 1, 7, device=dev))


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("H,Hkv,N,causal", [(8, 2, 256, False), (8, 1, 333, True), (6, 3, 129, False),
                                           (4, 2, 1024, True)])
def test_gqa_backward(fa, dev, D, H, Hkv, N, causal):
    """K/V of H_kv heads: dK, dV are the sums over each KV head's query heads of
    the oracle's gradients for the repeated K/V (no new arithmetic)."""
    B = 2
    rng = np.random.default_rng(H * 100 + Hkv + N + D)
    Q = rng.standard_normal((B, H, N, D)).astype(np.float32)
    K = rng.standard_normal((B, Hkv, N, D)).astype(np.float32)
    V = rng.standard_normal((B, Hkv, N, D)).astype(np.float32)
    G = rng.standard_normal((B, H, N, D)).astype(np.float32)
    tq, tk, tv, tg = (torch.from_numpy(x).to(dev) for x in (Q, K, V, G))
    O, L = fa.forward(tq, tk, tv, causal=causal)
    dQ, dK, dV = fa.backward(tq, tk, tv, O, tg, L, causal=causal)
    torch.cuda.synchronize()
    assert dK.shape == (B, Hkv, N, D) and dV.shape == (B, Hkv, N, D) and dQ.shape == (B, H, N, D)
    g = H // Hkv
    rQ, rK, rV = naive_attention_backward(half_cast(Q), np.repeat(half_cast(K), g, axis=1),
                                          np.repeat(half_cast(V), g, axis=1), half_cast(G), causal)
    rK = rK.reshape(B, Hkv, g, N, D).sum(axis=2)
    rV = rV.reshape(B, Hkv, g, N, D).sum(axis=2)
    # sums of g per-head gradients: the absolute budget grows with g
    _compare([t.cpu().numpy() for t in (dQ, dK, dV)], [rQ, rK, rV], TIGHT_ATOL * g, TIGHT_RTOL,
             f"GQA H{H} Hkv{Hkv} N{N} D{D} causal={causal}")
