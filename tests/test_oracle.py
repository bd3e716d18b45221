"""CPU tier: pin the oracle (oracle/naive.py) before trusting it as the checker.

Each oracle function is checked against something it does not share code
with: the float64 golden fixtures (explicit loops, tests/golden/make_golden.py),
a pure-Python brute force, closed forms and invariants. The mutation tests at
the end plant plausible mistakes in copies of the oracle and show that the
pinning checks catch each of them.
"""
import math
import pathlib

import numpy as np
import pytest

from oracle import naive as orc

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"


def _f64(x):
    return np.asarray(x, dtype=np.float64)


# ---------------------------------------------------------------- fixtures
@pytest.mark.parametrize("name", sorted(p.stem for p in GOLDEN.glob("fwd_*.npz")))
def test_oracle_matches_golden_fwd(name):
    z = np.load(GOLDEN / f"{name}.npz")
    q, k, v = z["q"][None], z["k"][None], z["v"][None]
    O, L = orc.naive_attention(orc.half_cast(q), orc.half_cast(k), orc.half_cast(v),
                               causal=bool(z["causal"]))
    vmax = float(np.abs(z["v"].astype(np.float32)).max())
    np.testing.assert_allclose(O[0], z["o"], atol=2e-6 * max(vmax, 1.0), rtol=0)
    np.testing.assert_allclose(L[0], z["l"], atol=2e-5, rtol=2e-6)
    O64, L64 = orc.naive_attention(q, k, v, causal=bool(z["causal"]), dtype=np.float64)
    np.testing.assert_allclose(O64[0], z["o"], atol=1e-12)
    np.testing.assert_allclose(L64[0], z["l"], atol=1e-12)


@pytest.mark.parametrize("name", sorted(p.stem for p in GOLDEN.glob("decode_*.npz")))
def test_oracle_matches_golden_decode(name):
    z = np.load(GOLDEN / f"{name}.npz")
    O, L = orc.decode_attention(z["q"], z["k_pool"], z["v_pool"], z["page_table"], z["ctx_lens"],
                                dtype=np.float64)
    np.testing.assert_allclose(O, z["o"], atol=1e-12)
    np.testing.assert_allclose(L, z["l"], atol=1e-12)
    for S in (1, 2, 3, 16):
        Os, Ls = orc.split_partials(z["q"], z["k_pool"], z["v_pool"], z["page_table"],
                                    z["ctx_lens"], S, dtype=np.float64)
        Oc, Lc = orc.lse_combine(Os, Ls)
        np.testing.assert_allclose(Oc, z["o"], atol=1e-12)
        np.testing.assert_allclose(Lc, z["l"], atol=1e-12)


def test_oracle_matches_golden_combine():
    z = np.load(GOLDEN / "combine_b2_s5.npz")
    O, L = orc.lse_combine(_f64(z["part_o"]), _f64(z["part_lse"]))
    np.testing.assert_allclose(O, z["o"], atol=1e-12)
    np.testing.assert_allclose(L, z["l"], atol=1e-12)


# ---------------------------------------------------------------- brute force
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("N,D", [(1, 8), (5, 16), (23, 64)])
def test_oracle_vs_bruteforce(N, D, causal):
    Q, K, V = orc.make_fwd_inputs(1, 2, N, D, seed=N + D)
    O, L = orc.naive_attention(orc.half_cast(Q), orc.half_cast(K), orc.half_cast(V), causal=causal)
    for h in range(2):
        Ob, Lb = orc.attention_bruteforce(_f64(Q[0, h]), _f64(K[0, h]), _f64(V[0, h]), causal)
        np.testing.assert_allclose(O[0, h], np.array(Ob), atol=2e-6)
        np.testing.assert_allclose(L[0, h], np.array(Lb), atol=2e-5)


# ---------------------------------------------------------------- closed forms
def test_closed_form_single_key():
    Q, K, V = orc.make_fwd_inputs(2, 3, 1, 64, seed=1)
    O, L = orc.naive_attention(Q, K, V, dtype=np.float64)
    np.testing.assert_array_equal(O, _f64(V))
    np.testing.assert_allclose(L, (_f64(Q) * _f64(K)).sum(-1) / 8.0, atol=1e-12)


def test_closed_form_zero_query():
    _, K, V = orc.make_fwd_inputs(1, 2, 50, 64, seed=2)
    Q = np.zeros_like(K)
    O, L = orc.naive_attention(Q, K, V, dtype=np.float64)
    np.testing.assert_allclose(O, np.broadcast_to(_f64(V).mean(axis=2, keepdims=True), O.shape),
                               atol=1e-12)
    np.testing.assert_allclose(L, np.full(L.shape, math.log(50)), atol=1e-12)


def test_closed_form_equal_keys():
    Q, K, V = orc.make_fwd_inputs(1, 1, 40, 64, seed=3)
    K[:] = K[:, :, :1, :]
    O, L = orc.naive_attention(Q, K, V, dtype=np.float64)
    s = (_f64(Q[0, 0]) @ _f64(K[0, 0, 0])) / 8.0
    np.testing.assert_allclose(O[0, 0], np.broadcast_to(_f64(V[0, 0]).mean(0), (40, 64)), atol=1e-12)
    np.testing.assert_allclose(L[0, 0], s + math.log(40), atol=1e-12)


def test_closed_form_constant_values():
    Q, K, _ = orc.make_fwd_inputs(1, 2, 33, 64, seed=4)
    V = np.full(Q.shape, 0.75, dtype=np.float16)
    O, _ = orc.naive_attention(Q, K, V, dtype=np.float64)
    np.testing.assert_allclose(O, 0.75, atol=1e-12)


def test_causal_first_and_last_rows():
    Q, K, V = orc.make_fwd_inputs(1, 2, 30, 64, seed=5)
    Oc, Lc = orc.naive_attention(Q, K, V, causal=True, dtype=np.float64)
    On, Ln = orc.naive_attention(Q, K, V, causal=False, dtype=np.float64)
    np.testing.assert_array_equal(Oc[:, :, 0], _f64(V[:, :, 0]))
    np.testing.assert_allclose(Lc[:, :, 0], (_f64(Q[:, :, 0]) * _f64(K[:, :, 0])).sum(-1) / 8.0,
                               atol=1e-12)
    np.testing.assert_allclose(Oc[:, :, -1], On[:, :, -1], atol=1e-12)
    np.testing.assert_allclose(Lc[:, :, -1], Ln[:, :, -1], atol=1e-12)
    # causal row i equals non-causal attention over the prefix [0, i]
    i = 17
    Op, Lp = orc.naive_attention(Q[:, :, : i + 1], K[:, :, : i + 1], V[:, :, : i + 1],
                                 dtype=np.float64)
    np.testing.assert_allclose(Oc[:, :, i], Op[:, :, i], atol=1e-12)
    np.testing.assert_allclose(Lc[:, :, i], Lp[:, :, i], atol=1e-12)


def test_key_permutation_invariance():
    Q, K, V = orc.make_fwd_inputs(1, 2, 45, 64, seed=6)
    perm = np.random.default_rng(0).permutation(45)
    O1, L1 = orc.naive_attention(Q, K, V, dtype=np.float64)
    O2, L2 = orc.naive_attention(Q, K[:, :, perm], V[:, :, perm], dtype=np.float64)
    np.testing.assert_allclose(O1, O2, atol=1e-12)
    np.testing.assert_allclose(L1, L2, atol=1e-12)


def test_softmax_rows_sum_to_one_and_shift_invariance():
    Q, K, V = orc.make_fwd_inputs(1, 1, 25, 64, seed=8)
    V1 = np.ones_like(V)
    O, _ = orc.naive_attention(Q, K, V1, dtype=np.float64)
    np.testing.assert_allclose(O, 1.0, atol=1e-12)       # rows of P sum to 1
    # adding a constant to every logit of a row shifts L by that constant
    Q2 = Q.astype(np.float64)
    K2 = np.concatenate([K.astype(np.float64), np.ones((1, 1, 25, 1))], axis=-1)
    Qa = np.concatenate([Q2, np.full((1, 1, 25, 1), 3.0)], axis=-1)
    Oa, La = orc.naive_attention(Qa, K2, V.astype(np.float64), dtype=np.float64)
    Ob, Lb = orc.naive_attention(np.concatenate([Q2, np.zeros((1, 1, 25, 1))], -1), K2,
                                 V.astype(np.float64), dtype=np.float64)
    np.testing.assert_allclose(Oa, Ob, atol=1e-12)
    np.testing.assert_allclose(La - Lb, 3.0 / math.sqrt(65), atol=1e-12)


# ---------------------------------------------------------------- decode
def _small_decode(seed=31, B=4, H=3, D=64, ctx=(1, 16, 17, 70)):
    rng = np.random.default_rng(seed)
    pages = [(c + 15) // 16 for c in ctx]
    P = sum(pages)
    perm = rng.permutation(P).astype(np.int32)
    table = np.zeros((B, max(pages)), np.int32)
    off = 0
    for b in range(B):
        table[b, :pages[b]] = perm[off:off + pages[b]]
        off += pages[b]
    q = rng.standard_normal((B, H, D)).astype(np.float16)
    kp = rng.standard_normal((P, H, 16, D)).astype(np.float16)
    vp = rng.standard_normal((P, H, 16, D)).astype(np.float16)
    return q, kp, vp, table, np.array(ctx, np.int32)


def test_gather_pages_matches_index_walk():
    q, kp, vp, table, ctx = _small_decode()
    for b in range(len(ctx)):
        for h in range(q.shape[1]):
            g = orc.gather_pages(kp, table, int(ctx[b]), b, h)
            walk = np.stack([kp[table[b, j // 16], h, j % 16] for j in range(ctx[b])])
            np.testing.assert_array_equal(g, walk)


def test_decode_equals_naive_over_gathered_keys():
    q, kp, vp, table, ctx = _small_decode()
    O, L = orc.decode_attention(q, kp, vp, table, ctx, dtype=np.float64)
    for b in range(len(ctx)):
        for h in range(q.shape[1]):
            k = orc.gather_pages(kp, table, int(ctx[b]), b, h)
            v = orc.gather_pages(vp, table, int(ctx[b]), b, h)
            On, Ln = orc.naive_attention(q[b, h][None, None, None], k[None, None],
                                         v[None, None], dtype=np.float64)
            np.testing.assert_allclose(O[b, h], On[0, 0, 0], atol=1e-12)
            np.testing.assert_allclose(L[b, h], Ln[0, 0, 0], atol=1e-12)


@pytest.mark.parametrize("S", [1, 2, 5, 16])
def test_split_combine_equals_unsplit(S):
    q, kp, vp, table, ctx = _small_decode()
    O, L = orc.decode_attention(q, kp, vp, table, ctx, dtype=np.float64)
    Os, Ls = orc.split_partials(q, kp, vp, table, ctx, S, dtype=np.float64)
    Oc, Lc = orc.lse_combine(Os, Ls)
    np.testing.assert_allclose(Oc, O, atol=1e-12)
    np.testing.assert_allclose(Lc, L, atol=1e-12)
    if S == 1:
        np.testing.assert_allclose(Os[:, :, 0], O, atol=1e-12)


def test_split_bounds_cover_pages_once():
    for ctx in (1, 15, 16, 17, 100, 32768):
        for S in (1, 3, 16):
            b = orc.split_bounds(ctx, 16, S)
            covered = [p for p0, p1 in b for p in range(p0, p1)]
            assert covered == list(range((ctx + 15) // 16))


def test_combine_empty_splits():
    Os = np.zeros((1, 1, 4, 8))
    Ls = np.full((1, 1, 4), -np.inf)
    O, L = orc.lse_combine(Os, Ls)
    assert np.all(O == 0) and np.isneginf(L).all()
    Os[0, 0, 2] = 1.5
    Ls[0, 0, 2] = 0.3
    O, L = orc.lse_combine(Os, Ls)
    np.testing.assert_allclose(O[0, 0], 1.5)
    np.testing.assert_allclose(L[0, 0], 0.3)


def test_decode_meta_is_a_permutation():
    ctx, table, P = orc.make_decode_meta(B=32, seed=5)
    pages = (ctx + 15) // 16
    used = np.concatenate([table[b, :pages[b]] for b in range(32)])
    assert sorted(used.tolist()) == list(range(P))
    assert ctx.min() >= 512 and ctx.max() <= 32768


def test_ragged_inputs_are_not_tile_multiples():
    N, Q, K, V = orc.make_ragged_inputs(B=1, H=1, D=64, seed=7)
    assert 1000 <= N <= 5000 and N % 32 and N % 64 and N % 128
    assert Q.dtype == np.float16 and Q.shape == (1, 1, N, 64)
    assert np.abs(Q.astype(np.float32)).max() > 6  # the std-3 rows are present


def test_generators_are_deterministic():
    a = orc.make_fwd_inputs(1, 2, 10, 64, seed=9)
    b = orc.make_fwd_inputs(1, 2, 10, 64, seed=9)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)


# ---------------------------------------------------------------- mutations
def _mut_scale(Q, K, V, causal=False, dtype=np.float32):       # 1/D instead of 1/sqrt(D)
    return orc.naive_attention(Q * np.float32(1 / math.sqrt(Q.shape[-1])), K, V, causal, dtype)


def _mut_transpose_v(Q, K, V, causal=False, dtype=np.float32):  # V read as V^T on square heads
    return orc.naive_attention(Q, K, np.swapaxes(V, -1, -2).copy(), causal, dtype)


def _mut_causal_offbyone(Q, K, V, causal=False, dtype=np.float32):  # j < i instead of j <= i
    if not causal:
        return orc.naive_attention(Q, K, V, False, dtype)
    O, L = orc.naive_attention(Q, K, V, True, dtype)
    Q2 = np.asarray(Q, dtype)
    O[:, :, 1:], L[:, :, 1:] = orc.naive_attention(Q2[:, :, 1:], K[:, :, :-1], V[:, :, :-1], True, dtype)
    return O, L


def _mut_lse_log2(Q, K, V, causal=False, dtype=np.float32):     # L in log2 instead of ln
    O, L = orc.naive_attention(Q, K, V, causal, dtype)
    return O, L / np.float32(math.log(2))


@pytest.mark.parametrize("mut", [_mut_scale, _mut_transpose_v, _mut_causal_offbyone, _mut_lse_log2])
def test_planted_mistakes_are_caught(mut):
    caught = False
    for name in sorted(p.stem for p in GOLDEN.glob("fwd_*.npz")):
        z = np.load(GOLDEN / f"{name}.npz")
        if mut is _mut_transpose_v and z["q"].shape[1] != z["q"].shape[2]:
            continue
        q, k, v = z["q"][None], z["k"][None], z["v"][None]
        O, L = mut(orc.half_cast(q), orc.half_cast(k), orc.half_cast(v), bool(z["causal"]))
        vmax = float(np.abs(z["v"].astype(np.float32)).max())
        if not (np.allclose(O[0], z["o"], atol=2e-6 * max(vmax, 1.0))
                and np.allclose(L[0], z["l"], atol=2e-5, rtol=2e-6)):
            caught = True
    if mut is _mut_transpose_v:
        # square head (N == D) case built here, checked against brute force
        Q, K, V = orc.make_fwd_inputs(1, 1, 16, 16, seed=99)
        O, _ = mut(orc.half_cast(Q), orc.half_cast(K), orc.half_cast(V))
        Ob, _ = orc.attention_bruteforce(_f64(Q[0, 0]), _f64(K[0, 0]), _f64(V[0, 0]))
        caught = caught or not np.allclose(O[0, 0], np.array(Ob), atol=2e-6)
    assert caught


def test_planted_combine_mistake_is_caught():
    z = np.load(GOLDEN / "combine_b2_s5.npz")
    Os, Ls = _f64(z["part_o"]), _f64(z["part_lse"])
    # mistake: weights exp(L_s) normalised by count instead of by their sum
    M = Ls.max(-1, keepdims=True)
    w = np.where(np.isfinite(Ls), np.exp(Ls - M), 0)
    bad = (w[..., None] * Os).sum(-2) / np.isfinite(Ls).sum(-1, keepdims=True)
    assert not np.allclose(bad, z["o"], atol=1e-6)


# ---------------------------------------------------------------- backward
def _fd_grads(Q, K, V, G, causal, eps=1e-6):
    """Central finite differences of sum(naive_attention(Q, K, V) * G), float64."""
    def loss(q, k, v):
        O, _ = orc.naive_attention(q, k, v, causal, np.float64)
        return float((O * G).sum())

    out = []
    for which in range(3):
        args = [Q.copy(), K.copy(), V.copy()]
        g = np.zeros_like(args[which])
        for idx in np.ndindex(*g.shape):
            a = args[which]
            keep = a[idx]
            a[idx] = keep + eps
            hi = loss(*args)
            a[idx] = keep - eps
            lo = loss(*args)
            a[idx] = keep
            g[idx] = (hi - lo) / (2 * eps)
        out.append(g)
    return out


def _bwd_inputs(seed, B=1, H=2, N=6, D=4):
    rng = np.random.default_rng(seed)
    return [rng.standard_normal((B, H, N, D)) for _ in range(4)]


@pytest.mark.parametrize("causal", [False, True])
def test_backward_matches_finite_differences(causal):
    Q, K, V, G = _bwd_inputs(7)
    ref = _fd_grads(Q, K, V, G, causal)
    got = orc.naive_attention_backward(Q, K, V, G, causal, np.float64)
    for name, r, g in zip("QKV", ref, got):
        np.testing.assert_allclose(g, r, atol=1e-7, rtol=1e-6, err_msg=f"d{name}")
    # float32 (the tests' precision) stays within 1e-5 of float64
    got32 = orc.naive_attention_backward(Q, K, V, G, causal)
    for g32, g in zip(got32, got):
        np.testing.assert_allclose(g32, g, atol=1e-5)


def test_backward_closed_forms():
    Q, K, V, G = _bwd_inputs(8, N=5)
    dQ, dK, dV = orc.naive_attention_backward(Q, K, V, G, False, np.float64)
    # sum over keys of dS is zero per row, so sum_j dK_j = 0 and the gradient
    # with respect to a common shift of all keys vanishes
    np.testing.assert_allclose(dK.sum(axis=2), 0, atol=1e-12)
    # dV columns sum to the dO columns (P rows sum to one)
    np.testing.assert_allclose(dV.sum(axis=2), G.sum(axis=2), atol=1e-12)
    # causal: row 0 attends only key 0, so dQ[0] = 0 and dV[0] gets dO[0] in full
    dQc, dKc, dVc = orc.naive_attention_backward(Q, K, V, G, True, np.float64)
    np.testing.assert_allclose(dQc[:, :, 0], 0, atol=1e-12)
    # the last key is seen only by the last query: dV[N-1] = P[N-1, N-1] * dO[N-1]
    # with P[N-1, N-1] = exp(q.k / sqrt(4) - L[N-1])
    s = (Q[:, :, -1] * K[:, :, -1]).sum(-1) / 2.0 - orc.naive_attention(
        Q, K, V, True, np.float64)[1][:, :, -1]
    np.testing.assert_allclose(dVc[:, :, -1], np.exp(s)[..., None] * G[:, :, -1], atol=1e-12)


def _mut_bwd_no_di(Q, K, V, dO, causal=False, dtype=np.float64):     # dS = P * dP
    Q, K, V, dO = (np.asarray(a, dtype) for a in (Q, K, V, dO))
    dQ, dK, dV = orc.naive_attention_backward(Q, K, V, dO, causal, dtype)
    O, _ = orc.naive_attention(Q, K, V, causal, dtype)
    Di = (dO * O).sum(-1, keepdims=True)
    # adding back P * Di through dQ = dS K scale drops the -Di term
    S = np.einsum("bhid,bhjd->bhij", Q, K) * Q.shape[-1] ** -0.5
    if causal:
        S = np.where(np.arange(S.shape[-1])[None, :] > np.arange(S.shape[-2])[:, None], -np.inf, S)
    P, _ = orc._softmax_lse(S)
    return dQ + np.einsum("bhij,bhjd->bhid", P * Di, K) * Q.shape[-1] ** -0.5, dK, dV


def _mut_bwd_dk_unscaled(Q, K, V, dO, causal=False, dtype=np.float64):  # dK without scale
    dQ, dK, dV = orc.naive_attention_backward(Q, K, V, dO, causal, dtype)
    return dQ, dK * Q.shape[-1] ** 0.5, dV


def _mut_bwd_dv_untransposed(Q, K, V, dO, causal=False, dtype=np.float64):  # dV = P dO
    S = np.einsum("bhid,bhjd->bhij", Q, K) * Q.shape[-1] ** -0.5
    if causal:
        S = np.where(np.arange(S.shape[-1])[None, :] > np.arange(S.shape[-2])[:, None], -np.inf, S)
    P, _ = orc._softmax_lse(S)
    dQ, dK, _ = orc.naive_attention_backward(Q, K, V, dO, causal, dtype)
    return dQ, dK, np.einsum("bhij,bhjd->bhid", P, dO)


@pytest.mark.parametrize("mut", [_mut_bwd_no_di, _mut_bwd_dk_unscaled, _mut_bwd_dv_untransposed])
def test_planted_backward_mistakes_are_caught(mut):
    Q, K, V, G = _bwd_inputs(9, N=5)
    for causal in (False, True):
        ref = _fd_grads(Q, K, V, G, causal)
        got = mut(Q, K, V, G, causal)
        if not all(np.allclose(g, r, atol=1e-6, rtol=1e-6) for g, r in zip(got, ref)):
            return
    pytest.fail("finite differences did not catch the planted mistake")


# ---------------------------------------------------------------- page writer
def _pool_case(seed=3, B=3, H=2, D=8, T=37, page_size=16):
    rng = np.random.default_rng(seed)
    max_pages = (T + 40 + page_size - 1) // page_size + 1
    num_pages = B * max_pages + 5
    perm = rng.permutation(num_pages).astype(np.int32)
    table = perm[:B * max_pages].reshape(B, max_pages)
    kp = rng.standard_normal((num_pages, H, page_size, D)).astype(np.float16)
    vp = rng.standard_normal((num_pages, H, page_size, D)).astype(np.float16)
    kn = rng.standard_normal((B, H, T, D)).astype(np.float16)
    vn = rng.standard_normal((B, H, T, D)).astype(np.float16)
    return kp, vp, table, kn, vn


def test_append_then_gather_returns_rows():
    kp, vp, table, kn, vn = _pool_case()
    B, H, T, _ = kn.shape
    kp2, vp2, bad = orc.append_pages(kp, vp, table, np.zeros(B, np.int32), kn, vn)
    assert not bad.any()
    for b in range(B):
        for h in range(H):
            np.testing.assert_array_equal(orc.gather_pages(kp2, table, T, b, h), kn[b, h])
            np.testing.assert_array_equal(orc.gather_pages(vp2, table, T, b, h), vn[b, h])
    # pages not in any sequence's first ceil(T/16) entries are untouched
    used = set(table[:, : (T + 15) // 16].ravel().tolist())
    for pid in range(kp.shape[0]):
        if pid not in used:
            np.testing.assert_array_equal(kp2[pid], kp[pid])


def test_append_in_two_steps_equals_one():
    kp, vp, table, kn, vn = _pool_case(seed=4)
    B, H, T, _ = kn.shape
    start = np.array([0, 5, 17], np.int32)
    one = orc.append_pages(kp, vp, table, start, kn, vn)
    cut = 13
    a = orc.append_pages(kp, vp, table, start, kn[:, :, :cut], vn[:, :, :cut])
    two = orc.append_pages(a[0], a[1], table, start + cut, kn[:, :, cut:], vn[:, :, cut:])
    np.testing.assert_array_equal(one[0], two[0])
    np.testing.assert_array_equal(one[1], two[1])
    # ragged counts: writing n_b tokens equals writing the truncated batch row by row
    lens = np.array([0, 9, 37], np.int32)
    r = orc.append_pages(kp, vp, table, start, kn, vn, lens)
    for b in range(B):
        rb = orc.append_pages(kp, vp, table[b:b + 1], start[b:b + 1], kn[b:b + 1, :, :lens[b]],
                              vn[b:b + 1, :, :lens[b]])
        used = table[b, start[b] // 16:(start[b] + max(lens[b], 1) + 15) // 16 + 1]
        for pid in used:
            np.testing.assert_array_equal(r[0][pid], rb[0][pid])


def test_append_invalid_pages_write_nothing():
    kp, vp, table, kn, vn = _pool_case(seed=5)
    B = kn.shape[0]
    bad_table = table.copy()
    bad_table[1, 0] = -1                      # sequence 1's first page invalid
    bad_table[2, 1] = kp.shape[0]             # sequence 2's second page past the pool
    start = np.array([0, 0, 0], np.int32)
    kp2, vp2, bad = orc.append_pages(kp, vp, bad_table, start, kn, vn)
    assert bad.tolist() == [0, 1, 1]
    # past the table: positions beyond max_pages * 16
    far = np.array([bad_table.shape[1] * 16 - 3, -1, 0], np.int32)
    _, _, bad2 = orc.append_pages(kp, vp, table, far, kn[:, :, :5], vn[:, :, :5])
    assert bad2.tolist() == [1, 1, 0]


@pytest.mark.parametrize("mistake", ["slot_from_page", "head_stride"])
def test_planted_append_mistakes_are_caught(mistake):
    kp, vp, table, kn, vn = _pool_case(seed=6)
    B, H, T, D = kn.shape
    bad_kp = np.array(kp, copy=True)
    for b in range(B):
        for t in range(T):
            pid = table[b, t // 16]
            if mistake == "slot_from_page":   # slot and page index swapped
                bad_kp[table[b, t % 16 if t % 16 < table.shape[1] else 0], :, t // 16] = kn[b, :, t]
            else:                             # heads written in reverse order
                bad_kp[pid, ::-1, t % 16] = kn[b, :, t]
    ok = all(np.array_equal(orc.gather_pages(bad_kp, table, T, b, h), kn[b, h])
             for b in range(B) for h in range(H))
    assert not ok


# ---------------------------------------------------------------- bf16 rounding
def test_bf16_cast_matches_torch_and_ties_to_even():
    import torch
    rng = np.random.default_rng(12)
    x = np.concatenate([rng.standard_normal(10000).astype(np.float32) * 10.0 ** rng.integers(-6, 6, 10000),
                        np.array([0.0, -0.0, 1.0, 65504.0, 3.0e38, 1e-40], np.float32)])
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(orc.bf16_cast(x), ref)
    # exact ties: 1 + 2^-8 lies halfway between 1 and 1 + 2^-7 -> even (1.0);
    # 1 + 3 * 2^-8 lies halfway between 1 + 2^-7 and 1 + 2^-6 -> even (1 + 2^-6)
    ties = np.array([1 + 2.0 ** -8, 1 + 3 * 2.0 ** -8], np.float32)
    np.testing.assert_array_equal(orc.bf16_cast(ties), np.array([1.0, 1 + 2.0 ** -6], np.float32))


def test_planted_bf16_truncation_is_caught():
    import torch
    x = np.random.default_rng(13).standard_normal(1000).astype(np.float32)
    trunc = (x.view(np.uint32) >> 16 << 16).view(np.float32)   # round toward zero
    assert not np.array_equal(trunc, torch.from_numpy(x).to(torch.bfloat16).float().numpy())


def test_bench_decode_metadata_matches_the_oracle_generator():
    """bench.py builds config 5's paging itself (the bench may not call the
    oracle outside its CPU-baseline leg); it must be the tests' metadata."""
    import importlib.util
    import pathlib
    path = pathlib.Path(__file__).resolve().parents[1] / "bench.py"
    spec = importlib.util.spec_from_file_location("fa_bench", path)
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    for seed in (5, 6):
        a = bench.decode_meta(B=32, seed=seed)
        b = orc.make_decode_meta(B=32, seed=seed)
        assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1]) and a[2] == b[2]


# --- fp16_p_forward: the reference kernel's fp16 rounding of P and O ---------

def _fp16(x):
    return np.asarray(x, np.float64).astype(np.float32).astype(np.float16).astype(np.float64)


def _fp16_p_loop(q, k, v, causal, normalise_by_rounded=False, rescale_o=True):
    """Pure-Python restatement, row by row, of the reference kernel's loop
    (cuda/flash_attn_fa3_db_full.cu:250-293, :330-339): 64-key tiles, m raised
    to the running max every tile, P = fl32(2^(fl32(s c - m))) summed unrounded
    into l and rounded to fp16 for O += P V, O = fp16(O / l). The keyword
    arguments plant the mistakes the pinning test must see."""
    N, D = q.shape
    c = float(np.float32(np.float32(1.4426950408889634) * np.float32(1.0 / math.sqrt(D))))
    out = np.zeros((N, v.shape[1]))
    for i in range(N):
        s = [float(np.float32(sum(float(q[i, d]) * float(k[j, d]) for d in range(D))))
             for j in range(k.shape[0])]
        if causal:
            s = [x if j <= i else -math.inf for j, x in enumerate(s)]
        m, l, lr, o = -math.inf, 0.0, 0.0, np.zeros(v.shape[1])
        for t0 in range(0, len(s), 64):
            tile = s[t0:t0 + 64]
            tm = float(np.float32(max(tile) * c)) if max(tile) > -math.inf else -math.inf
            mn = max(m, tm)
            alpha = 1.0 if mn == m else 2.0 ** (m - mn)
            l *= alpha
            lr *= alpha
            if rescale_o:
                o = o * alpha
            ms = mn if mn > -math.inf else 0.0
            for j, x in enumerate(tile):
                p = float(np.float32(2.0 ** float(np.float32(x * c - ms)))) if x > -math.inf else 0.0
                p16 = float(_fp16(p))
                l += p
                lr += p16
                o = o + p16 * v[t0 + j]
            m = mn
        out[i] = _fp16(o / (lr if normalise_by_rounded else l))
    return out


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("lazy", [True, False])
def test_fp16_p_forward_without_p_rounding_is_naive_attention(causal, lazy):
    """round_p=False: the running-max bookkeeping (lazy or per tile) is exact
    algebra, so O is the naive result rounded to fp16 (within one fp16 ulp,
    where the two round a value near a rounding boundary differently, plus
    fp32 noise of the terms where a row's terms cancel) and L is the naive L."""
    for N, amp in ((1, 1.0), (63, 1.0), (200, 3.0), (333, 1.0)):
        Q, K, V = (orc.half_cast(x)[0, 0] for x in orc.make_fwd_inputs(1, 1, N, 64, seed=N, amp=amp))
        Or, Lr = orc.naive_attention(Q[None, None], K[None, None], V[None, None], causal=causal,
                                     dtype=np.float64)
        O, L = orc.fp16_p_forward(Q, K, V, causal=causal, round_p=False, lazy_max=lazy)
        ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(Or[0, 0]), 2.0 ** -14))) - 10)
        assert (np.abs(O - Or[0, 0]) <= ulp + 1e-6 * np.abs(V).max()).all(), (N, amp)
        assert np.abs(L - Lr[0, 0]).max() <= 1e-5 * max(1.0, np.abs(Lr).max()), (N, amp)


@pytest.mark.parametrize("causal", [False, True])
def test_fp16_p_forward_matches_the_loop_and_catches_planted_mistakes(causal):
    """With the reference's per-tile max (lazy_max=False), fp16_p_forward is
    the row-by-row loop above on peaky inputs (std-3 Q and K: a few keys carry
    each row); normalising by the rounded sum, or dropping O's rescale, moves
    the loop's result away from it."""
    N, D = 150, 16
    Q, K, V = (orc.half_cast(x)[0, 0] for x in orc.make_fwd_inputs(1, 1, N, D, seed=5, amp=3.0))
    O, _ = orc.fp16_p_forward(Q, K, V, causal=causal, lazy_max=False)
    want = _fp16_p_loop(Q, K, V, causal)
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(want), 2.0 ** -14))) - 10)
    assert (np.abs(O - want) <= ulp).all()
    assert np.abs(O - want).max() <= 1e-3
    Or_, _ = orc.fp16_p_forward(Q, K, V, causal=causal, lazy_max=False, norm_rounded=True)
    want_r = _fp16_p_loop(Q, K, V, causal, normalise_by_rounded=True)
    assert (np.abs(Or_ - want_r) <= ulp).all()
    planted = [want_r, _fp16_p_loop(Q, K, V, causal, rescale_o=False)]
    for bad in planted:
        assert np.abs(bad - O).max() > 2 * np.abs(want - O).max() + 1e-6


def test_fp16_p_forward_is_a_convex_combination():
    """Whatever the running-max rule, every O element lies within the range of
    its V column (up to P's and O's rounding)."""
    N, D = 500, 64
    Q, K, V = (orc.half_cast(x)[0, 0] for x in orc.make_fwd_inputs(1, 1, N, D, seed=9, amp=3.0))
    for lazy in (True, False):
        O, _ = orc.fp16_p_forward(Q, K, V, lazy_max=lazy)
        lo, hi = V.min(axis=0), V.max(axis=0)
        slack = 2.0 ** -10 * np.abs(V).max(axis=0)
        assert (O >= lo - slack).all() and (O <= hi + slack).all()
