"""GPU tier: grouped KV heads (GQA/MQA) and packed variable-length sequences.

Both widen the forward's boundary (README.md:326 lists "varlen, GQA, MQA" as
not covered by the reference). The expected values come from the pinned
oracle with no new arithmetic: GQA is naive attention with each KV head
repeated for its query-head group; varlen is naive attention of each
sequence on its own. Tolerances are the forward's (tests/test_fwd_gpu.py):
O max-abs <= 2e-3 plus half an fp16 ulp, L relative <= 1e-4.
"""
import numpy as np
import pytest
import torch

from oracle import decode_attention, half_cast, naive_attention, naive_attention_backward

from test_fwd_gpu import _check

pytestmark = pytest.mark.gpu


def _randn(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("Hkv", [1, 2, 8])
@pytest.mark.parametrize("N,causal", [(128, False), (333, True), (1024, False), (1024, True)])
def test_gqa_forward(fa, dev, D, Hkv, N, causal):
    B, H = 2, 8
    Q = _randn((B, H, N, D), 1)
    K = _randn((B, Hkv, N, D), 2)
    V = _randn((B, Hkv, N, D), 3)
    tq, tk, tv = (torch.from_numpy(x).to(dev) for x in (Q, K, V))
    O, L = fa.forward(tq, tk, tv, causal=causal)
    O2 = fa.forward_only(tq, tk, tv, causal=causal)
    torch.cuda.synchronize()
    assert torch.equal(O, O2)
    g = H // Hkv
    Or, Lr = naive_attention(half_cast(Q), np.repeat(half_cast(K), g, axis=1),
                             np.repeat(half_cast(V), g, axis=1), causal=causal)
    _check(O, L, Or, Lr, tag=f"GQA H{H} Hkv{Hkv} N{N} D{D} causal={causal}")


@pytest.mark.parametrize("Hkv", [4, 1])
def test_gqa_causal_single_wave(fa, dev, Hkv):
    """B1 H16 N2048 D64 causal (one wave of 128-row blocks on 256 CUs, so the
    default path runs the 64-row kernel), here with K/V heads shared by
    groups of query heads."""
    B, H, N, D = 1, 16, 2048, 64
    Q = _randn((B, H, N, D), 11)
    K = _randn((B, Hkv, N, D), 12)
    V = _randn((B, Hkv, N, D), 13)
    tq, tk, tv = (torch.from_numpy(x).to(dev) for x in (Q, K, V))
    O, L = fa.forward(tq, tk, tv, causal=True)
    torch.cuda.synchronize()
    g = H // Hkv
    Or, Lr = naive_attention(half_cast(Q), np.repeat(half_cast(K), g, axis=1),
                             np.repeat(half_cast(V), g, axis=1), causal=True)
    _check(O, L, Or, Lr, tag=f"GQA causal H{H} Hkv{Hkv} N{N} D{D}")


def test_gqa_with_all_heads_equals_mha(fa, dev):
    Q, K, V = (_randn((1, 4, 300, 64), s) for s in (4, 5, 6))
    tq, tk, tv = (torch.from_numpy(x).to(dev).half() for x in (Q, K, V))
    O1, L1 = fa.forward(tq, tk, tv)
    # the same K/V given as a GQA group of 2 that happens to hold equal heads
    k2 = tk[:, ::2].contiguous()
    v2 = tv[:, ::2].contiguous()
    O2, L2 = fa.forward(tq, k2, v2)
    O3, L3 = fa.forward(tq, k2.repeat_interleave(2, dim=1), v2.repeat_interleave(2, dim=1))
    assert torch.equal(O2, O3) and torch.equal(L2, L3)
    assert O1.shape == O2.shape


def _cu(lengths):
    return np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("Hkv", [4, 2])
def test_varlen_forward(fa, dev, D, causal, Hkv):
    H = 4
    lengths = [1, 100, 0, 257, 1024, 63, 128]
    cu = _cu(lengths)
    total = int(cu[-1])
    q = _randn((H, total, D), 7)
    k = _randn((Hkv, total, D), 8)
    v = _randn((Hkv, total, D), 9)
    tq, tk, tv, tcu = (torch.from_numpy(x).to(dev) for x in (q, k, v, cu))
    O, L = fa.forward_varlen(tq, tk, tv, tcu, max(lengths), causal=causal)
    torch.cuda.synchronize()
    assert O.shape == (H, total, D) and L.shape == (H, total)
    g = H // Hkv
    for b, n in enumerate(lengths):
        if n == 0:
            continue
        s0, s1 = cu[b], cu[b + 1]
        Or, Lr = naive_attention(half_cast(q[None, :, s0:s1]),
                                 np.repeat(half_cast(k[None, :, s0:s1]), g, axis=1),
                                 np.repeat(half_cast(v[None, :, s0:s1]), g, axis=1), causal=causal)
        _check(O[None, :, s0:s1], L[None, :, s0:s1], Or, Lr,
               tag=f"varlen seq {b} (n={n}) D{D} causal={causal} Hkv{Hkv}")


def test_varlen_single_sequence_matches_dense(fa, dev):
    H, N, D = 2, 512, 64
    q, k, v = (_randn((H, N, D), s) for s in (10, 11, 12))
    tq, tk, tv = (torch.from_numpy(x).to(dev).half() for x in (q, k, v))
    cu = torch.tensor([0, N], dtype=torch.int32, device=dev)
    Ov, Lv = fa.forward_varlen(tq, tk, tv, cu, N, causal=True)
    Od, Ld = fa.forward(tq[None], tk[None], tv[None], causal=True)
    assert (Ov.float() - Od[0].float()).abs().max().item() <= 1e-3
    assert (Lv - Ld[0]).abs().max().item() <= 1e-4


def test_varlen_rows_outside_sequences_and_malformed_bounds(fa, dev):
    """Trailing rows past cu[B] keep O = 0 and L = -inf (an empty sequence
    adds no rows); out-of-range bounds are clamped."""
    H, D = 2, 64
    total = 300
    q, k, v = (torch.from_numpy(_randn((H, total, D), s)).to(dev).half() for s in (13, 14, 15))
    cu = torch.tensor([0, 100, 100, 200], dtype=torch.int32, device=dev)
    O, L = fa.forward_varlen(q, k, v, cu, 100)
    assert torch.count_nonzero(O[:, 200:]).item() == 0
    assert torch.isneginf(L[:, 200:]).all()
    assert torch.isfinite(L[:, :200]).all()
    # decreasing and past-the-end bounds: nothing is read or written outside
    bad = torch.tensor([0, 250, 100, 10_000], dtype=torch.int32, device=dev)
    O2, _ = fa.forward_varlen(q, k, v, bad, 256)
    torch.cuda.synchronize()
    assert torch.isfinite(O2.float()).all()


def test_gqa_decode(fa, dev):
    B, H, Hkv, D = 4, 8, 2, 128
    rng = np.random.default_rng(16)
    ctx = np.array([1, 77, 300, 1000], np.int32)
    pages = (ctx + 15) // 16
    table = np.zeros((B, pages.max()), np.int32)
    perm = rng.permutation(int(pages.sum())).astype(np.int32)
    off = 0
    for b in range(B):
        table[b, :pages[b]] = perm[off:off + pages[b]]
        off += pages[b]
    q = rng.standard_normal((B, H, D)).astype(np.float16)
    kp = rng.standard_normal((int(pages.sum()), Hkv, 16, D)).astype(np.float16)
    vp = rng.standard_normal((int(pages.sum()), Hkv, 16, D)).astype(np.float16)
    tq, tkp, tvp, ttab, tctx = (torch.from_numpy(x).to(dev) for x in (q, kp, vp, table, ctx))
    O, L = fa.decode_paged(tq, tkp, tvp, ttab, tctx, 4)
    g = H // Hkv
    Or, Lr = decode_attention(q, np.repeat(kp, g, axis=1), np.repeat(vp, g, axis=1), table, ctx)
    assert np.abs(O.float().cpu().numpy() - Or).max() <= 2e-3
    assert (np.abs(L.cpu().numpy() - Lr) / np.maximum(np.abs(Lr), 1)).max() <= 1e-4
    with pytest.raises(RuntimeError, match="decode_partials takes pools with H heads"):
        fa.decode_partials(tq, tkp, tvp, ttab, tctx, 4)


def test_gqa_rejects_bad_head_counts(fa, dev):
    q = torch.zeros(1, 6, 64, 64, device=dev)
    kv = torch.zeros(1, 4, 64, 64, device=dev)
    with pytest.raises(RuntimeError, match="multiple"):
        fa.forward(q, kv, kv)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("H,Hkv", [(8, 4), (8, 2), (12, 2), (6, 2), (16, 2), (32, 2), (40, 2),
                                   (32, 1)])
def test_gqa_decode_groups(fa, dev, D, H, Hkv):
    """Groups of 2 to 32 query heads per KV head (a workgroup takes up to 16
    of them: groups of 20 and 32 span two workgroups, groups of 3 and 6 leave
    columns of the 16 unused) against the decode oracle over repeated pools,
    including an invalid page id (NaN for that sequence only)."""
    B = 3
    rng = np.random.default_rng(H * 10 + Hkv + D)
    ctx = np.array([5, 160, 700], np.int32)
    pages = (ctx + 15) // 16
    table = np.zeros((B, pages.max()), np.int32)
    perm = rng.permutation(int(pages.sum())).astype(np.int32)
    off = 0
    for b in range(B):
        table[b, :pages[b]] = perm[off:off + pages[b]]
        off += pages[b]
    q = rng.standard_normal((B, H, D)).astype(np.float16)
    kp = rng.standard_normal((int(pages.sum()), Hkv, 16, D)).astype(np.float16)
    vp = rng.standard_normal((int(pages.sum()), Hkv, 16, D)).astype(np.float16)
    tq, tkp, tvp, tctx = (torch.from_numpy(x).to(dev) for x in (q, kp, vp, ctx))
    for splits in (1, 5, 16):
        O, L = fa.decode_paged(tq, tkp, tvp, torch.from_numpy(table).to(dev), tctx, splits)
        g = H // Hkv
        Or, Lr = decode_attention(q, np.repeat(kp, g, axis=1), np.repeat(vp, g, axis=1), table, ctx)
        assert np.abs(O.float().cpu().numpy() - Or).max() <= 2e-3, f"splits {splits}"
        assert (np.abs(L.cpu().numpy() - Lr) / np.maximum(np.abs(Lr), 1)).max() <= 1e-4
    bad = table.copy()
    bad[1, 2] = 10 ** 6
    O, L = fa.decode_paged(tq, tkp, tvp, torch.from_numpy(bad).to(dev), tctx, 4)
    On = O.float().cpu().numpy()
    assert np.isnan(On[1]).all() and np.isfinite(On[0]).all() and np.isfinite(On[2]).all()


# Backward of the packed layout: each sequence against the oracle's backward
# of that sequence alone (K/V repeated per group, dK/dV summed per KV head),
# at the dense backward's bound (tests/test_bwd_gpu.py): |g - g_ref| <=
# 5e-3 + 5e-3 |g_ref|, the absolute part times the group for dK/dV.
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("Hkv", [4, 2])
def test_varlen_backward(fa, dev, D, causal, Hkv):
    H = 4
    lengths = [1, 100, 0, 257, 300, 63, 128]
    cu = _cu(lengths)
    total = int(cu[-1]) + 5                  # 5 trailing rows outside every sequence
    q, o_g = _randn((H, total, D), 20), _randn((H, total, D), 23)
    k, v = _randn((Hkv, total, D), 21), _randn((Hkv, total, D), 22)
    tq, tk, tv, tg, tcu = (torch.from_numpy(x).to(dev) for x in (q, k, v, o_g, cu))
    O, L = fa.forward_varlen(tq, tk, tv, tcu, max(lengths), causal=causal)
    dQ, dK, dV = fa.backward_varlen(tq, tk, tv, O, tg, L, tcu, max(lengths), causal=causal)
    torch.cuda.synchronize()
    assert dQ.shape == (H, total, D) and dK.shape == (Hkv, total, D) and dV.shape == dK.shape
    g = H // Hkv
    got = [t.cpu().numpy() for t in (dQ, dK, dV)]
    for b, n in enumerate(lengths):
        if n == 0:
            continue
        s0, s1 = cu[b], cu[b + 1]
        rQ, rK, rV = naive_attention_backward(
            half_cast(q[None, :, s0:s1]), np.repeat(half_cast(k[None, :, s0:s1]), g, axis=1),
            np.repeat(half_cast(v[None, :, s0:s1]), g, axis=1), half_cast(o_g[None, :, s0:s1]),
            causal)
        rK = rK.reshape(1, Hkv, g, n, D).sum(axis=2)
        rV = rV.reshape(1, Hkv, g, n, D).sum(axis=2)
        for name, x, r, atol in (("dQ", got[0], rQ, 5e-3), ("dK", got[1], rK, 5e-3 * g),
                                 ("dV", got[2], rV, 5e-3 * g)):
            err = np.abs(x[None, :, s0:s1] - r)
            assert (err <= atol + 5e-3 * np.abs(r)).all(), \
                f"{name} seq {b} (n={n}) D{D} causal={causal} Hkv{Hkv}: max err {err.max():.3e}"
    for x in got:
        assert not x[:, cu[-1]:].any(), "rows outside every sequence must stay zero"


def test_varlen_backward_single_sequence_matches_dense(fa, dev):
    H, N, D = 2, 384, 64
    q, k, v, gr = (torch.from_numpy(_randn((H, N, D), s)).to(dev).half() for s in (30, 31, 32, 33))
    cu = torch.tensor([0, N], dtype=torch.int32, device=dev)
    Ov, Lv = fa.forward_varlen(q, k, v, cu, N, causal=True)
    gv = fa.backward_varlen(q, k, v, Ov, gr, Lv, cu, N, causal=True)
    Od, Ld = fa.forward(q[None], k[None], v[None], causal=True)
    gd = fa.backward(q[None], k[None], v[None], Od, gr[None], Ld, causal=True)
    for a, b in zip(gv, gd):
        assert (a - b[0]).abs().max().item() <= 1e-3
