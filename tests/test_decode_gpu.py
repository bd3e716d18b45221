"""GPU tier: split-KV paged decode and the logsumexp combine against the oracle.

No reference counterpart exists (the reference has no decode path); the
oracle (oracle/naive.py: decode_attention, split_partials, lse_combine) is
pinned on the CPU by tests/test_oracle.py. Bars:
* gather: bit-exact. A one-hot query selects a single token whose V row is
  returned unchanged, so O equals the V row the page table points at, bit for
  bit; permuting the page ids (and moving the pages with them) leaves O and L
  bitwise unchanged.
* values: O max-abs <= 2e-3, L relative <= 1e-4 (|dL| / max(|L|, 1)),
  against fp32 math on the same fp16 inputs.
"""
import pathlib

import numpy as np
import pytest
import torch

from oracle import (decode_attention, lse_combine, make_decode_meta, naive_attention,
                    split_partials)

pytestmark = pytest.mark.gpu
GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"


def _dev(dev, *xs):
    return [torch.from_numpy(np.ascontiguousarray(x)).to(dev) for x in xs]


def _small(seed, B, H, D, ctx, extra_pages=0):
    rng = np.random.default_rng(seed)
    pages = [(c + 15) // 16 for c in ctx]
    P = sum(pages) + extra_pages
    perm = rng.permutation(P).astype(np.int32)
    table = np.zeros((B, max(max(pages), 1)), np.int32)
    off = 0
    for b in range(B):
        table[b, :pages[b]] = perm[off:off + pages[b]]
        off += pages[b]
    q = rng.standard_normal((B, H, D)).astype(np.float16)
    kp = rng.standard_normal((P, H, 16, D)).astype(np.float16)
    vp = rng.standard_normal((P, H, 16, D)).astype(np.float16)
    return q, kp, vp, table, np.array(ctx, np.int32)


def _check(O, L, Or, Lr, tag=""):
    O = O.float().cpu().numpy()
    L = L.cpu().numpy()
    assert np.abs(O - Or).max() <= 2e-3, f"{tag} O {np.abs(O - Or).max():.3e}"
    rel = np.abs(L - Lr) / np.maximum(np.abs(Lr), 1.0)
    assert rel.max() <= 1e-4, f"{tag} L rel {rel.max():.3e}"


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("S", [1, 3, 16])
def test_decode_small_vs_oracle(fa, dev, D, S):
    q, kp, vp, table, ctx = _small(1 + D + S, B=5, H=3, D=D, ctx=[1, 15, 16, 17, 300], extra_pages=2)
    tq, tk, tv, tt, tc = _dev(dev, q, kp, vp, table, ctx)
    O, L = fa.decode_paged(tq, tk, tv, tt, tc, num_splits=S)
    Or, Lr = decode_attention(q, kp, vp, table, ctx)
    _check(O, L, Or, Lr, tag=f"D{D} S{S}")
    po, pl = fa.decode_partials(tq, tk, tv, tt, tc, num_splits=S)
    Ors, Lrs = split_partials(q, kp, vp, table, ctx, S)
    assert np.array_equal(np.isneginf(pl.cpu().numpy()), np.isneginf(Lrs)), "empty splits differ"
    fin = np.isfinite(Lrs)
    assert np.abs(po.cpu().numpy()[fin] - Ors[fin]).max() <= 2e-3
    assert (np.abs(pl.cpu().numpy()[fin] - Lrs[fin]) / np.maximum(np.abs(Lrs[fin]), 1)).max() <= 1e-4


@pytest.mark.parametrize("name", sorted(p.stem for p in GOLDEN.glob("decode_*.npz")))
def test_decode_golden(fa, dev, name):
    z = np.load(GOLDEN / f"{name}.npz")
    tq, tk, tv, tt, tc = _dev(dev, z["q"], z["k_pool"], z["v_pool"], z["page_table"], z["ctx_lens"])
    for S in (1, 4, 16):
        O, L = fa.decode_paged(tq, tk, tv, tt, tc, num_splits=S)
        _check(O, L, z["o"], z["l"], tag=f"{name} S{S}")


def test_combine_golden(fa, dev):
    z = np.load(GOLDEN / "combine_b2_s5.npz")
    po, pl = _dev(dev, z["part_o"], z["part_lse"])
    O, L = fa.lse_combine(po, pl)
    _check(O, L, z["o"], z["l"], tag="combine")
    Or, Lr = lse_combine(z["part_o"], z["part_lse"])
    _check(O, L, Or, Lr, tag="combine vs oracle")


def test_gather_bit_exact_one_hot(fa, dev):
    """q is a one-hot with a huge weight on channel 0; exactly one token per
    sequence has K[...,0] = 1, every other K is 0 on that channel, so P is
    one-hot and O must equal that token's V row bit for bit."""
    D, H, B = 128, 4, 6
    ctx = [16, 17, 100, 1000, 33, 500]
    rng = np.random.default_rng(3)
    q, kp, vp, table, ctxa = _small(4, B, H, D, ctx, extra_pages=5)
    q[:] = 0
    q[:, :, 0] = 2000.0                     # logit gap 2000/sqrt(128) ~ 177 > fp32 exp range
    kp[:] = 0
    targets = []
    for b in range(B):
        j = int(rng.integers(0, ctx[b]))
        targets.append(j)
        pid = table[b, j // 16]
        kp[pid, :, j % 16, 0] = 1.0
    tq, tk, tv, tt, tc = _dev(dev, q, kp, vp, table, ctxa)
    for S in (1, 5, 16):
        O, _ = fa.decode_paged(tq, tk, tv, tt, tc, num_splits=S)
        O = O.cpu().numpy()
        for b, j in enumerate(targets):
            want = vp[table[b, j // 16], :, j % 16, :]     # CPU gather of the same pool
            assert np.array_equal(O[b], want), f"seq {b} token {j} S{S}"


def test_page_permutation_bitwise_invariance(fa, dev):
    """Relabel the pages (move pool rows, rewrite the table): identical bits out."""
    q, kp, vp, table, ctx = _small(9, B=4, H=2, D=128, ctx=[40, 700, 129, 16], extra_pages=7)
    P = kp.shape[0]
    relabel = np.random.default_rng(10).permutation(P).astype(np.int32)
    kp2 = np.empty_like(kp)
    vp2 = np.empty_like(vp)
    kp2[relabel] = kp
    vp2[relabel] = vp
    table2 = relabel[table]
    a = fa.decode_paged(*_dev(dev, q, kp, vp, table, ctx), num_splits=8)
    b = fa.decode_paged(*_dev(dev, q, kp2, vp2, table2, ctx), num_splits=8)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_split_count_invariance(fa, dev):
    q, kp, vp, table, ctx = _small(11, B=3, H=2, D=128, ctx=[2000, 37, 513])
    args = _dev(dev, q, kp, vp, table, ctx)
    O1, L1 = fa.decode_paged(*args, num_splits=1)
    for S in (2, 7, 16):
        O2, L2 = fa.decode_paged(*args, num_splits=S)
        assert (O1.float() - O2.float()).abs().max().item() <= 2e-3
        assert ((L1 - L2).abs() / L1.abs().clamp_min(1)).max().item() <= 1e-4
    # one split: the combine pass returns the split partial itself
    po, pl = fa.decode_partials(*args, num_splits=1)
    assert torch.equal(pl[:, :, 0], L1)
    assert torch.equal(po[:, :, 0].half(), O1)


@pytest.mark.parametrize("B,Hkv", [(40, 4), (300, 4), (300, 2)])
def test_sequence_order_is_a_permutation(fa, dev, B, Hkv):
    """Workgroups take sequences longest first (ranked in the kernel for
    B <= 256, identity order above): every sequence is still decoded exactly
    once, repeated and zero lengths included, against the oracle."""
    rng = np.random.default_rng(B + Hkv)
    ctx = rng.integers(0, 60, B)
    ctx[::7] = 33                                   # ties broken by index
    ctx[3] = 0
    H, D = 4, 64
    pages = (ctx + 15) // 16
    P = int(pages.sum()) + 1
    perm = rng.permutation(P).astype(np.int32)
    table = np.zeros((B, max(int(pages.max()), 1)), np.int32)
    off = 0
    for b in range(B):
        table[b, :pages[b]] = perm[off:off + pages[b]]
        off += pages[b]
    q = rng.standard_normal((B, H, D)).astype(np.float16)
    kp = rng.standard_normal((P, Hkv, 16, D)).astype(np.float16)
    vp = rng.standard_normal((P, Hkv, 16, D)).astype(np.float16)
    O, L = fa.decode_paged(*_dev(dev, q, kp, vp, table, ctx.astype(np.int32)), num_splits=3)
    g = H // Hkv
    Or, Lr = decode_attention(q, np.repeat(kp, g, axis=1), np.repeat(vp, g, axis=1), table, ctx)
    O, L = O.float().cpu().numpy(), L.cpu().numpy()
    assert np.abs(O - Or).max() <= 2e-3, f"B{B} Hkv{Hkv} O {np.abs(O - Or).max():.3e}"
    assert np.array_equal(np.isneginf(L), np.isneginf(Lr))   # the empty sequence
    fin = np.isfinite(Lr)
    assert (np.abs(L[fin] - Lr[fin]) / np.maximum(np.abs(Lr[fin]), 1.0)).max() <= 1e-4


def test_bad_page_ids_give_nan_not_fault(fa, dev):
    """Out-of-range page ids and over-long contexts poison only their sequence."""
    q, kp, vp, table, ctx = _small(12, B=3, H=2, D=64, ctx=[20, 40, 30])
    table = table.copy()
    table[1, 1] = kp.shape[0] + 100         # beyond the pool
    ctx = ctx.copy()
    ctx[2] = table.shape[1] * 16 + 50       # beyond the table row
    O, L = fa.decode_paged(*_dev(dev, q, kp, vp, table, ctx), num_splits=4)
    O, L = O.float().cpu().numpy(), L.cpu().numpy()
    assert np.isnan(O[1]).all() and np.isnan(L[1]).all()
    assert np.isnan(O[2]).all() and np.isnan(L[2]).all()
    Or, Lr = decode_attention(q[:1], kp, vp, table[:1], ctx[:1])
    assert np.abs(O[0] - Or[0]).max() <= 2e-3


def test_zero_length_context(fa, dev):
    q, kp, vp, table, ctx = _small(13, B=2, H=2, D=64, ctx=[0, 20])
    O, L = fa.decode_paged(*_dev(dev, q, kp, vp, table, ctx), num_splits=4)
    assert (O[0] == 0).all() and torch.isneginf(L[0]).all()


def test_config5_full_size(fa, dev):
    """Config 5 at full size: B=32, H=32, D=128, ctx ~ U[512, 32768], 16-token
    pages under a random permutation, 16 splits. The pool is filled on the GPU;
    the oracle checks six (b, h) pairs by gathering their pages to the host."""
    B, H, D = 32, 32, 128
    ctx, table, P = make_decode_meta(B=B, seed=5)
    g = torch.Generator(device=dev).manual_seed(5)
    kp = torch.randn(P, H, 16, D, device=dev, dtype=torch.float16, generator=g)
    vp = torch.randn(P, H, 16, D, device=dev, dtype=torch.float16, generator=g)
    q = torch.randn(B, H, D, device=dev, dtype=torch.float16, generator=g)
    tt, tc = _dev(dev, table, ctx)
    O, L = fa.decode_paged(q, kp, vp, tt, tc, num_splits=16)
    torch.cuda.synchronize()
    assert torch.isfinite(O.float()).all() and torch.isfinite(L).all()
    for b, h in ((0, 0), (3, 31), (int(np.argmax(ctx)), 5), (int(np.argmin(ctx)), 17), (20, 9),
                 (31, 30)):
        n_pages = (int(ctx[b]) + 15) // 16
        ids = torch.from_numpy(table[b, :n_pages].astype(np.int64)).to(dev)
        kb = kp[ids, h].reshape(-1, D)[: ctx[b]].cpu().numpy()
        vb = vp[ids, h].reshape(-1, D)[: ctx[b]].cpu().numpy()
        qb = q[b, h].cpu().numpy()
        # the GPU pool was gathered on the device by page id: the oracle sees
        # the contiguous keys of this (b, h)
        Or, Lr = naive_attention(qb[None, None, None], kb[None, None], vb[None, None])
        Or, Lr = Or[:, :, 0], Lr[:, :, 0]
        _check(O[b:b + 1, h:h + 1], L[b:b + 1, h:h + 1], Or, Lr, tag=f"config5 b{b} h{h}")


@pytest.mark.parametrize("D,Hkv,dtype", [(64, 4, torch.float16), (128, 4, torch.float16),
                                         (64, 1, torch.float16), (128, 2, torch.float16),
                                         (128, 1, torch.float16), (128, 4, torch.bfloat16),
                                         (128, 1, torch.bfloat16)])
def test_garbage_past_context_is_ignored(fa, dev, D, Hkv, dtype):
    """Slots past ctx in a sequence's last page hold whatever the pool held
    (pools come from torch.empty; kv_append writes only up to the context).
    NaN and Inf there must not reach O or L: the result equals the oracle's,
    which gathers only the first ctx tokens, for the one-head-per-workgroup
    kernel (Hkv = H) and the grouped kernels (Hkv < H; Hkv = 1 at D = 128 is
    the four-head kernel whose lanes hold two tokens of a page, t and t + 8,
    so the slots past ctx reach both of a lane's tokens)."""
    H = 4
    ctx = [1, 15, 17, 40, 300, 33]
    q, kp, vp, table, ctxa = _small(21 + D + Hkv, B=len(ctx), H=Hkv, D=D, ctx=ctx, extra_pages=1)
    q = np.random.default_rng(22).standard_normal((len(ctx), H, D)).astype(np.float16)
    if dtype == torch.bfloat16:   # values exactly representable in both formats
        q = (np.round(q.astype(np.float32) * 8) / 8).astype(np.float16)
        kp = (np.round(kp.astype(np.float32) * 8) / 8).astype(np.float16)
        vp = (np.round(vp.astype(np.float32) * 8) / 8).astype(np.float16)
    kg, vg = kp.copy(), vp.copy()
    for b, n in enumerate(ctx):
        last = table[b, (n - 1) // 16]
        if n % 16:
            kg[last, :, n % 16:, ::2] = np.inf
            kg[last, :, n % 16:, 1::2] = np.nan
            vg[last, :, n % 16:, ::3] = np.nan
            vg[last, :, n % 16:, 1::3] = np.inf
            vg[last, :, n % 16:, 2::3] = -np.inf
    tq, tk, tv, tt, tc = _dev(dev, q, kg, vg, table, ctxa)
    tq, tk, tv = tq.to(dtype), tk.to(dtype), tv.to(dtype)
    g = H // Hkv
    Or, Lr = decode_attention(q, np.repeat(kp, g, axis=1), np.repeat(vp, g, axis=1), table, ctxa)
    for S in (1, 3):
        O, L = fa.decode_paged(tq, tk, tv, tt, tc, num_splits=S)
        assert torch.isfinite(O.float()).all() and torch.isfinite(L).all(), f"S{S}: non-finite"
        Of, Lf = O.float().cpu().numpy(), L.cpu().numpy()
        tol = 2e-3 if dtype == torch.float16 else 1e-2
        assert np.abs(Of - Or).max() <= tol, f"S{S} O {np.abs(Of - Or).max():.3e}"
        assert (np.abs(Lf - Lr) / np.maximum(np.abs(Lr), 1.0)).max() <= 1e-4
