"""GPU tier: the KV-cache page writer (kv_append) against the oracle's scatter.

The writer is a copy, so the bar is bit-exact: every slot of both pools,
including the slots the call must not touch, equals the oracle's result
(oracle.append_pages). Cases: start positions off page boundaries, tokens
crossing pages, ragged new_lens, T = 0, invalid page ids and positions (flag
set, nothing written), a decode after the append (the writer produces the
format the decode reads), and a full config-3-sized prefill reshaped into
pages, checked by gathering it back on the GPU.
"""
import numpy as np
import pytest
import torch

from oracle import append_pages, decode_attention

pytestmark = pytest.mark.gpu


def _dev(dev, *xs):
    return [torch.from_numpy(np.ascontiguousarray(x)).to(dev) for x in xs]


def _case(seed, B, H, T, D, extra_pages=8):
    rng = np.random.default_rng(seed)
    max_pages = (T + 64) // 16 + 2
    num_pages = B * max_pages + extra_pages
    perm = rng.permutation(num_pages).astype(np.int32)
    table = perm[:B * max_pages].reshape(B, max_pages).copy()
    kp = rng.standard_normal((num_pages, H, 16, D)).astype(np.float16)
    vp = rng.standard_normal((num_pages, H, 16, D)).astype(np.float16)
    kn = rng.standard_normal((B, H, T, D)).astype(np.float16)
    vn = rng.standard_normal((B, H, T, D)).astype(np.float16)
    start = rng.integers(0, 60, size=B).astype(np.int32)
    return kp, vp, table, kn, vn, start


def _run(fa, dev, kp, vp, table, kn, vn, start, lens=None):
    tkp, tvp, ttab, tkn, tvn, tst = _dev(dev, kp, vp, table, kn, vn, start)
    tl = None if lens is None else _dev(dev, lens)[0]
    bad = fa.kv_append(tkn, tvn, tkp, tvp, ttab, tst, tl)
    torch.cuda.synchronize()
    return tkp.cpu().numpy(), tvp.cpu().numpy(), bad.cpu().numpy()


def _check(got, want, tag):
    gk, gv, gb = got
    wk, wv, wb = want
    assert np.array_equal(gk.view(np.uint16), wk.view(np.uint16)), f"{tag}: k_pool differs"
    assert np.array_equal(gv.view(np.uint16), wv.view(np.uint16)), f"{tag}: v_pool differs"
    assert np.array_equal(gb, wb), f"{tag}: bad flags {gb} != {wb}"


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("B,H,T", [(1, 1, 1), (3, 2, 37), (4, 8, 100), (2, 3, 257)])
def test_matches_oracle(fa, dev, B, H, T, D):
    kp, vp, table, kn, vn, start = _case(B * 100 + T + D, B, H, T, D)
    want = append_pages(kp, vp, table, start, kn, vn)
    _check(_run(fa, dev, kp, vp, table, kn, vn, start), want, f"B{B} H{H} T{T} D{D}")


@pytest.mark.parametrize("D", [64, 128])
def test_ragged_lengths(fa, dev, D):
    kp, vp, table, kn, vn, start = _case(7, 5, 2, 50, D)
    lens = np.array([0, 1, 17, 50, 99], np.int32)      # 99 is clamped to T
    want = append_pages(kp, vp, table, start, kn, vn, lens)
    _check(_run(fa, dev, kp, vp, table, kn, vn, start, lens), want, "ragged")
    neg = np.array([-3, 5, 0, 50, 2], np.int32)         # negative counts write nothing
    want = append_pages(kp, vp, table, start, kn, vn, neg)
    _check(_run(fa, dev, kp, vp, table, kn, vn, start, neg), want, "negative lens")


def test_zero_tokens_is_a_noop(fa, dev):
    kp, vp, table, kn, vn, start = _case(8, 2, 2, 0, 64)
    got = _run(fa, dev, kp, vp, table, kn, vn, start)
    _check(got, (kp, vp, np.zeros(2, np.int32)), "T=0")


def test_invalid_pages_and_positions(fa, dev):
    kp, vp, table, kn, vn, start = _case(9, 4, 2, 40, 64)
    start[0], start[1] = 10, 0       # positions 10..49 and 0..39
    table[0, 1] = -5                 # invalid id in the middle of sequence 0
    table[1, 0] = kp.shape[0]        # one past the pool
    start[2] = table.shape[1] * 16 - 7   # runs past the table
    start[3] = -2                    # negative start: first two tokens dropped
    want = append_pages(kp, vp, table, start, kn, vn)
    assert want[2].tolist() == [1, 1, 1, 1]
    _check(_run(fa, dev, kp, vp, table, kn, vn, start), want, "invalid")


@pytest.mark.parametrize("D", [64, 128])
def test_append_then_decode(fa, dev, D):
    """Prefill through kv_append, one decode step, one more append, decode again."""
    B, H = 3, 4
    rng = np.random.default_rng(D)
    ctx = np.array([1, 40, 130], np.int32)
    max_pages = 10
    num_pages = B * max_pages
    table = rng.permutation(num_pages).astype(np.int32).reshape(B, max_pages)
    k_all = rng.standard_normal((B, H, 140, D)).astype(np.float16)
    v_all = rng.standard_normal((B, H, 140, D)).astype(np.float16)
    kp = np.zeros((num_pages, H, 16, D), np.float16)
    vp = np.zeros_like(kp)
    tkp, tvp, ttab = _dev(dev, kp, vp, table)
    tk, tv = _dev(dev, k_all, v_all)
    bad = fa.kv_append(tk[:, :, :130].contiguous(), tv[:, :, :130].contiguous(), tkp, tvp, ttab,
                       torch.zeros(B, dtype=torch.int32, device=dev),
                       torch.from_numpy(ctx).to(dev))
    assert int(bad.sum()) == 0
    q = rng.standard_normal((B, H, D)).astype(np.float16)
    tq = _dev(dev, q)[0]
    O, L = fa.decode_paged(tq, tkp, tvp, ttab, torch.from_numpy(ctx).to(dev), 4)
    Or, Lr = decode_attention(q, tkp.cpu().numpy(), tvp.cpu().numpy(), table, ctx)
    assert np.abs(O.float().cpu().numpy() - Or).max() <= 2e-3
    assert (np.abs(L.cpu().numpy() - Lr) / np.maximum(np.abs(Lr), 1)).max() <= 1e-4
    # append one generated token per sequence at position ctx[b], decode over ctx + 1
    nk = _dev(dev, rng.standard_normal((B, H, 1, D)).astype(np.float16))[0]
    nv = _dev(dev, rng.standard_normal((B, H, 1, D)).astype(np.float16))[0]
    bad = fa.kv_append(nk, nv, tkp, tvp, ttab, torch.from_numpy(ctx).to(dev))
    assert int(bad.sum()) == 0
    ctx1 = ctx + 1
    O, L = fa.decode_paged(tq, tkp, tvp, ttab, torch.from_numpy(ctx1).to(dev), 4)
    kp_h, vp_h = tkp.cpu().numpy(), tvp.cpu().numpy()
    Or, Lr = decode_attention(q, kp_h, vp_h, table, ctx1)
    assert np.abs(O.float().cpu().numpy() - Or).max() <= 2e-3
    # the new token sits in slot ctx % 16 of page table[b][ctx // 16]
    for b in range(B):
        pid, slot = table[b, ctx[b] // 16], ctx[b] % 16
        assert np.array_equal(kp_h[pid, :, slot], nk[b, :, 0].cpu().numpy())


def test_prefill_into_pages_config3_size(fa, dev):
    """B4 H16 N4096 D128 reshaped into pages, read back by gathering on the GPU."""
    B, H, N, D = 4, 16, 4096, 128
    g = torch.Generator(device=dev).manual_seed(3)
    k = torch.randn(B, H, N, D, device=dev, generator=g).half()
    v = torch.randn(B, H, N, D, device=dev, generator=g).half()
    pages = N // 16
    num_pages = B * pages
    table = torch.randperm(num_pages, device=dev, generator=g).to(torch.int32).view(B, pages)
    kp = torch.empty(num_pages, H, 16, D, dtype=torch.half, device=dev)
    vp = torch.empty_like(kp)
    bad = fa.kv_append(k, v, kp, vp, table, torch.zeros(B, dtype=torch.int32, device=dev))
    assert int(bad.sum()) == 0
    # pool[table[b, p], h, s] == k[b, h, 16 p + s]
    back_k = kp[table.long()].permute(0, 2, 1, 3, 4).reshape(B, H, N, D)
    back_v = vp[table.long()].permute(0, 2, 1, 3, 4).reshape(B, H, N, D)
    assert torch.equal(back_k, k) and torch.equal(back_v, v)


def test_rejects_bad_arguments(fa, dev):
    kp = torch.zeros(4, 2, 16, 64, dtype=torch.half, device=dev)
    kn = torch.zeros(1, 2, 3, 64, dtype=torch.half, device=dev)
    tab = torch.zeros(1, 2, dtype=torch.int32, device=dev)
    st = torch.zeros(1, dtype=torch.int32, device=dev)
    with pytest.raises(RuntimeError, match="float16"):
        fa.kv_append(kn.float(), kn.float(), kp, kp, tab, st)
    with pytest.raises(RuntimeError, match="page_size must be 16"):
        p8 = torch.zeros(4, 2, 8, 64, dtype=torch.half, device=dev)
        fa.kv_append(kn, kn, p8, p8.clone(), tab, st)
    with pytest.raises(RuntimeError, match="int32"):
        fa.kv_append(kn, kn, kp, kp.clone(), tab.long(), st)


@pytest.mark.parametrize("D,Hkv", [(64, 8), (128, 2)])
def test_decode_agrees_with_causal_forward(fa, dev, D, Hkv):
    """The serving invariant between the two paths: K and V written into pages
    by kv_append, then decoding the query of position t over the first t + 1
    tokens gives row t of the causal forward over the same Q, K, V (both
    against the same fp32 oracle at the forward's bars: O within 2e-3 each, so
    4e-3 apart at most; L within 1e-4 relative)."""
    B, H, N = 2, 8, 1000
    g = torch.Generator(device=dev).manual_seed(D + Hkv)
    q = torch.randn(B, H, N, D, device=dev, generator=g).half()
    k = torch.randn(B, Hkv, N, D, device=dev, generator=g).half()
    v = torch.randn(B, Hkv, N, D, device=dev, generator=g).half()
    O, L = fa.forward(q, k, v, causal=True)
    pages = (N + 15) // 16
    table = torch.randperm(B * pages, device=dev, generator=g).to(torch.int32).view(B, pages)
    kp = torch.zeros(B * pages, Hkv, 16, D, dtype=torch.half, device=dev)
    vp = torch.zeros_like(kp)
    bad = fa.kv_append(k, v, kp, vp, table, torch.zeros(B, dtype=torch.int32, device=dev))
    assert int(bad.sum()) == 0
    for t in (0, 15, 16, 517, N - 1):
        ctx = torch.full((B,), t + 1, dtype=torch.int32, device=dev)
        Od, Ld = fa.decode_paged(q[:, :, t].contiguous(), kp, vp, table, ctx, 16)
        torch.cuda.synchronize()
        d_o = (Od.float() - O[:, :, t].float()).abs().max().item()
        d_l = ((Ld - L[:, :, t]).abs() / L[:, :, t].abs().clamp(min=1)).max().item()
        assert d_o <= 4e-3, f"t {t}: O differs by {d_o:.2e}"
        assert d_l <= 1e-4, f"t {t}: L differs by {d_l:.2e}"
