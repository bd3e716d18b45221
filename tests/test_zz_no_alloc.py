"""GPU tier: fa_decode_paged_noalloc_f16, the paged decode that allocates nothing.

It runs the kernels of fa_decode_paged_gqa_f16 with the split partials in the
library's static device array instead of a caller workspace, so its O and L
must equal that entry point's bit for bit. Both are called through the C ABI
(ctypes, raw device pointers). Two calls in a row, the second smaller, show
that nothing left in the array by one call leaks into the next; a call near
the array's limit touches its far end; a call captured in a HIP graph replays
correctly after the device's first call. O and L are also held to the oracle
(oracle/naive.py: decode_attention) at the decode bars: O max-abs <= 2e-3,
L relative <= 1e-4.
"""
import numpy as np
import pytest
import torch

from oracle import decode_attention

pytestmark = pytest.mark.gpu


def _case(seed, B, H, Hkv, D, ctx):
    rng = np.random.default_rng(seed)
    pages = [(c + 15) // 16 for c in ctx]
    P = max(sum(pages), 1) + 3
    perm = rng.permutation(P).astype(np.int32)
    table = np.zeros((B, max(max(pages), 1)), np.int32)
    off = 0
    for b in range(B):
        table[b, :pages[b]] = perm[off:off + pages[b]]
        off += pages[b]
    q = rng.standard_normal((B, H, D)).astype(np.float16)
    kp = rng.standard_normal((P, Hkv, 16, D)).astype(np.float16)
    vp = rng.standard_normal((P, Hkv, 16, D)).astype(np.float16)
    return q, kp, vp, table, np.asarray(ctx, np.int32)


def _to(dev, *xs):
    return [torch.from_numpy(np.ascontiguousarray(x)).to(dev) for x in xs]


def _run(lib, fn, tq, tk, tv, tt, tc, Hkv, S, stream, workspace):
    B, H, D = tq.shape
    o = torch.full((B, H, D), float("nan"), device=tq.device, dtype=torch.float16)
    lse = torch.full((B, H), float("nan"), device=tq.device, dtype=torch.float32)
    head = (tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), tt.data_ptr(), tc.data_ptr(),
            B, H, Hkv, D, 16, tt.shape[1], tk.shape[0], S)
    if workspace:
        n = lib.fa_decode_workspace_floats(B, H, D, S)
        ws = torch.empty(n, device=tq.device, dtype=torch.float32)
        st = fn(*head, ws.data_ptr(), ws.data_ptr() + 4 * B * H * S * D, o.data_ptr(),
                lse.data_ptr(), stream)
    else:
        st = fn(*head, o.data_ptr(), lse.data_ptr(), stream)
    assert st == 0, lib.fa_status_str(st)
    torch.cuda.synchronize()
    return o, lse


def _compare(lib, dev, case, Hkv, S, stream, tag):
    q, kp, vp, table, ctx = case
    tq, tk, tv, tt, tc = _to(dev, q, kp, vp, table, ctx)
    print(f"[no-alloc] {tag}: B{q.shape[0]} H{q.shape[1]} Hkv{Hkv} D{q.shape[2]} S{S}", flush=True)
    o_na, l_na = _run(lib, lib.fa_decode_paged_noalloc_f16, tq, tk, tv, tt, tc, Hkv, S, stream,
                      workspace=False)
    o_ws, l_ws = _run(lib, lib.fa_decode_paged_gqa_f16, tq, tk, tv, tt, tc, Hkv, S, stream,
                      workspace=True)
    assert torch.equal(o_na, o_ws), f"{tag}: O differs from fa_decode_paged_gqa_f16"
    assert torch.equal(l_na, l_ws), f"{tag}: L differs from fa_decode_paged_gqa_f16"
    g = q.shape[1] // Hkv
    Or, Lr = decode_attention(q, np.repeat(kp, g, axis=1), np.repeat(vp, g, axis=1), table, ctx)
    O = o_na.float().cpu().numpy()
    L = l_na.cpu().numpy()
    live = ctx > 0
    assert np.abs(O - Or).max() <= 2e-3, f"{tag}: O max-abs {np.abs(O - Or).max():.3e}"
    rel = np.abs(L[live] - Lr[live]) / np.maximum(np.abs(Lr[live]), 1.0)
    assert rel.max() <= 1e-4, f"{tag}: L rel {rel.max():.3e}"
    assert np.all(np.isneginf(L[~live])) and np.all(O[~live] == 0)


def test_two_calls_second_smaller_match_workspace_entry(capi, dev):
    lib = capi.load()
    stream = torch.cuda.current_stream().cuda_stream
    rng = np.random.default_rng(71)
    big = _case(72, B=6, H=16, Hkv=4, D=128,
                ctx=rng.integers(1, 3000, size=6).tolist())
    _compare(lib, dev, big, Hkv=4, S=16, stream=stream, tag="first call")
    small = _case(73, B=3, H=4, Hkv=4, D=64, ctx=[0, 17, 250])
    _compare(lib, dev, small, Hkv=4, S=3, stream=stream, tag="second call, smaller")


def test_near_the_limit_on_a_side_stream(capi, dev):
    """B*H*S*(D+1) within 6% of the array's size, on a stream other than the default."""
    lib = capi.load()
    B, H, S, D = 64, 32, 15, 128
    assert B * H * S * (D + 1) <= capi.DECODE_SCRATCH_FLOATS < B * H * (S + 1) * (D + 1)
    case = _case(74, B=B, H=H, Hkv=8, D=D, ctx=[1 + (7 * b) % 60 for b in range(B)])
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        _compare(lib, dev, case, Hkv=8, S=S, stream=side.cuda_stream, tag="near the limit")


def test_rejects_beyond_the_limit(capi, dev):
    lib = capi.load()
    q, kp, vp, table, ctx = _case(75, B=2, H=2, Hkv=2, D=64, ctx=[5, 9])
    tq, tk, tv, tt, tc = _to(dev, q, kp, vp, table, ctx)
    o = torch.zeros(2, 2, 64, device=dev, dtype=torch.float16)
    # H = 65535 query heads with 16 splits need 65535*16*65 floats > 2^22; the
    # size check comes before any launch, so the small buffers are never read.
    st = lib.fa_decode_paged_noalloc_f16(tq.data_ptr(), tk.data_ptr(), tv.data_ptr(),
                                         tt.data_ptr(), tc.data_ptr(), 1, 65535, 65535, 64, 16,
                                         tt.shape[1], tk.shape[0], 16, o.data_ptr(), None, None)
    assert st == capi.STATUS["FA_ERR_SCRATCH_SIZE"]
    assert b"FA_DECODE_SCRATCH_FLOATS" in lib.fa_status_str(st)
    torch.cuda.synchronize()
    assert torch.count_nonzero(o) == 0


def test_captured_in_a_hip_graph(capi, dev):
    """After one call outside capture (which resolves the array's address on
    this device), a call captured in a HIP graph replays correctly: every
    replay, with eager work and synchronisations between them and new q
    values copied into the captured buffer, equals fa_decode_paged_gqa_f16 on
    the same inputs bit for bit. The entry point records only kernels (no
    memset node, no allocation)."""
    lib = capi.load()
    B, H, Hkv, D, S = 5, 8, 2, 128, 6
    q, kp, vp, table, ctx = _case(76, B=B, H=H, Hkv=Hkv, D=D, ctx=[1, 40, 700, 16, 2100])
    tq, tk, tv, tt, tc = _to(dev, q, kp, vp, table, ctx)
    head = lambda: (tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), tt.data_ptr(), tc.data_ptr(),  # noqa: E731
                    B, H, Hkv, D, 16, tt.shape[1], tk.shape[0], S)
    o = torch.zeros(B, H, D, device=dev, dtype=torch.float16)
    lse = torch.zeros(B, H, device=dev, dtype=torch.float32)
    stream = torch.cuda.current_stream().cuda_stream
    assert lib.fa_decode_paged_noalloc_f16(*head(), o.data_ptr(), lse.data_ptr(), stream) == 0
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        cs = torch.cuda.current_stream().cuda_stream
        st = lib.fa_decode_paged_noalloc_f16(*head(), o.data_ptr(), lse.data_ptr(), cs)
    assert st == 0, lib.fa_status_str(st)
    rng = np.random.default_rng(77)
    for rep in range(4):
        new_q = rng.standard_normal((B, H, D)).astype(np.float16)
        tq.copy_(torch.from_numpy(new_q).to(dev))
        o.fill_(float("nan"))
        lse.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        o_ws, l_ws = _run(lib, lib.fa_decode_paged_gqa_f16, tq, tk, tv, tt, tc, Hkv, S, stream,
                          workspace=True)
        assert torch.equal(o, o_ws), f"replay {rep}: O differs"
        assert torch.equal(lse, l_ws), f"replay {rep}: L differs"
        _ = (torch.randn(256, 256, device=dev) @ torch.randn(256, 256, device=dev)).sum().item()
