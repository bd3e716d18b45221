"""CPU tier: the C-ABI library loads, exports every declared symbol, and rejects
bad arguments before any HIP call (the reference's argument checks,
cuda/flash_attn_fa3_db_full.cu:352-363, restated as status codes)."""
import ctypes as C

import pytest


def test_library_exports_every_header_symbol(capi):
    lib = capi.load()
    names = capi.header_symbols()
    assert "fa_fwd_f16" in names and "fa_decode_paged_f16" in names and "fa_probe_chain" in names
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    assert set(names) == set(capi.SIGNATURES), "ctypes signatures out of sync with include/*.h"


def test_abi_version_and_status_strings(capi):
    lib = capi.load()
    assert lib.fa_abi_version() == 1
    assert lib.fa_status_str(0) == b"ok"
    assert b"64 or 128" in lib.fa_status_str(capi.STATUS["FA_ERR_HEAD_DIM"])
    assert b"N must be > 0" == lib.fa_status_str(capi.STATUS["FA_ERR_SEQ_LEN"])
    assert b"HIP" in lib.fa_status_str(-1)


A = 0x10000   # a fake, 16-byte aligned address: never dereferenced by validation


@pytest.mark.parametrize("args,code", [
    ((0, A, A, A, 1, 1, 64, 64), "FA_ERR_NULL_POINTER"),
    ((A, A, A, 0, 1, 1, 64, 64), "FA_ERR_NULL_POINTER"),
    ((A, A, A, A, 1, 1, 64, 32), "FA_ERR_HEAD_DIM"),
    ((A, A, A, A, 1, 1, 64, 96), "FA_ERR_HEAD_DIM"),
    ((A, A, A, A, 1, 1, 0, 64), "FA_ERR_SEQ_LEN"),
    ((A, A, A, A, 1, 1, -5, 64), "FA_ERR_SEQ_LEN"),
    ((A, A, A, A, 0, 1, 64, 64), "FA_ERR_BATCH_HEADS"),
    ((A, A, A, A, 1, 0, 64, 64), "FA_ERR_BATCH_HEADS"),
    ((A + 2, A, A, A, 1, 1, 64, 64), "FA_ERR_ALIGNMENT"),
    ((A, A, A, A, 1, 1, 1 << 25, 128), "FA_ERR_TOO_LARGE"),
    ((A, A, A, A, 1 << 20, 1 << 20, 128, 64), "FA_ERR_TOO_LARGE"),
    ((A, A, A, A, 1, 8, 4096, 64), "FA_OK"),
    ((A, A, A, A, 4, 16, 4096, 128), "FA_OK"),
    ((A, A, A, A, 1, 1, 1, 64), "FA_OK"),
])
def test_validate_fwd(capi, args, code):
    lib = capi.load()
    assert lib.fa_validate_fwd(*args) == capi.STATUS[code]


def test_fwd_rejects_before_touching_the_device(capi):
    lib = capi.load()
    # invalid arguments return their status without any HIP call (no GPU here)
    assert lib.fa_fwd_f16(A, A, A, A, None, 1, 1, 64, 80, 0, None) == capi.STATUS["FA_ERR_HEAD_DIM"]
    assert lib.fa_fwd_f16(A, A, A, A, A + 2, 1, 1, 64, 64, 0, None) == capi.STATUS["FA_ERR_ALIGNMENT"]
    assert lib.fa_fwd_f16(A, 0, A, A, None, 1, 1, 64, 64, 1, None) == capi.STATUS["FA_ERR_NULL_POINTER"]


def _dec(**kw):
    base = dict(q=A, k=A, v=A, pt=A, ctx=A, B=32, H=32, D=128, ps=16, maxp=2048, np_=33000, S=16)
    base.update(kw)
    b = base
    return (b["q"], b["k"], b["v"], b["pt"], b["ctx"], b["B"], b["H"], b["D"], b["ps"], b["maxp"],
            b["np_"], b["S"])


@pytest.mark.parametrize("kw,code", [
    (dict(), "FA_OK"),
    (dict(pt=0), "FA_ERR_NULL_POINTER"),
    (dict(D=96), "FA_ERR_HEAD_DIM"),
    (dict(B=0), "FA_ERR_BATCH_HEADS"),
    (dict(ps=32), "FA_ERR_PAGE_SIZE"),
    (dict(S=0), "FA_ERR_NUM_SPLITS"),
    (dict(S=17), "FA_ERR_NUM_SPLITS"),
    (dict(maxp=0), "FA_ERR_MAX_PAGES"),
    (dict(np_=0), "FA_ERR_NUM_PAGES"),
    (dict(k=A + 8), "FA_ERR_ALIGNMENT"),
    (dict(ctx=A + 2), "FA_ERR_ALIGNMENT"),
    (dict(H=70000), "FA_ERR_TOO_LARGE"),
])
def test_validate_decode(capi, kw, code):
    lib = capi.load()
    assert lib.fa_validate_decode(*_dec(**kw)) == capi.STATUS[code]


def test_noalloc_decode_rejects_before_touching_the_device(capi):
    lib = capi.load()
    fn = lib.fa_decode_paged_noalloc_f16
    head = (A, A, A, A, A)
    # 64 * 32 * 16 * (128 + 1) floats of partials exceed the 2^22 of the array
    assert 64 * 32 * 16 * 129 > capi.DECODE_SCRATCH_FLOATS
    assert fn(*head, 64, 32, 32, 128, 16, 2048, 33000, 16, A, A, None) == \
        capi.STATUS["FA_ERR_SCRATCH_SIZE"]
    assert fn(*head, 32, 32, 5, 128, 16, 2048, 33000, 16, A, A, None) == \
        capi.STATUS["FA_ERR_KV_HEADS"]
    assert fn(*head, 32, 32, 8, 128, 16, 2048, 33000, 16, None, A, None) == \
        capi.STATUS["FA_ERR_NULL_POINTER"]
    assert fn(*head, 32, 32, 8, 128, 16, 2048, 33000, 17, A, A, None) == \
        capi.STATUS["FA_ERR_NUM_SPLITS"]


def test_decode_rejects_before_touching_the_device(capi):
    lib = capi.load()
    args = _dec(S=20)
    assert lib.fa_decode_paged_f16(*args, A, A, A, A, None) == capi.STATUS["FA_ERR_NUM_SPLITS"]
    assert lib.fa_decode_split_f16(*_dec(), 0, A, None) == capi.STATUS["FA_ERR_NULL_POINTER"]
    assert lib.fa_lse_combine_f32(A, A, 1, 1, 64, 0, A, None, None) == capi.STATUS["FA_ERR_NUM_SPLITS"]
    assert lib.fa_decode_workspace_floats(32, 32, 128, 16) == 32 * 32 * 16 * 129


def test_torch_binding_checks_mirror_reference(fa):
    """The reference checks is_cuda first (cuda/flash_attn_fa3_db_full.cu:352)."""
    import torch
    x = torch.zeros(1, 1, 8, 64)
    with pytest.raises(RuntimeError, match="Q/K/V must be CUDA tensors"):
        fa.forward(x, x, x)
    with pytest.raises(RuntimeError, match="Q/K/V must be CUDA tensors"):
        fa.forward_only(x, x, x, causal=True)
    with pytest.raises(RuntimeError, match="must be CUDA tensors"):
        fa.decode_paged(torch.zeros(1, 1, 64, dtype=torch.half),
                        torch.zeros(1, 1, 16, 64, dtype=torch.half),
                        torch.zeros(1, 1, 16, 64, dtype=torch.half),
                        torch.zeros(1, 1, dtype=torch.int32), torch.ones(1, dtype=torch.int32))


def test_package_loads_native_libraries(fa):
    libs = fa.loaded_libraries()
    assert any(p.endswith("libfa_mi355x.so") for p in libs)
    assert any("_fa_torch" in p for p in libs)


def _bwd(**kw):
    b = dict(q=A, k=A, v=A, o=A, do=A, lse=A, dq=A, dk=A, dv=A, ws=A, B=1, H=8, N=4096, D=64)
    b.update(kw)
    return tuple(b[k] for k in ("q", "k", "v", "o", "do", "lse", "dq", "dk", "dv", "ws",
                                "B", "H", "N", "D"))


@pytest.mark.parametrize("kw,code", [
    (dict(), "FA_OK"),
    (dict(D=128, B=4, H=16), "FA_OK"),
    (dict(N=1), "FA_OK"),
    (dict(do=0), "FA_ERR_NULL_POINTER"),
    (dict(lse=0), "FA_ERR_NULL_POINTER"),
    (dict(ws=0), "FA_ERR_NULL_POINTER"),
    (dict(dv=0), "FA_ERR_NULL_POINTER"),
    (dict(q=0), "FA_ERR_NULL_POINTER"),
    (dict(D=96), "FA_ERR_HEAD_DIM"),
    (dict(N=0), "FA_ERR_SEQ_LEN"),
    (dict(H=0), "FA_ERR_BATCH_HEADS"),
    (dict(do=A + 8), "FA_ERR_ALIGNMENT"),
    (dict(dk=A + 4), "FA_ERR_ALIGNMENT"),
    (dict(lse=A + 2), "FA_ERR_ALIGNMENT"),
    (dict(lse=A + 4), "FA_OK"),
    (dict(B=1 << 20, H=1 << 20, N=128), "FA_ERR_TOO_LARGE"),
])
def test_validate_bwd(capi, kw, code):
    lib = capi.load()
    assert lib.fa_validate_bwd(*_bwd(**kw)) == capi.STATUS[code]


def test_bwd_rejects_before_touching_the_device(capi):
    lib = capi.load()
    assert lib.fa_bwd_f16(*_bwd(D=80), 0, None) == capi.STATUS["FA_ERR_HEAD_DIM"]
    assert lib.fa_bwd_f16(*_bwd(ws=0), 1, None) == capi.STATUS["FA_ERR_NULL_POINTER"]
    assert lib.fa_bwd_workspace_floats(2, 8, 4096) == 2 * 2 * 8 * 4096
    assert lib.fa_bwd_workspace_floats(0, 8, 4096) == 0


def test_torch_backward_checks_mirror_reference(fa):
    """The reference checks Q then dO for is_cuda (cuda/flash_attn_kernel.cu:425-426)."""
    import torch
    x = torch.zeros(1, 1, 8, 64)
    with pytest.raises(RuntimeError, match="Q must be a CUDA tensor"):
        fa.backward(x, x, x, x, x, torch.zeros(1, 1, 8))


def _kv(**kw):
    b = dict(kn=A, vn=A, pt=A, st=A, nl=None, kp=A, vp=A, bad=None, B=32, H=8, T=1, D=128, ps=16,
             maxp=2048, np_=65536)
    b.update(kw)
    return tuple(b[k] for k in ("kn", "vn", "pt", "st", "nl", "kp", "vp", "bad", "B", "H", "T",
                                "D", "ps", "maxp", "np_"))


@pytest.mark.parametrize("kw,code", [
    (dict(), "FA_OK"),
    (dict(T=0), "FA_OK"),
    (dict(T=0, kn=0, vn=0), "FA_OK"),
    (dict(T=1, kn=0), "FA_ERR_NULL_POINTER"),
    (dict(nl=A, bad=A, T=4096, D=64), "FA_OK"),
    (dict(T=-1), "FA_ERR_SEQ_LEN"),
    (dict(kp=0), "FA_ERR_NULL_POINTER"),
    (dict(st=0), "FA_ERR_NULL_POINTER"),
    (dict(D=96), "FA_ERR_HEAD_DIM"),
    (dict(B=0), "FA_ERR_BATCH_HEADS"),
    (dict(ps=32), "FA_ERR_PAGE_SIZE"),
    (dict(maxp=0), "FA_ERR_MAX_PAGES"),
    (dict(np_=0), "FA_ERR_NUM_PAGES"),
    (dict(vn=A + 8), "FA_ERR_ALIGNMENT"),
    (dict(nl=A + 2), "FA_ERR_ALIGNMENT"),
    (dict(H=70000), "FA_ERR_TOO_LARGE"),
])
def test_validate_kv_append(capi, kw, code):
    lib = capi.load()
    assert lib.fa_validate_kv_append(*_kv(**kw)) == capi.STATUS[code]


def test_kv_append_rejects_before_touching_the_device(capi):
    lib = capi.load()
    assert lib.fa_kv_append_f16(*_kv(ps=8), None) == capi.STATUS["FA_ERR_PAGE_SIZE"]
    assert lib.fa_kv_append_f16(*_kv(T=0), None) == capi.STATUS["FA_OK"]   # no launch


@pytest.mark.parametrize("args,code", [
    ((A, A, A, A, 2, 8, 2, 1024, 64), "FA_OK"),
    ((A, A, A, A, 2, 8, 1, 1024, 128), "FA_OK"),
    ((A, A, A, A, 2, 8, 3, 1024, 64), "FA_ERR_KV_HEADS"),
    ((A, A, A, A, 2, 8, 0, 1024, 64), "FA_ERR_KV_HEADS"),
    ((A, A, A, A, 2, 8, 16, 1024, 64), "FA_ERR_KV_HEADS"),
    ((A, A, A, A, 2, 8, 2, 1024, 96), "FA_ERR_HEAD_DIM"),
])
def test_validate_fwd_gqa(capi, args, code):
    lib = capi.load()
    assert lib.fa_validate_fwd_gqa(*args) == capi.STATUS[code]


@pytest.mark.parametrize("args,code", [
    ((A, A, A, A, A, 7, 4, 2, 1024, 1573, 64), "FA_OK"),
    ((A, A, A, A, A, 7, 4, 2, 1024, 0, 128), "FA_OK"),
    ((A, A, A, A, 0, 7, 4, 2, 1024, 1573, 64), "FA_ERR_NULL_POINTER"),
    ((A, A, A, A, A + 2, 7, 4, 2, 1024, 1573, 64), "FA_ERR_ALIGNMENT"),
    ((A, A, A, A, A, 7, 4, 3, 1024, 1573, 64), "FA_ERR_KV_HEADS"),
    ((A, A, A, A, A, 7, 4, 2, 0, 1573, 64), "FA_ERR_SEQ_LEN"),
    ((A, A, A, A, A, 7, 4, 2, 1024, -1, 64), "FA_ERR_SEQ_LEN"),
    ((A, A, A, A, A, 0, 4, 2, 1024, 1573, 64), "FA_ERR_BATCH_HEADS"),
    ((A, A, A, A, A, 7, 4, 2, 1 << 24, 1573, 64), "FA_ERR_TOO_LARGE"),
])
def test_validate_fwd_varlen(capi, args, code):
    lib = capi.load()
    assert lib.fa_validate_fwd_varlen(*args) == capi.STATUS[code]


def test_gqa_entry_points_reject_before_touching_the_device(capi):
    lib = capi.load()
    assert lib.fa_fwd_gqa_f16(A, A, A, A, None, 1, 8, 3, 64, 64, 0, None) == capi.STATUS["FA_ERR_KV_HEADS"]
    assert lib.fa_fwd_varlen_f16(A, A, A, A, None, 0, 1, 8, 8, 64, 64, 64, 0, None) == \
        capi.STATUS["FA_ERR_NULL_POINTER"]
    args = list(_dec())
    # (q, k, v, pt, ctx, B, H, D, ps, maxp, np_, S) -> insert H_kv after H
    gqa = args[:7] + [5] + args[7:] + [A, A, A, None, None]
    assert lib.fa_decode_paged_gqa_f16(*gqa) == capi.STATUS["FA_ERR_KV_HEADS"]
    assert lib.fa_status_str(capi.STATUS["FA_ERR_KV_HEADS"]) == b"H must be a positive multiple of H_kv"


def test_bwd_gqa_workspace_and_rejections(capi):
    lib = capi.load()
    assert lib.fa_bwd_gqa_workspace_floats(2, 8, 8, 4096, 64) == 2 * 2 * 8 * 4096
    n = 2 * 1 * 3 * 5
    assert lib.fa_bwd_gqa_workspace_floats(1, 3, 1, 5, 64) == (n + 3) // 4 * 4 + 2 * 3 * 5 * 64
    assert lib.fa_bwd_gqa_workspace_floats(1, 3, 2, 5, 64) == 0
    args = list(_bwd(H=8))
    gqa = args[:12] + [3] + args[12:]          # insert H_kv after H
    assert lib.fa_bwd_gqa_f16(*gqa, 0, None) == capi.STATUS["FA_ERR_KV_HEADS"]
    gqa = args[:12] + [2] + args[12:]
    gqa[9] = A + 4                             # workspace only 4-byte aligned
    assert lib.fa_bwd_gqa_f16(*gqa, 0, None) == capi.STATUS["FA_ERR_ALIGNMENT"]
    # the bf16 backward shares the checks
    assert lib.fa_bwd_bf16(*gqa, 0, None) == capi.STATUS["FA_ERR_ALIGNMENT"]
    gqa = args[:12] + [3] + args[12:]
    assert lib.fa_bwd_bf16(*gqa, 0, None) == capi.STATUS["FA_ERR_KV_HEADS"]
    gqa[0] = None
    assert lib.fa_bwd_bf16(*gqa, 0, None) == capi.STATUS["FA_ERR_NULL_POINTER"]


def test_validate_bwd_varlen(capi):
    lib = capi.load()
    ok = [A] * 11 + [3, 8, 2, 512, 1000, 64]
    assert lib.fa_validate_bwd_varlen(*ok) == capi.STATUS["FA_OK"]
    bad = list(ok); bad[10] = None                     # cu_seqlens
    assert lib.fa_validate_bwd_varlen(*bad) == capi.STATUS["FA_ERR_NULL_POINTER"]
    bad = list(ok); bad[4] = None                      # dout
    assert lib.fa_validate_bwd_varlen(*bad) == capi.STATUS["FA_ERR_NULL_POINTER"]
    bad = list(ok); bad[13] = 3                        # H_kv does not divide H
    assert lib.fa_validate_bwd_varlen(*bad) == capi.STATUS["FA_ERR_KV_HEADS"]
    bad = list(ok); bad[16] = 96
    assert lib.fa_validate_bwd_varlen(*bad) == capi.STATUS["FA_ERR_HEAD_DIM"]
    bad = list(ok); bad[6] = A + 8                     # dq not 16-byte aligned
    assert lib.fa_validate_bwd_varlen(*bad) == capi.STATUS["FA_ERR_ALIGNMENT"]
    bad = list(ok); bad[14] = 0                        # max_seqlen
    assert lib.fa_validate_bwd_varlen(*bad) == capi.STATUS["FA_ERR_SEQ_LEN"]
    # the entry point rejects before touching the device
    assert lib.fa_bwd_varlen_f16(*bad, 0, None) == capi.STATUS["FA_ERR_SEQ_LEN"]


def test_bf16_decode_and_page_writer_reject_before_touching_the_device(capi):
    """The bf16 entry points run the fp16 ones' checks first (no launch)."""
    lib = capi.load()
    args = list(_dec())
    gqa = args[:7] + [5] + args[7:] + [A, A, A, None, None]     # H_kv 5 does not divide H
    assert lib.fa_decode_paged_bf16(*gqa) == capi.STATUS["FA_ERR_KV_HEADS"]
    bad_s = list(_dec(S=20))
    gqa = bad_s[:7] + [bad_s[6]] + bad_s[7:] + [A, A, A, None, None]
    assert lib.fa_decode_paged_bf16(*gqa) == capi.STATUS["FA_ERR_NUM_SPLITS"]
    ok = list(_dec())
    gqa = ok[:7] + [ok[6]] + ok[7:] + [0, A, A, None, None]      # no part_o
    assert lib.fa_decode_paged_bf16(*gqa) == capi.STATUS["FA_ERR_NULL_POINTER"]
    assert lib.fa_kv_append_bf16(*_kv(ps=8), None) == capi.STATUS["FA_ERR_PAGE_SIZE"]
    assert lib.fa_kv_append_bf16(*_kv(T=0), None) == capi.STATUS["FA_OK"]   # no launch


def test_read_probe_rejects_before_touching_the_device(capi):
    """fa_probe_read_bw and fa_probe_gather_bw check their pointers, sizes,
    alignment and grid first."""
    lib = capi.load()
    assert lib.fa_probe_read_bw(None, 1024, 8, A, None) == 1
    assert lib.fa_probe_read_bw(A, 1024, 8, None, None) == 1
    assert lib.fa_probe_read_bw(A, 1000, 8, A, None) == 2     # not a multiple of 16
    assert lib.fa_probe_read_bw(A, 0, 8, A, None) == 2
    assert lib.fa_probe_read_bw(A, 1024, 0, A, None) == 2     # no workgroups
    assert lib.fa_probe_read_bw(A + 8, 1024, 8, A, None) == 2  # 8-byte aligned only
    g = lib.fa_probe_gather_bw   # (k, v, table, pages, pages_per_wg, nontemporal, sink, stream)
    assert g(None, A, A, 16, 4, 1, A, None) == 1
    assert g(A, A, None, 16, 4, 1, A, None) == 1
    assert g(A, A, A, 16, 4, 1, None, None) == 1
    assert g(A, A, A, 0, 4, 1, A, None) == 2          # no pages
    assert g(A, A, A, 16, 0, 1, A, None) == 2         # no pages per workgroup
    assert g(A, A + 8, A, 16, 4, 1, A, None) == 2     # pool not 16-byte aligned


def test_kernel_and_split_choice_follow_the_cu_count(capi):
    """The forward's kernel variant and key-split count come from the device's
    compute-unit count (read at launch), not from a built-in 256: the same
    shape on a 256-CU MI355X and on a 32-CU partition (one XCD) chooses
    differently, and both choices follow the measured crossovers."""
    lib = capi.load()
    choose, plan = lib.fa_probe_choose_variant, lib.fa_probe_splitkv_plan_cus
    # D = 128 always runs the 128-row kernel
    assert choose(128, 0, 8, 4096, 256) == 204 and choose(128, 1, 1, 64, 32) == 204
    # D = 64 at 256 CUs: fewer 128-row blocks than CUs -> the 64-row kernel
    assert choose(64, 0, 8, 2048, 256) == 408      # 128 blocks < 256
    assert choose(64, 0, 8, 4096, 256) == 204      # 256 blocks = one per CU
    assert choose(64, 1, 8, 4096, 256) == 408      # causal, exactly one wave, N >= 2048
    assert choose(64, 1, 16, 4096, 256) == 204     # causal, two waves
    assert choose(64, 1, 32, 1024, 256) == 204     # causal, one wave but N < 2048
    # the same shapes on a 32-CU device: 128 and 256 blocks fill it several times
    assert choose(64, 0, 8, 2048, 32) == 204
    assert choose(64, 1, 8, 4096, 32) == 204
    assert choose(64, 0, 1, 2048, 32) == 408       # 16 blocks < 32
    assert choose(64, 0, 1, 4096, 32) == 204       # exactly 32 blocks
    assert choose(64, 1, 1, 4096, 32) == 408       # causal, one wave of 32
    # bad arguments
    assert choose(96, 0, 8, 4096, 256) == 0 and choose(64, 0, 8, 4096, 0) == 0
    # split-KV plan: D = 128 long sequences over few heads split to fill the CUs
    assert plan(1, 1, 16384, 128, 0, 256) == 2     # 128 blocks, 256 tiles / 32 = 8 -> ceil(256/128)
    assert plan(1, 1, 16384, 128, 0, 32) == 1      # 128 blocks >= 32 CUs
    assert plan(1, 1, 4096, 128, 0, 256) == 2      # 32 blocks: 8 by CUs, 64 tiles / 32 = 2
    assert plan(1, 1, 4096, 128, 0, 64) == 2
    assert plan(1, 1, 2048, 128, 0, 256) == 1      # 32 tiles: too few per split
    assert plan(1, 8, 4096, 128, 0, 256) == 1      # 256 blocks fill 256 CUs
    assert plan(1, 8, 4096, 128, 0, 512) == 2      # but not a 512-CU device
    assert plan(1, 1, 16384, 64, 0, 256) == 1      # D = 64 never splits
    assert plan(1, 3, 8192, 128, 0, 256) == 1      # 192 blocks: two splits would not fit one wave
    # causal D = 128: the longest row block sets the time; splits down to 8 tiles
    assert plan(1, 1, 8192, 128, 1, 256) == 4      # 64 blocks, 128 tiles
    assert plan(1, 1, 2048, 128, 1, 256) == 4      # 16 blocks, 32 tiles: 8 per split
    assert plan(1, 4, 4096, 128, 1, 256) == 2      # 128 blocks, 64 tiles
    assert plan(1, 8, 2048, 128, 1, 256) == 1      # 128 blocks, 32 tiles: 2 splits lose
    assert plan(1, 3, 8192, 128, 1, 256) == 1      # 192 blocks
    assert plan(1, 1, 16384, 64, 1, 256) == 1      # D = 64 never splits
