"""GPU tier: on-device checks of the matrix-core and LDS layouts the forward
kernel is built on, with negative controls (the method of the reference's
tests/test_mma_probe.py:18-57, rebuilt for gfx950 instructions)."""
import torch
import pytest

pytestmark = pytest.mark.gpu


def _rand(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).half()


def test_mfma32_layout(fa, dev):
    a, b = _rand((32, 16), 1).to(dev), _rand((16, 32), 2).to(dev)
    ref = a.float().cpu() @ b.float().cpu()
    got = fa.probe.probe_mfma32(a, b, 0).cpu()
    assert (got - ref).abs().max().item() < 1e-3
    bad = fa.probe.probe_mfma32(a, b, 1).cpu()
    assert (bad - ref).abs().max().item() > 0.5, "negative control must be LARGE"


def test_mfma16_layout(fa, dev):
    a, b = _rand((16, 32), 3).to(dev), _rand((32, 16), 4).to(dev)
    ref = a.float().cpu() @ b.float().cpu()
    got = fa.probe.probe_mfma16(a, b, 0).cpu()
    assert (got - ref).abs().max().item() < 1e-3
    bad = fa.probe.probe_mfma16(a, b, 1).cpu()
    assert (bad - ref).abs().max().item() > 0.5


def test_permlane32_swap(fa, dev):
    x = torch.arange(64, dtype=torch.float32) * 1.5 - 7
    out = fa.probe.probe_permlane(x.to(dev)).cpu()
    partner = x.view(2, 32).flip(0).reshape(-1)
    r0 = torch.where(torch.arange(64) < 32, x, partner)
    r1 = torch.where(torch.arange(64) < 32, partner, x)
    assert torch.equal(out[0], r0) and torch.equal(out[1], r1)
    assert torch.equal(out[2], torch.maximum(x, partner))
    assert torch.equal(out[3], x + partner)


def test_ds_read_tr16_semantics(fa, dev):
    """Lane s of each 16-lane group reading 8 bytes at 8*l receives the 4 halves
    at element offsets 64*g + 16*e + s (a column of a 4x16 row-major block)."""
    src = torch.arange(256, dtype=torch.int16)
    out = fa.probe.probe_tr16_raw(src.to(dev)).cpu().to(torch.int64)
    exp = torch.empty(64, 4, dtype=torch.int64)
    for l in range(64):
        g, s = divmod(l, 16)
        for e in range(4):
            exp[l, e] = 64 * g + 16 * e + s
    assert torch.equal(out, exp), f"tr16 layout differs:\n{out[:16]}"


@pytest.mark.parametrize("D", [64, 128])
def test_operand_fragments_exact(fa, dev, D):
    tile = (torch.arange(64 * D, dtype=torch.int32) % 30011).to(torch.int16).view(torch.half)
    tile = tile.view(64, D)
    kout, vout = fa.probe.probe_frags(tile.to(dev))
    kout = kout.cpu().view(torch.int16)
    vout = vout.cpu().view(torch.int16)
    t = tile.view(torch.int16)
    for kb in range(2):
        for kk in range(D // 16):
            for l in range(64):
                row = 32 * kb + (l % 32)
                col = 16 * kk + 8 * (l // 32)
                assert torch.equal(kout[kb, kk, l], t[row, col:col + 8]), (kb, kk, l)
    for j in range(4):
        for db in range(D // 32):
            for l in range(64):
                keys = [16 * j + 8 * (i // 4) + 4 * (l // 32) + (i % 4) for i in range(8)]
                exp = t[keys, 32 * db + (l % 32)]
                assert torch.equal(vout[j, db, l], exp), (j, db, l)


@pytest.mark.parametrize("D", [64, 128])
def test_qk_pv_chain(fa, dev, D):
    q = (_rand((32, D), 5) * 0.25).to(dev)
    k = (_rand((64, D), 6) * 0.25).to(dev)
    v = _rand((64, D), 7).to(dev)
    s = q.float().cpu() @ k.float().cpu().T
    ref = s.half().float() @ v.float().cpu()
    got = fa.probe.probe_chain(q, k, v).cpu()
    # fp32 accumulation order may flip an fp16 rounding of S: ~1 ulp of P times |v|
    assert (got - ref).abs().max().item() < 5e-3
    # negative control: pairing P with V rows in a different key order is far off
    perm = torch.arange(64).view(4, 16).flip(1).reshape(-1)
    bad = s.half().float() @ v.float().cpu()[perm]
    assert (got - bad).abs().max().item() > 0.1


def test_read_bandwidth_probe_runs(fa, dev):
    """The read-bandwidth probe streams a buffer without writing the sink
    (all-zero input folds to 0, not the sink's trigger value)."""
    x = torch.zeros(16 << 20, dtype=torch.int32, device=dev)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    for blocks in (1, 64, 4096):
        fa.probe.probe_read_bw(x, sink, blocks)
    torch.cuda.synchronize()
    assert sink.item() == 0
    # The loads read the data: one 16-byte vector whose words fold to the
    # trigger value, in the chunk of the last of 64 workgroups, sets the sink.
    x.view(-1, 4)[-1, 0] = 0x9e3779b9 - (1 << 32)
    fa.probe.probe_read_bw(x, sink, 64)
    torch.cuda.synchronize()
    assert sink.item() == 0x9e3779b9 - (1 << 32)


@pytest.mark.parametrize("nontemporal", [True, False])
def test_gather_bandwidth_probe_reads_every_page(fa, dev, nontemporal):
    """The gather probe reads each page of both pools once through the table
    (all-zero pools leave the sink alone; one trigger vector in the V page a
    table entry names sets it), and clamps out-of-range ids into the pool."""
    pages = 300
    k = torch.zeros(pages * 1024, dtype=torch.int32, device=dev)
    v = torch.zeros(pages * 1024, dtype=torch.int32, device=dev)
    g = torch.Generator().manual_seed(3)
    table = torch.randperm(pages, generator=g).to(torch.int32).to(dev)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    for per in (1, 7, 65, 300):
        fa.probe.probe_gather_bw(k, v, table, sink, per, nontemporal)
    torch.cuda.synchronize()
    assert sink.item() == 0
    target = int(table[-1].item())                  # the page of the last table entry
    v.view(pages, 256, 4)[target, 200, 0] = 0x9e3779b9 - (1 << 32)
    fa.probe.probe_gather_bw(k, v, table, sink, 65, nontemporal)
    torch.cuda.synchronize()
    assert sink.item() == 0x9e3779b9 - (1 << 32)
    # out-of-range ids read page 0 or the last page instead
    sink.zero_()
    v.zero_()
    bad = torch.zeros(pages, dtype=torch.int32, device=dev)   # every entry page 0 ...
    bad[5], bad[6] = pages + 1000, -7                          # ... but these two
    v.view(pages, 256, 4)[pages - 1, 3, 0] = 0x9e3779b9 - (1 << 32)
    fa.probe.probe_gather_bw(k, v, bad, sink, 65, nontemporal)
    torch.cuda.synchronize()
    assert sink.item() == 0x9e3779b9 - (1 << 32)
