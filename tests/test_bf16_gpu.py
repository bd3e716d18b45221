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

from oracle import bf16_cast, naive_attention

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
