"""GPU tier: cross-check against PyTorch-ROCm's SDPA (an independent GPU kernel).

The reference's headline compares its forward with SDPA-Flash
(bench/bench_fa3_headline.py:1-91); bench.py reproduces that paired timing.
This test only checks that both produce the same O on those inputs, within
the sum of two fp16-output budgets (2 x 2e-3). The parity bar itself is the
CPU oracle (tests/test_fwd_gpu.py); skipped if this torch build has neither
the flash nor the memory-efficient SDPA backend.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _backend(dev):
    from torch.nn.attention import SDPBackend, sdpa_kernel
    import torch.nn.functional as F
    x = torch.randn(1, 1, 64, 64, device=dev, dtype=torch.float16)
    for be in (SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION):
        try:
            with sdpa_kernel(be):
                F.scaled_dot_product_attention(x, x, x)
            return be
        except RuntimeError:
            continue
    return None


@pytest.mark.parametrize("N", [1024, 2048, 4096])
@pytest.mark.parametrize("causal", [False, True])
def test_matches_sdpa(fa, dev, N, causal):
    from torch.nn.attention import sdpa_kernel
    import torch.nn.functional as F
    be = _backend(dev)
    if be is None:
        pytest.skip("no flash or memory-efficient SDPA backend in this torch build")
    g = torch.Generator(device=dev).manual_seed(N)
    Q, K, V = (torch.randn(1, 8, N, 64, device=dev, dtype=torch.float16, generator=g)
               for _ in range(3))
    O, _ = fa.forward(Q, K, V, causal=causal)
    with sdpa_kernel(be):
        Os = F.scaled_dot_product_attention(Q, K, V, is_causal=causal)
    diff = (O.float() - Os.float()).abs().max().item()
    print(f"N={N} causal={causal} backend={be.name}: max |O - O_sdpa| = {diff:.2e}")
    assert diff <= 4e-3
