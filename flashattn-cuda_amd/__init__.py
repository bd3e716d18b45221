"""MI355X (gfx950) FlashAttention forward and split-KV paged decode.

Drop-in for the reference's torch-extension module
(cuda/flash_attn_fa3_db_full.cu:405-418):

    O, L = forward(Q, K, V)           # O fp16 [B,H,N,D], L fp32 [B,H,N]
    O = forward_only(Q, K, V)         # bitwise the same O, no L

Both accept ``causal=True``, D in {64, 128} and K/V with fewer heads than Q
(GQA/MQA: [B, H_kv, N, D], H a multiple of H_kv); ``forward_varlen`` takes
packed variable-length sequences. The backward of the
reference's first module (cuda/flash_attn_kernel.cu:417-503):

    dQ, dK, dV = backward(Q, K, V, O, dO, L)   # fp32 [B,H,N,D]

New entry points:

    bad = kv_append(k_new, v_new, k_pool, v_pool, page_table, start_pos)   # in place
    O, L = decode_paged(q, k_pool, v_pool, page_table, ctx_lens, num_splits=16)
    part_o, part_lse = decode_partials(...);  O, L = lse_combine(part_o, part_lse)

Every call runs the hand-written HIP kernels of ``libfa_mi355x.so`` through
the C ABI in include/fa_mi355x.h. There is no fallback: importing this package
without the built extension raises ImportError.
"""
from __future__ import annotations

import importlib.machinery
import importlib.util
import os
import pathlib
import sysconfig

import torch  # noqa: F401  (loads the HIP runtime the extension links against)

_HERE = pathlib.Path(__file__).resolve().parent
_EXT = _HERE / ("_fa_torch" + sysconfig.get_config_var("EXT_SUFFIX"))
LIB_PATH = _HERE / "libfa_mi355x.so"


def _load_ext():
    if not _EXT.exists() or not LIB_PATH.exists():
        raise ImportError(
            f"flashattn-cuda_amd is not built ({_EXT.name} / {LIB_PATH.name} missing); "
            f"run `python {_HERE / 'build.py'}`")
    loader = importlib.machinery.ExtensionFileLoader("_fa_torch", str(_EXT))
    spec = importlib.util.spec_from_file_location("_fa_torch", str(_EXT), loader=loader)
    mod = importlib.util.module_from_spec(spec)
    loader.exec_module(mod)
    return mod


_C = _load_ext()
EXT_PATH = _EXT


def forward(Q, K, V, causal: bool = False):
    """[O, L]: O = softmax(Q K^T / sqrt(D)) V (fp16), L = row logsumexp (fp32)."""
    return _C.forward(Q, K, V, causal)


def forward_bf16(Q, K, V, causal: bool = False, want_L: bool = True):
    """bfloat16 forward: [O bf16 [B,H,N,D], L fp32 [B,H,N]] ([O] if not want_L)."""
    return _C.forward_bf16(Q, K, V, causal, want_L)


def forward_varlen(q, k, v, cu_seqlens, max_seqlen: int, causal: bool = False):
    """[O, L] of B packed sequences, head-major: q [H, total, D], k/v [H_kv, total, D].

    Sequence b is rows cu_seqlens[b] .. cu_seqlens[b+1] (int32 [B+1]) of every
    head and attends only within itself; max_seqlen must cover every sequence.
    Rows past cu_seqlens[B] belong to no sequence: O = 0 and L = -inf there.
    """
    return _C.forward_varlen(q, k, v, cu_seqlens, max_seqlen, causal)


def forward_only(Q, K, V, causal: bool = False):
    """O only; bitwise equal to forward(...)[0]."""
    return _C.forward_only(Q, K, V, causal)


def backward(Q, K, V, O, dO, L, causal: bool = False):
    """[dQ, dK, dV] (fp32 [B,H,N,D]) of sum(O * dO), from forward()'s O and L.

    The reference's backward(Q, K, V, O, dO, L) (cuda/flash_attn_kernel.cu:417-503).
    """
    return _C.backward(Q, K, V, O, dO, L, causal)


def backward_bf16(Q, K, V, O, dO, L, causal: bool = False):
    """[dQ, dK, dV] (fp32) of forward_bf16(): inputs in bfloat16, P and dS
    rounded to bf16 for their products; K/V may have fewer heads (GQA)."""
    return _C.backward_bf16(Q, K, V, O, dO, L, causal)


def backward_varlen(q, k, v, o, dO, L, cu_seqlens, max_seqlen: int, causal: bool = False):
    """[dQ, dK, dV] (fp32, head-major packed like forward_varlen's inputs) of
    forward_varlen(); rows outside every sequence are zeros."""
    return _C.backward_varlen(q, k, v, o, dO, L, cu_seqlens, max_seqlen, causal)


def kv_append(k_new, v_new, k_pool, v_pool, page_table, start_pos, new_lens=None):
    """Write k_new/v_new [B,H,T,D] into the pools at start_pos[b] + t, in place
    (all four fp16, or all four bf16).

    Returns bad int32 [B]: 1 where a token of the sequence had no valid page
    (that token is not written).
    """
    return _C.kv_append(k_new, v_new, k_pool, v_pool, page_table, start_pos, new_lens)


def decode_paged(q, k_pool, v_pool, page_table, ctx_lens, num_splits: int = 16):
    """[O, L] of one query token per sequence over its paged K/V (split pass + combine).

    q and the pools are all fp16 or all bf16; O has q's dtype, L is fp32.
    """
    return _C.decode_paged(q, k_pool, v_pool, page_table, ctx_lens, num_splits)


def decode_partials(q, k_pool, v_pool, page_table, ctx_lens, num_splits: int = 16):
    """[part_o fp32 [B,H,S,D], part_lse fp32 [B,H,S]] of the split pass alone."""
    return _C.decode_partials(q, k_pool, v_pool, page_table, ctx_lens, num_splits)


def lse_combine(part_o, part_lse):
    """[O fp16 [B,H,D], L fp32 [B,H]] merged from split partials."""
    return _C.lse_combine(part_o, part_lse)


def loaded_libraries():
    """Paths of this package's native libraries mapped into the process."""
    out = []
    try:
        with open(f"/proc/{os.getpid()}/maps") as f:
            for line in f:
                p = line.split()[-1]
                if p.startswith(str(_HERE)) and p.endswith(".so") and p not in out:
                    out.append(p)
    except OSError:
        pass
    return out


probe = _C  # probe_mfma32, probe_mfma16, probe_tr16_raw, probe_frags, probe_chain
