"""Writes the small golden fixtures under tests/golden/.

The reference ships no golden vectors (its tests compare against the naive
oracle computed in the same run, tests/test_fa3_db_full.py:28-45), so these
fixtures are computed here, in float64, by explicit Python loops over the
definitions (no numpy linear algebra), from seeded fp16 inputs:

* fwd_*.npz     : q, k, v fp16 [H, N, D]; o, l float64 [H, N]  (+ causal flag)
                  o = softmax(q k^T / sqrt(D)) v, l = logsumexp  (ref/naive_attn.py:23-38)
* decode_*.npz  : q [B,H,D], k_pool/v_pool [P,H,16,D] fp16, page_table, ctx_lens;
                  o [B,H,D], l [B,H] float64 from an explicit per-token page walk
* combine.npz   : part_o [B,H,S,D], part_lse [B,H,S] (with empty splits);
                  o, l float64 of the logsumexp merge

Run: python tests/golden/make_golden.py
"""
from __future__ import annotations

import math
import pathlib

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent


def attn_rows(q, k, v, causal):
    n, d = q.shape
    scale = 1.0 / math.sqrt(d)
    O = np.zeros((n, v.shape[1]))
    L = np.zeros(n)
    for i in range(n):
        keys = range(i + 1) if causal else range(k.shape[0])
        s = [sum(float(q[i, t]) * float(k[j, t]) for t in range(d)) * scale for j in keys]
        m = max(s)
        w = [math.exp(x - m) for x in s]
        z = sum(w)
        for jj, j in enumerate(keys):
            for t in range(v.shape[1]):
                O[i, t] += w[jj] / z * float(v[j, t])
        L[i] = m + math.log(z)
    return O, L


def fwd_case(name, H, N, D, seed, causal, amp=1.0):
    rng = np.random.default_rng(seed)
    q, k, v = ((rng.standard_normal((H, N, D)) * amp).astype(np.float16) for _ in range(3))
    O = np.zeros((H, N, D))
    L = np.zeros((H, N))
    for h in range(H):
        O[h], L[h] = attn_rows(q[h], k[h], v[h], causal)
    np.savez_compressed(HERE / f"{name}.npz", q=q, k=k, v=v, o=O, l=L,
                        causal=np.array(causal), seed=np.array(seed))


def decode_case(name, B, H, D, ctx, seed):
    rng = np.random.default_rng(seed)
    ps = 16
    pages = [(c + ps - 1) // ps for c in ctx]
    P = sum(pages) + 3                      # a few pages no sequence uses
    perm = rng.permutation(P)
    table = np.zeros((B, max(pages)), dtype=np.int32)
    off = 0
    for b in range(B):
        table[b, :pages[b]] = perm[off:off + pages[b]]
        off += pages[b]
    q = rng.standard_normal((B, H, D)).astype(np.float16)
    kp = rng.standard_normal((P, H, ps, D)).astype(np.float16)
    vp = rng.standard_normal((P, H, ps, D)).astype(np.float16)
    O = np.zeros((B, H, D))
    L = np.zeros((B, H))
    for b in range(B):
        for h in range(H):
            krows, vrows = [], []
            for j in range(ctx[b]):          # explicit token -> (page, slot) walk
                pid = int(table[b, j // ps])
                krows.append(kp[pid, h, j % ps])
                vrows.append(vp[pid, h, j % ps])
            o, l = attn_rows(q[b, h][None, :], np.array(krows), np.array(vrows), False)
            O[b, h], L[b, h] = o[0], l[0]
    np.savez_compressed(HERE / f"{name}.npz", q=q, k_pool=kp, v_pool=vp, page_table=table,
                        ctx_lens=np.array(ctx, dtype=np.int32), o=O, l=L)


def combine_case(name, B, H, S, D, seed):
    rng = np.random.default_rng(seed)
    po = rng.standard_normal((B, H, S, D)).astype(np.float32)
    pl = (rng.standard_normal((B, H, S)) * 4).astype(np.float32)
    pl[0, 0, 1:] = -np.inf                  # one non-empty split
    pl[1 % B, H - 1, ::2] = -np.inf         # alternate empty splits
    po[np.isinf(pl)] = 0.0
    O = np.zeros((B, H, D))
    L = np.zeros((B, H))
    for b in range(B):
        for h in range(H):
            ls = [float(x) for x in pl[b, h] if np.isfinite(x)]
            m = max(ls)
            L[b, h] = m + math.log(sum(math.exp(x - m) for x in ls))
            for s in range(S):
                if np.isfinite(pl[b, h, s]):
                    O[b, h] += math.exp(float(pl[b, h, s]) - L[b, h]) * po[b, h, s].astype(np.float64)
    np.savez_compressed(HERE / f"{name}.npz", part_o=po, part_lse=pl, o=O, l=L)


def main():
    fwd_case("fwd_n37_d64", H=2, N=37, D=64, seed=11, causal=False)
    fwd_case("fwd_n37_d64_causal", H=2, N=37, D=64, seed=12, causal=True)
    fwd_case("fwd_n1_d64", H=1, N=1, D=64, seed=13, causal=False)
    fwd_case("fwd_n20_d128", H=1, N=20, D=128, seed=14, causal=False)
    fwd_case("fwd_n20_d128_causal_amp3", H=1, N=20, D=128, seed=15, causal=True, amp=3.0)
    decode_case("decode_b3_d64", B=3, H=2, D=64, ctx=[5, 40, 17], seed=21)
    decode_case("decode_b2_d128", B=2, H=2, D=128, ctx=[33, 16], seed=22)
    combine_case("combine_b2_s5", B=2, H=2, S=5, D=64, seed=23)


if __name__ == "__main__":
    main()
