"""CPU oracle for the FlashAttention forward/backward, paged decode and page writer: TEST INFRASTRUCTURE ONLY.

Importable only from tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg. The HIP product path never routes through it.
"""
from .naive import (  # noqa: F401
    LN2, append_pages, attention_bruteforce, bf16_cast, decode_attention, gather_pages, half_cast,
    fp16_p_forward, lse_combine, make_decode_meta, make_fwd_inputs, make_ragged_inputs,
    naive_attention, naive_attention_backward, ragged_n, randn_f16, split_bounds, split_partials,
)
