"""CPU oracle for the attention hot path (test infrastructure, never product code).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package.  ``attention`` is the numpy float32 restatement of the
reference's algorithm; ``f64`` loads the float64 brute force written in C
(attn_f64.c) that pins it.
"""
from .attention import (CHUNK, LOG2E, append_slots, attention_fp32, attention_gqa,  # noqa: F401
                        attention_varlen, decode_kv_bytes,
                        decode_partition, gather_kv, make_paged_cache, merge_partials, paged_decode_fp32,
                        paged_decode_splitk, prefill_flops, reshape_and_cache, round_partition,
                        split_partials)
