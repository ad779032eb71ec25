"""CPU oracle for the flashattn_cuda hot path (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package; the product path never does.
"""

from .attention import (  # noqa: F401
    HEAD_DIM,
    attention_cpu,
    attention_flops,
    choose_decode_split,
    decode,
    decode_bytes,
    decode_gqa,
    fp16_half_ulp,
    fp16_rounding_floor,
    kv_append,
    legacy_attention,
    make_decode_inputs,
    make_prefill_inputs,
    prefill,
    prefill_gqa,
    repeat_kv,
    stable_softmax,
)
