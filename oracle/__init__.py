"""CPU oracle for the flash-GQA hot path (TEST INFRASTRUCTURE ONLY).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg
may import this package, and only as the checker (or the timed CPU baseline).
The product (``cuda_llm_ops_amd``) never imports it.
"""
from .oracle import (  # noqa: F401
    attention_backward_f64,
    attention_f64,
    bf16_to_f32,
    decode,
    decode_paged,
    f32_to_bf16,
    fp8e4m3_to_f32,
    lib,
    normal_bf16,
    prefill,
    prefill_backward,
    prefill_mla,
    prefill_swa,
    sparse_prefill,
)
