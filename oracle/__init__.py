"""The oracle: a CPU restatement of BlockStreamer's gpt-oss MoE expert path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import this package, and only to check
results against (or, for ``cpu_baseline``, as the timed CPU port).  The product
package ``blockstreamer_amd`` never imports it.
"""

from .oracle import (  # noqa: F401
    FP4_VALUES,
    apply_gate_ref,
    attention_ref,
    dequant_c,
    dequant_torch,
    bits_equal_or_both_nan,
    dequantize_expert_ref,
    dequant_table_c,
    e2m3_decode,
    e4m3_decode,
    experts_mx6_ref,
    experts_mx_ref,
    experts_ref,
    mlp_ref,
    mxfp6_split_dequant_ref,
    mxfp6_split_ref,
    mxfp8_dequant_ref,
    mxfp8_quant_ref,
    mxfp8_split_dequant_ref,
    mxfp8_split_ref,
    rmsnorm_bwd_ref,
    rmsnorm_ref,
    router_ref,
    to_kpair_ref,
    topk_softmax_ref,
)
