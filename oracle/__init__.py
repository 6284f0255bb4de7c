"""CPU oracle for the GeneT5 MoE layer forward — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker; the product (genet5_amd) never does.

The reference (97YearsOldProgrammer/GeneT5) has no MoE code (its lib/blocks
holds a dense FeedForward only), so this package restates the layer the
benchmark names: the expert body is FeedForward.forward
(lib/blocks/_component.py:48-52) with activation 'silu' (:31) — gate = wi_0,
up = wi_1 (:42-43, split order lib/model/build.py:30-34) — and the router is
16 experts top-2 (README.md:12).  See oracle/moe_oracle.py for each function's
pin.  oracle/attn_oracle.py restates the encoder's varlen ALiBi attention
(flash_attn_varlen_func as lib/blocks/_flash_att.py:76-88 calls it).
"""
from .attn_oracle import attention_varlen  # noqa: F401
from .moe_oracle import (  # noqa: F401
    add_rmsnorm,
    add_rmsnorm_np,
    combine,
    combine_c,
    dispatch,
    dispatch_c,
    expert_forward,
    input_grad_c,
    moe_backward,
    moe_forward,
    router_logits,
    router_logits_np,
    topk_gates,
    topk_gates_c,
)
