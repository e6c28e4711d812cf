"""CPU oracle for the fused-MoE hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the algorithm of the reference's pre-routed
fused expert MLP (problem_detail.json:50, xpuoj_data/race_stress2.py:29-48) plus
the build-defined routing, alignment, combine and W8A8 steps that the reference
does not implement.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker or as
the timed CPU baseline.  The product package ``muxi_race_amd`` never imports
it: the HIP library is the only compute path.

Pinning (how each function is checked independently of its own formula):

* ``route_topk``        -- brute-force rank counting + scipy softmax closed form
                           (tests/test_oracle_routing.py).
* ``router_logits``     -- one-hot token rows select router-weight columns
                           (catches a transposed operand) and a float64 numpy
                           product (tests/test_oracle_routing.py).
* ``align`` / ``metadata_from_group_sizes`` -- hand-written known answers
                           (problem_detail.json:40 example, RB:82-101 cases) and
                           permutation/padding invariants (tests/test_oracle_align.py).
* ``prerouted_forward`` -- permutation-matrix closed form (catches transposed
                           operands and raw/padded index mix-ups), an fp64 scalar
                           loop on tiny inputs, E=1 dense SwiGLU, zero-size
                           experts, V=0, NaN-poisoned padding, power-of-two
                           linearity (tests/test_oracle_core.py).
* ``prerouted_forward_blocks`` -- equals ``prerouted_forward`` on harness
                           metadata (random splits); hand-derived answers for
                           swapped / trailing / out-of-range / short gidx
                           (tests/test_oracle_blocks.py).
* ``combine``           -- closed form on one-hot inputs (tests/test_oracle_core.py).
* ``quantize_rows_int8`` / ``w8a8_forward`` -- exact integer checks on
                           hand-made rows, round-half-away edge cases, and the
                           fp16 oracle within the north-star W8A8 gate
                           (tests/test_oracle_w8a8.py).
* ``fp8_e4m3_codes`` / ``quantize_rows_fp8`` / ``pow2_scales`` / ``w8a8_forward(fmt="fp8")`` --
                           torch's own float8_e4m3fn conversion on every code
                           boundary and midpoint (ties to even), hand-made
                           codes, the e4m3 value table against the format's
                           definition, power-of-two scales against brute
                           force over j, and the fp16 oracle within the W8A8
                           gate (tests/test_oracle_fp8.py).
* ``fused_moe_forward(shared=)`` -- exact doubling closed form and the dense
                           SwiGLU difference (tests/test_oracle_core.py).
* ``fused_moe_forward(expert_range=)`` -- one shard over all experts is the
                           full layer exactly, disjoint shards sum to it, dense
                           fp64 per-token sums (tests/test_oracle_core.py).
* ``fused_moe_forward(routing=)`` -- the router's own ids / weights reproduce
                           the logits path bitwise (layer and shard), -1 or
                           foreign ids equal zero weights exactly, dense fp64
                           per-token sums with unnormalised weights
                           (tests/test_oracle_core.py).
* ``stratified_tokens`` -- (a sampler, not arithmetic) every block of the
                           routing's align holds a sampled token's pair, every
                           expert's first and last pair is sampled
                           (tests/test_oracle_align.py).
"""

from .moe_ref import (  # noqa: F401
    router_logits,
    route_topk,
    align,
    metadata_from_group_sizes,
    prerouted_forward,
    prerouted_forward_blocks,
    gather_rows,
    combine,
    fused_moe_forward,
    quantize_rows_int8,
    quantize_rows_fp8,
    pow2_scales,
    fp8_e4m3_codes,
    FP8_E4M3_VALUES,
    w8a8_forward,
    silu_mul,
)
from .sampling import stratified_tokens  # noqa: F401
