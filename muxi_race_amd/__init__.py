"""muxi_race_amd -- MI355X (gfx950) fused Mixture-of-Experts FFN.

Hand-written HIP kernels behind a C ABI (include/moe_gfx950.h), called from
Python through ctypes on torch's current HIP stream.

    from muxi_race_amd import run_kernel, fused_moe
"""

from .moe import (  # noqa: F401
    MoeError,
    W8A8Weights,
    fused_moe,
    fused_moe_routed,
    fused_workspace_bytes,
    moe_align,
    pick_block_m,
    quantize_rows_w8,
    quantize_w8a8_weights,
    route_hidden,
    route_topk,
    run_kernel,
)

from .weights import load_w8a8, save_w8a8  # noqa: F401,E402

__version__ = "0.1.0"
