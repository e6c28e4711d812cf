"""ctypes binding of libmoe_gfx950.so (C ABI in include/moe_gfx950.h).

torch is imported before the library is opened so that the library's
libamdhip64.so.7 dependency binds to the HIP runtime torch already loaded (one
runtime per process).  There is no fallback: if the library is missing or does
not load, every entry point raises.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch  # noqa: F401  (must precede dlopen of the HIP library)

LIB_PATH = Path(__file__).resolve().with_name("libmoe_gfx950.so")

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int

# name -> (restype, argtypes); mirrors include/moe_gfx950.h exactly
SIGNATURES = {
    "moe_version": (_int, []),
    "moe_last_error_string": (ctypes.c_char_p, []),
    "moe_prerouted_workspace_bytes": (_i64, [_i64, _i64]),
    "moe_run_prerouted": (_int, [_p, _p, _p, _p, _p, _int, _p, _p, _p, _p, _p,
                                 _i64, _i64, _i64, _i64, _i64, _i64, _p, _i64, _p]),
    "moe_run_prerouted_events": (_int, [_p, _p, _p, _p, _p, _int, _p, _p, _p, _p, _p,
                                        _i64, _i64, _i64, _i64, _i64, _i64, _p, _i64, _p, _p]),
    "moe_route_topk": (_int, [_p, _p, _i64, _i64, _i64, _p, _p, _p]),
    "moe_align_capacity_rows": (_i64, [_i64, _i64, _i64, _i64]),
    "moe_align_scratch_bytes": (_i64, [_i64, _i64, _i64]),
    "moe_router_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "moe_route_hidden": (_int, [_p, _p, _p, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _i64, _p]),
    "moe_fused_hidden_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64, _i64]),
    "moe_fused_forward_hidden": (_int, [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64,
                                        _p, _i64, _p, _p, _p]),
    "moe_fused_ex_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64, _i64, _int, _int]),
    "moe_fused_forward_ex": (_int, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64,
                                    _i64, _i64, _i64, _p, _i64, _p, _p, _p, _p]),
    "moe_fused_shard_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64, _i64, _i64]),
    "moe_fused_forward_shard": (_int, [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                       _i64, _p, _i64, _p, _p, _p, _p]),
    "moe_fused_routed_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64, _i64, _i64]),
    "moe_fused_forward_routed": (_int, [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                        _i64, _p, _i64, _p, _p]),
    "moe_fused_shared_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64, _i64]),
    "moe_fused_forward_shared": (_int, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64,
                                        _i64, _i64, _p, _i64, _p, _p, _p]),
    "moe_align": (_int, [_p, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _p, _p, _i64, _p]),
    "moe_fused_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64, _i64, _int]),
    "moe_pick_block_m": (_i64, [_i64, _i64, _i64]),
    "moe_fused_forward": (_int, [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64,
                                 _i64, _p, _i64, _p, _p, _p]),
    "moe_fused_forward_noalloc": (_int, [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64,
                                         _i64, _p, _p, _p]),
    "moe_fused_forward_events": (_int, [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64,
                                        _i64, _i64, _p, _i64, _p, _p, _p, _p]),
    "moe_quantize_rows_w8": (_int, [_p, _i64, _i64, _p, _p, _p]),
    "moe_quantize_rows_fp8": (_int, [_p, _i64, _i64, _p, _p, _p]),
    "moe_fused_forward_fp8": (_int, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64,
                                     _i64, _p, _i64, _p, _p, _p, _p]),
    "moe_fused_forward_w8a8": (_int, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64,
                                      _i64, _i64, _i64, _i64, _p, _i64, _p, _p, _p]),
    "moe_fused_forward_w8a8_events": (_int, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64,
                                             _i64, _i64, _i64, _i64, _p, _i64, _p, _p, _p, _p]),
}

_LIB = None


class MoeError(RuntimeError):
    """A non-zero moe_status returned by the HIP library."""


def lib() -> ctypes.CDLL:
    """The loaded library (raises if it was never built)."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH.name} is not built: run `python -m muxi_race_amd.build` "
                "(or __graft_entry__.build()); there is no non-HIP fallback")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = handle
    return _LIB


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().moe_last_error_string()
        raise MoeError(f"{what} failed (status {rc}): {msg.decode() if msg else ''}")
