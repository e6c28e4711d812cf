"""CPU checks of the C ABI: the library loads, exports exactly what
include/moe_gfx950.h declares (with matching arity), and host-side validation
rejects bad arguments before any GPU call."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "moe_gfx950.h"


def _declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"\b(moe_\w+)\s*\(([^;{]*?)\)\s*;", text):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_header_declares_entry_points():
    decl = _declared()
    for name in ("moe_run_prerouted", "moe_route_topk", "moe_align", "moe_fused_forward",
                 "moe_fused_forward_w8a8", "moe_quantize_rows_w8", "moe_last_error_string"):
        assert name in decl


def test_library_exports_every_declared_symbol():
    from muxi_race_amd._lib import SIGNATURES, lib
    L = lib()
    decl = _declared()
    assert set(decl) == set(SIGNATURES), set(decl) ^ set(SIGNATURES)
    for name, arity in decl.items():
        assert hasattr(L, name), name
        assert len(SIGNATURES[name][1]) == arity, (name, arity)


def test_host_validation_without_gpu():
    from muxi_race_amd._lib import lib
    L = lib()
    assert L.moe_version() >= 1
    nul = ctypes.c_void_p(0)
    # P = 0 is a no-op (reference fast exit), no device access
    rc = L.moe_run_prerouted(nul, nul, nul, nul, nul, 0, nul, nul, nul, nul, nul,
                             0, 128, 128, 4, 0, 0, nul, 0, nul)
    assert rc == 0
    # H not a multiple of 128
    rc = L.moe_run_prerouted(nul, nul, nul, nul, nul, 0, nul, nul, nul, nul, nul,
                             128, 100, 128, 4, 10, 1, nul, 0, nul)
    assert rc == -2 and b"multiples of 128" in L.moe_last_error_string()
    # null pointers
    rc = L.moe_run_prerouted(nul, nul, nul, nul, nul, 0, nul, nul, nul, nul, nul,
                             128, 128, 128, 4, 10, 1, nul, 0, nul)
    assert rc == -1
    rc = L.moe_route_topk(nul, nul, 4, 2000, 2, nul, nul, nul)
    assert rc == -2
    rc = L.moe_fused_forward(nul, nul, nul, nul, nul, nul, nul, 4, 128, 128, 8, 2, 48,
                             nul, 0, nul, nul, nul)
    assert rc == -2 and b"block_m" in L.moe_last_error_string()
    rc = L.moe_quantize_rows_w8(nul, 4, 12, nul, nul, nul)
    assert rc == -1
    # shared expert: exactly one of logits / w_router, and k + 1 <= 32
    one = ctypes.c_void_p(256)
    rc = L.moe_fused_forward_shared(nul, one, one, nul, nul, nul, nul, one, one, one, nul, 4, 128, 128, 64, 2,
                                    0, nul, 0, nul, nul, nul)
    assert rc == -1 and b"exactly one" in L.moe_last_error_string()
    rc = L.moe_fused_forward_shared(nul, one, nul, nul, nul, nul, nul, one, one, one, nul, 4, 128, 128, 64, 32,
                                    0, nul, 0, nul, nul, nul)
    assert rc == -2 and b"top_k" in L.moe_last_error_string()
    rc = L.moe_fused_forward_shared(nul, one, nul, nul, nul, nul, nul, one, nul, one, nul, 4, 128, 128, 64, 2,
                                    0, nul, 0, nul, nul, nul)
    assert rc == -1
    # weight strides that overlap rows or experts, or break 16-byte alignment
    H, I = 128, 256
    for st in ((100, 0, 0, 0), (0, 0, 200, 0), (132, 0, 0, 0), (-8, 0, 0, 0), (0, 128 * 255, 0, 0),
               (0, 0, 0, 128 * 256 - 8), (0, 4 + I * H, 0, 0)):
        arr = (ctypes.c_int64 * 4)(*st)
        rc = L.moe_fused_forward_ex(one, one, nul, nul, one, one, one, nul, nul, nul, arr, one, 4, H, I, 8, 2, 0,
                                    one, 1 << 30, nul, nul, nul, nul)
        assert rc == -1 and b"weight strides" in L.moe_last_error_string(), st


def test_routed_entry_host_validation_without_gpu():
    """moe_fused_forward_routed rejects a missing routing, an expert range past
    the routing's experts and a bad block_m on the host; an empty batch is a
    no-op; its workspace is the shard's (same layout)."""
    from muxi_race_amd._lib import lib
    L = lib()
    nul, one = ctypes.c_void_p(0), ctypes.c_void_p(256)
    args = lambda ids, w, T, E_total, b, E_local, bm: (one, ids, w, one, one, one, one, T, 128, 128, E_total, 2, b,
                                                       E_local, bm, one, 1 << 30, nul, nul)
    rc = L.moe_fused_forward_routed(*args(nul, nul, 4, 8, 0, 8, 0))
    assert rc == -1 and b"null" in L.moe_last_error_string()
    rc = L.moe_fused_forward_routed(*args(one, nul, 4, 8, 0, 8, 0))
    assert rc == -1
    rc = L.moe_fused_forward_routed(*args(one, one, 4, 8, 4, 8, 0))   # experts [4, 12) of 8
    assert rc == -1 and b"expert shard" in L.moe_last_error_string()
    rc = L.moe_fused_forward_routed(*args(one, one, 4, 8, 0, 8, 48))
    assert rc == -2 and b"block_m" in L.moe_last_error_string()
    rc = L.moe_fused_forward_routed(*args(one, one, 4, 0, 0, 8, 0))
    assert rc == -1 and b"E_total" in L.moe_last_error_string()
    assert L.moe_fused_forward_routed(*args(nul, nul, 0, 8, 0, 8, 0)) == 0  # T = 0
    assert L.moe_fused_routed_workspace_bytes(2736, 7168, 2048, 256, 8, 32, 0) == \
        L.moe_fused_shard_workspace_bytes(2736, 7168, 2048, 256, 8, 32, 0)


def test_capacity_and_workspace_sizes():
    from muxi_race_amd._lib import lib
    L = lib()
    # P + min(E, P) * (bm - 1), rounded down to whole blocks
    assert L.moe_align_capacity_rows(4096, 8, 256, 128) == (32768 + 256 * 127) // 128 * 128
    assert L.moe_align_capacity_rows(1, 1, 256, 32) == 32
    assert L.moe_prerouted_workspace_bytes(256, 512) == 256 * 512 * 2
    assert L.moe_pick_block_m(4096, 256, 8) == 128
    assert L.moe_pick_block_m(32, 256, 8) == 32
    ws = L.moe_fused_workspace_bytes(4096, 7168, 2048, 256, 8, 128, 0)
    assert ws >= 32768 * 7168 * 2 + 65280 * 2048 * 2
    assert L.moe_fused_ex_workspace_bytes(4096, 7168, 2048, 256, 8, 128, 1, 1) == \
        L.moe_fused_shared_workspace_bytes(4096, 7168, 2048, 256, 8, 128)
    assert L.moe_fused_ex_workspace_bytes(4096, 7168, 2048, 256, 8, 128, 0, 0) == \
        L.moe_fused_workspace_bytes(4096, 7168, 2048, 256, 8, 128, 0)
    # the shared expert is expert E, choice k: the fused layout for (E + 1, k + 1)
    # plus the router's partial sums
    assert L.moe_fused_shared_workspace_bytes(4096, 7168, 2048, 256, 8, 128) == \
        L.moe_fused_workspace_bytes(4096, 7168, 2048, 257, 9, 128, 0) + L.moe_router_workspace_bytes(4096, 7168, 256)


def test_256_row_padding_policy():
    """With block_m = 0 the library pads experts to 256 rows only where
    256-row items run faster: H a multiple of 256 and >= 192 routed rows per
    expert on average (mixtral, w8a8), never at dsv3's 128."""
    from muxi_race_amd._lib import lib
    L = lib()
    ws = lambda T, H, I, E, k, bm, f: L.moe_fused_workspace_bytes(T, H, I, E, k, bm, f)
    cap = L.moe_align_capacity_rows
    # mixtral (512 rows per expert): fp16 pads
    assert cap(2048, 2, 8, 256) > cap(2048, 2, 8, 128)
    assert ws(2048, 4096, 14336, 8, 2, 0, 0) > ws(2048, 4096, 14336, 8, 2, 128, 0)
    # w8a8 (192 rows per expert): every format pads; 191 rows per expert does not
    for f in (0, 1, 2):
        assert ws(2048, 7168, 2048, 64, 6, 0, f) > ws(2048, 7168, 2048, 64, 6, 128, f)
        assert ws(2037, 7168, 2048, 64, 6, 0, f) == ws(2037, 7168, 2048, 64, 6, 128, f)
    # dsv3 (128 rows per expert): nothing pads
    for f in (0, 1, 2):
        assert ws(4096, 7168, 2048, 256, 8, 0, f) == ws(4096, 7168, 2048, 256, 8, 128, f)
    # H not a multiple of 256: no padding
    assert ws(2048, 4224, 14336, 8, 2, 0, 0) == ws(2048, 4224, 14336, 8, 2, 128, 0)


@pytest.mark.parametrize("define,sources", [
    ("MOE_S2_SCATTER", ("grouped_gemm.hip", "capi.hip")),
    ("MOE_S1_TRIPLE", ("grouped_gemm.hip",)),
])
def test_measured_variant_compiles(tmp_path, define, sources):
    """Variants kept as committed compile-time flags for their A/B must keep
    compiling for gfx950: the Stage 2 scatter-reduce (MOE_S2_SCATTER=1: packed
    fp16 atomics into the token-ordered output, no combine) and Stage 1's
    triple items (MOE_S1_TRIPLE=1: an odd multi-block expert's last three
    blocks as one item per half weight tile)."""
    import subprocess
    from muxi_race_amd.build import CSRC, HIP_FLAGS, _hipcc
    try:
        hipcc = _hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    for src in sources:
        cmd = [hipcc, *HIP_FLAGS, f"-D{define}=1", "-c", str(CSRC / src), "-o", str(tmp_path / (src + ".o"))]
        r = subprocess.run(cmd, capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-2000:]
