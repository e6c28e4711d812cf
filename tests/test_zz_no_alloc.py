"""moe_fused_forward_noalloc (the allocation-free fused forward, static 64 MiB
scratch per GPU) against moe_fused_forward with a caller workspace, through
the C ABI: bitwise equal outputs and routing on two calls in a row, the second
smaller (the scratch still holds the first call's contents), and a clear
MOE_ERR_WORKSPACE for a problem beyond the scratch."""
import ctypes

import pytest
import torch

from _cases import moe_inputs

pytestmark = pytest.mark.gpu
P = ctypes.c_void_p


def _ptr(t):
    return P(0 if t is None else t.data_ptr())


def _both(L, inp, T):
    H, I, E, k = inp["H"], inp["I"], inp["E"], inp["k"]
    x, lg = inp["x"][:T].contiguous(), inp["logits"][:T].contiguous()
    stream = P(torch.cuda.current_stream().cuda_stream)
    res = []
    for noalloc in (False, True):
        out = torch.full((T, H), float("nan"), dtype=torch.float16, device="cuda")
        ids = torch.full((T, k), -1, dtype=torch.int32, device="cuda")
        w = torch.full((T, k), float("nan"), dtype=torch.float32, device="cuda")
        head = [_ptr(x), _ptr(lg), _ptr(inp["bias"]), _ptr(inp["wg"]), _ptr(inp["wu"]), _ptr(inp["wd"]), _ptr(out),
                T, H, I, E, k, 0]
        if noalloc:
            rc = L.moe_fused_forward_noalloc(*head, _ptr(ids), _ptr(w), stream)
        else:
            nbytes = L.moe_fused_workspace_bytes(T, H, I, E, k, 0, 0)
            ws = torch.full((nbytes,), 0xFF, dtype=torch.uint8, device="cuda")  # NaN-poisoned workspace
            rc = L.moe_fused_forward(*head, _ptr(ws), ws.numel(), _ptr(ids), _ptr(w), stream)
        assert rc == 0, L.moe_last_error_string()
        torch.cuda.synchronize()
        res.append((out, ids, w))
    return res


def test_noalloc_equals_fused_forward_on_two_calls():
    from muxi_race_amd._lib import lib
    L = lib()
    inp = moe_inputs("decode", 91)  # T = 32 at H 7168, I 2048, E 256, top-8 (Zipf routing)
    for T in (32, 8):               # the second call is smaller
        (o_ref, i_ref, w_ref), (o, i, w) = _both(L, inp, T)
        assert bool(torch.isfinite(o_ref).all())
        assert torch.equal(i, i_ref) and torch.equal(w, w_ref), f"T={T}: routing differs"
        assert torch.equal(o, o_ref), f"T={T}: output differs from moe_fused_forward"


def test_noalloc_rejects_a_problem_beyond_the_scratch():
    from muxi_race_amd._lib import lib
    L = lib()
    nul = P(0)
    T, H, I, E, k = 4096, 7168, 2048, 256, 8  # dsv3: ~0.75 GB of workspace
    need = L.moe_fused_workspace_bytes(T, H, I, E, k, 0, 0)
    assert need > 64 << 20
    rc = L.moe_fused_forward_noalloc(nul, nul, nul, nul, nul, nul, nul, T, H, I, E, k, 0, nul, nul,
                                     P(torch.cuda.current_stream().cuda_stream))
    msg = L.moe_last_error_string().decode()
    assert rc == -3 and "static scratch holds 67108864" in msg, (rc, msg)
