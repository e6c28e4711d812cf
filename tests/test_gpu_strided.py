"""Strided weights (rows and experts apart: the two halves of a fused
[E, 2I, H] gate/up tensor, rows padded, experts with gaps) give bitwise the
dense-weight result: the kernels read the same values in the same order, only
from other addresses.  Gaps are NaN-filled, so a read of one shows.  Also
checked against the oracle once, and with the shared expert and the router
GEMM."""
import pytest
import torch

from _cases import moe_inputs
from conftest import assert_close
from oracle import fused_moe_forward

pytestmark = pytest.mark.gpu


def _gapped(w, row_extra, expert_extra):
    """View of w [E, N, K] with rows K + row_extra and experts
    N * (K + row_extra) + expert_extra elements apart, gaps NaN."""
    E, N, K = w.shape
    ld = K + row_extra
    es = N * ld + expert_extra
    buf = torch.full((E * es,), float("nan"), dtype=w.dtype, device=w.device)
    v = buf.as_strided((E, N, K), (es, ld, 1))
    v.copy_(w)
    return v


def _run(inp, wg, wu, wd, **kw):
    from muxi_race_amd import fused_moe
    out, (ids, w) = fused_moe(inp["x"], inp["logits"], wg, wu, wd, inp["k"], expert_bias=inp["bias"],
                              return_routing=True, **kw)
    torch.cuda.synchronize()
    return out, ids, w


@pytest.mark.parametrize("name,bm", [("small", 0), ("small", 32), ("small", 64), ("small", 128), ("decode", 0),
                                     ("mixtral", 0), ("mixtral-1536", 0)])
def test_strided_is_bitwise_dense(name, bm):
    # mixtral-1536: 384 routed rows per expert, so the 256-row padding and 256-row Stage 1 items
    T = {"mixtral": 256, "mixtral-1536": 1536}.get(name)
    inp = moe_inputs(name.split("-")[0], 61, T=T)
    ref = _run(inp, inp["wg"], inp["wu"], inp["wd"], block_m=bm)
    # gate / up as the halves of one [E, 2I, H] tensor (expert stride 2*I*H)
    w13 = torch.cat([inp["wg"], inp["wu"]], dim=1)
    I = inp["I"]
    got = _run(inp, w13[:, :I], w13[:, I:], inp["wd"], block_m=bm)
    for a, b in zip(ref, got):
        assert torch.equal(a, b), "w13"
    del w13
    for rx, ex in ((8, 0), (0, 64), (72, 136)):
        got = _run(inp, _gapped(inp["wg"], rx, ex), _gapped(inp["wu"], rx, ex), _gapped(inp["wd"], ex, rx),
                   block_m=bm)
        for a, b in zip(ref, got):
            assert torch.equal(a, b), (rx, ex)


def test_strided_against_oracle():
    inp = moe_inputs("decode", 62)
    out, _, _ = _run(inp, _gapped(inp["wg"], 64, 0), _gapped(inp["wu"], 64, 0), _gapped(inp["wd"], 64, 0))
    ref = fused_moe_forward(inp["x"].cpu(), inp["logits"].cpu(), inp["wg"], inp["wu"], inp["wd"], inp["k"],
                            inp["bias"].cpu())
    assert_close(out, ref, what="decode strided")


def test_strided_with_shared_expert_and_router():
    from muxi_race_amd import fused_moe
    inp = moe_inputs("small", 63, T=300)
    g = torch.Generator(device="cuda").manual_seed(63)
    H, I, E = inp["H"], inp["I"], inp["E"]
    sh = [torch.randn(s, generator=g, device="cuda", dtype=torch.float16) * 0.02 for s in ((I, H), (I, H), (H, I))]
    wr = (torch.randn((E, H), generator=g, device="cuda") / H ** 0.5).half()
    dense = fused_moe(inp["x"], None, inp["wg"], inp["wu"], inp["wd"], inp["k"], router_weight=wr,
                      shared_expert=sh, return_routing=True)
    pw = [_gapped(inp[n], 40, 16) for n in ("wg", "wu", "wd")]
    psh = [_gapped(t[None], 40, 0)[0] for t in sh]
    strided = fused_moe(inp["x"], None, *pw, inp["k"], router_weight=wr, shared_expert=psh, return_routing=True)
    torch.cuda.synchronize()
    assert torch.equal(dense[0], strided[0])
    assert torch.equal(dense[1][0], strided[1][0]) and torch.equal(dense[1][1], strided[1][1])
    with pytest.raises(ValueError):  # shared rows must follow the routed row strides
        fused_moe(inp["x"], None, *pw, inp["k"], router_weight=wr, shared_expert=sh)
    with pytest.raises(ValueError):  # gate and up share their strides
        fused_moe(inp["x"], inp["logits"], pw[0], inp["wu"], pw[2], inp["k"])
    with pytest.raises(ValueError):  # overlapping experts
        fused_moe(inp["x"], inp["logits"], *[t.as_strided(t.shape, (t.stride(1), t.stride(1), 1)) for t in pw[:2]],
                  pw[2], inp["k"])
