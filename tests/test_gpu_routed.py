"""A routing given by the caller (fused_moe_routed / moe_fused_forward_routed):
the library's own routing fed back reproduces fused_moe bitwise; an
expert-parallel dispatch on one GPU (the tokens with a choice in the shard,
gathered, with their global ids and weights) matches the oracle's shard on
those tokens and, scattered back, the full layer; foreign and negative ids and
unnormalised weights match the oracle; argument errors raise."""
import numpy as np
import pytest
import torch

from _cases import moe_inputs
from conftest import assert_close
from oracle import fused_moe_forward

pytestmark = pytest.mark.gpu


def _route(inp):
    from muxi_race_amd import route_topk
    return route_topk(inp["logits"], inp["k"], inp["bias"])


@pytest.mark.parametrize("name", ["small", "decode", "mixtral"])
def test_own_routing_fed_back_is_fused_moe_bitwise(name):
    from muxi_race_amd import fused_moe, fused_moe_routed
    inp = moe_inputs(name, 101, T={"mixtral": 512}.get(name))
    ref = fused_moe(inp["x"], inp["logits"], inp["wg"], inp["wu"], inp["wd"], inp["k"], expert_bias=inp["bias"])
    ids, w = _route(inp)
    got = fused_moe_routed(inp["x"], ids, w, inp["wg"], inp["wu"], inp["wd"])
    torch.cuda.synchronize()
    assert torch.equal(got, ref)


def _dispatch(ids, b, n):
    """Tokens with at least one choice in experts [b, b + n): what the
    dispatch exchange delivers to the GPU holding them."""
    mine = ((ids >= b) & (ids < b + n)).any(dim=1)
    return torch.nonzero(mine).flatten()


@pytest.mark.parametrize("name,G", [("small", 4), ("decode", 8), ("dsv3", 8)])
def test_dispatched_shards_match_oracle_and_sum_to_full(name, G):
    from muxi_race_amd import fused_moe, fused_moe_routed
    inp = moe_inputs(name, 102, T={"dsv3": 1024}.get(name))
    E, T, H = inp["E"], inp["T"], inp["H"]
    full = fused_moe(inp["x"], inp["logits"], inp["wg"], inp["wu"], inp["wd"], inp["k"], expert_bias=inp["bias"])
    ids, w = _route(inp)
    n = E // G
    total = torch.zeros((T, H), dtype=torch.float32, device="cuda")
    for g in range(G):
        b = g * n
        tok = _dispatch(ids, b, n)
        out = torch.full((tok.numel(), H), float("nan"), dtype=torch.float16, device="cuda")
        if tok.numel():
            fused_moe_routed(inp["x"][tok].contiguous(), ids[tok].contiguous(), w[tok].contiguous(),
                             inp["wg"][b:b + n], inp["wu"][b:b + n], inp["wd"][b:b + n], expert_begin=b,
                             num_experts=E, out=out)
        torch.cuda.synchronize()
        total[tok] += out.float()
        if g in (0, G - 1) and tok.numel():
            pick = torch.from_numpy(np.sort(np.random.default_rng(g).choice(tok.numel(), min(tok.numel(), 24),
                                                                             replace=False))).cuda()
            ref = fused_moe_forward(inp["x"][tok[pick]].cpu(), None, inp["wg"][b:b + n], inp["wu"][b:b + n],
                                    inp["wd"][b:b + n], inp["k"], expert_range=(b, n),
                                    routing=(ids[tok[pick]].cpu(), w[tok[pick]].cpu()))
            assert_close(out[pick], ref, what=f"{name} dispatched shard {g}/{G}")
            assert torch.isfinite(out).all()
    # each part is rounded to fp16 once: the sum differs from the full layer by those roundings
    assert_close(total, full.float(), what=f"{name}: sum of {G} dispatched shards")


def test_foreign_and_negative_ids_and_unnormalised_weights():
    from muxi_race_amd import fused_moe_routed
    inp = moe_inputs("small", 103, T=200)
    T, k = inp["T"], inp["k"]
    g = torch.Generator().manual_seed(7)
    ids = torch.randint(-1, 12, (T, k), generator=g, dtype=torch.int32)  # a 12-expert routing
    w = torch.rand((T, k), generator=g) * 3
    ids[:7] = 20  # tokens with no choice here at all
    b, n = 2, 4
    got = fused_moe_routed(inp["x"], ids.cuda(), w.cuda(), inp["wg"][b:b + n], inp["wu"][b:b + n],
                           inp["wd"][b:b + n], expert_begin=b, num_experts=12)
    torch.cuda.synchronize()
    ref = fused_moe_forward(inp["x"].cpu(), None, inp["wg"][b:b + n], inp["wu"][b:b + n], inp["wd"][b:b + n], k,
                            expert_range=(b, n), routing=(ids, w))
    assert_close(got, ref, what="foreign / negative ids")
    assert (got[:7] == 0).all()


def test_routed_argument_errors():
    from muxi_race_amd import MoeError, fused_moe_routed
    inp = moe_inputs("small", 104, T=64)
    ids, w = _route(inp)
    wg, wu, wd = inp["wg"], inp["wu"], inp["wd"]
    with pytest.raises(TypeError):
        fused_moe_routed(inp["x"], ids.long(), w, wg, wu, wd)             # int64 ids
    with pytest.raises(ValueError):
        fused_moe_routed(inp["x"], ids[:-1], w[:-1], wg, wu, wd)          # rows != tokens
    with pytest.raises(ValueError):
        fused_moe_routed(inp["x"], ids, w, wg, wu, wd, expert_begin=2, num_experts=inp["E"])  # past E
    with pytest.raises((ValueError, MoeError)):
        fused_moe_routed(inp["x"], ids, w, wg[:, :, :-1], wu, wd)         # bad weight shape


def test_routed_edge_cases():
    """An empty batch returns at once; a token that lists the same expert twice
    gets both pairs (two rows summed, as the oracle's align keeps both); k = 1
    with weights of 1 is the plain per-expert MLP."""
    from muxi_race_amd import fused_moe_routed
    inp = moe_inputs("small", 105, T=96)
    T, H, E = inp["T"], inp["H"], inp["E"]
    wg, wu, wd = inp["wg"], inp["wu"], inp["wd"]
    empty = fused_moe_routed(inp["x"][:0], torch.zeros((0, 2), dtype=torch.int32, device="cuda"),
                             torch.zeros((0, 2), device="cuda"), wg, wu, wd)
    assert empty.shape == (0, H)
    g = torch.Generator().manual_seed(11)
    ids = torch.randint(0, E, (T, 3), generator=g, dtype=torch.int32)
    ids[:, 1] = ids[:, 0]  # every token lists its first expert twice
    w = torch.rand((T, 3), generator=g)
    got = fused_moe_routed(inp["x"], ids.cuda(), w.cuda(), wg, wu, wd)
    ref = fused_moe_forward(inp["x"].cpu(), None, wg, wu, wd, 3, expert_range=(0, E), routing=(ids, w))
    assert_close(got, ref, what="duplicate choices")
    one = torch.randint(0, E, (T, 1), generator=g, dtype=torch.int32)
    got1 = fused_moe_routed(inp["x"], one.cuda(), torch.ones((T, 1), device="cuda"), wg, wu, wd)
    torch.cuda.synchronize()
    xd = inp["x"].cpu().double()
    exp = torch.zeros(T, H, dtype=torch.float64)
    for e in range(E):
        rows = (one[:, 0] == e).nonzero().flatten()
        if rows.numel():
            g_ = xd[rows] @ wg[e].cpu().double().T
            u_ = xd[rows] @ wu[e].cpu().double().T
            exp[rows] = (torch.sigmoid(g_) * g_ * u_) @ wd[e].cpu().double().T
    assert_close(got1, exp, what="k = 1, weight 1: the per-expert MLP")
