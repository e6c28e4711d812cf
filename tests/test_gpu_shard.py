"""Expert-parallel shards on one GPU (fused_moe(expert_range=)): each shard
against the oracle's shard, the shards' partial outputs summing to the full
layer, and the global routing returned unchanged."""
import numpy as np
import pytest
import torch

from _cases import moe_inputs
from conftest import assert_close
from oracle import fused_moe_forward

pytestmark = pytest.mark.gpu


def _shard(inp, b, n, **kw):
    from muxi_race_amd import fused_moe
    return fused_moe(inp["x"], inp["logits"], inp["wg"][b:b + n], inp["wu"][b:b + n], inp["wd"][b:b + n],
                     inp["k"], expert_bias=inp["bias"], expert_range=(b, n), return_routing=True, **kw)


@pytest.mark.parametrize("name,G", [("small", 2), ("small", 8), ("decode", 8), ("dsv3", 8), ("mixtral", 4)])
def test_shards_sum_to_full_and_match_oracle(name, G):
    from muxi_race_amd import fused_moe
    # mixtral at T=1536: 384 routed rows per expert over the whole layer, so every
    # shard runs on the 256-row padding
    inp = moe_inputs(name, 91, T={"dsv3": 1024, "mixtral": 1536}.get(name))
    E, T = inp["E"], inp["T"]
    full, (fids, fw) = fused_moe(inp["x"], inp["logits"], inp["wg"], inp["wu"], inp["wd"], inp["k"],
                                 expert_bias=inp["bias"], return_routing=True)
    n = E // G
    parts = []
    rows = torch.from_numpy(np.sort(np.random.default_rng(T).choice(T, min(T, 16), replace=False)))
    bias = None if inp["bias"] is None else inp["bias"].cpu()
    for g in range(G):
        out, (ids, w) = _shard(inp, g * n, n)
        torch.cuda.synchronize()
        assert torch.equal(ids, fids) and torch.equal(w, fw)
        parts.append(out.float())
        if g in (0, G - 1):
            ref = fused_moe_forward(inp["x"][rows.cuda()].cpu(), inp["logits"][rows.cuda()].cpu(),
                                    inp["wg"][g * n:(g + 1) * n], inp["wu"][g * n:(g + 1) * n],
                                    inp["wd"][g * n:(g + 1) * n], inp["k"], bias, expert_range=(g * n, n))
            assert_close(out[rows.cuda()], ref, what=f"{name} shard {g}/{G}")
    total = sum(parts)
    # each part is rounded to fp16 once: the sum differs from the full layer by those roundings
    assert_close(total, full.float(), what=f"{name}: sum of {G} shards")


def test_shard_with_no_pairs_is_zero_and_errors():
    inp = moe_inputs("small", 92, T=64)
    inp["logits"][:, 4:] -= 100.0  # nobody picks experts 4..7
    out, _ = _shard(inp, 4, 4)
    torch.cuda.synchronize()
    assert (out == 0).all()
    with pytest.raises(ValueError):
        _shard(inp, 6, 4)                  # past the routed experts
    with pytest.raises(ValueError):
        _shard(inp, 0, 2, block_m=0, shared_expert=(inp["wg"][0], inp["wu"][0], inp["wd"][0]))
