"""GPU parity of fused_moe with a DeepSeek-style always-on shared expert
(expert E, weight 1, appended to every token as choice k) against the CPU
oracle: routing ids bit-exact with the shared column, outputs within the fp16
tolerance, on the small, decode, mixtral and dsv3 configs, every output
element compared.  Outputs are NaN-poisoned and must come back finite."""
import numpy as np
import pytest
import torch

from _cases import moe_inputs, stratified_tokens
from conftest import assert_close
from oracle import fused_moe_forward, route_topk

pytestmark = pytest.mark.gpu


def _shared_weights(inp, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    H, I = inp["H"], inp["I"]
    mk = lambda shape: torch.randn(shape, generator=g, device="cuda", dtype=torch.float16) * 0.02
    return mk((I, H)), mk((I, H)), mk((H, I))


def _check(inp, shared, sample=None, block_m=0, what=""):
    from muxi_race_amd import fused_moe
    out = torch.full((inp["T"], inp["H"]), float("nan"), dtype=torch.float16, device="cuda")
    out, (ids, w) = fused_moe(inp["x"], inp["logits"], inp["wg"], inp["wu"], inp["wd"], inp["k"],
                              expert_bias=inp["bias"], block_m=block_m, return_routing=True,
                              shared_expert=shared, out=out)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all()), "non-finite values left in the NaN-poisoned output"
    T, E, k = inp["T"], inp["E"], inp["k"]
    bias = None if inp["bias"] is None else inp["bias"].cpu()
    rid, rw = route_topk(inp["logits"].cpu().numpy(), k, None if bias is None else bias.numpy())
    assert tuple(ids.shape) == (T, k + 1)
    np.testing.assert_array_equal(ids[:, :k].cpu().numpy(), rid)
    np.testing.assert_allclose(w[:, :k].cpu().numpy(), rw, rtol=1e-5, atol=1e-7)
    assert (ids[:, k] == E).all() and (w[:, k] == 1.0).all()
    rows = torch.arange(T) if sample is None else torch.from_numpy(stratified_tokens(ids.cpu().numpy(), seed=T))
    print(f"{what}: {len(rows)} of {T} tokens checked", flush=True)
    ref = fused_moe_forward(inp["x"][rows.cuda()].cpu(), inp["logits"][rows.cuda()].cpu(), inp["wg"], inp["wu"],
                            inp["wd"], k, bias, shared=[s.cpu() for s in shared])
    assert_close(out[rows.cuda()], ref, what=what)
    return out


@pytest.mark.parametrize("bm", [0, 32, 64, 128])
def test_small(bm):
    inp = moe_inputs("small", 41, T=512)
    _check(inp, _shared_weights(inp, 1), block_m=bm, what=f"small bm={bm}")


def test_decode_full():
    inp = moe_inputs("decode", 42)
    _check(inp, _shared_weights(inp, 2), what="decode")


def test_mixtral_full():
    inp = moe_inputs("mixtral", 43)
    _check(inp, _shared_weights(inp, 3), what="mixtral")


def test_dsv3_full():
    inp = moe_inputs("dsv3", 44)
    _check(inp, _shared_weights(inp, 4), what="dsv3")


def test_single_token():
    inp = moe_inputs("small", 45, T=1)
    _check(inp, _shared_weights(inp, 5), what="T=1")


def test_from_hidden_equals_from_logits():
    from muxi_race_amd import fused_moe, route_hidden
    inp = moe_inputs("decode", 46)
    shared = _shared_weights(inp, 6)
    g = torch.Generator().manual_seed(6)
    wr = (torch.randn((inp["E"], inp["H"]), generator=g) / inp["H"] ** 0.5).half().cuda()
    _, _, logits = route_hidden(inp["x"], wr, inp["k"], inp["bias"], return_logits=True)
    a, (ia, wa) = fused_moe(inp["x"], None, inp["wg"], inp["wu"], inp["wd"], inp["k"], expert_bias=inp["bias"],
                            router_weight=wr, return_routing=True, shared_expert=shared)
    b, (ib, wb) = fused_moe(inp["x"], logits, inp["wg"], inp["wu"], inp["wd"], inp["k"], expert_bias=inp["bias"],
                            return_routing=True, shared_expert=shared)
    torch.cuda.synchronize()
    assert torch.equal(ia, ib) and torch.equal(wa, wb)
    assert torch.equal(a, b)


def test_rejects_bad_shapes():
    from muxi_race_amd import fused_moe
    inp = moe_inputs("small", 47, T=4)
    sg, su, sd = _shared_weights(inp, 7)
    with pytest.raises(ValueError):
        fused_moe(inp["x"], inp["logits"], inp["wg"], inp["wu"], inp["wd"], inp["k"], shared_expert=(sg, su, sg))
    with pytest.raises(ValueError):
        fused_moe(inp["x"], inp["logits"], inp["wg"], inp["wu"], inp["wd"], inp["k"], shared_expert=(sg, su))
