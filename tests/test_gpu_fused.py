"""GPU parity of fused_moe (route -> align -> Stage1 -> Stage2 -> combine)
against the CPU oracle, on every BASELINE config.  Every call writes into a
NaN-poisoned output that must come back finite everywhere.  Every config's
whole output is compared with the oracle (remote_bench.py:262-280 checks the
whole output too); only T = 32768 is checked on a stratified token set
(oracle/sampling.py stratified_tokens: the first and last pair of every
touched expert and the first row of every block, so every item of both stages
feeds a checked element; tokens are independent, so the oracle on those rows,
with the full expert weights, is exact for them)."""
import numpy as np
import pytest
import torch

from _cases import moe_inputs, stratified_tokens
from conftest import assert_close
from oracle import fused_moe_forward, route_topk

pytestmark = pytest.mark.gpu


def _gpu(inp, block_m=0):
    from muxi_race_amd import fused_moe
    out = torch.full((inp["T"], inp["H"]), float("nan"), dtype=torch.float16, device="cuda")
    out, (ids, w) = fused_moe(inp["x"], inp["logits"], inp["wg"], inp["wu"], inp["wd"], inp["k"],
                              expert_bias=inp["bias"], block_m=block_m, return_routing=True, out=out)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all()), "non-finite values left in the NaN-poisoned output"
    return out, ids, w


def _check(inp, sample=None, block_m=0, what="", **strat):
    """sample None: every token; "strat": stratified_tokens(**strat)."""
    out, ids, w = _gpu(inp, block_m)
    T = inp["T"]
    bias = None if inp["bias"] is None else inp["bias"].cpu()
    # routing indices are bit-exact for every token
    rid, rw = route_topk(inp["logits"].cpu().numpy(), inp["k"], None if bias is None else bias.numpy())
    np.testing.assert_array_equal(ids.cpu().numpy(), rid)
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=1e-5, atol=1e-7)
    rows = torch.arange(T) if sample is None else torch.from_numpy(stratified_tokens(rid, seed=T, **strat))
    print(f"{what}: {len(rows)} of {T} tokens checked", flush=True)
    ref = fused_moe_forward(inp["x"][rows.cuda()].cpu(), inp["logits"][rows.cuda()].cpu(),
                            inp["wg"], inp["wu"], inp["wd"], inp["k"], bias)
    assert_close(out[rows.cuda()], ref, what=what)
    return out


def test_small_full():
    _check(moe_inputs("small", 1), what="small")


@pytest.mark.parametrize("bm", [32, 64, 128])
def test_block_m_variants(bm):
    inp = moe_inputs("small", 2, T=512)
    _check(inp, block_m=bm, what=f"bm={bm}")


def test_decode_full():
    _check(moe_inputs("decode", 3), what="decode")


def test_mixtral_full():
    _check(moe_inputs("mixtral", 4), what="mixtral")


def test_mixtral_ragged():
    # H = 4096 takes Stage 2's 256-wide N tiles; T = 700 leaves ragged last blocks
    _check(moe_inputs("mixtral", 9, T=700), block_m=128, what="mixtral T=700")


def test_dsv3_full():
    _check(moe_inputs("dsv3", 5), what="dsv3")


def test_edge_single_token_and_single_expert():
    inp = moe_inputs("small", 6, T=1)
    _check(inp, what="T=1")
    inp = moe_inputs("small", 7, T=300)
    inp["logits"][:, 3] += 100.0  # every token picks expert 3 first -> 3 blocks of one expert
    _check(inp, block_m=128, what="one hot expert")


def test_repeat_is_bitwise_deterministic():
    inp = moe_inputs("small", 8, T=256)
    a, _, _ = _gpu(inp)
    for _ in range(3):
        b, _, _ = _gpu(inp)
        assert torch.equal(a, b)


def test_two_streams_do_not_share_scratch():
    """Calls on two streams (default priority) may overlap: each gets its own
    workspace, so both results equal the one-stream results."""
    from muxi_race_amd import fused_moe
    a_in, b_in = moe_inputs("small", 10, T=384), moe_inputs("decode", 11)
    ra, _, _ = _gpu(a_in)
    rb, _, _ = _gpu(b_in)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    outs = []
    for _ in range(3):
        with torch.cuda.stream(s1):
            oa = fused_moe(a_in["x"], a_in["logits"], a_in["wg"], a_in["wu"], a_in["wd"], a_in["k"],
                           expert_bias=a_in["bias"])
        with torch.cuda.stream(s2):
            ob = fused_moe(b_in["x"], b_in["logits"], b_in["wg"], b_in["wu"], b_in["wd"], b_in["k"],
                           expert_bias=b_in["bias"])
        outs.append((oa, ob))
    torch.cuda.synchronize()
    for oa, ob in outs:
        assert torch.equal(oa, ra) and torch.equal(ob, rb)


def _random_case(T, H, I, E, k, seed, bias=True):
    g = torch.Generator().manual_seed(seed)
    return dict(x=torch.randn(T, H, generator=g).half().cuda(), logits=torch.randn(T, E, generator=g).cuda(),
                bias=(torch.randn(E, generator=g) * 0.5).cuda() if bias else None,
                wg=(torch.randn(E, I, H, generator=g) * 0.05).half().cuda(),
                wu=(torch.randn(E, I, H, generator=g) * 0.05).half().cuda(),
                wd=(torch.randn(E, H, I, generator=g) * 0.05).half().cuda(), k=k, T=T, H=H, I=I, E=E)


@pytest.mark.parametrize("T,H,I,E,k", [
    (1, 128, 128, 1, 1),        # smallest legal problem
    (3, 128, 256, 1024, 32),    # widest routing: E = 1024 experts, k = 32 choices
    (257, 256, 128, 32, 32),    # every token takes every expert (k = E)
    (129, 384, 640, 5, 3),      # odd expert count, H and I not powers of two
    # more than 256 experts (no absorbed rows): ~109 rows each on paired
    # 128-row items, and ~218 each on 256-row items (H a multiple of 256)
    (4096, 128, 256, 300, 8),
    (8192, 256, 256, 300, 8),
])
def test_extreme_shapes(T, H, I, E, k):
    _check(_random_case(T, H, I, E, k, T + E), what=f"T={T} H={H} I={I} E={E} k={k}")


def test_256_row_padding_ragged():
    """fp16 experts with >= 192 routed rows on average and H a multiple of 256:
    align pads experts to 256 rows, Stage 1 runs 256-row items, Stage 2
    128-row (paired) items.  Skewed biases give full, partial and empty
    256-row blocks, 128-row halves with no rows, and two empty experts."""
    inp = _random_case(1536, 512, 384, 8, 2, 77, bias=False)
    inp["bias"] = torch.tensor([2.5, 2.0, 1.0, 0.5, 0.0, -0.5, -40.0, -40.0], device="cuda")
    from muxi_race_amd import pick_block_m
    assert pick_block_m(1536, 8, 2) == 128
    _check(inp, what="fp16, 256-row padding")


def test_empty_batch():
    from muxi_race_amd import fused_moe
    inp = _random_case(1, 128, 128, 4, 2, 5)
    x = inp["x"][:0]
    out, (ids, w) = fused_moe(x, inp["logits"][:0], inp["wg"], inp["wu"], inp["wd"], 2, return_routing=True)
    torch.cuda.synchronize()
    assert out.shape == (0, 128) and ids.shape == (0, 2) and w.shape == (0, 2)


def test_large_batch_sampled():
    """A large prefill batch: dsv3 shape at T = 32768 (262144 routed pairs, the
    64-workgroup align, 3.8 GB of per-pair rows), checked on sampled tokens."""
    inp = moe_inputs("dsv3", 12, T=32768)
    _check(inp, sample="strat", what="dsv3 T=32768", max_block_starts=256, extra=32)
