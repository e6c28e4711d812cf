"""GPU router and moe_align: indices bit-exact against the CPU oracle on every
BASELINE config's logits and on tie-heavy / edge inputs."""
import numpy as np
import pytest
import torch

from _cases import CONFIGS, moe_inputs
from oracle import align, route_topk

pytestmark = pytest.mark.gpu


def _route_both(logits, k, bias):
    from muxi_race_amd import route_topk as gpu_route
    ids, w = gpu_route(logits, k, bias)
    torch.cuda.synchronize()
    rid, rw = route_topk(logits.cpu().numpy(), k, None if bias is None else bias.cpu().numpy())
    return ids.cpu().numpy(), w.cpu().numpy(), rid, rw


def _logits_for(name, seed):
    T, H, I, E, k, bias_kind = CONFIGS[name]
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn((T, E), generator=g)
    bias = None
    if bias_kind == "normal":
        bias = torch.randn((E,), generator=g) * 0.5
    elif bias_kind == "zipf":
        bias = -1.2 * torch.log(torch.arange(E, dtype=torch.float32) + 1)
    return logits.cuda(), (None if bias is None else bias.cuda()), k, E


@pytest.mark.parametrize("name", list(CONFIGS))
def test_routing_bit_exact(name):
    logits, bias, k, E = _logits_for(name, 100)
    ids, w, rid, rw = _route_both(logits, k, bias)
    np.testing.assert_array_equal(ids, rid)
    np.testing.assert_allclose(w, rw, rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("E,k", [(8, 2), (64, 6), (256, 8), (1000, 32), (3, 3), (1, 1), (8, 8), (5, 1), (65, 32)])
def test_routing_ties(E, k):
    g = torch.Generator().manual_seed(E)
    logits = (torch.randn((257, E), generator=g) * 2).round() / 2  # many exact ties
    logits[0] = 0.0  # all-equal row -> experts 0..k-1
    ids, w, rid, rw = _route_both(logits.cuda(), k, None)
    np.testing.assert_array_equal(ids, rid)
    np.testing.assert_array_equal(ids[0], np.arange(k))
    np.testing.assert_allclose(w, rw, rtol=1e-5, atol=1e-7)


def _align_both(ids_np, E, bm, many_workgroups=True):
    from muxi_race_amd import moe_align
    got = moe_align(torch.from_numpy(ids_np).cuda(), E, bm, many_workgroups=many_workgroups)
    torch.cuda.synchronize()
    ref = align(ids_np, E, bm)
    rows = int(ref["group_padded_offsets"][-1])
    assert int(got["group_padded_offsets"][-1]) == rows
    np.testing.assert_array_equal(got["sorted_pair_ids"][:rows].cpu().numpy(), ref["sorted_pair_ids"])
    np.testing.assert_array_equal(got["block_expert"][:rows // bm].cpu().numpy(), ref["block_expert"])
    for key in ("group_sizes", "group_offsets", "group_padded_offsets"):
        np.testing.assert_array_equal(got[key].cpu().numpy(), ref[key])


@pytest.mark.parametrize("name", list(CONFIGS))
@pytest.mark.parametrize("bm", [32, 128, 256])
@pytest.mark.parametrize("many", [True, False])  # several workgroups (large P) or one
def test_align_bit_exact(name, bm, many):
    logits, bias, k, E = _logits_for(name, 200)
    rid, _ = route_topk(logits.cpu().numpy(), k, None if bias is None else bias.cpu().numpy())
    _align_both(rid, E, bm, many)


def test_align_edges():
    rng = np.random.default_rng(0)
    _align_both(np.zeros((3000, 1), np.int32), 4, 128)            # one expert takes all
    _align_both(np.array([[5]], np.int32), 1024, 64)              # one pair, E = 1024
    _align_both(np.zeros((0, 2), np.int32), 8, 128)               # no tokens
    ids = np.stack([rng.choice(1024, 8, replace=False) for _ in range(5000)]).astype(np.int32)
    _align_both(ids, 1024, 32)                                     # many chunks, wide E (8 waves)
    _align_both(np.full((70000, 2), 7, np.int32), 16, 128)         # 64 workgroups, one hot expert
    small = np.stack([rng.choice(1000, 8, replace=False) for _ in range(300)]).astype(np.int32)
    _align_both(small, 1000, 32)                                   # small batch, wide E (8 waves)
    _align_both(rng.integers(0, 256, (37, 7)).astype(np.int32), 256, 16)   # ragged small batch
    _align_both(rng.integers(0, 8, (1024, 8)).astype(np.int32), 8, 128)    # 512 pairs per wave (limit)


@pytest.mark.parametrize("T,k,E,bm", [(301, 3, 16, 64), (4000, 2, 16, 128)])
def test_align_drops_out_of_range_ids(T, k, E, bm):
    """Pairs whose id lies outside [0, E) are not placed.  Reference: the
    oracle's align with those pairs sent to an extra last expert E, whose rows
    come after every kept expert's and so leave theirs unchanged."""
    from muxi_race_amd import moe_align
    ids = np.random.default_rng(T).integers(-3, E + 3, (T, k)).astype(np.int32)
    ref = align(np.where((ids >= 0) & (ids < E), ids, E).astype(np.int32), E + 1, bm)
    got = moe_align(torch.from_numpy(ids).cuda(), E, bm)
    torch.cuda.synchronize()
    rows = int(ref["group_padded_offsets"][E])
    assert int(got["group_padded_offsets"][E]) == rows
    np.testing.assert_array_equal(got["sorted_pair_ids"][:rows].cpu().numpy(), ref["sorted_pair_ids"][:rows])
    np.testing.assert_array_equal(got["block_expert"][:rows // bm].cpu().numpy(), ref["block_expert"][:rows // bm])
    np.testing.assert_array_equal(got["group_sizes"].cpu().numpy(), ref["group_sizes"][:E])
    np.testing.assert_array_equal(got["group_offsets"].cpu().numpy()[:E], ref["group_offsets"][:E])
    np.testing.assert_array_equal(got["group_padded_offsets"].cpu().numpy(), ref["group_padded_offsets"][:E + 1])


def test_align_many_workgroups_matches_one_on_dropped_ids():
    """Out-of-range ids are dropped (the oracle rejects them): both GPU paths
    must still agree bit for bit on a ragged batch spread over 14 workgroups."""
    from muxi_race_amd import moe_align
    ids = torch.from_numpy(np.random.default_rng(1).integers(-3, 19, (9001, 3)).astype(np.int32)).cuda()
    a = moe_align(ids, 16, 64, many_workgroups=True)
    b = moe_align(ids, 16, 64, many_workgroups=False)
    torch.cuda.synchronize()
    rows = int(b["group_padded_offsets"][-1])
    assert int(a["group_padded_offsets"][-1]) == rows
    assert torch.equal(a["sorted_pair_ids"][:rows], b["sorted_pair_ids"][:rows])
    assert torch.equal(a["block_expert"][:rows // 64], b["block_expert"][:rows // 64])
    for key in ("group_sizes", "group_offsets", "group_padded_offsets"):
        assert torch.equal(a[key], b[key])


def test_routing_signed_zero_and_nan_order():
    """-0.0 and +0.0 are equal logits (ties to the lower expert), and a NaN
    logit ranks below every number, as in the oracle's stable sort of -v.
    Ids only: a NaN in the row makes the oracle's softmax NaN."""
    from muxi_race_amd import route_topk as gpu_route
    E, k = 70, 6
    g = torch.Generator().manual_seed(5)
    logits = torch.randn((64, E), generator=g)
    logits[0] = 0.0
    logits[0, ::2] = -0.0                      # alternating signed zeros: experts 0..5
    logits[1, :] = -1.0
    logits[1, [3, 9, 40]] = float("nan")       # NaNs never beat -1
    logits[2, :8] = float("nan")               # NaN in the first 8 experts: after every number
    logits[3, : E - 2] = float("nan")          # only 2 numbers: they come first, then NaNs by index
    ids, _ = gpu_route(logits.cuda(), k, None)
    torch.cuda.synchronize()
    rid, _ = route_topk(logits.numpy(), k)
    np.testing.assert_array_equal(ids.cpu().numpy(), rid)
    np.testing.assert_array_equal(ids[0].cpu().numpy(), np.arange(k))
    np.testing.assert_array_equal(ids[3, :2].cpu().numpy(), [E - 2, E - 1])
