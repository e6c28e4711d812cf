"""Pins oracle.align / metadata_from_group_sizes with hand-written known answers
(problem_detail.json:40 example; remote_bench.py:82-101 construction) and
invariants."""
import numpy as np
import pytest

from oracle import align, metadata_from_group_sizes, route_topk


def test_spec_example_metadata():
    """problem_detail.json:40: E=2, group_sizes=[3,2], group_offsets=[0,3]:
    expert 0 owns rows 0..2, expert 1 starts at padded row 128."""
    go, gpo, gidx = metadata_from_group_sizes([3, 2], 128)
    np.testing.assert_array_equal(go, [0, 3, 5])
    np.testing.assert_array_equal(gpo, [0, 128, 256])
    np.testing.assert_array_equal(gidx, [0, 1])


def test_known_answer_with_empty_and_boundary_experts():
    # sizes 0 / 129 / 128 / 1: empty expert gets no block; 129 needs two blocks
    go, gpo, gidx = metadata_from_group_sizes([0, 129, 128, 1], 128)
    np.testing.assert_array_equal(go, [0, 0, 129, 257, 258])
    np.testing.assert_array_equal(gpo, [0, 0, 256, 384, 512])
    np.testing.assert_array_equal(gidx, [1, 1, 2, 3])


def test_known_answer_block32():
    go, gpo, gidx = metadata_from_group_sizes([33, 0, 32], 32)
    np.testing.assert_array_equal(go, [0, 33, 33, 65])
    np.testing.assert_array_equal(gpo, [0, 64, 64, 96])
    np.testing.assert_array_equal(gidx, [0, 0, 2])


def test_align_known_answer():
    # T=3 tokens, k=2: pairs p = t*2 + j
    ids = np.array([[2, 0], [0, 1], [2, 1]], dtype=np.int32)
    al = align(ids, 3, 4)
    # expert 0: pairs 1, 2 ; expert 1: pairs 3, 5 ; expert 2: pairs 0, 4; sentinel 6
    np.testing.assert_array_equal(al["sorted_pair_ids"], [1, 2, 6, 6, 3, 5, 6, 6, 0, 4, 6, 6])
    np.testing.assert_array_equal(al["block_expert"], [0, 1, 2])
    np.testing.assert_array_equal(al["group_sizes"], [2, 2, 2])
    np.testing.assert_array_equal(al["group_offsets"], [0, 2, 4, 6])
    np.testing.assert_array_equal(al["group_padded_offsets"], [0, 4, 8, 12])


@pytest.mark.parametrize("T,k,E,bm", [(1, 1, 1, 128), (50, 2, 8, 32), (300, 8, 64, 128), (7, 3, 300, 64), (700, 8, 16, 256)])
def test_align_invariants(rng, T, k, E, bm):
    ids = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    al = align(ids, E, bm)
    P = T * k
    sp, gs, go, gpo = (al[n] for n in ("sorted_pair_ids", "group_sizes", "group_offsets", "group_padded_offsets"))
    assert sp.shape[0] == gpo[-1] and gpo[-1] % bm == 0
    valid = sp[sp < P]
    assert sorted(valid.tolist()) == list(range(P)), "valid rows are a permutation of the pairs"
    flat = ids.reshape(-1)
    for e in range(E):
        rows = sp[gpo[e]:gpo[e + 1]]
        n = int(gs[e])
        assert (gpo[e + 1] - gpo[e]) == -(-n // bm) * bm
        assert (flat[rows[:n]] == e).all(), "rows of expert e hold pairs routed to e"
        assert (np.diff(rows[:n]) > 0).all(), "ascending pair order inside an expert"
        assert (rows[n:] == P).all(), "padding rows hold the sentinel"
        assert go[e + 1] - go[e] == n
    assert (np.diff(al["block_expert"]) >= 0).all()
    assert al["block_expert"].shape[0] == gpo[-1] // bm


def test_align_capacity_bound(rng):
    """P_pad <= P + min(E, P) * (bm - 1): the bound the GPU workspace uses."""
    for _ in range(20):
        E = int(rng.integers(1, 64))
        k = int(rng.integers(1, min(E, 8) + 1))
        T = int(rng.integers(0, 200))
        bm = int(rng.choice([32, 64, 128, 256]))
        ids = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32) \
            if T else np.zeros((0, k), np.int32)
        al = align(ids, E, bm)
        P = T * k
        assert al["group_padded_offsets"][-1] <= P + min(E, P) * (bm - 1)


def test_stratified_tokens_cover_every_block():
    """The checkers' token sample holds, for every block of the align, a token
    with a pair in that block, and every touched expert's first and last pair
    (random dsv3-like routing, block sizes 128 and 256)."""
    from oracle import stratified_tokens
    rng = np.random.default_rng(3)
    T, E, k = 1024, 64, 6
    ids, _ = route_topk(rng.standard_normal((T, E)).astype(np.float32), k,
                        (rng.standard_normal(E) * 0.8).astype(np.float32))
    for bm in (128, 256):
        rows = stratified_tokens(ids, block=bm, extra=0)
        picked = np.zeros(T, bool)
        picked[rows] = True
        al = align(ids, E, bm)
        sp, P = al["sorted_pair_ids"], T * k
        for b in range(len(sp) // bm):
            blk = sp[b * bm:(b + 1) * bm]
            blk = blk[blk < P]
            if blk.size:
                assert picked[blk // k].any(), f"block {b} (bm={bm}) has no sampled token"
        gs, go = al["group_sizes"], al["group_offsets"]
        for e in range(E):
            if gs[e]:
                first = sp[al["group_padded_offsets"][e]]
                last = sp[al["group_padded_offsets"][e] + gs[e] - 1]
                assert picked[first // k] and picked[last // k]
    assert len(stratified_tokens(ids, block=128, extra=0, max_block_starts=4)) < len(rows)
