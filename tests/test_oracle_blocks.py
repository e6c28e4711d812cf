"""Pins oracle.prerouted_forward_blocks -- the reference operator's per-block
form (block b -> expert group_idx_for_bx[b], submission.py:1444-1447,
:1283-1299, :2115) -- against the independently pinned expert loop
(prerouted_forward) and hand-derived answers for metadata the harness never
builds."""
import numpy as np
import torch

from _cases import random_group_sizes
from oracle import metadata_from_group_sizes, prerouted_forward, prerouted_forward_blocks


def _weights(E, H, I, seed):
    g = torch.Generator().manual_seed(seed)
    return [(torch.randn(shape, generator=g) * 0.3).half() for shape in ((E, I, H), (E, I, H), (E, H, I))]


def test_equals_expert_loop_on_harness_metadata():
    """On remote_bench.py:82-101 metadata the block form is the SPEC loop."""
    H, I = 32, 16
    for seed in range(4):
        sizes = random_group_sizes(6, 900, 4000 + seed)
        go, gpo, gidx = metadata_from_group_sizes(sizes, 128)
        P = int(gpo[-1])
        g = torch.Generator().manual_seed(seed)
        x = torch.randn(P, H, generator=g).half()
        routed = torch.rand(int(go[-1]), generator=g)
        wg, wu, wd = _weights(6, H, I, seed)
        a = prerouted_forward(x, wg, wu, wd, routed, sizes, go, gpo, gidx)
        b = prerouted_forward_blocks(x, wg, wu, wd, routed, sizes, go, gpo, gidx)
        assert torch.equal(a, b)


def _mlp1(x, wg, wu, wd, routed):
    """One expert's rows through the expert loop (E = 1, one group)."""
    n = x.shape[0]
    go, gpo, gidx = metadata_from_group_sizes([n], 128)
    pad = torch.zeros(int(gpo[-1]), x.shape[1], dtype=x.dtype)
    pad[:n] = x
    return prerouted_forward(pad, wg[None], wu[None], wd[None], routed, [n], go, gpo, gidx)[:n]


def test_swapped_block_experts():
    """gs = [128, 128], gpo = [0, 128, 256], gidx = [1, 0]: block 0 runs
    expert 1 at token offset -128, so all 128 rows are valid and take
    routed[128 - 128 + i] = routed[i]; block 1 runs expert 0 at offset 128 and
    has no valid row."""
    H, I = 16, 8
    wg, wu, wd = _weights(2, H, I, 1)
    g = torch.Generator().manual_seed(2)
    x = torch.randn(256, H, generator=g).half()
    routed = torch.rand(256, generator=g)
    out = prerouted_forward_blocks(x, wg, wu, wd, routed, [128, 128], [0, 128, 256], [0, 128, 256], [1, 0])
    exp0 = _mlp1(x[:128], wg[1], wu[1], wd[1], routed[:128])
    assert torch.equal(out[:128], exp0)
    assert (out[128:] == 0).all()


def test_trailing_short_and_out_of_range_blocks():
    """Sizes [3, 130] (blocks 0 | 1, 2), two trailing blocks past gpo[E] that
    name expert 1 (offset past its rows: zero), one naming expert 7 (outside
    [0, E): zero), and a gidx one block short of P: the last block's rows keep
    the initial contents of out."""
    H, I = 16, 8
    wg, wu, wd = _weights(2, H, I, 3)
    sizes = [3, 130]
    go, gpo, _ = metadata_from_group_sizes(sizes, 128)
    gidx = [0, 1, 1, 1, 7]  # blocks 3 and 4 lie past gpo[E] = 384; P holds 7 blocks
    P = 7 * 128
    g = torch.Generator().manual_seed(4)
    x = torch.randn(P, H, generator=g).half()
    routed = torch.rand(int(go[-1]), generator=g)
    init = torch.full((P, H), 5.0, dtype=torch.float16)
    out = prerouted_forward_blocks(x, wg, wu, wd, routed, sizes, go, gpo, gidx, out=init)
    assert torch.equal(out[:3], _mlp1(x[:3], wg[0], wu[0], wd[0], routed[:3]))
    assert torch.equal(out[128:258], _mlp1(x[128:258], wg[1], wu[1], wd[1], routed[3:133]))
    assert (out[3:128] == 0).all() and (out[258:640] == 0).all()
    assert (out[640:] == 5.0).all()


def test_clamped_routed_index():
    """A block placed before its expert's padded start (offset -128) reads
    routed[clamp(go[e] - 128 + i, 0, V - 1)]: with go[e] = 0, routed[0] for
    every row, which the one-row expert loop reproduces row by row."""
    H, I = 16, 8
    wg, wu, wd = _weights(2, H, I, 5)
    g = torch.Generator().manual_seed(6)
    x = torch.randn(256, H, generator=g).half()
    routed = torch.rand(10, generator=g)
    # expert 1: 10 rows at padded start 128, raw start 0; block 0 names it
    out = prerouted_forward_blocks(x, wg, wu, wd, routed, [0, 10], [0, 0, 10], [0, 128, 256], [1, 1])
    # block 0: offset -128, n = min(128, 138) = 128 valid rows, routed index clamp(i - 128) = 0
    exp = _mlp1(x[:128], wg[1], wu[1], wd[1], routed[:1].expand(128).contiguous())
    assert torch.equal(out[:128], exp)
    # block 1: offset 0, 10 valid rows with routed[0..9]
    assert torch.equal(out[128:138], _mlp1(x[128:138], wg[1], wu[1], wd[1], routed))
    assert (out[138:] == 0).all()
