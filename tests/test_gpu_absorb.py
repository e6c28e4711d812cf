"""GPU parity of absorbed rows.  When an expert's last block holds at most 32
routed rows (after at least one other block), the schedule gives that block
no items: the expert's first item group takes those rows as extra token rows
(moe_common.h schedule_absorbed; fp16 256-row items and 128-row paired
items of both stages, E <= 256).  Exact per-expert counts straddle the rule:
1 and 32 rows past a block boundary are absorbed, 33 are not, and so are
single-block experts, empty ones and exact multiples.  They run under the
256-row padding (block_m 0 picks it here: H % 256 == 0, >= 192 rows per
expert) and the 128-row padding, with top-1 and top-2 routing.  Every output
is compared whole with the oracle, from a NaN-poisoned buffer."""
import numpy as np
import pytest
import torch

from _cases import exact_routing_inputs
from conftest import assert_close
from oracle import fused_moe_forward

pytestmark = pytest.mark.gpu

# per-expert routed rows; with 256-row blocks 257, 288, 513, 543 are absorbed
# in Stage 1, and with 128-row blocks 257, 288, 513, 543, 385 and 160 (fused
# launches let a two-block expert's pair become one item with the rows)
COUNTS = [257, 288, 289, 545, 513, 543, 256, 1, 0, 33, 160, 161, 385, 417]
H, I = 256, 256


def _inputs(k, seed, counts=COUNTS):
    return exact_routing_inputs(k, seed, counts, H, I)


@pytest.mark.parametrize("k", [1, 2])
@pytest.mark.parametrize("bm", [0, 128])
def test_absorbed_rows_full_output(k, bm):
    from muxi_race_amd import fused_moe
    x, logits, wg, wu, wd = _inputs(k, seed=31 + k)
    T = x.shape[0]
    out = torch.full((T, H), float("nan"), dtype=torch.float16, device="cuda")
    out = fused_moe(x.cuda(), logits.cuda(), wg.cuda(), wu.cuda(), wd.cuda(), k, block_m=bm, out=out)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all()), "non-finite values left in the NaN-poisoned output"
    ref = fused_moe_forward(x, logits, wg, wu, wd, k)
    assert_close(out, ref, what=f"absorbed rows k={k} bm={bm}")


def test_absorbed_rows_many_experts():
    """E = 150 (the expert scan's third chunk), top-2, the default block_m
    (128-row padding at ~140 rows per expert): Stage 1 paired 128-row items
    absorb too.  Experts of 129-160 rows (one block and up to 32 rows: the pair
    becomes one item) and of 257-288 (two blocks and up to 32) next to ones
    that stay as they are."""
    from muxi_race_amd import fused_moe
    rng = np.random.default_rng(5)
    counts = list(COUNTS) + [int(rng.choice([0, rng.integers(1, 40), rng.integers(129, 161), rng.integers(161, 257),
                                             rng.integers(257, 289)])) for _ in range(136)]
    counts[-1] += sum(counts) % 2
    x, logits, wg, wu, wd = _inputs(2, 41, counts)
    T = x.shape[0]
    out = torch.full((T, H), float("nan"), dtype=torch.float16, device="cuda")
    out = fused_moe(x.cuda(), logits.cuda(), wg.cuda(), wu.cuda(), wd.cuda(), 2, out=out)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all()), "non-finite values left in the NaN-poisoned output"
    assert_close(out, fused_moe_forward(x, logits, wg, wu, wd, 2), what="absorbed rows E=150")


def test_absorbed_rows_repeatable():
    """Two calls give bitwise the same output (the absorbed rows' items and
    the rest are fixed by the metadata alone)."""
    from muxi_race_amd import fused_moe
    x, logits, wg, wu, wd = (t.cuda() for t in _inputs(2, seed=40))
    a = fused_moe(x, logits, wg, wu, wd, 2)
    b = fused_moe(x, logits, wg, wu, wd, 2)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_absorbed_rows_prerouted_padding_zero():
    """run_kernel keeps its pairs (absorb = 2): runs of three or more blocks
    whose last block holds <= 32 rows (257, 288, 513, 385 here) are absorbed,
    129-160-row groups are not.  The absorbed blocks' padding rows must still
    come back exactly 0 from a NaN-poisoned output, with NaN in x's padding
    rows (problem_detail.json:50 note 4)."""
    from _cases import prerouted_inputs
    from muxi_race_amd import run_kernel
    from oracle import prerouted_forward
    sizes = [257, 288, 289, 513, 3, 0, 385, 130, 160]
    args = list(prerouted_inputs(sizes, 512, 256, seed=77))
    x, gpo = args[0], args[7].cpu().tolist()
    pad = torch.ones(x.shape[0], dtype=torch.bool)
    for e, n in enumerate(sizes):
        pad[gpo[e]:gpo[e] + n] = False
    x[pad.to(x.device)] = float("nan")
    out = torch.full(x.shape, float("nan"), dtype=torch.float16, device=x.device)
    run_kernel(*args, out)
    torch.cuda.synchronize()
    assert_close(out, prerouted_forward(*args), what="prerouted absorbed rows")
    assert (out[pad.to(out.device)] == 0).all()


def test_absorbed_rows_256_row_items_many_experts():
    """E = 80 at ~270 rows per expert (block_m 0 picks the 256-row padding):
    both stages on 256-row items, with the expert scan over two chunks.
    Experts of 257-288 and 513-544 rows are absorbed, 289+ and 545+ are not."""
    from muxi_race_amd import fused_moe
    rng = np.random.default_rng(9)
    counts = [int(rng.choice([rng.integers(257, 289), rng.integers(289, 400), rng.integers(513, 545),
                              rng.integers(100, 256), 0])) for _ in range(80)]
    counts[-1] += sum(counts) % 2
    assert sum(counts) / len(counts) >= 192
    x, logits, wg, wu, wd = _inputs(2, 43, counts)
    T = x.shape[0]
    out = torch.full((T, H), float("nan"), dtype=torch.float16, device="cuda")
    out = fused_moe(x.cuda(), logits.cuda(), wg.cuda(), wu.cuda(), wd.cuda(), 2, out=out)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all()), "non-finite values left in the NaN-poisoned output"
    assert_close(out, fused_moe_forward(x, logits, wg, wu, wd, 2), what="absorbed rows E=80, 256-row items")


@pytest.mark.parametrize("bm", [0, 128])
def test_last_blocks_beyond_absorption(bm):
    """Last blocks of 33-64 rows stay items of their own (absorption takes at
    most 32 rows; splitting 33-64 over two item groups measured slower at
    dsv3) next to absorbed and plain experts: 424, 572, 562, 296, 600 and
    others, top-1, the 256-row (bm 0) and 128-row paddings; pre-routed too,
    with NaN-poisoned padding."""
    from muxi_race_amd import fused_moe
    counts = [424, 572, 562, 296, 600, 250, 0, 31, 200]
    x, logits, wg, wu, wd = _inputs(1, 44, counts)
    T = x.shape[0]
    out = torch.full((T, H), float("nan"), dtype=torch.float16, device="cuda")
    out = fused_moe(x.cuda(), logits.cuda(), wg.cuda(), wu.cuda(), wd.cuda(), 1, block_m=bm, out=out)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all()), "non-finite values left in the NaN-poisoned output"
    assert_close(out, fused_moe_forward(x, logits, wg, wu, wd, 1), what=f"last blocks of 33-64 rows bm={bm}")
    if bm == 128:
        from _cases import prerouted_inputs
        from muxi_race_amd import run_kernel
        from oracle import prerouted_forward
        sizes = [424, 572, 296, 3, 0, 562]
        args = list(prerouted_inputs(sizes, 512, 256, seed=45))
        xp, gpo = args[0], args[7].cpu().tolist()
        pad = torch.ones(xp.shape[0], dtype=torch.bool)
        for e, n in enumerate(sizes):
            pad[gpo[e]:gpo[e] + n] = False
        xp[pad.to(xp.device)] = float("nan")
        o = torch.full(xp.shape, float("nan"), dtype=torch.float16, device=xp.device)
        run_kernel(*args, o)
        torch.cuda.synchronize()
        assert_close(o, prerouted_forward(*args), what="prerouted last blocks of 33-64 rows")
        assert (o[pad.to(o.device)] == 0).all()
