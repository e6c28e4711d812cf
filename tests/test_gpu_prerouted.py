"""GPU parity of the drop-in run_kernel (pre-routed fused expert MLP) against
the CPU oracle (problem_detail.json:50), on the reference harness's shapes
(remote_bench.py:21-29), the tail list (OPTIMIZATION_LOG.md:63), random splits
(race_stress2.py:114-133), NaN poisoning and repeat determinism."""
import pytest
import torch

from _cases import RB_CASES, TAIL_SIZES, prerouted_inputs, random_group_sizes, rb_group_sizes
from conftest import assert_close
from oracle import metadata_from_group_sizes, prerouted_forward

pytestmark = pytest.mark.gpu


def _run(args, fill=float("nan")):
    from muxi_race_amd import run_kernel
    x = args[0]
    out = torch.full(x.shape, fill, dtype=torch.float16, device=x.device)
    run_kernel(*args, out)
    torch.cuda.synchronize()
    return out


def _check(args, what):
    out = _run(args)
    ref = prerouted_forward(*args)
    assert_close(out, ref, what=what)
    return out


@pytest.mark.parametrize("case", [0, 5, 6, 4, 1, 2, 3])
def test_rb_cases(case):
    cfg = RB_CASES[case]
    sizes = rb_group_sizes(cfg)
    args = prerouted_inputs(sizes, cfg["hidden"], cfg["intermediate"], seed=20260901 + case)
    _check(args, f"rb case {case}")


def test_tail_sizes():
    args = prerouted_inputs(TAIL_SIZES, 1024, 512, seed=63)
    _check(args, "tail sizes")


@pytest.mark.parametrize("seed", range(6))
def test_random_splits(seed):
    sizes = random_group_sizes(32, 4544, 999000 + seed * 17)
    args = prerouted_inputs(sizes, 512, 256, seed=555000 + seed * 19, init="ns")
    _check(args, f"split seed {seed}")


def test_routed_fp16():
    args = prerouted_inputs([100, 0, 260, 5], 256, 384, seed=4, routed_dtype=torch.float16)
    _check(args, "routed fp16")


def test_nan_poisoned_padding_output_and_workspace():
    """Padding rows of x are NaN, `out` and the cached workspace start as NaN;
    padding rows must come back exactly 0 and everything finite
    (OPTIMIZATION_LOG.md:2193-2198: select, never multiply by 0)."""
    from muxi_race_amd import moe as moe_mod
    sizes = [3, 0, 129, 127, 1]
    args = list(prerouted_inputs(sizes, 256, 256, seed=9))
    x, gs, gpo = args[0], sizes, args[7].cpu().tolist()
    pad = torch.ones(x.shape[0], dtype=torch.bool)
    for e, n in enumerate(gs):
        pad[gpo[e]:gpo[e] + n] = False
    x[pad.to(x.device)] = float("nan")
    _run(args)  # populate the workspace cache
    for buf in moe_mod._WORKSPACE.values():
        buf.fill_(0xFF)  # 0xFFFF is an fp16 NaN
    ref = prerouted_forward(*args)
    for _ in range(3):
        out = _run(args)
        assert_close(out, ref, what="nan poisoned")
        assert (out[pad.to(out.device)] == 0).all()


def test_repeat_is_bitwise_deterministic():
    args = prerouted_inputs([200, 77, 0, 300], 512, 512, seed=12)
    a = _run(args)
    for _ in range(5):
        b = _run(args)
        assert torch.equal(a, b)


def test_all_padding_rows_are_zero():
    """group_sizes all 0 with P = 128 padded rows: out is written as all zeros
    (the reference's zero-output path, submission.py:2130-2153)."""
    dev = "cuda"
    E, H, I = 2, 256, 128
    x = torch.randn(128, H, device=dev).half()
    w = torch.randn(E, I, H, device=dev).half()
    wd = torch.randn(E, H, I, device=dev).half()
    routed = torch.zeros(0, device=dev)
    gs = torch.zeros(E, dtype=torch.int32, device=dev)
    go = torch.zeros(E + 1, dtype=torch.int32, device=dev)
    gpo = torch.zeros(E + 1, dtype=torch.int32, device=dev)
    gidx = torch.zeros(1, dtype=torch.int32, device=dev)
    out = _run((x, w, w, wd, routed, gs, go, gpo, gidx))
    assert (out == 0).all()


def test_empty_problem_is_a_no_op():
    from muxi_race_amd import run_kernel
    dev = "cuda"
    E, H, I = 2, 256, 128
    x = torch.empty(0, H, device=dev, dtype=torch.float16)
    w = torch.zeros(E, I, H, device=dev, dtype=torch.float16)
    wd = torch.zeros(E, H, I, device=dev, dtype=torch.float16)
    z = torch.zeros(E + 1, dtype=torch.int32, device=dev)
    out = torch.empty(0, H, device=dev, dtype=torch.float16)
    run_kernel(x, w, w, wd, torch.zeros(0, device=dev), z[:E], z, z, z[:0], out)
    torch.cuda.synchronize()


def test_rejects_bad_metadata_dtype():
    """int64 metadata segfaulted the reference (OPTIMIZATION_LOG.md:2174-2176);
    here it is a TypeError before any launch."""
    from muxi_race_amd import run_kernel
    args = list(prerouted_inputs([5], 128, 128, seed=1))
    args[5] = args[5].long()
    with pytest.raises(TypeError):
        run_kernel(*args, torch.empty_like(args[0]))


def _meta_tensors(sizes, go, gpo, gidx, dev="cuda"):
    return [torch.tensor(list(a), dtype=torch.int32, device=dev) for a in (sizes, go, gpo, gidx)]


def _block_case(sizes, go, gpo, gidx, P, H, I, seed, V=None):
    g = torch.Generator().manual_seed(seed)
    E = len(sizes)
    x = torch.randn(P, H, generator=g).half().cuda()
    ws = [(torch.randn(shape, generator=g) * 0.05).half().cuda() for shape in ((E, I, H), (E, I, H), (E, H, I))]
    routed = torch.rand(int(go[-1]) if V is None else V, generator=g).cuda()
    return [x, *ws, routed, *_meta_tensors(sizes, go, gpo, gidx)]


@pytest.mark.parametrize("name,sizes,go,gpo,gidx,P", [
    # two trailing blocks past gpo[E] naming the last expert: their rows are 0
    ("trailing", [3, 300], [0, 3, 303], [0, 128, 512], [0, 1, 1, 1, 1, 1], 6 * 128),
    # gidx one block shorter than P: the last block is left untouched
    ("short", [3, 300], [0, 3, 303], [0, 128, 512], [0, 1, 1, 1], 5 * 128),
    # swapped experts: block 0 runs expert 1 at token offset -128
    ("swapped", [128, 128], [0, 128, 256], [0, 128, 256], [1, 0], 256),
    # non-monotone runs (pairs form inside each run) and an out-of-range value
    ("runs", [256, 384, 100], [0, 256, 640, 740], [0, 256, 640, 768],
     [0, 0, 1, 1, 1, 2, 0, 0, 9], 9 * 128),
])
def test_group_idx_for_bx_maps_blocks(name, sizes, go, gpo, gidx, P):
    """Block b runs expert group_idx_for_bx[b] over min(nblk, P / 128) blocks
    (problem_detail.json:50 note 5; submission.py:1444, :2115), against the
    oracle's per-block form; rows past the launched blocks keep their NaN."""
    from oracle import prerouted_forward_blocks
    args = _block_case(sizes, go, gpo, gidx, P, 256, 384, seed=len(name))
    out = _run(args)
    nan_init = torch.full((P, 256), float("nan"), dtype=torch.float16)
    ref = prerouted_forward_blocks(*[a.cpu() for a in args], out=nan_init)
    launched = min(len(gidx), P // 128) * 128
    assert_close(out[:launched], ref[:launched], what=f"gidx {name}")
    assert torch.isnan(out[launched:].float()).all()
    if name == "trailing":
        assert (out[512:] == 0).all()


def test_group_idx_for_bx_equals_expert_loop_on_harness_metadata():
    """On remote_bench.py:82-101 metadata the per-block map is the expert loop:
    the two oracles agree and the GPU matches both (multi-block experts pair)."""
    from oracle import prerouted_forward_blocks
    sizes = [0, 700, 1, 128, 129, 255]
    args = prerouted_inputs(sizes, 512, 256, seed=31, init="ns")
    out = _run(args)
    ref = prerouted_forward(*args)
    assert torch.equal(ref, prerouted_forward_blocks(*[a.cpu() for a in args]))
    assert_close(out, ref, what="harness metadata")
