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
