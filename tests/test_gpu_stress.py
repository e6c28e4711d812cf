"""Repeat and split stress of the HIP path, after the reference's race stress
(xpuoj_data/race_stress2.py:98-133): many back-to-back calls at full size,
each output compared bitwise with the first, stopping at the first mismatch;
and run_kernel over 40 random group splits x 3 repetitions at the harness's
case-2 shape, every repetition checked against an fp32 reference.

The kernels' LDS rings rely on s_waitcnt counts, fence-less barriers and the
in-order retirement of direct-to-LDS loads; a race there would show up as an
intermittent bit difference between repeats, which these loops look for."""
import os

import numpy as np
import pytest
import torch

from _cases import RB_CASES, moe_inputs, prerouted_inputs, random_group_sizes, rb_group_sizes, stratified_tokens
from _torch_ref import prerouted_reference
from conftest import ATOL_F16, RTOL_F16, assert_close
from oracle import metadata_from_group_sizes, prerouted_forward

pytestmark = pytest.mark.gpu
# race_stress2.py's Phase A runs 2000 calls; MOE_STRESS_REPEATS=2000 does the same
REPEATS = int(os.environ.get("MOE_STRESS_REPEATS", "200"))  # calls per repeat test
BATCH = 8  # calls enqueued back to back between comparisons


def _close_on_device(got, ref, what):
    """The fp16 gate |d| <= atol + rtol |ref| (non-finite fails), evaluated on
    the device; the CPU assert_close reports the first failure."""
    g = got.float()
    ok = torch.isfinite(g) & ((g - ref).abs() <= ATOL_F16 + RTOL_F16 * ref.abs())
    if not bool(ok.all()):
        assert_close(got, ref, what=what)


def _repeat_bitwise(call, first, what):
    """REPEATS calls in batches of BATCH distinct outputs, each equal to `first`."""
    outs = [torch.empty_like(first) for _ in range(BATCH)]
    done = 0
    while done < REPEATS:
        n = min(BATCH, REPEATS - done)
        for i in range(n):
            call(outs[i])
        torch.cuda.synchronize()
        for i in range(n):
            if not torch.equal(outs[i], first):
                d = (outs[i].float() - first.float()).abs()
                bad = int((d != 0).sum() + (torch.isnan(outs[i]) != torch.isnan(first)).sum())
                raise AssertionError(f"{what}: call {done + i} differs from the first in {bad} elements, "
                                     f"max|d|={float(d.nan_to_num().max()):.4g}")
        done += n
    print(f"{what}: {REPEATS} calls bitwise equal", flush=True)


@pytest.mark.parametrize("name", ["dsv3", "mixtral"])
def test_fused_repeat_bitwise(name):
    """REPEATS back-to-back fused forwards at a full BASELINE config equal the
    first bitwise (which is itself checked against the oracle on a stratified
    token set)."""
    from muxi_race_amd import fused_moe
    from oracle import fused_moe_forward, route_topk
    inp = moe_inputs(name, 500 + len(name))
    args = (inp["x"], inp["logits"], inp["wg"], inp["wu"], inp["wd"], inp["k"])
    first = fused_moe(*args, expert_bias=inp["bias"])
    torch.cuda.synchronize()
    bias = None if inp["bias"] is None else inp["bias"].cpu()
    rid, _ = route_topk(inp["logits"].cpu().numpy(), inp["k"], None if bias is None else bias.numpy())
    rows = torch.from_numpy(stratified_tokens(rid, seed=1, max_block_starts=64, extra=8)).cuda()
    ref = fused_moe_forward(inp["x"][rows].cpu(), inp["logits"][rows].cpu(), inp["wg"], inp["wu"], inp["wd"],
                            inp["k"], bias)
    assert_close(first[rows], ref, what=f"{name} first call")
    _repeat_bitwise(lambda o: fused_moe(*args, expert_bias=inp["bias"], out=o), first, name)


def test_run_kernel_repeat_bitwise():
    """REPEATS back-to-back run_kernel calls at the harness's case 3 (E64 H7168
    I2048, 9088 rows) equal the first bitwise; the first matches the fp32
    reference in every element."""
    from muxi_race_amd import run_kernel
    cfg = RB_CASES[3]
    args = prerouted_inputs(rb_group_sizes(cfg), cfg["hidden"], cfg["intermediate"], seed=20260904)
    first = torch.full(args[0].shape, float("nan"), dtype=torch.float16, device="cuda")
    run_kernel(*args, first)
    torch.cuda.synchronize()
    ref = prerouted_reference(*args[:8])
    _close_on_device(first, ref, "case 3 first call")
    _repeat_bitwise(lambda o: run_kernel(*args, o), first, "run_kernel case 3")


def test_torch_reference_matches_oracle():
    """The device fp32 reference used below agrees with the CPU oracle."""
    sizes = random_group_sizes(8, 900, 77)
    args = prerouted_inputs(sizes, 512, 256, seed=78, init="ns")
    a = prerouted_reference(*args[:8]).cpu()
    b = prerouted_forward(*args, out_fp32=True)
    torch.testing.assert_close(a, b, rtol=1e-4, atol=1e-5)


def test_run_kernel_random_splits():
    """race_stress2.py Phase B: 40 random splits of the case-2 rows over 32
    experts (sizes uniform in [0, min(remaining, 400)], :15-26), fresh seeded
    inputs per split (weights N(0, 0.02), routed weights fp16, :63-80), three
    repetitions each, every one within the fp16 gate of the fp32 reference
    and bitwise equal to the first.  Stops at the first failing split."""
    from muxi_race_amd import run_kernel
    cfg = RB_CASES[2]
    E, H, I, valid = cfg["experts"], cfg["hidden"], cfg["intermediate"], cfg["valid"]
    for s in range(40):
        sizes = random_group_sizes(E, valid, 999000 + s * 17)
        go, gpo, gidx = metadata_from_group_sizes(sizes, 128)
        P = int(gpo[-1])
        g = torch.Generator(device="cuda").manual_seed(555000 + s * 19 + 2)
        mk = lambda shape, sc: torch.randn(shape, generator=g, device="cuda", dtype=torch.float16) * sc
        x = mk((P, H), 1.0)
        wg, wu, wd = mk((E, I, H), 0.02), mk((E, I, H), 0.02), mk((E, H, I), 0.02)
        routed = torch.rand((int(go[-1]),), generator=g, device="cuda").half()
        meta = [torch.tensor(np.asarray(a, np.int32), device="cuda") for a in (sizes, go, gpo, gidx)]
        ref = prerouted_reference(x, wg, wu, wd, routed, *meta[:3])
        first = None
        for r in range(3):
            out = torch.full((P, H), float("nan"), dtype=torch.float16, device="cuda")
            run_kernel(x, wg, wu, wd, routed, *meta, out)
            torch.cuda.synchronize()
            _close_on_device(out, ref, f"split {s} rep {r} sizes {sizes}")
            if first is None:
                first = out
            else:
                assert torch.equal(out, first), f"split {s} rep {r} differs from rep 0"
    print("40 splits x 3 repetitions within the fp16 gate", flush=True)
