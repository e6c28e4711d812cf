"""Committed golden fixtures (tests/golden/*.npz, made by make_golden.py):
the CPU oracle must reproduce them (regression pin), and the GPU path must
match them at the north-star tolerance through the C ABI."""
from pathlib import Path

import numpy as np
import pytest
import torch

from conftest import assert_close
from oracle import fused_moe_forward, prerouted_forward, quantize_rows_int8, route_topk, w8a8_forward

G = Path(__file__).resolve().parent / "golden"


def _load(name):
    return dict(np.load(G / name, allow_pickle=False))


PRE_KEYS = ("x", "w_gate", "w_up", "w_down", "routed", "group_sizes", "group_offsets",
            "group_padded_offsets", "group_idx_for_bx")


def test_oracle_reproduces_prerouted_fixture():
    d = _load("prerouted_small.npz")
    out = prerouted_forward(*(d[k] for k in PRE_KEYS)).float()
    torch.testing.assert_close(out, torch.from_numpy(d["out"]).float(), rtol=1e-3, atol=1e-3)
    pad = np.ones(d["x"].shape[0], bool)
    for e, n in enumerate(d["group_sizes"]):
        pad[d["group_padded_offsets"][e]:d["group_padded_offsets"][e] + n] = False
    assert (d["out"][pad] == 0).all()


def test_oracle_reproduces_fused_fixture():
    d = _load("fused_small.npz")
    k = int(d["top_k"])
    ids, w = route_topk(d["logits"], k, d["bias"])
    np.testing.assert_array_equal(ids, d["ids"])
    np.testing.assert_allclose(w, d["weights"], rtol=1e-6)
    out = fused_moe_forward(torch.from_numpy(d["x"]), torch.from_numpy(d["logits"]),
                            torch.from_numpy(d["w_gate"]), torch.from_numpy(d["w_up"]),
                            torch.from_numpy(d["w_down"]), k, torch.from_numpy(d["bias"]))
    torch.testing.assert_close(out.float(), torch.from_numpy(d["out"]).float(), rtol=1e-3, atol=1e-3)
    qg, sg = quantize_rows_int8(d["w_gate"])
    np.testing.assert_array_equal(qg, d["q_gate"])
    np.testing.assert_array_equal(sg, d["s_gate"])
    qu, su = quantize_rows_int8(d["w_up"])
    qd, sd = quantize_rows_int8(d["w_down"])
    out8 = w8a8_forward(torch.from_numpy(d["x"]), torch.from_numpy(d["logits"]), qg, sg, qu, su, qd, sd,
                        k, torch.from_numpy(d["bias"]))
    torch.testing.assert_close(out8.float(), torch.from_numpy(d["out_w8a8"]).float(), rtol=1e-3, atol=1e-3)


@pytest.mark.gpu
def test_gpu_matches_prerouted_fixture():
    from muxi_race_amd import run_kernel
    d = _load("prerouted_small.npz")
    t = [torch.from_numpy(d[k]).cuda() for k in PRE_KEYS]
    out = torch.full(d["out"].shape, float("nan"), dtype=torch.float16, device="cuda")
    run_kernel(*t, out)
    torch.cuda.synchronize()
    assert_close(out, torch.from_numpy(d["out"]), what="prerouted fixture")


@pytest.mark.gpu
def test_gpu_matches_fused_fixture():
    from muxi_race_amd import fused_moe, quantize_w8a8_weights
    d = _load("fused_small.npz")
    k = int(d["top_k"])
    c = {n: torch.from_numpy(d[n]).cuda() for n in ("x", "logits", "bias", "w_gate", "w_up", "w_down")}
    out, (ids, w) = fused_moe(c["x"], c["logits"], c["w_gate"], c["w_up"], c["w_down"], k,
                              expert_bias=c["bias"], return_routing=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(ids.cpu().numpy(), d["ids"])
    assert_close(out, torch.from_numpy(d["out"]), what="fused fixture")
    qw = quantize_w8a8_weights(c["w_gate"], c["w_up"], c["w_down"])
    np.testing.assert_array_equal(qw.q_gate.cpu().numpy(), d["q_gate"])
    out8 = fused_moe(c["x"], c["logits"], None, None, None, k, expert_bias=c["bias"], w8a8=qw)
    torch.cuda.synchronize()
    assert_close(out8, torch.from_numpy(d["out_w8a8"]), what="w8a8 fixture")


EXT = ("x", "bias", "w_router", "w_gate", "w_up", "w_down", "w_gate_shared", "w_up_shared", "w_down_shared")


def test_oracle_reproduces_extensions_fixture():
    from oracle import fp8_e4m3_codes, quantize_rows_fp8, router_logits  # noqa: F401
    d = _load("extensions_small.npz")
    k = int(d["top_k"])
    t = torch.from_numpy
    lg = router_logits(d["x"], d["w_router"])
    np.testing.assert_allclose(lg, d["logits"], rtol=1e-6, atol=1e-6)
    ids, w = route_topk(d["logits"], k, d["bias"])
    np.testing.assert_array_equal(ids, d["ids"])
    base = (t(d["x"]), t(d["logits"]))
    out = fused_moe_forward(*base, t(d["w_gate"]), t(d["w_up"]), t(d["w_down"]), k, t(d["bias"]))
    torch.testing.assert_close(out.float(), t(d["out_router"]).float(), rtol=1e-3, atol=1e-3)
    sh = (t(d["w_gate_shared"]), t(d["w_up_shared"]), t(d["w_down_shared"]))
    out = fused_moe_forward(*base, t(d["w_gate"]), t(d["w_up"]), t(d["w_down"]), k, t(d["bias"]), shared=sh)
    torch.testing.assert_close(out.float(), t(d["out_shared"]).float(), rtol=1e-3, atol=1e-3)
    out = fused_moe_forward(*base, t(d["w_gate"][2:6]), t(d["w_up"][2:6]), t(d["w_down"][2:6]), k, t(d["bias"]),
                            expert_range=(2, 4))
    torch.testing.assert_close(out.float(), t(d["out_shard"]).float(), rtol=1e-3, atol=1e-3)
    qg, sg = quantize_rows_fp8(d["w_gate"])
    np.testing.assert_array_equal(qg, d["q_gate_fp8"])
    np.testing.assert_array_equal(sg, d["s_gate_fp8"])
    qu, su = quantize_rows_fp8(d["w_up"])
    qd, sd = quantize_rows_fp8(d["w_down"])
    out = w8a8_forward(*base, qg, sg, qu, su, qd, sd, k, t(d["bias"]), fmt="fp8")
    torch.testing.assert_close(out.float(), t(d["out_fp8"]).float(), rtol=1e-3, atol=1e-3)


@pytest.mark.gpu
def test_gpu_matches_extensions_fixture():
    from muxi_race_amd import fused_moe, quantize_w8a8_weights, route_hidden
    d = _load("extensions_small.npz")
    k = int(d["top_k"])
    c = {n: torch.from_numpy(d[n]).cuda() for n in EXT + ("logits",)}
    ids, _, lg = route_hidden(c["x"], c["w_router"], k, c["bias"], return_logits=True)
    torch.cuda.synchronize()
    np.testing.assert_allclose(lg.cpu().numpy(), d["logits"], rtol=1e-4, atol=1e-4)
    np.testing.assert_array_equal(ids.cpu().numpy(), d["ids"])
    w3 = (c["w_gate"], c["w_up"], c["w_down"])
    out = fused_moe(c["x"], None, *w3, k, expert_bias=c["bias"], router_weight=c["w_router"])
    assert_close(out, torch.from_numpy(d["out_router"]), what="router fixture")
    sh = (c["w_gate_shared"], c["w_up_shared"], c["w_down_shared"])
    out = fused_moe(c["x"], c["logits"], *w3, k, expert_bias=c["bias"], shared_expert=sh)
    assert_close(out, torch.from_numpy(d["out_shared"]), what="shared-expert fixture")
    out = fused_moe(c["x"], c["logits"], *(w[2:6] for w in w3), k, expert_bias=c["bias"], expert_range=(2, 4))
    assert_close(out, torch.from_numpy(d["out_shard"]), what="shard fixture")
    qw = quantize_w8a8_weights(*w3, fmt="fp8")
    np.testing.assert_array_equal(qw.q_gate.view(torch.uint8).cpu().numpy(), d["q_gate_fp8"])
    out = fused_moe(c["x"], c["logits"], None, None, None, k, expert_bias=c["bias"], w8a8=qw)
    torch.cuda.synchronize()
    assert_close(out, torch.from_numpy(d["out_fp8"]), what="fp8 fixture")
