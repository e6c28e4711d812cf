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
