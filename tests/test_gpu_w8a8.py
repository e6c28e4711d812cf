"""GPU W8A8: quantiser bit-exact against the oracle; fused W8A8 elementwise
against the W8A8 oracle (same quantised arithmetic) and within the north-star
gate (relative L2 <= 5e-2) against the fp16 oracle."""
import numpy as np
import pytest
import torch

from _cases import moe_inputs, skewed_8bit_case
from conftest import assert_close
from oracle import fused_moe_forward, quantize_rows_int8, w8a8_forward

pytestmark = pytest.mark.gpu
W8A8_REL_L2 = 5e-2


@pytest.mark.parametrize("K", [1024, 2048 + 8, 7168, 8200])  # register path (4, 8, 16 chunks) and two-pass
def test_quantize_rows_bit_exact(K):
    from muxi_race_amd import quantize_rows_w8
    g = torch.Generator().manual_seed(K)
    w = (torch.randn(300, K, generator=g) * 0.02).half()
    w[0] = 0.0
    w[1, :4] = torch.tensor([127.0, 2.5, -2.5, 0.5]).half()
    w[1, 4:] = 0.0
    q, s = quantize_rows_w8(w.cuda())
    torch.cuda.synchronize()
    rq, rs = quantize_rows_int8(w)
    np.testing.assert_array_equal(q.cpu().numpy(), rq)
    np.testing.assert_array_equal(s.cpu().numpy(), rs)
    np.testing.assert_array_equal(q[1, :4].cpu().numpy(), [127, 3, -3, 1])


def _run(inp, sample=None, block_m=0):
    from muxi_race_amd import fused_moe, quantize_w8a8_weights
    qw = quantize_w8a8_weights(inp["wg"], inp["wu"], inp["wd"])
    out = fused_moe(inp["x"], inp["logits"], None, None, None, inp["k"], expert_bias=inp["bias"], w8a8=qw,
                    block_m=block_m)
    torch.cuda.synchronize()
    T = inp["T"]
    rows = torch.arange(T) if sample is None else torch.from_numpy(
        np.sort(np.random.default_rng(T).choice(T, sample, replace=False)))
    r = rows.cuda()
    x, lg = inp["x"][r].cpu(), inp["logits"][r].cpu()
    bias = None if inp["bias"] is None else inp["bias"].cpu()
    ref8 = w8a8_forward(x, lg, qw.q_gate.cpu().numpy(), qw.s_gate.cpu().numpy(), qw.q_up.cpu().numpy(),
                        qw.s_up.cpu().numpy(), qw.q_down.cpu().numpy(), qw.s_down.cpu().numpy(),
                        inp["k"], bias)
    ref16 = fused_moe_forward(x, lg, inp["wg"], inp["wu"], inp["wd"], inp["k"], bias)
    got = out[r].float().cpu()
    assert_close(got, ref8, what="w8a8 vs w8a8 oracle")
    rel = float((got - ref16.float()).norm() / ref16.float().norm())
    assert rel < W8A8_REL_L2, f"relative L2 vs fp16 oracle {rel:.4f}"
    return rel


@pytest.mark.parametrize("bm", [0, 32, 128])
def test_w8a8_small(bm):
    _run(moe_inputs("small", 21), block_m=bm)


def test_w8a8_skewed_ragged():
    """int8 over the 256-row padding (Stage 1 on 256-row items, Stage 2 on
    128-row ones): an empty expert, partial and multi-block experts."""
    _run(skewed_8bit_case(22))


def test_w8a8_config_sampled():
    _run(moe_inputs("w8a8", 22), sample=16)
