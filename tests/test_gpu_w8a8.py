"""GPU W8A8: quantiser bit-exact against the oracle; fused W8A8 elementwise
against the W8A8 oracle (same quantised arithmetic) and within the north-star
gate (relative L2 <= 5e-2) against the fp16 oracle.

Elementwise against the fp16 oracle the W8A8 path is reported, not gated at
100%: per-row weight int8 and per-token int8 of both activations (x and the
SiLU*up intermediate) at H = 7168, I = 2048 leave ~3% relative L2, and about
a fifth of the elements fall outside |d| <= 1e-2 + 5e-2 |ref| (a property of
the quantisation scheme, the same for the oracle's own W8A8 arithmetic: 0.76
inside on a T = 128, E = 8 slice of these dimensions).  The fraction inside
is printed and held above 0.80: the lowest case, the w8a8 config's whole
output (2048 tokens), measures 0.818.  Full-size outputs are NaN-poisoned and
must come back finite; the w8a8 config's whole output is compared."""
import numpy as np
import pytest
import torch

from _cases import moe_inputs, scale_contrast_case, skewed_8bit_case, stratified_tokens
from conftest import assert_close
from oracle import fused_moe_forward, quantize_rows_int8, route_topk, w8a8_forward

pytestmark = pytest.mark.gpu
W8A8_REL_L2 = 5e-2
W8A8_ELEMENTWISE_FLOOR = 0.80  # fraction within 1e-2 + 5e-2 |ref| of the fp16 oracle (measured >= 0.818)


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
    T = inp["T"]
    out = torch.full((T, inp["H"]), float("nan"), dtype=torch.float16, device="cuda")
    out = fused_moe(inp["x"], inp["logits"], None, None, None, inp["k"], expert_bias=inp["bias"], w8a8=qw,
                    block_m=block_m, out=out)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all()), "non-finite values left in the NaN-poisoned output"
    bias = None if inp["bias"] is None else inp["bias"].cpu()
    if sample is None:
        rows = torch.arange(T)
    else:
        rid, _ = route_topk(inp["logits"].cpu().numpy(), inp["k"], None if bias is None else bias.numpy())
        rows = torch.from_numpy(stratified_tokens(rid, seed=T))
    r = rows.cuda()
    x, lg = inp["x"][r].cpu(), inp["logits"][r].cpu()
    ref8 = w8a8_forward(x, lg, qw.q_gate.cpu().numpy(), qw.s_gate.cpu().numpy(), qw.q_up.cpu().numpy(),
                        qw.s_up.cpu().numpy(), qw.q_down.cpu().numpy(), qw.s_down.cpu().numpy(),
                        inp["k"], bias)
    ref16 = fused_moe_forward(x, lg, inp["wg"], inp["wu"], inp["wd"], inp["k"], bias).float()
    got = out[r].float().cpu()
    assert_close(got, ref8, what="w8a8 vs w8a8 oracle")
    rel = float((got - ref16).norm() / ref16.norm())
    inside = float(((got - ref16).abs() <= 1e-2 + 5e-2 * ref16.abs()).float().mean())
    print(f"w8a8 vs fp16 oracle on {len(rows)} tokens: rel L2 {rel:.4f}, "
          f"{inside:.4f} of elements within 1e-2 + 5e-2|ref|", flush=True)
    assert rel < W8A8_REL_L2, f"relative L2 vs fp16 oracle {rel:.4f}"
    assert inside >= W8A8_ELEMENTWISE_FLOOR, f"only {inside:.4f} of elements within 1e-2 + 5e-2|ref|"
    return rel


@pytest.mark.parametrize("bm", [0, 32, 128])
def test_w8a8_small(bm):
    _run(moe_inputs("small", 21), block_m=bm)


@pytest.mark.parametrize("bm", [0, 128])
def test_w8a8_skewed_ragged(bm):
    """An empty expert, partial and multi-block experts, over the library's
    256-row padding (both stages on 256-row items) and over 128-row blocks
    (Stage 1 pairs the blocks of multi-block experts, Stage 2 too)."""
    _run(skewed_8bit_case(22), block_m=bm)


def test_w8a8_config_full():
    _run(moe_inputs("w8a8", 22))


@pytest.mark.parametrize("fmt", ["int8", "fp8"])
def test_intermediate_scale_blocks(fmt):
    """I = 256 with h's second 128-column block ~1000x its first (the oracle's
    scale-contrast case), against the 8-bit oracle elementwise.  int8 takes
    one scale per row: the small block's codes are 0 and out[:, 0] (which
    reads only that block) is exactly 0.  fp8 takes per-(row, 128-column)
    scales and keeps the small block."""
    from muxi_race_amd import fused_moe, quantize_w8a8_weights
    from oracle import quantize_rows_fp8
    qfn = quantize_rows_int8 if fmt == "int8" else quantize_rows_fp8
    x, lg, wg, wu, wd, ref, _, k = scale_contrast_case(qfn)
    qw = quantize_w8a8_weights(wg.cuda(), wu.cuda(), wd.cuda(), fmt=fmt)
    out = fused_moe(x.cuda(), lg.cuda(), None, None, None, k, w8a8=qw).float().cpu()
    torch.cuda.synchronize()
    codes = lambda t: (t.view(torch.uint8) if fmt == "fp8" else t).cpu().numpy()
    ref8 = w8a8_forward(x, lg, codes(qw.q_gate), qw.s_gate.cpu().numpy(), codes(qw.q_up), qw.s_up.cpu().numpy(),
                        codes(qw.q_down), qw.s_down.cpu().numpy(), k, fmt=fmt).float()
    assert_close(out, ref8, what=f"{fmt} scale contrast vs oracle")
    if fmt == "int8":
        assert float(out[:, 0].abs().max()) == 0.0
    else:
        rel0 = float((out[:, 0] - ref[:, 0]).norm() / ref[:, 0].norm())
        assert rel0 < 8e-2, rel0


def test_int8_invariant_under_intermediate_permutation():
    """int32 accumulation over the whole of K and one intermediate scale per
    row: permuting the I columns (gate/up rows and w_down columns alike, across
    128-column blocks) leaves the int8 output bit-identical."""
    from muxi_race_amd import fused_moe, quantize_w8a8_weights
    inp = moe_inputs("small", 23)
    I = inp["I"]
    perm = torch.randperm(I, generator=torch.Generator().manual_seed(23)).cuda()
    outs = []
    for p in (None, perm):
        wg, wu, wd = inp["wg"], inp["wu"], inp["wd"]
        if p is not None:
            wg, wu, wd = wg[:, p].contiguous(), wu[:, p].contiguous(), wd[:, :, p].contiguous()
        qw = quantize_w8a8_weights(wg, wu, wd)
        outs.append(fused_moe(inp["x"], inp["logits"], None, None, None, inp["k"], expert_bias=inp["bias"], w8a8=qw))
    torch.cuda.synchronize()
    assert bool(torch.isfinite(outs[0]).all()) and torch.equal(outs[0], outs[1])
