"""Size-independent properties at the BASELINE configs' full sizes.

Token-permutation equivariance.  Each output row depends only on its own
token: its routing, its gathered rows multiplied in a fixed K order, and a
fixed choice-order sum.  A permutation of the tokens changes which tokens
share an expert's blocks, which land in paired, single or absorbed rows, and
every row's place in the expert-sorted order.  So permuting the rows of x and
of the logits must permute the output rows, the routing ids and the routing
weights bit for bit, in every config and format.  A gather, padding,
absorbed-row or combine mapping mistake breaks this at sizes the CPU oracle
cannot check whole."""
import pytest
import torch

from _cases import moe_inputs

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name,fmt", [("small", None), ("decode", None), ("mixtral", None), ("dsv3", None),
                                      ("w8a8", "int8"), ("w8a8", "fp8")])
def test_token_permutation_equivariance(name, fmt):
    from muxi_race_amd import fused_moe, quantize_w8a8_weights
    inp = moe_inputs(name, 301)
    perm = torch.randperm(inp["T"], generator=torch.Generator().manual_seed(302)).cuda()
    kw = dict(expert_bias=inp["bias"], return_routing=True)
    if fmt is None:
        w = (inp["wg"], inp["wu"], inp["wd"])
    else:
        kw["w8a8"] = quantize_w8a8_weights(inp["wg"], inp["wu"], inp["wd"], fmt=fmt)
        w = (None, None, None)
    out, (ids, wts) = fused_moe(inp["x"], inp["logits"], *w, inp["k"], **kw)
    outp, (idsp, wtsp) = fused_moe(inp["x"][perm].contiguous(), inp["logits"][perm].contiguous(), *w,
                                   inp["k"], **kw)
    torch.cuda.synchronize()
    assert torch.equal(ids[perm], idsp) and torch.equal(wts[perm], wtsp), "routing not per-token"
    assert torch.isfinite(out).all()
    diff = (out[perm] != outp).any(dim=1)
    assert not diff.any(), f"{name} {fmt or 'fp16'}: {int(diff.sum())} of {inp['T']} rows differ after permutation"
