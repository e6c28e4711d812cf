"""Size-independent properties at the BASELINE configs' full sizes.

Token-permutation equivariance.  Each output row depends only on its own
token: its routing, its gathered rows multiplied in a fixed K order, and a
fixed choice-order sum.  A permutation of the tokens changes which tokens
share an expert's blocks, which land in paired, single or absorbed rows, and
every row's place in the expert-sorted order.  So permuting the rows of x and
of the logits must permute the output rows, the routing ids and the routing
weights bit for bit, in every config and format.  A gather, padding,
absorbed-row or combine mapping mistake breaks this at sizes the CPU oracle
cannot check whole.  The same holds within one call: tokens that repeat other
tokens must get their rows bit for bit."""
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


@pytest.mark.parametrize("name,fmt", [("mixtral", None), ("dsv3", None), ("w8a8", "int8"), ("w8a8", "fp8")])
def test_identical_tokens_get_identical_rows(name, fmt):
    """A quarter of the tokens repeat other tokens (x row and logits row):
    they are routed alike but sit at other places of the sorted order (other
    blocks, paired / single / absorbed rows), and each copy's output row must
    equal the original's bit for bit, in one call."""
    from muxi_race_amd import fused_moe, quantize_w8a8_weights
    inp = moe_inputs(name, 303)
    T = inp["T"]
    g = torch.Generator().manual_seed(304)
    dst = torch.randperm(T, generator=g)[: T // 4]
    src = torch.randint(0, T, (T // 4,), generator=g)
    keep = ~torch.isin(src, dst)  # a source row is never overwritten
    dst, src = dst[keep].cuda(), src[keep].cuda()
    x, lg = inp["x"].clone(), inp["logits"].clone()
    x[dst] = x[src]
    lg[dst] = lg[src]
    kw = dict(expert_bias=inp["bias"])
    if fmt is None:
        w = (inp["wg"], inp["wu"], inp["wd"])
    else:
        kw["w8a8"] = quantize_w8a8_weights(inp["wg"], inp["wu"], inp["wd"], fmt=fmt)
        w = (None, None, None)
    out = fused_moe(x, lg, *w, inp["k"], **kw)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    diff = (out[dst] != out[src]).any(dim=1)
    assert not diff.any(), f"{name} {fmt or 'fp16'}: {int(diff.sum())} of {dst.numel()} copies differ"
