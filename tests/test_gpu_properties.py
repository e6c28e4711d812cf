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
tokens must get their rows bit for bit.  And for the reference operator
(run_kernel), rows permuted inside each expert's group; and through the router
GEMM, the shared expert and an expert-parallel shard."""
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


@pytest.mark.parametrize("case", [1, 2, 3])
def test_run_kernel_row_permutation_equivariance(case):
    """The reference operator (run_kernel) on its published cases: permuting
    the valid rows inside each expert's group, with their raw-order routing
    weights, permutes the output rows bit for bit (padding rows stay 0)."""
    from _cases import RB_CASES, prerouted_inputs, rb_group_sizes
    from muxi_race_amd import run_kernel
    cfg = RB_CASES[case]
    sizes = rb_group_sizes(cfg)
    x, wg, wu, wd, routed, gs, go, gpo, gidx = prerouted_inputs(sizes, cfg["hidden"], cfg["intermediate"],
                                                                seed=305 + case)
    P = x.shape[0]
    g = torch.Generator().manual_seed(306 + case)
    rp = torch.arange(P)                     # padded row -> source padded row
    vp = torch.arange(routed.numel())        # raw index -> source raw index
    for e, n in enumerate(sizes):
        s = torch.randperm(n, generator=g)
        p0, v0 = int(gpo[e]), int(go[e])
        rp[p0:p0 + n] = p0 + s
        vp[v0:v0 + n] = v0 + s
    rp, vp = rp.cuda(), vp.cuda()
    outs = []
    for xx, rr in ((x, routed), (x[rp].contiguous(), routed[vp].contiguous())):
        out = torch.full_like(x, float("nan"))
        run_kernel(xx, wg, wu, wd, rr, gs, go, gpo, gidx, out)
        outs.append(out)
    torch.cuda.synchronize()
    assert torch.isfinite(outs[0]).all()
    diff = (outs[0][rp] != outs[1]).any(dim=1)
    assert not diff.any(), f"case {case}: {int(diff.sum())} of {P} rows differ after permutation"


@pytest.mark.parametrize("name,mode", [("dsv3", "router"), ("decode", "router"), ("dsv3", "shared"),
                                       ("mixtral", "shared"), ("dsv3", "shard")])
def test_permutation_equivariance_other_entries(name, mode):
    """The same token-permutation property through the router GEMM (logits
    computed in the call from x and a router weight), with the always-on
    shared expert, and for one expert-parallel shard (experts 32-63 of 256)."""
    from muxi_race_amd import fused_moe
    inp = moe_inputs(name, 307)
    T, E, H, I = inp["T"], inp["E"], inp["H"], inp["I"]
    perm = torch.randperm(T, generator=torch.Generator().manual_seed(308)).cuda()
    g = torch.Generator(device="cuda").manual_seed(309)
    w = (inp["wg"], inp["wu"], inp["wd"])
    kw = dict(expert_bias=inp["bias"], return_routing=True)
    if mode == "router":
        kw["router_weight"] = (torch.randn((E, H), generator=g, device="cuda") / H ** 0.5).half()
    elif mode == "shared":
        kw["shared_expert"] = tuple(torch.randn(s, generator=g, device="cuda", dtype=torch.float16) * 0.02
                                    for s in ((I, H), (I, H), (H, I)))
    else:
        b, n = 32, 32
        w = tuple(t[b:b + n] for t in w)
        kw["expert_range"] = (b, n)

    def run(x, lg):
        return fused_moe(x, None if mode == "router" else lg, *w, inp["k"], **kw)

    out, (ids, wts) = run(inp["x"], inp["logits"])
    outp, (idsp, wtsp) = run(inp["x"][perm].contiguous(), inp["logits"][perm].contiguous())
    torch.cuda.synchronize()
    assert torch.equal(ids[perm], idsp) and torch.equal(wts[perm], wtsp), "routing not per-token"
    assert torch.isfinite(out).all()
    diff = (out[perm] != outp).any(dim=1)
    assert not diff.any(), f"{name} {mode}: {int(diff.sum())} of {T} rows differ after permutation"
