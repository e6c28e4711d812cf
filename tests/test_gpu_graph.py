"""The fused forward issues no memset and no allocation inside the library, so
a caller can capture it in a HIP graph (torch.cuda.graph).  Each case is
captured once and replayed several times with unrelated eager work and
synchronisations between replays; every replay must equal the eager result
bitwise."""
import pytest
import torch

from _cases import moe_inputs, skewed_8bit_case

pytestmark = pytest.mark.gpu


def _replays_match(fn, n=3):
    eager = fn().clone()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # warm the capture stream's workspace outside the capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    noise = torch.randn(1024, 1024, device="cuda")
    for i in range(n):
        _ = noise @ noise  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i} differs from the eager result"


@pytest.mark.parametrize("name", ["small", "decode"])
def test_fp16_forward_replays(name):
    from muxi_race_amd import fused_moe
    inp = moe_inputs(name, 101)
    _replays_match(lambda: fused_moe(inp["x"], inp["logits"], inp["wg"], inp["wu"], inp["wd"], inp["k"],
                                     expert_bias=inp["bias"]))


def test_256_row_padding_replays():
    """fp16 Stage 1 and fp8 Stage 2 on 256-row items (the 256-row padding)."""
    from muxi_race_amd import fused_moe, quantize_w8a8_weights
    g = torch.Generator().manual_seed(104)
    T, H, I, E, k = 1536, 512, 384, 8, 2  # 384 routed rows per expert
    x, lg = torch.randn(T, H, generator=g).half().cuda(), torch.randn(T, E, generator=g).cuda()
    w = [(torch.randn(shape, generator=g) * 0.05).half().cuda() for shape in ((E, I, H), (E, I, H), (E, H, I))]
    _replays_match(lambda: fused_moe(x, lg, *w, k))
    inp = skewed_8bit_case(105)
    qw = quantize_w8a8_weights(inp["wg"], inp["wu"], inp["wd"], fmt="fp8")
    _replays_match(lambda: fused_moe(inp["x"], inp["logits"], None, None, None, inp["k"],
                                     expert_bias=inp["bias"], w8a8=qw))


@pytest.mark.parametrize("fmt", ["int8", "fp8"])
def test_8bit_forward_replays(fmt):
    from muxi_race_amd import fused_moe, quantize_w8a8_weights
    inp = moe_inputs("small", 102, T=300)
    qw = quantize_w8a8_weights(inp["wg"], inp["wu"], inp["wd"], fmt=fmt)
    _replays_match(lambda: fused_moe(inp["x"], inp["logits"], None, None, None, inp["k"], w8a8=qw))


def test_router_and_shared_expert_replays():
    from muxi_race_amd import fused_moe
    inp = moe_inputs("decode", 103)
    g = torch.Generator(device="cuda").manual_seed(103)
    H, I, E = inp["H"], inp["I"], inp["E"]
    wr = (torch.randn((E, H), generator=g, device="cuda") / H ** 0.5).half()
    sh = [torch.randn(s, generator=g, device="cuda", dtype=torch.float16) * 0.02 for s in ((I, H), (I, H), (H, I))]
    _replays_match(lambda: fused_moe(inp["x"], None, inp["wg"], inp["wu"], inp["wd"], inp["k"],
                                     expert_bias=inp["bias"], router_weight=wr, shared_expert=sh))


def test_capture_on_the_warm_stream_keeps_its_workspace():
    """A graph captured on the stream the caller warmed up on keeps a
    workspace of its own: an eager call on that stream that needs a larger one
    does not free memory the graph's replays still write (tensors allocated
    afterwards keep their values, and every replay still equals eager)."""
    from muxi_race_amd import fused_moe
    small = moe_inputs("small", 106, T=64)
    big = moe_inputs("small", 107, T=2048)

    def f_small():
        return fused_moe(small["x"], small["logits"], small["wg"], small["wu"], small["wd"], small["k"])

    eager = f_small().clone()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        f_small()  # eager warm-up on the capture stream itself
        s.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            out = f_small()
        fused_moe(big["x"], big["logits"], big["wg"], big["wu"], big["wd"], big["k"])  # larger workspace
        s.synchronize()
        fill = [torch.full((32768,), 7.0, device="cuda") for _ in range(64)]  # reuse freed blocks
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for i in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i} differs from the eager result"
        assert all(bool((f == 7.0).all()) for f in fill), f"replay {i} wrote into freed memory"
