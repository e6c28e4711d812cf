"""Weights quantised on the GPU, saved, and loaded back onto the GPU run
bitwise like the freshly quantised ones (int8 and fp8)."""
import pytest
import torch

from _cases import moe_inputs

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("fmt", ["int8", "fp8"])
def test_saved_weights_run_identically(tmp_path, fmt):
    from muxi_race_amd import fused_moe, load_w8a8, quantize_w8a8_weights, save_w8a8
    inp = moe_inputs("small", 81, T=200)
    qw = quantize_w8a8_weights(inp["wg"], inp["wu"], inp["wd"], fmt=fmt)
    path = str(tmp_path / "layer.safetensors")
    save_w8a8(path, qw)
    lw = load_w8a8(path, device="cuda")
    a = fused_moe(inp["x"], inp["logits"], None, None, None, inp["k"], w8a8=qw)
    b = fused_moe(inp["x"], inp["logits"], None, None, None, inp["k"], w8a8=lw)
    torch.cuda.synchronize()
    assert lw.fmt == fmt and torch.equal(a, b)
