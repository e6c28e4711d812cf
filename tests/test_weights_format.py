"""On-disk W8A8 format: save -> load round trip is bit-identical (codes and
scales, int8 and fp8), and the loader rejects foreign or inconsistent files.
CPU only: the oracle's quantisers produce the same codes as the GPU's (pinned
bit-exact in the GPU quantiser tests)."""
import numpy as np
import pytest
import torch

from oracle import quantize_rows_fp8, quantize_rows_int8


def _weights(fmt, E=3, H=256, I=128):
    from muxi_race_amd import W8A8Weights
    g = torch.Generator().manual_seed(5)
    ws = [(torch.randn(s, generator=g) * 0.02).half() for s in ((E, I, H), (E, I, H), (E, H, I))]
    quant = quantize_rows_int8 if fmt == "int8" else quantize_rows_fp8
    parts = []
    for w in ws:
        q, s = quant(w)
        q = torch.from_numpy(q)
        parts += [q if fmt == "int8" else q.view(torch.float8_e4m3fn), torch.from_numpy(s)]
    return W8A8Weights(*parts)


@pytest.mark.parametrize("fmt", ["int8", "fp8"])
def test_round_trip_is_bit_identical(tmp_path, fmt):
    from muxi_race_amd import load_w8a8, save_w8a8
    w = _weights(fmt)
    path = str(tmp_path / f"layer.{fmt}.safetensors")
    save_w8a8(path, w)
    r = load_w8a8(path, device="cpu")
    assert r.fmt == fmt
    for n in ("q_gate", "s_gate", "q_up", "s_up", "q_down", "s_down"):
        a, b = getattr(w, n), getattr(r, n)
        assert a.dtype == b.dtype and a.shape == b.shape
        assert torch.equal(a.view(torch.uint8) if a.dtype == torch.float8_e4m3fn else a,
                           b.view(torch.uint8) if b.dtype == torch.float8_e4m3fn else b), n


def test_loader_rejects_foreign_and_inconsistent_files(tmp_path):
    from safetensors.torch import save_file
    from muxi_race_amd import load_w8a8, save_w8a8
    p = str(tmp_path / "x.safetensors")
    save_file({"a": torch.zeros(2)}, p, metadata={"format": "other"})
    with pytest.raises(ValueError, match="not a"):
        load_w8a8(p, device="cpu")
    w = _weights("int8")
    save_w8a8(p, w)
    # same tag, wrong shape of one tensor
    t = {n: getattr(w, n) for n in ("q_gate", "s_gate", "q_up", "s_up", "q_down", "s_down")}
    t["s_up"] = t["s_up"][:, :-1].contiguous()
    meta = {"format": "muxi_race_amd.w8a8", "version": "1", "fmt": "int8", "experts": "3", "hidden": "256",
            "intermediate": "128"}
    save_file(t, p, metadata=meta)
    with pytest.raises(ValueError, match="s_up"):
        load_w8a8(p, device="cpu")
    # int8 tag over fp8 codes
    w8 = _weights("fp8")
    save_file({n: getattr(w8, n) for n in t}, p, metadata=meta)
    with pytest.raises(ValueError, match="q_gate"):
        load_w8a8(p, device="cpu")
    # mismatched code dtypes are refused at save time
    bad = _weights("int8")
    bad.q_up = w8.q_up
    with pytest.raises(ValueError, match="q_up"):
        save_w8a8(p, bad)
