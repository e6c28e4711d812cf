"""Host-side workspace cache rules (muxi_race_amd.moe._workspace), on the CPU:
the stream and graph-capture queries are replaced by stand-ins, and the
buffers are CPU tensors."""
import types

import pytest
import torch

from muxi_race_amd import moe


@pytest.fixture
def fake_cuda(monkeypatch):
    state = types.SimpleNamespace(stream=1, capturing=False)
    monkeypatch.setattr(torch.cuda, "current_stream",
                        lambda dev=None: types.SimpleNamespace(cuda_stream=state.stream))
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: state.capturing)
    monkeypatch.setattr(moe, "_WORKSPACE", {})
    monkeypatch.setattr(moe, "_CAPTURED_RETIRED", [])
    return state


def test_reuse_and_growth_per_stream(fake_cuda):
    dev = torch.device("cpu")
    a = moe._workspace(dev, ("fused", None), 1000)
    assert a.numel() >= 1000 and moe._workspace(dev, ("fused", None), 800) is a  # reused
    b = moe._workspace(dev, ("fused", None), 5000)
    assert b is not a and b.numel() >= 5000  # grown
    assert moe._workspace(dev, ("fused", "fp8"), 10) is not b  # another use
    fake_cuda.stream = 2
    assert moe._workspace(dev, ("fused", None), 10) is not b  # another stream
    assert moe._CAPTURED_RETIRED == []  # eager buffers are not kept once replaced


def test_capture_gets_its_own_buffer_and_keeps_replaced_ones(fake_cuda):
    dev = torch.device("cpu")
    eager = moe._workspace(dev, ("fused", None), 1000)
    fake_cuda.capturing = True
    cap = moe._workspace(dev, ("fused", None), 1000)
    assert cap is not eager  # never the eager buffer, though it is large enough
    assert moe._workspace(dev, ("fused", None), 500) is cap  # captures share theirs
    fake_cuda.capturing = False
    grown = moe._workspace(dev, ("fused", None), 100000)  # eager growth leaves the captured one alone
    assert grown is not cap and moe._CAPTURED_RETIRED == []
    fake_cuda.capturing = True
    cap2 = moe._workspace(dev, ("fused", None), 100000)
    assert cap2 is not cap and cap2 is not grown
    assert len(moe._CAPTURED_RETIRED) == 1 and moe._CAPTURED_RETIRED[0] is cap  # kept alive
