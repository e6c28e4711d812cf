"""CPU checks of bench.py's host-side pieces: the CPU baseline times the
oracle's complete fused forward on a token sample and reports it in the
contract's shape; the flag rejecting more than one GPU exits with a message."""
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))


def test_cpu_baseline_shape_and_sample():
    import bench
    inp = bench.make_inputs("small", "cpu")
    res = bench.cpu_baseline(inp, tokens=64)
    assert set(res) >= {"value", "unit", "cores", "kind", "sample", "ms", "ms_full_batch_at_this_rate"}
    assert res["unit"] == "TFLOP/s" and res["kind"] == "port" and res["cores"] >= 1
    assert res["value"] > 0 and res["ms"] > 0
    # half of the batch's tokens -> the full-batch estimate is twice the sample's time
    assert abs(res["ms_full_batch_at_this_rate"] - 2 * res["ms"]) <= 0.2
    assert "tokens [0, 64) of 128" in res["sample"] and "combine" in res["sample"]


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
