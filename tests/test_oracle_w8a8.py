"""Pins the W8A8 oracle: hand-made quantisation known answers (rounding
convention of submission_v321_int8_fixed.py:184-198), exact integer GEMM, and
the north-star gate against the fp16 oracle."""
import numpy as np
import torch

from _cases import scale_contrast_case
from oracle import fused_moe_forward, quantize_rows_int8, w8a8_forward
from oracle.moe_ref import _int_matmul

W8A8_REL_L2 = 5e-2  # north-star W8A8 gate, applied to the relative L2 error


def test_quantize_known_answers():
    w = np.array([[0.5, -1.0, 0.25, 0.0],
                  [0.0, 0.0, 0.0, 0.0],
                  [127.0, 2.5, -2.5, 0.5]], dtype=np.float32)
    q, s = quantize_rows_int8(w)
    # row 0: amax 1 -> inv 127: 63.5 -> 64, -127, 31.75 -> 32, 0
    np.testing.assert_array_equal(q[0], [64, -127, 32, 0])
    np.testing.assert_array_equal(q[1], [0, 0, 0, 0])
    # row 2: amax 127 -> inv 1: halves round away from zero
    np.testing.assert_array_equal(q[2], [127, 3, -3, 1])
    np.testing.assert_array_equal(s, np.float32([1 / 127, 0, 1]).astype(np.float32))


def test_quantize_fp32_add_convention():
    """trunc(v + 0.5) is evaluated in fp32: 0.49999997 + 0.5 rounds to 1.0,
    so it quantises to 1 (the reference formulation), not 0."""
    w = np.array([[127.0, 0.49999997, -0.49999997, 1.4999999]], dtype=np.float32)
    q, _ = quantize_rows_int8(w)
    np.testing.assert_array_equal(q[0], [127, 1, -1, 1])


def test_quantize_bounds_and_dequant_error(rng):
    w = (rng.standard_normal((64, 300)) * 0.02).astype(np.float16)
    q, s = quantize_rows_int8(w)
    assert q.dtype == np.int8 and np.abs(q.astype(np.int32)).max() <= 127
    assert (np.abs(q).max(axis=1) == 127).all(), "the row maximum maps to +-127"
    err = np.abs(q.astype(np.float32) * s[:, None] - w.astype(np.float32))
    assert (err <= s[:, None] * 0.5 * (1 + 1e-4)).all(), "error within half a step (+fp32 rounding)"


def test_int_matmul_exact(rng):
    a = rng.integers(-127, 128, size=(5, 7168)).astype(np.int8)
    b = rng.integers(-127, 128, size=(3, 7168)).astype(np.int8)
    got = _int_matmul(a, b)
    exp = [[sum(int(x) * int(y) for x, y in zip(a[i], b[j])) for j in range(3)] for i in range(5)]
    np.testing.assert_array_equal(got, np.array(exp))


def test_w8a8_against_fp16_oracle():
    g = torch.Generator().manual_seed(11)
    T, H, I, E, k = 64, 512, 256, 8, 3
    x = torch.randn(T, H, generator=g).half()
    lg = torch.randn(T, E, generator=g)
    wg = (torch.randn(E, I, H, generator=g) * 0.02).half()
    wu = (torch.randn(E, I, H, generator=g) * 0.02).half()
    wd = (torch.randn(E, H, I, generator=g) * 0.02).half()
    ref = fused_moe_forward(x, lg, wg, wu, wd, k).float()
    qg, sg = quantize_rows_int8(wg)
    qu, su = quantize_rows_int8(wu)
    qd, sd = quantize_rows_int8(wd)
    out = w8a8_forward(x, lg, qg, sg, qu, su, qd, sd, k).float()
    rel = float((out - ref).norm() / ref.norm())
    assert 1e-3 < rel < W8A8_REL_L2, rel  # quantisation is visible but inside the gate


def test_w8a8_exact_on_representable_inputs():
    """Inputs already on the int8 grid (x and weights = integer * 2^-n with a
    row maximum of 127 steps) quantise losslessly, so gate/up are exact; with
    I = 128 the intermediate has one scale block per row."""
    rng = np.random.default_rng(3)
    T, H, I, E, k = 8, 128, 128, 2, 1
    xi = rng.integers(-127, 128, size=(T, H)).astype(np.float32)
    xi[:, 0] = 127
    x = torch.from_numpy((xi / 64).astype(np.float16))
    wi = rng.integers(-127, 128, size=(E, I, H)).astype(np.float32)
    wi[:, :, 0] = 127
    wg = torch.from_numpy((wi / 4096).astype(np.float16))
    qg, sg = quantize_rows_int8(wg)
    np.testing.assert_array_equal(qg, wi.astype(np.int8))
    qx, sx = quantize_rows_int8(x)
    np.testing.assert_array_equal(qx, xi.astype(np.int8))
    lg = torch.zeros(T, E)
    lg[:, 1] = 1.0
    wdi = rng.integers(-127, 128, size=(E, H, I)).astype(np.float32)
    wdi[:, :, 0] = 127
    wd = torch.from_numpy((wdi / 4096).astype(np.float16))
    qd, sd = quantize_rows_int8(wd)
    out = w8a8_forward(x, lg, qg, sg, qg, sg, qd, sd, k).float()
    ref = fused_moe_forward(x, lg, wg, wg, wd, k).float()
    # only the intermediate requantisation remains (h = silu(g)*g is heavy
    # tailed, ~1.3% here): error well under the gate
    assert float((out - ref).norm() / ref.norm()) < 2e-2


def test_w8a8_intermediate_scale_is_per_128_columns():
    """Per-(row, 128-column) intermediate scales keep the small block: out[:, 0]
    stays within 5% of the fp16 oracle.  One scale per row would quantise the
    small block (|h| < amax / 254) to 0 and give out[:, 0] = 0 exactly; taking
    the scales in the wrong block order would multiply it by ~1000."""
    x, lg, wg, wu, wd, ref, q, k = scale_contrast_case(quantize_rows_int8)
    (qg, sg), (qu, su), (qd, sd) = q
    out = w8a8_forward(x, lg, qg, sg, qu, su, qd, sd, k).float()
    h_small = ref[:, 0].abs()
    assert (h_small > 1e-3).all(), "the small block contributes"
    big = ref[:, 1].abs().mean() / ref[:, 0].abs().mean()
    assert big > 300, f"block contrast only {float(big):.0f}x"
    rel0 = float((out[:, 0] - ref[:, 0]).norm() / ref[:, 0].norm())
    rel1 = float((out[:, 1] - ref[:, 1]).norm() / ref[:, 1].norm())
    assert rel0 < 5e-2 and rel1 < 5e-2, (rel0, rel1)
    # the same data with one scale over both blocks loses the small block
    out_row = w8a8_forward(x, lg, qg, sg, qu, su, qd, sd, k, scale_block=256).float()
    assert float(out_row[:, 0].abs().max()) == 0.0
