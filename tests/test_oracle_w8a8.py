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
    row maximum of 127 steps) quantise losslessly, so gate/up are exact."""
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
    # tailed, ~1.3% here, plus h's fp16 rounding): error well under the gate
    assert float((out - ref).norm() / ref.norm()) < 2e-2


def test_w8a8_int8_intermediate_scale_is_per_row():
    """int8 quantises h with one scale per routed row.  In the scale-contrast
    case (I = 256, h's second 128-column block ~1000x its first) the small
    block's codes are all 0 (|h| < amax / 254), so out[:, 0], which reads only
    that block, is exactly 0, while out[:, 1] stays within 5% of the fp16
    oracle.  Per-(row, 128-column) scales would keep the small block (out[:, 0]
    within ~1% of the fp16 oracle, as fp8's do); a scale taken from the wrong
    row would break out[:, 1]."""
    x, lg, wg, wu, wd, ref, q, k = scale_contrast_case(quantize_rows_int8)
    (qg, sg), (qu, su), (qd, sd) = q
    out = w8a8_forward(x, lg, qg, sg, qu, su, qd, sd, k).float()
    assert (ref[:, 0].abs() > 1e-3).all(), "the small block contributes in fp16"
    big = ref[:, 1].abs().mean() / ref[:, 0].abs().mean()
    assert big > 300, f"block contrast only {float(big):.0f}x"
    assert float(out[:, 0].abs().max()) == 0.0
    rel1 = float((out[:, 1] - ref[:, 1]).norm() / ref[:, 1].norm())
    assert rel1 < 5e-2, rel1
    # the fp8 path keeps per-(row, 128-column) scales: the small block survives
    from oracle import quantize_rows_fp8
    x, lg, wg, wu, wd, ref, q8, k = scale_contrast_case(quantize_rows_fp8)
    (qg, sg), (qu, su), (qd, sd) = q8
    out8 = w8a8_forward(x, lg, qg, sg, qu, su, qd, sd, k, fmt="fp8").float()
    rel0 = float((out8[:, 0] - ref[:, 0]).norm() / ref[:, 0].norm())
    assert rel0 < 8e-2, rel0


def test_w8a8_int8_invariant_under_intermediate_permutation():
    """One scale over the whole row makes the int8 result independent of the
    order of the I columns: permuting gate/up rows and w_down columns by the
    same permutation (here one that moves columns across 128-column blocks)
    gives a bit-identical output.  Per-block scales would not: the blocks'
    maxima change."""
    g = torch.Generator().manual_seed(12)
    T, H, I, E, k = 24, 256, 384, 4, 2
    x = torch.randn(T, H, generator=g).half()
    lg = torch.randn(T, E, generator=g)
    wg = (torch.randn(E, I, H, generator=g) * 0.05)
    wu = (torch.randn(E, I, H, generator=g) * 0.05)
    wg[:, :128] *= 8.0  # uneven column blocks, so per-block and per-row scales differ
    wg, wu = wg.half(), wu.half()
    wd = (torch.randn(E, H, I, generator=g) * 0.05).half()
    perm = torch.randperm(I, generator=g)
    q = [quantize_rows_int8(w) for w in (wg, wu, wd)]
    qp = [quantize_rows_int8(w) for w in (wg[:, perm], wu[:, perm], wd[:, :, perm])]
    out = w8a8_forward(x, lg, *q[0], *q[1], *q[2], k)
    outp = w8a8_forward(x, lg, *qp[0], *qp[1], *qp[2], k)
    assert float(out.float().abs().max()) > 0 and torch.equal(out, outp)
    # the same permutation moves fp8's per-(row, 128-column) block maxima, so
    # its result changes: the check tells the two contracts apart
    from oracle import quantize_rows_fp8
    q8 = [quantize_rows_fp8(w) for w in (wg, wu, wd)]
    q8p = [quantize_rows_fp8(w) for w in (wg[:, perm], wu[:, perm], wd[:, :, perm])]
    o8 = w8a8_forward(x, lg, *q8[0], *q8[1], *q8[2], k, fmt="fp8")
    o8p = w8a8_forward(x, lg, *q8p[0], *q8p[1], *q8p[2], k, fmt="fp8")
    assert not torch.equal(o8, o8p)
