"""Pins the fp8 (OCP e4m3) oracle: the encoder against torch's own
float8_e4m3fn conversion on every code value, every midpoint between
neighbouring codes (ties to even) and the floats just beside them; the value
table against torch's decode; hand-made codes; exact float64 products of e4m3
values; and the fp8 W8A8 forward against the fp16 oracle."""
import numpy as np
import torch

from oracle import FP8_E4M3_VALUES, fp8_e4m3_codes, fused_moe_forward, quantize_rows_fp8, w8a8_forward
from oracle.moe_ref import _exact_matmul

FP8_REL_L2 = 8e-2  # e4m3 keeps 3 mantissa bits: ~2-4% per operand, two GEMMs


def _torch_codes(v):
    return torch.from_numpy(np.asarray(v, np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_value_table_matches_torch_decode():
    dec = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy().astype(np.float64)
    np.testing.assert_array_equal(np.isnan(dec), np.isnan(FP8_E4M3_VALUES))
    ok = ~np.isnan(dec)
    np.testing.assert_array_equal(dec[ok], FP8_E4M3_VALUES[ok])


def test_encoder_on_every_boundary_matches_torch():
    pos = np.unique(FP8_E4M3_VALUES[:0x7F][~np.isnan(FP8_E4M3_VALUES[:0x7F])])  # 0 .. 448
    mids = (pos[:-1] + pos[1:]) / 2                                        # ties: round to even
    pts = np.concatenate([pos, mids]).astype(np.float32)
    pts = np.concatenate([pts, np.nextafter(pts, np.float32(np.inf)), np.nextafter(pts, np.float32(0))])
    pts = pts[(pts >= 0) & (pts < 464)]
    pts = np.concatenate([pts, -pts]).astype(np.float32)
    np.testing.assert_array_equal(fp8_e4m3_codes(pts), _torch_codes(pts))
    rng = np.random.default_rng(0)
    r = (rng.standard_normal(200000) * 10.0 ** rng.uniform(-4, 2, 200000)).astype(np.float32)
    r = r[np.abs(r) < 448]
    np.testing.assert_array_equal(fp8_e4m3_codes(r), _torch_codes(r))


def test_encoder_known_codes():
    v = np.float32([1.0, 448.0, 2.0 ** -9, -2.0, 0.0, 1.0625, 1.1875, 450.0, 2.0 ** -10, 3 * 2.0 ** -10])
    # 1.0625 is halfway between 1.0 (0x38) and 1.125 (0x39): even -> 0x38;
    # 1.1875 between 0x39 and 1.25 (0x3A): even -> 0x3A; 450 saturates to 448;
    # 2^-10 ties to 0, 3*2^-10 ties to 2*2^-9 (code 2)
    np.testing.assert_array_equal(fp8_e4m3_codes(v), [0x38, 0x7E, 0x01, 0xC0, 0x00, 0x38, 0x3A, 0x7E, 0x00, 0x02])


def test_quantize_rows_fp8():
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((64, 300)) * 0.02).astype(np.float16)
    w[0] = 0
    q, s = quantize_rows_fp8(w)
    assert q.dtype == np.uint8 and s[0] == 0 and (q[0] == 0).all()
    assert (np.abs(FP8_E4M3_VALUES[q[1:]]).max(axis=1) == 448).all(), "the row maximum maps to 448"
    deq = FP8_E4M3_VALUES[q] * s[:, None]
    wf = w.astype(np.float64)
    big = np.abs(wf) >= s[:, None] * 2.0 ** -6   # normal range of the scaled row
    assert (np.abs(deq - wf)[big] <= np.abs(wf)[big] * 2.0 ** -4 * (1 + 1e-6)).all(), "half an ulp (3 bits)"


def test_exact_matmul_of_e4m3_values():
    rng = np.random.default_rng(2)
    a = FP8_E4M3_VALUES[rng.choice(np.r_[0:0x7F, 0x80:0xFF], size=(4, 7168))]
    b = FP8_E4M3_VALUES[rng.choice(np.r_[0:0x7F, 0x80:0xFF], size=(3, 7168))]
    got = _exact_matmul(a, b)
    # every value is an integer multiple of 2^-9: integer arithmetic is exact
    ai, bi = (a * 512).astype(np.int64), (b * 512).astype(np.int64)
    exp = np.array([[int(np.dot(ai[i].astype(object), bi[j].astype(object))) for j in range(3)] for i in range(4)])
    np.testing.assert_array_equal(got * 2.0 ** 18, exp.astype(np.float64))


def test_fp8_forward_against_fp16_oracle():
    g = torch.Generator().manual_seed(11)
    T, H, I, E, k = 64, 512, 256, 8, 3
    x = torch.randn(T, H, generator=g).half()
    lg = torch.randn(T, E, generator=g)
    wg = (torch.randn(E, I, H, generator=g) * 0.02).half()
    wu = (torch.randn(E, I, H, generator=g) * 0.02).half()
    wd = (torch.randn(E, H, I, generator=g) * 0.02).half()
    ref = fused_moe_forward(x, lg, wg, wu, wd, k).float()
    qg, sg = quantize_rows_fp8(wg)
    qu, su = quantize_rows_fp8(wu)
    qd, sd = quantize_rows_fp8(wd)
    out = w8a8_forward(x, lg, qg, sg, qu, su, qd, sd, k, fmt="fp8").float()
    rel = float((out - ref).norm() / ref.norm())
    assert 5e-3 < rel < FP8_REL_L2, rel


def test_pow2_scales_brute_force():
    """pow2_scales(amax) is the smallest 2**j (j >= -127) with amax <= 448 * 2**j,
    checked by trying every j, on random magnitudes and the edges amax = 448 * 2**j
    (and the floats beside it)."""
    from oracle import pow2_scales
    rng = np.random.default_rng(7)
    a = (10.0 ** rng.uniform(-40, 30, 3000)).astype(np.float32)
    edges = np.float32([448.0 * 2.0 ** j for j in (-20, -1, 0, 3)])
    a = np.concatenate([a, edges, np.nextafter(edges, np.float32(np.inf)), np.nextafter(edges, np.float32(0))])
    a = np.concatenate([a, np.float32([0.0, 1e-45, 2.0 ** -130])])
    s = pow2_scales(a)
    for amax, sc in zip(a.astype(np.float64), s.astype(np.float64)):
        if amax == 0:
            assert sc == 0
            continue
        js = [j for j in range(-127, 128) if amax <= 448.0 * 2.0 ** j]
        assert sc == 2.0 ** js[0], (amax, sc)
    ok = (a > 2.0 ** -100)
    assert ((a[ok] / s[ok] > 224) & (a[ok] / s[ok] <= 448)).all()


def test_pow2_fp8_rows_are_exact_scalings():
    from oracle import quantize_rows_fp8
    rng = np.random.default_rng(8)
    w = (rng.standard_normal((50, 128)) * 10.0 ** rng.uniform(-3, 3, (50, 1))).astype(np.float32)
    q, s = quantize_rows_fp8(w, pow2=True)
    assert (np.log2(s) == np.round(np.log2(s))).all()
    # the codes are those of w / s (exact division by a power of two)
    np.testing.assert_array_equal(q, fp8_e4m3_codes((w / s[:, None]).astype(np.float32)))
    assert (np.abs(FP8_E4M3_VALUES[q]).max(axis=1) >= 224).all()  # (224, 448] before rounding
