"""Seeded input builders shared by the GPU tests.

Shapes and distributions follow BASELINE.json's configs and the reference's
harness conventions (xpuoj_data/remote_bench.py:21-29 cases, :60-75 group
sizes, :78-155 inputs; race_stress2.py:15-26 random splits).
"""
from __future__ import annotations

import math

import numpy as np
import torch

from oracle import fused_moe_forward, metadata_from_group_sizes, stratified_tokens  # noqa: F401

# name -> (T, H, I, E, k, bias kind)
CONFIGS = {
    "small": (128, 1024, 512, 8, 2, None),
    "mixtral": (2048, 4096, 14336, 8, 2, None),
    "dsv3": (4096, 7168, 2048, 256, 8, "normal"),
    "decode": (32, 7168, 2048, 256, 8, "zipf"),
    "w8a8": (2048, 7168, 2048, 64, 6, None),
}

# remote_bench.py:21-29
RB_CASES = {
    0: dict(experts=1, hidden=128, intermediate=128, valid=127, high_experts=0, low_size=127),
    4: dict(experts=1, hidden=2048, intermediate=8192, valid=3072, high_experts=1, low_size=0),
    5: dict(experts=1, hidden=2048, intermediate=8192, valid=127, high_experts=0, low_size=127),
    6: dict(experts=1, hidden=2048, intermediate=128, valid=3072, high_experts=1, low_size=0),
    1: dict(experts=16, hidden=2048, intermediate=8192, valid=2272, high_experts=8, low_size=124),
    2: dict(experts=32, hidden=7168, intermediate=2048, valid=4544, high_experts=22, low_size=112),
    3: dict(experts=64, hidden=7168, intermediate=2048, valid=9088, high_experts=23, low_size=127),
}

# OPTIMIZATION_LOG.md:63 tail list
TAIL_SIZES = [0, 1, 31, 32, 63, 64, 127, 128, 129, 255, 256, 257]


def rb_group_sizes(cfg):
    """remote_bench.py:60-75: `low` experts of low_size, the rest share the
    remainder, then interleaved (even positions first)."""
    high = cfg["high_experts"]
    low = cfg["experts"] - high
    sizes = [cfg["low_size"]] * low
    remaining = cfg["valid"] - sum(sizes)
    if high:
        q, r = divmod(remaining, high)
        sizes.extend([q + (i < r) for i in range(high)])
    sizes = sizes[::2] + sizes[1::2]
    return sizes


def random_group_sizes(E, valid, seed):
    """race_stress2.py:15-26: E-1 sizes uniform in [0, min(remaining, 400)]."""
    g = torch.Generator().manual_seed(seed)
    sizes, remaining = [], valid
    for _ in range(E - 1):
        v = int(torch.randint(0, min(remaining, 400) + 1, (1,), generator=g).item())
        sizes.append(v)
        remaining -= v
    sizes.append(remaining)
    return sizes


def prerouted_inputs(sizes, H, I, seed, device="cuda", init="rb", routed_dtype=torch.float32):
    """Pre-routed operator inputs on `device` from a CPU-seeded generator
    (remote_bench.py:78-155 pattern).  init 'rb': weights N(0,1)/sqrt(I|H);
    'ns': N(0, 0.02)."""
    E = len(sizes)
    go, gpo, gidx = metadata_from_group_sizes(sizes, 128)
    P = int(gpo[-1])
    g = torch.Generator(device="cpu").manual_seed(seed)
    ws, wd_s = (1 / math.sqrt(I), 1 / math.sqrt(H)) if init == "rb" else (0.02, 0.02)
    big = E * I * H > (1 << 27)
    if big:  # generate on the device to keep host time bounded
        gd = torch.Generator(device=device).manual_seed(seed)
        mk = lambda shape, s: (torch.randn(shape, generator=gd, device=device, dtype=torch.float16) * s)
    else:
        mk = lambda shape, s: (torch.randn(shape, generator=g, dtype=torch.float16) * s).to(device)
    x = torch.randn((P, H), generator=g, dtype=torch.float16).to(device)
    wg = mk((E, I, H), ws)
    wu = mk((E, I, H), ws)
    wd = mk((E, H, I), wd_s)
    routed = torch.rand((int(go[-1]),), generator=g, dtype=torch.float32).to(routed_dtype).to(device)
    meta = [torch.tensor(np.asarray(a, dtype=np.int32), device=device) for a in (sizes, go, gpo, gidx)]
    return (x, wg, wu, wd, routed, *meta)


def moe_inputs(name, seed, device="cuda", T=None):
    """fused-MoE inputs for a BASELINE config (optionally with fewer tokens)."""
    T0, H, I, E, k, bias_kind = CONFIGS[name]
    T = T0 if T is None else T
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = torch.randn((T, H), generator=g, dtype=torch.float16).to(device)
    logits = torch.randn((T, E), generator=g, dtype=torch.float32).to(device)
    bias = None
    if bias_kind == "normal":
        bias = (torch.randn((E,), generator=g) * 0.5).to(device)
    elif bias_kind == "zipf":
        # expert rank = index: bias = -1.2 * ln(rank + 1)
        bias = (-1.2 * torch.log(torch.arange(E, dtype=torch.float32) + 1)).to(device)
    if E * I * H > (1 << 27):
        gd = torch.Generator(device=device).manual_seed(seed + 1)
        mk = lambda shape: torch.randn(shape, generator=gd, device=device, dtype=torch.float16) * 0.02
    else:
        mk = lambda shape: (torch.randn(shape, generator=g, dtype=torch.float16) * 0.02).to(device)
    wg = mk((E, I, H))
    wu = mk((E, I, H))
    wd = mk((E, H, I))
    return dict(x=x, logits=logits, bias=bias, wg=wg, wu=wu, wd=wd, k=k, T=T, H=H, I=I, E=E)


def skewed_8bit_case(seed, device="cuda"):
    """T=800, H=512 (a multiple of 256), 200 routed rows per expert: 128-row
    blocks picked, and the 8-bit paths pad experts to 256 rows.  Biases give an
    empty expert, experts of <= 128 rows (an empty second half) and
    multi-block experts."""
    g = torch.Generator().manual_seed(seed)
    T, H, I, E, k = 800, 512, 256, 8, 2
    return dict(x=torch.randn(T, H, generator=g).half().to(device), logits=torch.randn(T, E, generator=g).to(device),
                bias=torch.tensor([2.0, 1.5, 1.0, 0.0, -0.5, -1.0, -1.5, -40.0]).to(device),
                wg=(torch.randn(E, I, H, generator=g) * 0.05).half().to(device),
                wu=(torch.randn(E, I, H, generator=g) * 0.05).half().to(device),
                wd=(torch.randn(E, H, I, generator=g) * 0.05).half().to(device), k=k, T=T, H=H, I=I, E=E)


def scale_contrast_case(fmt_q):
    """I = 256 (two 128-column scale blocks of the intermediate): gate/up
    rows 0-127 ~N(0, 0.05^2), rows 128-255 30x larger, so h's second block is
    ~1000x the first.  w_down row 0 reads only block 0 and row 1 only block
    1, so out[:, 0] is made of the small block alone."""
    g = torch.Generator().manual_seed(5)
    T, H, I, E, k = 16, 128, 256, 1, 1
    x = torch.randn(T, H, generator=g).half()
    lg = torch.zeros(T, E)
    wg = torch.randn(E, I, H, generator=g) * 0.05
    wu = torch.randn(E, I, H, generator=g) * 0.05
    wg[:, 128:] *= 30.0
    wu[:, 128:] *= 30.0
    wg, wu = wg.half(), wu.half()
    wd = torch.zeros(E, H, I)
    wd[:, 0, :128] = torch.randn(128, generator=g) * 0.05
    wd[:, 1, 128:] = torch.randn(128, generator=g) * 0.05
    wd[:, 2:] = torch.randn(E, H - 2, I, generator=g) * 0.05
    wd = wd.half()
    ref = fused_moe_forward(x, lg, wg, wu, wd, k).float()
    q = [fmt_q(w) for w in (wg, wu, wd)]
    return x, lg, wg, wu, wd, ref, q, k


def exact_routing_inputs(k, seed, counts, H, I):
    """CPU x, logits and weights whose top-k routing gives expert e exactly
    counts[e] pairs (with k > 1 the k experts of a token differ)."""
    from oracle import route_topk
    g = torch.Generator().manual_seed(seed)
    E = len(counts)
    slots = np.repeat(np.arange(E), counts)  # expert-sorted pair slots
    P = len(slots)
    assert P % k == 0 and max(counts) < P // k
    T = P // k
    logits = torch.randn(T, E, generator=g) * 0.1
    perm = torch.randperm(T, generator=g).numpy()  # tokens in random order
    for j in range(k):
        # token perm[i] takes slot i + j*T: an expert's run is shorter than T,
        # so the k slots of a token name k different experts
        logits[perm, torch.from_numpy(slots[j * T:(j + 1) * T])] += 8.0 - j
    x = torch.randn(T, H, generator=g).half()
    wg = (torch.randn(E, I, H, generator=g) * 0.05).half()
    wu = (torch.randn(E, I, H, generator=g) * 0.05).half()
    wd = (torch.randn(E, H, I, generator=g) * 0.05).half()
    ids, _ = route_topk(logits.numpy(), k, None)
    np.testing.assert_array_equal(np.bincount(ids.ravel(), minlength=E), counts)
    return x, logits, wg, wu, wd
