"""Regenerate the golden fixtures in this directory (run from the repo root):

    python tests/golden/make_golden.py

The reference commits no golden tensors (its harness writes .pt files at run
time, xpuoj_data/remote_bench.py:254-257), so these fixtures hold seeded
inputs and the CPU oracle's outputs for small cases of each path: the
pre-routed operator on the problem_detail.json:40 layout (an empty expert and
a two-block expert added), the full fused MoE with an expert bias, and W8A8.
"""
from pathlib import Path
import sys

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle import (fused_moe_forward, metadata_from_group_sizes, prerouted_forward,  # noqa: E402
                    quantize_rows_int8, route_topk, w8a8_forward)

OUT = Path(__file__).resolve().parent


def prerouted():
    rng = np.random.default_rng(40)
    sizes = [3, 0, 130, 2]
    H, I = 128, 128
    go, gpo, gidx = metadata_from_group_sizes(sizes, 128)
    P = int(gpo[-1])
    x = rng.standard_normal((P, H)).astype(np.float16)
    wg = (rng.standard_normal((4, I, H)) / np.sqrt(I)).astype(np.float16)
    wu = (rng.standard_normal((4, I, H)) / np.sqrt(I)).astype(np.float16)
    wd = (rng.standard_normal((4, H, I)) / np.sqrt(H)).astype(np.float16)
    routed = rng.random(int(go[-1])).astype(np.float32)
    out = prerouted_forward(x, wg, wu, wd, routed, sizes, go, gpo, gidx).numpy()
    np.savez_compressed(OUT / "prerouted_small.npz", x=x, w_gate=wg, w_up=wu, w_down=wd, routed=routed,
                        group_sizes=np.asarray(sizes, np.int32), group_offsets=go,
                        group_padded_offsets=gpo, group_idx_for_bx=gidx, out=out)


def fused():
    rng = np.random.default_rng(41)
    T, H, I, E, k = 40, 128, 128, 4, 2
    x = rng.standard_normal((T, H)).astype(np.float16)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.5).astype(np.float32)
    wg = (rng.standard_normal((E, I, H)) * 0.05).astype(np.float16)
    wu = (rng.standard_normal((E, I, H)) * 0.05).astype(np.float16)
    wd = (rng.standard_normal((E, H, I)) * 0.05).astype(np.float16)
    ids, w = route_topk(logits, k, bias)
    out = fused_moe_forward(torch.from_numpy(x), torch.from_numpy(logits), torch.from_numpy(wg),
                            torch.from_numpy(wu), torch.from_numpy(wd), k, torch.from_numpy(bias)).numpy()
    qg, sg = quantize_rows_int8(wg)
    qu, su = quantize_rows_int8(wu)
    qd, sd = quantize_rows_int8(wd)
    out8 = w8a8_forward(torch.from_numpy(x), torch.from_numpy(logits), qg, sg, qu, su, qd, sd, k,
                        torch.from_numpy(bias)).numpy()
    np.savez_compressed(OUT / "fused_small.npz", x=x, logits=logits, bias=bias, w_gate=wg, w_up=wu,
                        w_down=wd, top_k=np.int32(k), ids=ids, weights=w, out=out, out_w8a8=out8,
                        q_gate=qg, s_gate=sg)


if __name__ == "__main__":
    torch.set_num_threads(1)
    prerouted()
    fused()
    for f in sorted(OUT.glob("*.npz")):
        print(f.name, f.stat().st_size)
