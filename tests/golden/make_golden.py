"""Regenerate the golden fixtures in this directory (run from the repo root):

    python tests/golden/make_golden.py

The reference commits no golden tensors (its harness writes .pt files at run
time, xpuoj_data/remote_bench.py:254-257), so these fixtures hold seeded
inputs and the CPU oracle's outputs for small cases of each path: the
pre-routed operator on the problem_detail.json:40 layout (an empty expert and
a two-block expert added), the full fused MoE with an expert bias, and W8A8;
and, for the paths beyond the reference's operator, fp8 W8A8 codes and output,
the router GEMM, the shared expert and an expert-parallel shard.
"""
from pathlib import Path
import sys

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle import (fused_moe_forward, metadata_from_group_sizes, prerouted_forward,  # noqa: E402
                    quantize_rows_fp8, quantize_rows_int8, route_topk, router_logits, w8a8_forward)

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


def extensions():
    rng = np.random.default_rng(42)
    T, H, I, E, k = 48, 256, 128, 8, 2
    x = rng.standard_normal((T, H)).astype(np.float16)
    bias = (rng.standard_normal(E) * 0.5).astype(np.float32)
    wr = (rng.standard_normal((E, H)) / np.sqrt(H)).astype(np.float16)
    wg = (rng.standard_normal((E, I, H)) * 0.05).astype(np.float16)
    wu = (rng.standard_normal((E, I, H)) * 0.05).astype(np.float16)
    wd = (rng.standard_normal((E, H, I)) * 0.05).astype(np.float16)
    sg = (rng.standard_normal((I, H)) * 0.05).astype(np.float16)
    su = (rng.standard_normal((I, H)) * 0.05).astype(np.float16)
    sd = (rng.standard_normal((H, I)) * 0.05).astype(np.float16)
    t = torch.from_numpy
    logits = router_logits(x, wr)                      # fp32 [T, E] from the router GEMM
    ids, w = route_topk(logits, k, bias)
    out_router = fused_moe_forward(t(x), t(logits), t(wg), t(wu), t(wd), k, t(bias)).numpy()
    out_shared = fused_moe_forward(t(x), t(logits), t(wg), t(wu), t(wd), k, t(bias),
                                   shared=(t(sg), t(su), t(sd))).numpy()
    out_shard = fused_moe_forward(t(x), t(logits), t(wg[2:6]), t(wu[2:6]), t(wd[2:6]), k, t(bias),
                                  expert_range=(2, 4)).numpy()
    qg, s_g = quantize_rows_fp8(wg)
    qu, s_u = quantize_rows_fp8(wu)
    qd, s_d = quantize_rows_fp8(wd)
    out_fp8 = w8a8_forward(t(x), t(logits), qg, s_g, qu, s_u, qd, s_d, k, t(bias), fmt="fp8").numpy()
    np.savez_compressed(OUT / "extensions_small.npz", x=x, bias=bias, w_router=wr, w_gate=wg, w_up=wu,
                        w_down=wd, w_gate_shared=sg, w_up_shared=su, w_down_shared=sd, top_k=np.int32(k),
                        logits=logits, ids=ids, weights=w, out_router=out_router, out_shared=out_shared,
                        out_shard=out_shard, q_gate_fp8=qg, s_gate_fp8=s_g, out_fp8=out_fp8)


if __name__ == "__main__":
    torch.set_num_threads(1)
    prerouted()
    fused()
    extensions()
    for f in sorted(OUT.glob("*.npz")):
        print(f.name, f.stat().st_size)
