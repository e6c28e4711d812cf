"""Device-side fp32 restatement of the reference operator for the stress
tests (problem_detail.json:50; xpuoj_data/race_stress2.py:29-48 runs the same
loop on the GPU).  Test infrastructure only: it is pinned against the CPU
oracle in tests/test_gpu_stress.py and never used by the product path."""
import torch
import torch.nn.functional as F


def prerouted_reference(x, wg, wu, wd, routed, gs, go, gpo):
    """fp32 [P, H] on x's device: rows of expert e's valid tokens get
    silu(x Wg^T) * (x Wu^T) Wd^T * routed[go[e] + i]; all other rows 0."""
    P, H = x.shape
    out = torch.zeros((P, H), dtype=torch.float32, device=x.device)
    sizes, offs, padds = gs.tolist(), go.tolist(), gpo.tolist()
    for e, n in enumerate(sizes):
        if n == 0:
            continue
        xe = x[padds[e]:padds[e] + n].float()
        g = F.linear(xe, wg[e].float())
        u = F.linear(xe, wu[e].float())
        y = F.linear(torch.sigmoid(g) * g * u, wd[e].float())
        out[padds[e]:padds[e] + n] = y * routed[offs[e]:offs[e] + n].float().unsqueeze(1)
    return out
