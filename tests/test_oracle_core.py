"""Pins oracle.prerouted_forward / combine / fused_moe_forward
(problem_detail.json:50 semantics) without retyping its formula."""
import math

import numpy as np
import pytest
import torch

from oracle import combine, fused_moe_forward, metadata_from_group_sizes, prerouted_forward, route_topk


def _silu(v):
    return v / (1.0 + math.exp(-v))


def _perm_matrix(perm):
    n = len(perm)
    m = np.zeros((n, n), dtype=np.float32)
    for i, p in enumerate(perm):
        m[i, p] = 1.0  # (x M^T)[i] = x[perm[i]]
    return m


def test_permutation_closed_form():
    """Wg = a*Pg, Wu = b*Pu, Wd = c*Pd with non-involutive permutations:
    out[r, j] = routed[go[e]+i] * c * silu(a*x[pg[pd[j]]]) * b*x[pu[pd[j]]].
    A transposed operand, a dropped factor or a padded/raw index mix-up changes
    the result."""
    n = 8
    sizes = [3, 0, 2, 5]
    E = len(sizes)
    go, gpo, gidx = metadata_from_group_sizes(sizes, 128)
    P = int(gpo[-1])
    rng = np.random.default_rng(7)
    x = rng.standard_normal((P, n)).astype(np.float16)
    perms = {}
    wg = np.zeros((E, n, n), np.float16)
    wu = np.zeros((E, n, n), np.float16)
    wd = np.zeros((E, n, n), np.float16)
    coef = [(0.5, 2.0, 0.25), (1.0, 1.0, 1.0), (2.0, 0.5, 1.5), (0.75, -1.0, 0.5)]
    for e in range(E):
        pg = [(i + 1 + e) % n for i in range(n)]
        pu = [(3 * i + 2) % n for i in range(n)]
        pd = [(5 * i + e) % n for i in range(n)]
        perms[e] = (pg, pu, pd)
        a, b, c = coef[e]
        wg[e] = a * _perm_matrix(pg)
        wu[e] = b * _perm_matrix(pu)
        wd[e] = c * _perm_matrix(pd)
    V = int(go[-1])
    routed = (1.0 + 0.125 * np.arange(V)).astype(np.float32)
    out = prerouted_forward(x, wg, wu, wd, routed, sizes, go, gpo, gidx, out_fp32=True).numpy()
    exp = np.zeros((P, n), np.float64)
    for e in range(E):
        pg, pu, pd = perms[e]
        a, b, c = coef[e]
        for i in range(sizes[e]):
            r = gpo[e] + i
            xr = x[r].astype(np.float64)
            for j in range(n):
                hi = pd[j]
                exp[r, j] = routed[go[e] + i] * c * _silu(a * xr[pg[hi]]) * (b * xr[pu[hi]])
    np.testing.assert_allclose(out, exp, rtol=2e-6, atol=1e-7)


def test_scalar_loop_fp64(rng):
    """Random tiny case against a plain fp64 triple loop."""
    H, I, sizes = 6, 5, [2, 1, 0, 3]
    E = len(sizes)
    go, gpo, gidx = metadata_from_group_sizes(sizes, 128)
    P = int(gpo[-1])
    x = rng.standard_normal((P, H)).astype(np.float16)
    wg = (rng.standard_normal((E, I, H)) * 0.5).astype(np.float16)
    wu = (rng.standard_normal((E, I, H)) * 0.5).astype(np.float16)
    wd = (rng.standard_normal((E, H, I)) * 0.5).astype(np.float16)
    routed = rng.random(int(go[-1])).astype(np.float16)
    out = prerouted_forward(x, wg, wu, wd, routed, sizes, go, gpo, gidx, out_fp32=True).numpy()
    for e in range(E):
        for i in range(sizes[e]):
            r = gpo[e] + i
            xr = [float(v) for v in x[r]]
            h = []
            for q in range(I):
                g = sum(xr[k] * float(wg[e, q, k]) for k in range(H))
                u = sum(xr[k] * float(wu[e, q, k]) for k in range(H))
                h.append(_silu(g) * u)
            for j in range(H):
                y = sum(h[q] * float(wd[e, j, q]) for q in range(I)) * float(routed[go[e] + i])
                assert abs(out[r, j] - y) <= 1e-5 * (1 + abs(y))
    mask = np.ones(P, bool)
    for e in range(E):
        mask[gpo[e]:gpo[e] + sizes[e]] = False
    assert (out[mask] == 0).all()


def test_single_expert_is_dense_swiglu(rng):
    H, I, n = 16, 24, 100
    go, gpo, gidx = metadata_from_group_sizes([n], 128)
    x = torch.from_numpy(rng.standard_normal((128, H)).astype(np.float16))
    wg = torch.from_numpy((rng.standard_normal((1, I, H)) * 0.3).astype(np.float16))
    wu = torch.from_numpy((rng.standard_normal((1, I, H)) * 0.3).astype(np.float16))
    wd = torch.from_numpy((rng.standard_normal((1, H, I)) * 0.3).astype(np.float16))
    routed = torch.ones(n)
    out = prerouted_forward(x, wg, wu, wd, routed, [n], go, gpo, gidx, out_fp32=True)
    xd = x[:n].double()
    dense = (torch.nn.functional.silu(xd @ wg[0].double().T) * (xd @ wu[0].double().T)) @ wd[0].double().T
    torch.testing.assert_close(out[:n].double(), dense, rtol=1e-5, atol=1e-6)
    assert (out[n:] == 0).all()


def test_nan_padding_and_empty_cases(rng):
    H, I, sizes = 8, 8, [1, 0, 127]
    go, gpo, gidx = metadata_from_group_sizes(sizes, 128)
    P = int(gpo[-1])
    x = rng.standard_normal((P, H)).astype(np.float16)
    pad = np.ones(P, bool)
    for e, n in enumerate(sizes):
        pad[gpo[e]:gpo[e] + n] = False
    x[pad] = np.nan
    w = (rng.standard_normal((3, I, H)) * 0.2).astype(np.float16)
    wdn = (rng.standard_normal((3, H, I)) * 0.2).astype(np.float16)
    routed = rng.random(int(go[-1])).astype(np.float32)
    out = prerouted_forward(x, w, w, wdn, routed, sizes, go, gpo, gidx)
    assert torch.isfinite(out).all()
    assert (out[torch.from_numpy(pad)] == 0).all()
    # V = 0: every row is padding
    go0, gpo0, gidx0 = metadata_from_group_sizes([0, 0, 0], 128)
    out0 = prerouted_forward(np.zeros((0, H), np.float16), w, w, wdn, np.zeros(0, np.float32), [0, 0, 0], go0, gpo0, gidx0)
    assert out0.shape == (0, H)


def test_routed_weight_linearity(rng):
    H, I, sizes = 16, 16, [5, 9]
    go, gpo, gidx = metadata_from_group_sizes(sizes, 128)
    P = int(gpo[-1])
    x = rng.standard_normal((P, H)).astype(np.float16)
    wg = (rng.standard_normal((2, I, H)) * 0.2).astype(np.float16)
    wd = (rng.standard_normal((2, H, I)) * 0.2).astype(np.float16)
    r = rng.random(14).astype(np.float32)
    # fp32 output: scaling by 2 is exact (fp16 subnormals would round differently)
    o1 = prerouted_forward(x, wg, wg, wd, r, sizes, go, gpo, gidx, out_fp32=True)
    o2 = prerouted_forward(x, wg, wg, wd, 2 * r, sizes, go, gpo, gidx, out_fp32=True)
    torch.testing.assert_close(o2, 2 * o1, rtol=0, atol=0)


def test_combine_closed_form():
    T, k, H = 3, 2, 4
    y = torch.zeros(T * k, H)
    for p in range(T * k):
        y[p, p % H] = float(p + 1)
    out = combine(y, T, k)
    exp = torch.zeros(T, H)
    for t in range(T):
        for j in range(k):
            p = t * k + j
            exp[t, p % H] += p + 1
    torch.testing.assert_close(out, exp, rtol=0, atol=0)


def test_fused_matches_dense_per_token(rng):
    """Full pipeline (route -> align -> gather -> grouped MLP -> combine) against
    a per-token dense formulation in fp64 that never sorts or pads."""
    T, H, I, E, k = 40, 32, 16, 6, 2
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float16))
    logits = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32))
    bias = torch.from_numpy((rng.standard_normal(E) * 0.5).astype(np.float32))
    wg = torch.from_numpy((rng.standard_normal((E, I, H)) * 0.2).astype(np.float16))
    wu = torch.from_numpy((rng.standard_normal((E, I, H)) * 0.2).astype(np.float16))
    wd = torch.from_numpy((rng.standard_normal((E, H, I)) * 0.2).astype(np.float16))
    for bm in (32, 128):
        out = fused_moe_forward(x, logits, wg, wu, wd, k, bias, block_m=bm)
        ids, w = route_topk(logits.numpy(), k, bias.numpy())
        exp = torch.zeros(T, H, dtype=torch.float64)
        for t in range(T):
            xt = x[t].double()
            for j in range(k):
                e = int(ids[t, j])
                g = wg[e].double() @ xt
                u = wu[e].double() @ xt
                exp[t] += float(w[t, j]) * (wd[e].double() @ (torch.sigmoid(g) * g * u))
        torch.testing.assert_close(out.double(), exp, rtol=2e-3, atol=2e-3)


def test_shared_expert_closed_forms(rng):
    """Shared expert: (1) with k = 1 and every token routed to expert 0, a
    shared expert equal to expert 0 doubles the output exactly (both terms have
    weight 1, fp32 sums, and fp16 scaling by 2 is exact); (2) the shared
    output minus the routed-only output is the dense SwiGLU MLP of x with the
    shared weights, computed per token in fp64 without routing or sorting."""
    T, H, I, E = 37, 32, 16, 5
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float16))
    wg = torch.from_numpy((rng.standard_normal((E, I, H)) * 0.2).astype(np.float16))
    wu = torch.from_numpy((rng.standard_normal((E, I, H)) * 0.2).astype(np.float16))
    wd = torch.from_numpy((rng.standard_normal((E, H, I)) * 0.2).astype(np.float16))
    logits = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32))
    hot = logits.clone()
    hot[:, 0] += 100.0
    base, aux = fused_moe_forward(x, hot, wg, wu, wd, 1, return_aux=True)
    assert (aux["ids"][:, 0] == 0).all()
    doubled, aux2 = fused_moe_forward(x, hot, wg, wu, wd, 1, shared=(wg[0], wu[0], wd[0]), return_aux=True)
    assert torch.equal(doubled, base * 2)
    np.testing.assert_array_equal(aux2["ids"][:, 1], np.full(T, E))
    np.testing.assert_array_equal(aux2["weights"][:, 1], np.ones(T, np.float32))

    sg = torch.from_numpy((rng.standard_normal((I, H)) * 0.2).astype(np.float16))
    su = torch.from_numpy((rng.standard_normal((I, H)) * 0.2).astype(np.float16))
    sd = torch.from_numpy((rng.standard_normal((H, I)) * 0.2).astype(np.float16))
    for k, bm in ((2, 32), (3, 128)):
        routed = fused_moe_forward(x, logits, wg, wu, wd, k, block_m=bm)
        both = fused_moe_forward(x, logits, wg, wu, wd, k, block_m=bm, shared=(sg, su, sd))
        xd = x.double()
        g, u = xd @ sg.double().T, xd @ su.double().T
        dense = (torch.sigmoid(g) * g * u) @ sd.double().T
        torch.testing.assert_close(both.double() - routed.double(), dense, rtol=2e-3, atol=3e-3)


def test_expert_shards_closed_forms(rng):
    """Expert shards: one shard over all experts is the full layer exactly; the
    partial outputs of disjoint shards covering all experts sum to the full
    layer (fp16 rounding of each part aside); a shard owning none of a
    token's choices gives that token 0."""
    T, H, I, E, k = 33, 32, 16, 8, 3
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float16))
    logits = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32))
    bias = torch.from_numpy((rng.standard_normal(E) * 0.5).astype(np.float32))
    wg = torch.from_numpy((rng.standard_normal((E, I, H)) * 0.2).astype(np.float16))
    wu = torch.from_numpy((rng.standard_normal((E, I, H)) * 0.2).astype(np.float16))
    wd = torch.from_numpy((rng.standard_normal((E, H, I)) * 0.2).astype(np.float16))
    full, aux = fused_moe_forward(x, logits, wg, wu, wd, k, bias, return_aux=True)
    whole = fused_moe_forward(x, logits, wg, wu, wd, k, bias, expert_range=(0, E))
    assert torch.equal(whole, full)
    parts = [fused_moe_forward(x, logits, wg[b:b + n], wu[b:b + n], wd[b:b + n], k, bias, expert_range=(b, n))
             for b, n in ((0, 3), (3, 1), (4, 4))]
    torch.testing.assert_close(sum(p.double() for p in parts), full.double(), rtol=0, atol=3e-3)
    ids = aux["ids"]
    none_in_1 = ~(ids == 3).any(axis=1)            # tokens without a choice of expert 3
    assert (parts[1][torch.from_numpy(none_in_1)] == 0).all()
    # a shard = the dense per-token sum over its own experts
    exp = torch.zeros(T, H, dtype=torch.float64)
    _, w = route_topk(logits.numpy(), k, bias.numpy())
    for t in range(T):
        for j in range(k):
            e = int(ids[t, j])
            if 4 <= e < 8:
                g, u = wg[e].double() @ x[t].double(), wu[e].double() @ x[t].double()
                exp[t] += float(w[t, j]) * (wd[e].double() @ (torch.sigmoid(g) * g * u))
    torch.testing.assert_close(parts[2].double(), exp, rtol=2e-3, atol=2e-3)


def test_given_routing_closed_forms(rng):
    """A routing given instead of logits (the step after an expert-parallel
    dispatch): (1) the router's own ids and weights reproduce the logits path
    bitwise, whole layer and shard; (2) ids marked -1 or naming another
    shard's experts add nothing, exactly as a weight of 0 would; (3) arbitrary,
    unnormalised weights give the dense fp64 per-token sum w * MLP over the
    in-range choices (a renormalisation or a dropped weight fails it)."""
    T, H, I, E, k = 29, 32, 16, 8, 3
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float16))
    logits = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32))
    wg = torch.from_numpy((rng.standard_normal((E, I, H)) * 0.2).astype(np.float16))
    wu = torch.from_numpy((rng.standard_normal((E, I, H)) * 0.2).astype(np.float16))
    wd = torch.from_numpy((rng.standard_normal((E, H, I)) * 0.2).astype(np.float16))
    ids, w = route_topk(logits.numpy(), k)
    full = fused_moe_forward(x, logits, wg, wu, wd, k)
    assert torch.equal(fused_moe_forward(x, None, wg, wu, wd, k, routing=(ids, w)), full)
    b, n = 2, 4
    shard = fused_moe_forward(x, logits, wg[b:b + n], wu[b:b + n], wd[b:b + n], k, expert_range=(b, n))
    given = fused_moe_forward(x, None, wg[b:b + n], wu[b:b + n], wd[b:b + n], k, expert_range=(b, n),
                              routing=(ids, w))
    assert torch.equal(given, shard)
    # out-of-range marks == zero weights
    ids2 = ids.copy()
    drop = rng.random(ids.shape) < 0.3
    ids2[drop] = -1
    w0 = np.where(drop, np.float32(0), w).astype(np.float32)
    a = fused_moe_forward(x, None, wg, wu, wd, k, expert_range=(0, E), routing=(ids2, w))
    z = fused_moe_forward(x, None, wg, wu, wd, k, routing=(ids, w0))
    assert torch.equal(a, z)
    # unnormalised weights, ids across a wider routing (E_total = 12)
    ids3 = rng.integers(-1, 12, size=(T, k)).astype(np.int32)
    w3 = (rng.random((T, k)) * 3).astype(np.float32)
    got = fused_moe_forward(x, None, wg[b:b + n], wu[b:b + n], wd[b:b + n], k, expert_range=(b, n),
                            routing=(ids3, w3))
    exp = torch.zeros(T, H, dtype=torch.float64)
    for t in range(T):
        for j in range(k):
            e = int(ids3[t, j])
            if b <= e < b + n:
                g, u = wg[e].double() @ x[t].double(), wu[e].double() @ x[t].double()
                exp[t] += float(w3[t, j]) * (wd[e].double() @ (torch.sigmoid(g) * g * u))
    torch.testing.assert_close(got.double(), exp, rtol=2e-3, atol=2e-3)
    with pytest.raises(ValueError):
        fused_moe_forward(x, None, wg, wu, wd, k, routing=(ids3, w3))  # out-of-range ids need a range
