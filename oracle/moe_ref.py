"""CPU restatement of the fused-MoE path (test infrastructure; see package doc).

Arrays are numpy for the integer/index work and torch-CPU float32 for the
expert GEMMs (the reference oracle itself is a torch fp32 loop,
problem_detail.json:50).  Nothing here touches a GPU.
"""

from __future__ import annotations

import numpy as np
import torch

LOG2E = 1.4426950408889634


# ---------------------------------------------------------------------------
# router GEMM (build-defined; the reference has no router, problem_detail.json
# :18 and :30): logits = x . w_router^T with fp16 inputs and fp32 accumulation
# ---------------------------------------------------------------------------
def router_logits(x, w_router) -> np.ndarray:
    """fp32 [T, E] logits of fp16 x [T, H] and w_router [E, H]."""
    xf = _as_t(x).float()
    wf = _as_t(w_router).float()
    return (xf @ wf.t()).numpy().astype(np.float32)


# ---------------------------------------------------------------------------
# routing: softmax -> top-k -> renormalise  (build-defined; the reference has no
# router, problem_detail.json:18 and :30)
# ---------------------------------------------------------------------------
def route_topk(logits: np.ndarray, k: int, bias: np.ndarray | None = None):
    """Return (ids int32 [T,k], weights float32 [T,k]).

    Selection ranks the fp32 biased logits ``v = logits + bias`` in descending
    order, ties broken towards the lower expert index.  Softmax is monotone, so
    this is the top-k of ``softmax(v)``; ranking the logits themselves keeps
    exp rounding from creating or breaking ties.  Weights are the softmax
    probabilities of the selected experts renormalised to sum to one, summed
    in selection order.
    """
    v = np.asarray(logits, dtype=np.float32)
    if bias is not None:
        v = (v + np.asarray(bias, dtype=np.float32)[None, :]).astype(np.float32)
    T, E = v.shape
    if not 1 <= k <= E:
        raise ValueError(f"top_k={k} outside [1, {E}]")
    # stable sort of -v: equal values keep ascending expert order
    order = np.argsort(-v, axis=1, kind="stable")
    ids = order[:, :k].astype(np.int32)
    m = v.max(axis=1, keepdims=True)
    ex = np.exp((v - m).astype(np.float32)).astype(np.float32)
    s = ex.sum(axis=1, dtype=np.float32, keepdims=True)
    p = (ex / s).astype(np.float32)
    psel = np.take_along_axis(p, ids.astype(np.int64), axis=1)
    denom = np.zeros((T, 1), dtype=np.float32)
    for j in range(k):  # selection order, float32
        denom = (denom + psel[:, j : j + 1]).astype(np.float32)
    w = (psel / denom).astype(np.float32)
    return ids, w


# ---------------------------------------------------------------------------
# alignment / group metadata (xpuoj_data/remote_bench.py:82-101 semantics)
# ---------------------------------------------------------------------------
def metadata_from_group_sizes(group_sizes, block_m: int = 128):
    """group_offsets, group_padded_offsets (E+1 each) and group_idx_for_bx.

    Restates remote_bench.py:82-101: offsets are [0, cumsum]; each expert is
    padded to a multiple of ``block_m`` rows; experts with no tokens get no
    blocks; block b belongs to the expert whose padded range contains it.
    """
    gs = np.asarray(group_sizes, dtype=np.int64)
    E = gs.shape[0]
    go = np.zeros(E + 1, dtype=np.int64)
    go[1:] = np.cumsum(gs)
    padded = (gs + block_m - 1) // block_m * block_m
    gpo = np.zeros(E + 1, dtype=np.int64)
    gpo[1:] = np.cumsum(padded)
    gidx = np.repeat(np.arange(E, dtype=np.int64), padded // block_m)
    return (go.astype(np.int32), gpo.astype(np.int32), gidx.astype(np.int32))


def align(ids: np.ndarray, num_experts: int, block_m: int):
    """moe_align: expert-sorted, block-padded permutation of routed pairs.

    Pair ``p = t*k + j`` (token t, choice j).  Pairs are grouped by expert in
    ascending expert order; inside an expert they keep ascending pair order.
    Each expert's group is padded to a multiple of ``block_m`` rows with the
    sentinel ``P = T*k``.  Returns a dict of int32 arrays: sorted_pair_ids
    [P_pad], block_expert [P_pad/block_m], group_sizes [E], group_offsets
    [E+1], group_padded_offsets [E+1].
    """
    flat = np.asarray(ids, dtype=np.int64).reshape(-1)
    P = flat.shape[0]
    E = int(num_experts)
    if P and (flat.min() < 0 or flat.max() >= E):
        raise ValueError("expert id out of range")
    gs = np.bincount(flat, minlength=E).astype(np.int64)
    go, gpo, gidx = metadata_from_group_sizes(gs, block_m)
    order = np.argsort(flat, kind="stable")  # by expert, then pair index
    sorted_ids = np.full(int(gpo[-1]), P, dtype=np.int64)
    for e in range(E):
        n = int(gs[e])
        if n:
            sorted_ids[gpo[e] : gpo[e] + n] = order[go[e] : go[e] + n]
    return dict(
        sorted_pair_ids=sorted_ids.astype(np.int32),
        block_expert=gidx,
        group_sizes=gs.astype(np.int32),
        group_offsets=go,
        group_padded_offsets=gpo,
    )


# ---------------------------------------------------------------------------
# pre-routed expert MLP (problem_detail.json:50; race_stress2.py:29-48)
# ---------------------------------------------------------------------------
def silu_mul(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    """sigmoid(g) * g * u in float32 (problem_detail.json:50 form)."""
    return torch.sigmoid(g) * g * u


def _as_t(a, dtype=None):
    t = a if isinstance(a, torch.Tensor) else torch.from_numpy(np.asarray(a))
    t = t.cpu()
    return t if dtype is None else t.to(dtype)


def prerouted_forward(x, w_gate, w_up, w_down, routed, group_sizes, group_offsets,
                      group_padded_offsets, group_idx_for_bx=None, *, out_fp32=False,
                      experts=None):
    """The reference's run_kernel semantics on the CPU.

    out = 0; for every expert e with n = group_sizes[e] > 0 the rows
    x[gpo[e] : gpo[e]+n] (padded order) go through silu(x Wg^T) * (x Wu^T),
    then Wd^T, then are scaled by routed[go[e] : go[e]+n] (raw order) and
    written back as float16 at the padded rows (problem_detail.json:50 notes
    1-6).  Padding rows stay 0.  Weights are converted to float32 one expert
    at a time.  ``experts`` restricts the loop (used for bounded timing
    samples); ``group_idx_for_bx`` is accepted for interface parity.
    """
    x = _as_t(x)
    P, H = x.shape
    out = torch.zeros((P, H), dtype=torch.float32)
    gs = _as_t(group_sizes).tolist()
    go = _as_t(group_offsets).tolist()
    gpo = _as_t(group_padded_offsets).tolist()
    routed = _as_t(routed)
    E = len(gs)
    for e in (range(E) if experts is None else experts):
        n = int(gs[e])
        if n == 0:
            continue
        ps, rs = int(gpo[e]), int(go[e])
        xe = x[ps : ps + n].float()
        g = xe @ _as_t(w_gate[e]).float().T
        u = xe @ _as_t(w_up[e]).float().T
        h = silu_mul(g, u)
        y = h @ _as_t(w_down[e]).float().T
        y = y * routed[rs : rs + n].float().unsqueeze(1)
        out[ps : ps + n] = y
    return out if out_fp32 else out.to(torch.float16)


def prerouted_forward_blocks(x, w_gate, w_up, w_down, routed, group_sizes, group_offsets,
                             group_padded_offsets, group_idx_for_bx, out=None, block_m: int = 128):
    """The reference operator's per-block form (submission.py:1444-1447,
    :1283-1299, :2115): the launch covers nblk = min(len(group_idx_for_bx),
    P // block_m) blocks; block b is expert e = group_idx_for_bx[b], with
    token offset o = b*block_m - gpo[e] and clamp(gs[e] - o, 0, block_m)
    valid rows; valid row i is the SwiGLU MLP of x's row times
    routed[clamp(go[e] + o + i, 0, V - 1)]; the block's other rows are 0.
    A block whose expert lies outside [0, E) is all 0 (the build's rule: the
    reference would read out of bounds).  Rows past the launched blocks keep
    ``out``'s contents (zeros when ``out`` is None).  Returns float16 [P, H].
    With group metadata from ``metadata_from_group_sizes`` this equals
    ``prerouted_forward`` (the problem_detail.json:50 loop)."""
    x = _as_t(x)
    P, H = x.shape
    res = torch.zeros((P, H), dtype=torch.float16) if out is None else _as_t(out).to(torch.float16).clone()
    gs = [int(v) for v in _as_t(group_sizes).tolist()]
    go = [int(v) for v in _as_t(group_offsets).tolist()]
    gpo = [int(v) for v in _as_t(group_padded_offsets).tolist()]
    gidx = [int(v) for v in _as_t(group_idx_for_bx).tolist()]
    routed = _as_t(routed).float()
    V = routed.numel()
    E = len(gs)
    nblk = min(len(gidx), P // block_m)
    wcache = {}
    for b in range(nblk):
        r0 = b * block_m
        blk = torch.zeros((block_m, H), dtype=torch.float32)
        e = gidx[b]
        if 0 <= e < E:
            o = r0 - gpo[e]
            n = max(0, min(block_m, gs[e] - o))
            if n:
                if e not in wcache:
                    wcache[e] = tuple(_as_t(w[e]).float() for w in (w_gate, w_up, w_down))
                wg, wu, wd = wcache[e]
                xe = x[r0 : r0 + n].float()
                h = silu_mul(xe @ wg.T, xe @ wu.T)
                idx = torch.clamp(torch.arange(n) + (go[e] + o), 0, max(V - 1, 0))
                scale = routed[idx] if V else torch.zeros(n)
                blk[:n] = (h @ wd.T) * scale.unsqueeze(1)
        res[r0 : r0 + block_m] = blk.to(torch.float16)
    return res


def gather_rows(x, sorted_pair_ids, top_k: int):
    """Expert-sorted activation rows: row r <- x[sorted_pair_ids[r] // top_k].

    Sentinel rows (id == T*top_k) become zero rows.
    """
    x = _as_t(x)
    T = x.shape[0]
    sp = _as_t(sorted_pair_ids).long()
    P = T * top_k
    valid = sp < P
    tok = torch.where(valid, sp // top_k, torch.zeros_like(sp))
    xs = x[tok].clone()
    xs[~valid] = 0
    return xs


def combine(y_pair: torch.Tensor, T: int, top_k: int) -> torch.Tensor:
    """out[t] = sum_j y_pair[t*k + j] (weights already applied), fp32 sum in
    choice order, returned as float32 [T, H]."""
    y = y_pair.float().reshape(T, top_k, -1)
    acc = torch.zeros_like(y[:, 0])
    for j in range(top_k):
        acc = acc + y[:, j]
    return acc


def fused_moe_forward(x, logits, w_gate, w_up, w_down, top_k: int, bias=None,
                      block_m: int = 128, *, return_aux=False, experts=None, shared=None, expert_range=None,
                      routing=None):
    """Full MoE: route -> align -> gather -> pre-routed MLP -> weighted combine.

    Returns float16 [T, H] (and the routing/alignment intermediates when
    ``return_aux``).  The pre-routed step is exactly ``prerouted_forward`` with
    routed weights taken in sorted-pair order, so the expert math is the
    reference's own loop.  ``shared`` = (w_gate_s [I, H], w_up_s [I, H],
    w_down_s [H, I]) adds an always-on expert: expert E, appended to every
    token as choice k with weight 1 (outside the top-k renormalisation), so
    the routing has k + 1 columns.  ``expert_range`` = (begin, count): an
    expert shard -- routing over all logits columns, weights of experts
    [begin, begin + count) only, and the sum over each token's choices routed
    there (other choices go to an appended all-zero expert with weight 0, which
    adds exactly 0).  ``routing`` = (ids int [T, k], weights float32 [T, k])
    replaces the router (logits and bias are then ignored): the weights are
    used as given, and with ``expert_range`` any id outside the range (another
    shard's expert, or a negative "no choice" mark) adds nothing, as for the
    other shards' choices above (build-defined: the step after an
    expert-parallel dispatch; the reference has no routing, problem_detail.json:18).
    """
    x = _as_t(x)
    T, H = x.shape
    E = int(w_gate.shape[0])
    if routing is not None:
        ids = np.asarray(_as_t(routing[0]).numpy(), dtype=np.int64).astype(np.int32)
        w = np.asarray(_as_t(routing[1]).float().numpy(), dtype=np.float32)
        if ids.shape != (T, top_k) or w.shape != (T, top_k):
            raise ValueError("routing must be ([T, k] ids, [T, k] weights)")
        if expert_range is None and ((ids < 0) | (ids >= E)).any():
            raise ValueError("routing ids outside [0, E) need an expert_range")
    else:
        ids, w = route_topk(_as_t(logits).float().numpy(), top_k,
                            None if bias is None else _as_t(bias).float().numpy())
    ids_global = ids
    if expert_range is not None:
        b, n = expert_range
        mine = (ids >= b) & (ids < b + n)
        ids = np.where(mine, ids - b, n).astype(np.int32)
        w = np.where(mine, w, np.float32(0)).astype(np.float32)
        z = lambda t: torch.cat([_as_t(t), torch.zeros_like(_as_t(t)[:1])])
        w_gate, w_up, w_down = z(w_gate), z(w_up), z(w_down)
        E = n + 1
    if shared is not None:
        ids = np.concatenate([ids, np.full((T, 1), E, np.int32)], axis=1)
        w = np.concatenate([w, np.ones((T, 1), np.float32)], axis=1)
        sg, su, sd = (_as_t(a) for a in shared)
        w_gate = torch.cat([_as_t(w_gate), sg[None]])
        w_up = torch.cat([_as_t(w_up), su[None]])
        w_down = torch.cat([_as_t(w_down), sd[None]])
        E, top_k = E + 1, top_k + 1
    al = align(ids, E, block_m)
    sp = al["sorted_pair_ids"]
    P = T * top_k
    xs = gather_rows(x, sp, top_k)
    # routed weights in raw (expert-grouped, unpadded) order
    valid_sorted = sp[sp < P]
    routed = torch.from_numpy(w.reshape(-1)[valid_sorted].copy())
    y_sorted = prerouted_forward(xs, w_gate, w_up, w_down, routed, al["group_sizes"],
                                 al["group_offsets"], al["group_padded_offsets"],
                                 out_fp32=True, experts=experts)
    y_pair = torch.zeros((P, H), dtype=torch.float32)
    vs = torch.from_numpy(sp.astype(np.int64))
    mask = vs < P
    y_pair[vs[mask]] = y_sorted[mask]
    out = combine(y_pair, T, top_k).to(torch.float16)
    if return_aux:
        return out, dict(ids=ids if expert_range is None else ids_global, weights=w, **al)
    return out


# ---------------------------------------------------------------------------
# W8A8 (build-defined; semantics follow xpuoj_data/submission_v321_int8_fixed.py
# :160-200 rounding and :311-325 per-(row, 128-column) intermediate scales)
# ---------------------------------------------------------------------------
def _round_half_away_fp32(v: np.ndarray) -> np.ndarray:
    """trunc(v + (v >= 0 ? 0.5 : -0.5)) with the add done in float32, as in
    submission_v321_int8_fixed.py:184-198."""
    v = v.astype(np.float32)
    half = np.where(v >= 0, np.float32(0.5), np.float32(-0.5)).astype(np.float32)
    return np.trunc((v + half).astype(np.float32))


def quantize_rows_int8(w):
    """Per-row symmetric int8: amax = max|w|, scale = amax/127,
    q = clamp(round_half_away(w * (127/amax)), -127, 127).  Rows with amax == 0
    quantise to 0 with scale 0.  Returns (q int8 [..., K], scale float32 [...])."""
    a = _as_t(w).float().numpy().astype(np.float32)
    amax = np.abs(a).max(axis=-1).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(amax > 0, np.float32(127.0) / amax, np.float32(0.0)).astype(np.float32)
    scale = (amax / np.float32(127.0)).astype(np.float32)
    v = (a * inv[..., None]).astype(np.float32)
    q = np.clip(_round_half_away_fp32(v), -127, 127).astype(np.int8)
    return q, scale


def fp8_e4m3_codes(v) -> np.ndarray:
    """OCP fp8 e4m3 codes (uint8) of float32 values, round to nearest even,
    saturating at +-448: normals round the fp32 mantissa to 3 bits (carry into
    the exponent) and rebias the exponent 127 -> 7; below 2**-6 the code is
    the nearest-even multiple of 2**-9."""
    v = np.asarray(v, dtype=np.float32)
    u = v.view(np.uint32)
    sign = ((u >> 24) & 0x80).astype(np.uint32)
    a = np.abs(v)
    au = a.view(np.uint32).astype(np.uint64)
    normal = ((au + 0x7FFFF + ((au >> 20) & 1)) >> 20).astype(np.int64) - (120 << 3)
    normal = np.minimum(normal, 0x7E)
    sub = np.rint((a * np.float32(512.0)).astype(np.float32)).astype(np.int64)
    code = np.where(a >= np.float32(0.015625), normal, sub)
    return (sign | code.astype(np.uint32)).astype(np.uint8)


def _fp8_table() -> np.ndarray:
    """float64 value of each of the 256 e4m3 codes (0x7F / 0xFF are NaN)."""
    c = np.arange(256)
    e, m = (c >> 3) & 0xF, c & 7
    mag = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1 + m / 8.0) * 2.0 ** (e - 7.0))
    mag = np.where((e == 15) & (m == 7), np.nan, mag)
    return np.where(c & 0x80, -mag, mag)


FP8_E4M3_VALUES = _fp8_table()


def pow2_scales(amax) -> np.ndarray:
    """Power-of-two fp8 block scales: 2**j with the smallest j >= -127 such
    that amax <= 448 * 2**j (amax = m * 2**e, m in [1, 2): j = e - 8 + [m >
    1.75]); 0 where amax == 0.  float32 (2**-127 is a denormal)."""
    amax = np.asarray(amax, dtype=np.float32)
    m, e = np.frexp(amax.astype(np.float64))       # amax = m * 2**e, m in [0.5, 1)
    j = (e - 1) - 8 + (2 * m > 1.75)
    j = np.maximum(j, -127)
    return np.where(amax > 0, np.ldexp(1.0, j), 0.0).astype(np.float32)


def quantize_rows_fp8(w, pow2: bool = False):
    """Per-row fp8 e4m3: amax = max|w|, scale = amax/448, code =
    e4m3(w * (448/amax)) (product rounded to fp32, then to e4m3 nearest even).
    With ``pow2`` the scale is ``pow2_scales(amax)`` and the code e4m3(w /
    scale), an exact scaling.  Rows with amax == 0 give code 0 and scale 0.
    Returns (codes uint8 [..., K], scale float32 [...])."""
    a = _as_t(w).float().numpy().astype(np.float32)
    amax = np.abs(a).max(axis=-1).astype(np.float32)
    if pow2:
        scale = pow2_scales(amax)
        with np.errstate(divide="ignore"):
            inv = np.where(scale > 0, 1.0 / scale.astype(np.float64), 0.0).astype(np.float32)
        return fp8_e4m3_codes((a * inv[..., None]).astype(np.float32)), scale
    with np.errstate(divide="ignore"):
        inv = np.where(amax > 0, np.float32(448.0) / amax, np.float32(0.0)).astype(np.float32)
    scale = (amax / np.float32(448.0)).astype(np.float32)
    return fp8_e4m3_codes((a * inv[..., None]).astype(np.float32)), scale


def _int_matmul(a: np.ndarray, b_t: np.ndarray) -> np.ndarray:
    """Exact int8 x int8 -> integer product a @ b_t.T (float64 BLAS is exact
    here: |sum| <= 127*127*K < 2**53)."""
    return np.rint(a.astype(np.float64) @ b_t.astype(np.float64).T).astype(np.int64)


def _exact_matmul(a: np.ndarray, b_t: np.ndarray) -> np.ndarray:
    """a @ b_t.T in float64 for 8-bit operand values (int8 or e4m3): exact,
    as the integer or 2**-18-grid sums stay below 2**53 ulps."""
    return np.asarray(a, dtype=np.float64) @ np.asarray(b_t, dtype=np.float64).T


def w8a8_forward(x, logits, wq_gate, s_gate, wq_up, s_up, wq_down, s_down, top_k: int,
                 bias=None, block_m: int = 128, *, scale_block: int = 128, experts=None, fmt="int8"):
    """W8A8 fused MoE on the CPU (the GPU path's arithmetic contract).

    x rows are quantised per token; gate/up are exact 8-bit GEMMs dequantised
    as (acc * s_x[t]) * s_w[e, n]; h = silu(g) * u.  Pairs are combined in
    choice order.

    fmt "int8" (wq_* int8): h is rounded to fp16 and quantised per row, like
    x (one scale per routed row, over all I columns); the down GEMM is one
    exact integer product over the whole of K, dequantised as
    ((acc * s_h[row]) * s_down[e, n]) * routing weight.

    fmt "fp8" (wq_* uint8, OCP e4m3 codes, whose products are exact in
    float64: 8 significant bits each, sums of at most 2**14 terms between
    2**-18 and 2**18; the GPU sums them in fp32): h is quantised per (row,
    ``scale_block`` columns) with power-of-two scales (``pow2_scales``), which
    the GPU's f8 MFMA applies itself; the down GEMM accumulates each column
    block's exact product times its row scale, in block order, then applies
    s_down[e, n] and the routing weight.
    """
    if fmt == "fp8":
        quant = quantize_rows_fp8
        val = lambda c: FP8_E4M3_VALUES[np.asarray(c, dtype=np.uint8)]
    else:
        quant = quantize_rows_int8
        val = lambda c: np.asarray(c)
    x = _as_t(x)
    T, H = x.shape
    E, I, _ = wq_gate.shape
    ids, w = route_topk(_as_t(logits).float().numpy(), top_k,
                        None if bias is None else _as_t(bias).float().numpy())
    al = align(ids, E, block_m)
    xq, sx = quant(x)
    xq = val(xq)
    P = T * top_k
    gs, go = al["group_sizes"], al["group_offsets"]
    order = al["sorted_pair_ids"]
    y_pair = np.zeros((P, H), dtype=np.float32)
    wflat = w.reshape(-1)
    for e in (range(E) if experts is None else experts):
        n = int(gs[e])
        if n == 0:
            continue
        pairs = order[al["group_padded_offsets"][e] : al["group_padded_offsets"][e] + n].astype(np.int64)
        tok = pairs // top_k
        a = xq[tok]
        g = (_exact_matmul(a, val(wq_gate[e])).astype(np.float32) * sx[tok][:, None]).astype(np.float32)
        g = (g * s_gate[e][None, :]).astype(np.float32)
        u = (_exact_matmul(a, val(wq_up[e])).astype(np.float32) * sx[tok][:, None]).astype(np.float32)
        u = (u * s_up[e][None, :]).astype(np.float32)
        h = silu_mul(torch.from_numpy(g), torch.from_numpy(u)).numpy().astype(np.float32)
        wd = val(wq_down[e])
        if fmt == "fp8":
            nb = I // scale_block
            hq, sh = quantize_rows_fp8(h.reshape(n, nb, scale_block), pow2=True)  # [n, nb, 128], [n, nb]
            hq = val(hq)
            acc = np.zeros((n, H), dtype=np.float32)
            for b in range(nb):
                part = _exact_matmul(hq[:, b, :], wd[:, b * scale_block:(b + 1) * scale_block])
                acc = (acc + part.astype(np.float32) * sh[:, b : b + 1]).astype(np.float32)
        else:
            hq, sh = quantize_rows_int8(h.astype(np.float16))  # [n, I], [n]
            acc = (_exact_matmul(hq, wd).astype(np.float32) * sh[:, None]).astype(np.float32)
        y = (acc * s_down[e][None, :]).astype(np.float32)
        y = (y * wflat[pairs][:, None]).astype(np.float32)
        y_pair[pairs] = y
    out = combine(torch.from_numpy(y_pair), T, top_k).to(torch.float16)
    return out
