"""Python host side of the fused-MoE operator.

``run_kernel`` keeps the reference's 10-argument operator interface
(problem_detail.json:24; 初审材料/源代码/submission.py:2098-2184): same names,
same argument meaning, ``out`` written in place, no synchronisation, a
workspace cached per (device, stream) and grown on demand, like
submission.py:2081-2095.  ``fused_moe`` is the north-star entry point
(hidden_states, router_logits, w_gate, w_up, w_down, top_k -> output).

Every function validates dtype / shape / contiguity / device on the host and
then calls the HIP library through its C ABI on torch's current stream.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from ._lib import MoeError, check, lib

__all__ = [
    "run_kernel", "fused_moe", "route_topk", "route_hidden", "moe_align", "quantize_rows_w8",
    "W8A8Weights", "quantize_w8a8_weights", "fused_workspace_bytes", "pick_block_m", "MoeError",
]

_WORKSPACE: dict = {}
_CAPTURED_RETIRED: list = []  # replaced buffers that captured graphs may still write


def _ptr(t):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _stream(dev: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _need(t: torch.Tensor, name: str, dtypes, ndim: int | None = None, device=None, strided_ok=False):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.dtype not in dtypes:
        raise TypeError(f"{name}: dtype {t.dtype} not in {dtypes}")
    if ndim is not None and t.dim() != ndim:
        raise ValueError(f"{name}: expected {ndim}-D, got shape {tuple(t.shape)}")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")
    if device is not None and t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")
    if strided_ok and t.dim() in (2, 3) and t.numel() > 0:
        # [.., N, K] with unit element stride, rows ld >= K apart and, for a
        # stack, experts es >= N * ld apart (views of wider or fused tensors)
        st, N, K = t.stride(), t.shape[-2], t.shape[-1]
        if st[-1] != 1 or st[-2] < K or (t.dim() == 3 and t.shape[0] > 1 and st[0] < N * st[-2]):
            raise ValueError(f"{name}: strides {tuple(st)} overlap rows or split them")
    elif not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _strides(t) -> tuple[int, int]:
    """(row stride, expert stride) in elements of an [E, N, K] weight stack."""
    es = t.stride(0) if t.shape[0] > 1 else t.shape[1] * t.stride(1)
    return t.stride(1), es


def _workspace(dev: torch.device, key, nbytes: int) -> torch.Tensor:
    """Scratch reused across calls, one per (device, stream, use): calls on
    different streams never share one (they may run concurrently), and a
    buffer is allocated on the stream that uses it, so replacing it by a
    larger one is ordered after that stream's earlier kernels.

    A call captured into a CUDA graph gets a buffer of its own (allocated
    during the capture, cached apart from the eager ones): every replay of the
    graph writes it, so an eager call that needs a larger buffer never frees
    one a graph still uses.  A captured buffer that a later, larger capture
    replaces is kept alive for the life of the process for the same reason.
    Replays of graphs that share a buffer must not overlap."""
    capturing = torch.cuda.is_current_stream_capturing()
    k = (dev.index, torch.cuda.current_stream(dev).cuda_stream, capturing, key)
    buf = _WORKSPACE.get(k)
    if buf is None or buf.numel() < nbytes:
        if buf is not None and capturing:
            _CAPTURED_RETIRED.append(buf)
        buf = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=dev)
        _WORKSPACE[k] = buf
    return buf


# ---------------------------------------------------------------------------
# reference operator interface
# ---------------------------------------------------------------------------
def run_kernel(stacked_expert_tokens, gate_w, up_w, down_w, routed_expert_weights, group_sizes,
               group_offsets, group_padded_offsets, group_idx_for_bx, out) -> None:
    """Pre-routed fused expert MLP, written into ``out`` (fp16 [P, H]).

    For each expert e with n = group_sizes[e] tokens, rows
    [group_padded_offsets[e], +n) of ``stacked_expert_tokens`` go through
    silu(x Wg[e]^T) * (x Wu[e]^T) Wd[e]^T and are scaled by
    routed_expert_weights[group_offsets[e] + i]; every other row of ``out`` is
    written as 0.  Reference: problem_detail.json:50, submission.py:2098-2184.

    Blocks of 128 rows map to experts through ``group_idx_for_bx`` (block b is
    expert group_idx_for_bx[b], submission.py:1444) and the call covers
    min(group_idx_for_bx.numel(), P / 128) blocks (submission.py:2115); rows
    past them are left untouched.  With the harness's metadata
    (remote_bench.py:82-101) that is every row.
    """
    x = stacked_expert_tokens
    _need(x, "stacked_expert_tokens", (torch.float16,), 2)
    dev = x.device
    P, H = x.shape
    _need(gate_w, "gate_w", (torch.float16,), 3, dev)
    E, I, H2 = gate_w.shape
    _need(up_w, "up_w", (torch.float16,), 3, dev)
    _need(down_w, "down_w", (torch.float16,), 3, dev)
    if H2 != H or tuple(up_w.shape) != (E, I, H) or tuple(down_w.shape) != (E, H, I):
        raise ValueError(f"weight shapes {tuple(gate_w.shape)}, {tuple(up_w.shape)}, "
                         f"{tuple(down_w.shape)} do not match x {tuple(x.shape)}")
    _need(routed_expert_weights, "routed_expert_weights", (torch.float32, torch.float16), 1, dev)
    for name, t, n in (("group_sizes", group_sizes, E), ("group_offsets", group_offsets, E + 1),
                       ("group_padded_offsets", group_padded_offsets, E + 1)):
        _need(t, name, (torch.int32,), 1, dev)
        if t.numel() != n:
            raise ValueError(f"{name}: expected {n} entries, got {t.numel()}")
    _need(group_idx_for_bx, "group_idx_for_bx", (torch.int32,), 1, dev)
    _need(out, "out", (torch.float16,), 2, dev)
    if tuple(out.shape) != (P, H):
        raise ValueError(f"out shape {tuple(out.shape)} != {(P, H)}")
    V = routed_expert_weights.numel()
    nblk = group_idx_for_bx.numel()
    L = lib()
    nbytes = L.moe_prerouted_workspace_bytes(P, I)
    # one buffer per (device, stream, capture state), grown on demand
    ws = _workspace(dev, ("prerouted",), nbytes) if P else None
    routed_dtype = 0 if routed_expert_weights.dtype == torch.float32 else 1
    with torch.cuda.device(dev):
        rc = L.moe_run_prerouted(
            _ptr(x), _ptr(gate_w), _ptr(up_w), _ptr(down_w), _ptr(routed_expert_weights),
            routed_dtype, _ptr(group_sizes), _ptr(group_offsets), _ptr(group_padded_offsets),
            _ptr(group_idx_for_bx), _ptr(out), P, H, I, E, V, nblk, _ptr(ws),
            0 if ws is None else ws.numel(), _stream(dev))
    check(rc, "run_kernel")


# ---------------------------------------------------------------------------
# routing / alignment building blocks
# ---------------------------------------------------------------------------
def route_topk(router_logits: torch.Tensor, top_k: int, expert_bias: torch.Tensor | None = None):
    """(ids int32 [T,k], weights fp32 [T,k]): top-k of logits(+bias), ties to
    the lower expert index, softmax weights renormalised over the k."""
    _need(router_logits, "router_logits", (torch.float32,), 2)
    dev = router_logits.device
    T, E = router_logits.shape
    if expert_bias is not None:
        _need(expert_bias, "expert_bias", (torch.float32,), 1, dev)
        if expert_bias.numel() != E:
            raise ValueError("expert_bias must have E entries")
    ids = torch.empty((T, top_k), dtype=torch.int32, device=dev)
    w = torch.empty((T, top_k), dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        rc = lib().moe_route_topk(_ptr(router_logits), _ptr(expert_bias), T, E, top_k, _ptr(ids),
                                  _ptr(w), _stream(dev))
    check(rc, "route_topk")
    return ids, w


def route_hidden(hidden_states: torch.Tensor, router_weight: torch.Tensor, top_k: int,
                 expert_bias: torch.Tensor | None = None, return_logits: bool = False):
    """Router GEMM + routing: logits = hidden_states . router_weight^T (fp16
    inputs, fp32 accumulation), then route_topk's softmax / top-k /
    renormalisation.  Returns (ids, weights) or (ids, weights, logits)."""
    x, wr = hidden_states, router_weight
    _need(x, "hidden_states", (torch.float16,), 2)
    dev = x.device
    _need(wr, "router_weight", (torch.float16,), 2, dev)
    T, H = x.shape
    E = wr.shape[0]
    if wr.shape[1] != H:
        raise ValueError("router_weight must be [E, H]")
    if expert_bias is not None:
        _need(expert_bias, "expert_bias", (torch.float32,), 1, dev)
        if expert_bias.numel() != E:
            raise ValueError("expert_bias must have E entries")
    L = lib()
    ids = torch.empty((T, top_k), dtype=torch.int32, device=dev)
    w = torch.empty((T, top_k), dtype=torch.float32, device=dev)
    logits = torch.empty((T, E), dtype=torch.float32, device=dev) if return_logits else None
    nbytes = int(L.moe_router_workspace_bytes(T, H, E))
    ws = _workspace(dev, ("router",), nbytes) if nbytes else None
    with torch.cuda.device(dev):
        rc = L.moe_route_hidden(_ptr(x), _ptr(wr), _ptr(expert_bias), T, H, E, top_k, _ptr(ids), _ptr(w),
                                _ptr(logits), _ptr(ws), 0 if ws is None else ws.numel(), _stream(dev))
    check(rc, "route_hidden")
    return (ids, w, logits) if return_logits else (ids, w)


def moe_align(topk_ids: torch.Tensor, num_experts: int, block_m: int, many_workgroups: bool = True):
    """Expert-sorted, block-padded pair permutation (see include/moe_gfx950.h).

    Returns a dict of device int32 tensors sized to the capacity bound;
    ``group_padded_offsets[E]`` is the number of rows actually used.  With
    ``many_workgroups`` a large batch is aligned by several workgroups (a
    scratch buffer is allocated for it); the result is identical either way.
    """
    _need(topk_ids, "topk_ids", (torch.int32,), 2)
    dev = topk_ids.device
    T, k = topk_ids.shape
    L = lib()
    cap = L.moe_align_capacity_rows(T, k, num_experts, block_m)
    sorted_ids = torch.empty(max(cap, 1), dtype=torch.int32, device=dev)
    bexp = torch.empty(max(cap // block_m, 1), dtype=torch.int32, device=dev)
    gs = torch.empty(num_experts, dtype=torch.int32, device=dev)
    go = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    gpo = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    nscratch = int(L.moe_align_scratch_bytes(T, k, num_experts)) if many_workgroups else 0
    scratch = torch.empty(max(nscratch, 16), dtype=torch.uint8, device=dev) if nscratch else None
    with torch.cuda.device(dev):
        rc = L.moe_align(_ptr(topk_ids), T, k, num_experts, block_m, _ptr(sorted_ids), _ptr(bexp),
                         _ptr(gs), _ptr(go), _ptr(gpo), _ptr(scratch) if nscratch else None, nscratch,
                         _stream(dev))
    check(rc, "moe_align")
    return dict(sorted_pair_ids=sorted_ids, block_expert=bexp, group_sizes=gs, group_offsets=go,
                group_padded_offsets=gpo)


def pick_block_m(T: int, E: int, top_k: int) -> int:
    return int(lib().moe_pick_block_m(T, E, top_k))


def fused_workspace_bytes(T, H, I, E, top_k, block_m=0, w8a8=False) -> int:
    """Workspace of fused_moe; w8a8: False (fp16), True / "int8", or "fp8"."""
    flag = 0 if not w8a8 else (2 if w8a8 == "fp8" else 1)
    return int(lib().moe_fused_workspace_bytes(T, H, I, E, top_k, block_m, flag))


# ---------------------------------------------------------------------------
# W8A8
# ---------------------------------------------------------------------------
def quantize_rows_w8(w: torch.Tensor, fmt: str = "int8"):
    """Per-row 8-bit quantisation of an fp16 tensor [..., K]: (q [..., K],
    scale fp32 [...]).  fmt "int8": q int8, scale = max|row|/127; "fp8": q
    torch.float8_e4m3fn (OCP e4m3, round to nearest even), scale = max|row|/448."""
    _need(w, "w", (torch.float16,))
    if fmt not in ("int8", "fp8"):
        raise ValueError(f"fmt must be 'int8' or 'fp8', got {fmt!r}")
    dev = w.device
    K = w.shape[-1]
    R = w.numel() // K if K else 0
    q = torch.empty(w.shape, dtype=torch.int8 if fmt == "int8" else torch.float8_e4m3fn, device=dev)
    s = torch.empty(w.shape[:-1], dtype=torch.float32, device=dev)
    fn = lib().moe_quantize_rows_w8 if fmt == "int8" else lib().moe_quantize_rows_fp8
    with torch.cuda.device(dev):
        rc = fn(_ptr(w), R, K, _ptr(q), _ptr(s), _stream(dev))
    check(rc, "quantize_rows_" + fmt)
    return q, s


@dataclass
class W8A8Weights:
    """Per-output-row 8-bit expert weights with fp32 scales: int8 codes, or
    fp8 e4m3 codes (torch.float8_e4m3fn) for the fp8 variant."""
    q_gate: torch.Tensor   # int8 | float8_e4m3fn [E, I, H]
    s_gate: torch.Tensor   # fp32 [E, I]
    q_up: torch.Tensor
    s_up: torch.Tensor
    q_down: torch.Tensor   # int8 | float8_e4m3fn [E, H, I]
    s_down: torch.Tensor   # fp32 [E, H]

    @property
    def fmt(self) -> str:
        return "fp8" if self.q_gate.dtype == torch.float8_e4m3fn else "int8"


def quantize_w8a8_weights(w_gate, w_up, w_down, fmt: str = "int8") -> W8A8Weights:
    qg, sg = quantize_rows_w8(w_gate, fmt)
    qu, su = quantize_rows_w8(w_up, fmt)
    qd, sd = quantize_rows_w8(w_down, fmt)
    return W8A8Weights(qg, sg, qu, su, qd, sd)


# ---------------------------------------------------------------------------
# north-star entry point
# ---------------------------------------------------------------------------
def fused_moe_routed(hidden_states, topk_ids, topk_weights, w_gate, w_up, w_down, *, expert_begin: int = 0,
                     num_experts: int | None = None, block_m: int = 0, out=None, stage_events=None):
    """The fused expert MLPs and weighted combine from a routing computed
    elsewhere: what one GPU runs after an expert-parallel dispatch (the
    received token rows, their global top-k ids and weights), or any caller
    whose router this library does not implement.  hidden_states fp16 [T, H],
    topk_ids int32 [T, k], topk_weights fp32 [T, k] (used as given, not
    renormalised), w_gate/w_up fp16 [E, I, H] and w_down fp16 [E, H, I] for
    experts [expert_begin, expert_begin + E).  Returns fp16 [T, H]: each token's
    sum, in choice order, of weight * expert MLP over its choices in that
    range; other ids (another GPU's experts, or -1 for "no choice") add
    nothing.  ``num_experts`` (the routing's expert count, default
    expert_begin + E) only sets the block rows the library picks."""
    x = hidden_states
    _need(x, "hidden_states", (torch.float16,), 2)
    dev = x.device
    T, H = x.shape
    _need(topk_ids, "topk_ids", (torch.int32,), 2, dev)
    _need(topk_weights, "topk_weights", (torch.float32,), 2, dev)
    if topk_ids.shape[0] != T or tuple(topk_weights.shape) != tuple(topk_ids.shape):
        raise ValueError("topk_ids and topk_weights must both be [T, k]")
    k = topk_ids.shape[1]
    for name, t in (("w_gate", w_gate), ("w_up", w_up), ("w_down", w_down)):
        _need(t, name, (torch.float16,), 3, dev)
    E, I = w_gate.shape[0], w_gate.shape[1]
    if tuple(w_gate.shape) != (E, I, H) or tuple(w_up.shape) != (E, I, H) or tuple(w_down.shape) != (E, H, I):
        raise ValueError("expert weight shapes do not match [E,I,H]/[E,I,H]/[E,H,I]")
    E_total = expert_begin + E if num_experts is None else int(num_experts)
    if expert_begin < 0 or expert_begin + E > E_total:
        raise ValueError(f"experts [{expert_begin}, {expert_begin + E}) outside the {E_total} routed experts")
    if out is None:
        out = torch.empty((T, H), dtype=torch.float16, device=dev)
    else:
        _need(out, "out", (torch.float16,), 2, dev)
        if tuple(out.shape) != (T, H):
            raise ValueError("out shape mismatch")
    L = lib()
    ws = _workspace(dev, ("fused", None),
                    L.moe_fused_routed_workspace_bytes(T, H, I, E_total, k, E, block_m))
    with torch.cuda.device(dev):
        rc = L.moe_fused_forward_routed(_ptr(x), _ptr(topk_ids), _ptr(topk_weights), _ptr(w_gate), _ptr(w_up),
                                        _ptr(w_down), _ptr(out), T, H, I, E_total, k, expert_begin, E, block_m,
                                        _ptr(ws), ws.numel(), _stream(dev), stage_events)
    check(rc, "fused_moe_routed")
    return out


def fused_moe(hidden_states, router_logits, w_gate, w_up, w_down, top_k: int, *,
              expert_bias=None, w8a8: W8A8Weights | None = None, block_m: int = 0, out=None,
              return_routing: bool = False, router_weight=None, shared_expert=None, expert_range=None):
    """Full MoE FFN: softmax/top-k/renormalise routing, expert SwiGLU MLPs,
    routing-weighted combine.  hidden_states fp16 [T, H], router_logits fp32
    [T, E], w_gate/w_up fp16 [E, I, H], w_down fp16 [E, H, I] (or ``w8a8``
    quantised weights, int8 or fp8, in which case w_gate/w_up/w_down may be
    None).
    With ``router_weight`` (fp16 [E, H]) and router_logits None (fp16 path
    only), the logits are computed in the same call by the router GEMM.
    ``shared_expert`` = (w_gate_s [I, H], w_up_s [I, H], w_down_s [H, I]) fp16
    adds an always-on expert with weight 1 in the same launches (fp16 path);
    the returned routing then has k + 1 columns, the last being (E, 1.0).
    fp16 weights may be strided views (rows and experts apart, e.g. the two
    halves of a fused [E, 2I, H] gate/up tensor): w_gate and w_up share their
    strides, the shared expert's rows use the routed experts' row strides.
    ``expert_range`` = (begin, count): one expert-parallel shard -- the logits
    cover all experts, the (dense fp16) weights only experts [begin, begin +
    count), and the result is this shard's partial sum (the shards' results
    add up to the full layer); the routing returned is the global one.
    Returns fp16 [T, H] (and (ids, weights) when ``return_routing``)."""
    x = hidden_states
    _need(x, "hidden_states", (torch.float16,), 2)
    dev = x.device
    T, H = x.shape
    if router_weight is not None:
        if router_logits is not None:
            raise ValueError("give router_logits or router_weight, not both")
        if w8a8 is not None:
            raise ValueError("router_weight is supported on the fp16 path")
        _need(router_weight, "router_weight", (torch.float16,), 2, dev)
        E = router_weight.shape[0]
        if router_weight.shape[1] != H:
            raise ValueError("router_weight must be [E, H]")
    else:
        _need(router_logits, "router_logits", (torch.float32,), 2, dev)
        E = router_logits.shape[1]
        if router_logits.shape[0] != T:
            raise ValueError("router_logits rows != tokens")
    E_route = E
    if expert_range is not None:
        if router_weight is not None or w8a8 is not None or shared_expert is not None:
            raise ValueError("expert_range takes router_logits and fp16 weights, without a shared expert")
        e_begin, E = (int(v) for v in expert_range)
        if e_begin < 0 or E < 1 or e_begin + E > E_route:
            raise ValueError(f"expert_range {expert_range} outside the {E_route} routed experts")
    if w8a8 is None:
        for name, t in (("w_gate", w_gate), ("w_up", w_up), ("w_down", w_down)):
            _need(t, name, (torch.float16,), 3, dev, strided_ok=True)
        if _strides(w_gate) != _strides(w_up):
            raise ValueError("w_gate and w_up must have the same strides")
        I = w_gate.shape[1]
        if tuple(w_gate.shape) != (E, I, H) or tuple(w_up.shape) != (E, I, H) or \
                tuple(w_down.shape) != (E, H, I):
            raise ValueError("expert weight shapes do not match [E,I,H]/[E,I,H]/[E,H,I]")
    else:
        q = w8a8
        qdt = q.q_gate.dtype
        if qdt not in (torch.int8, torch.float8_e4m3fn):
            raise TypeError(f"q_gate: dtype {qdt} is neither int8 nor float8_e4m3fn")
        _need(q.q_gate, "q_gate", (qdt,), 3, dev)
        _need(q.q_up, "q_up", (qdt,), 3, dev)
        _need(q.q_down, "q_down", (qdt,), 3, dev)
        for name, t in (("s_gate", q.s_gate), ("s_up", q.s_up), ("s_down", q.s_down)):
            _need(t, name, (torch.float32,), 2, dev)
        I = q.q_gate.shape[1]
        if tuple(q.q_gate.shape) != (E, I, H) or tuple(q.q_up.shape) != (E, I, H) or \
                tuple(q.q_down.shape) != (E, H, I) or tuple(q.s_gate.shape) != (E, I) or \
                tuple(q.s_up.shape) != (E, I) or tuple(q.s_down.shape) != (E, H):
            raise ValueError("W8A8 weight/scale shapes do not match")
    if shared_expert is not None:
        if w8a8 is not None:
            raise ValueError("shared_expert is supported on the fp16 path")
        if len(shared_expert) != 3:
            raise ValueError("shared_expert is (w_gate, w_up, w_down)")
        for name, t in zip(("w_gate_shared", "w_up_shared", "w_down_shared"), shared_expert):
            _need(t, name, (torch.float16,), 2, dev, strided_ok=True)
        sg_, su_, sd_ = shared_expert
        if tuple(sg_.shape) != (I, H) or tuple(su_.shape) != (I, H) or tuple(sd_.shape) != (H, I):
            raise ValueError("shared expert shapes do not match [I,H]/[I,H]/[H,I]")
        if sg_.stride(0) != w_gate.stride(1) or su_.stride(0) != w_up.stride(1) or sd_.stride(0) != w_down.stride(1):
            raise ValueError("shared expert rows must use the routed experts' row strides")
    if expert_bias is not None:
        _need(expert_bias, "expert_bias", (torch.float32,), 1, dev)
        if expert_bias.numel() != E_route:
            raise ValueError("expert_bias must have E entries")
    if out is None:
        out = torch.empty((T, H), dtype=torch.float16, device=dev)
    else:
        _need(out, "out", (torch.float16,), 2, dev)
        if tuple(out.shape) != (T, H):
            raise ValueError("out shape mismatch")
    L = lib()
    if expert_range is not None:
        if not (w_gate.is_contiguous() and w_up.is_contiguous() and w_down.is_contiguous()):
            raise ValueError("expert_range takes dense weights")
        bm = block_m  # 0: the library picks
        ws = _workspace(dev, ("fused", None), L.moe_fused_shard_workspace_bytes(T, H, I, E_route, top_k, E, bm))
        ids = torch.empty((T, top_k), dtype=torch.int32, device=dev) if return_routing else None
        wts = torch.empty((T, top_k), dtype=torch.float32, device=dev) if return_routing else None
        with torch.cuda.device(dev):
            rc = L.moe_fused_forward_shard(_ptr(x), _ptr(router_logits), _ptr(expert_bias), _ptr(w_gate),
                                           _ptr(w_up), _ptr(w_down), _ptr(out), T, H, I, E_route, top_k, e_begin, E,
                                           bm, _ptr(ws), ws.numel(), _ptr(ids), _ptr(wts), _stream(dev), None)
        check(rc, "fused_moe")
        return (out, (ids, wts)) if return_routing else out
    ncol = top_k + (shared_expert is not None)
    bm = block_m  # 0: the library picks the block rows (and a 256-row padding where that is faster)
    strided = w8a8 is None and not (w_gate.is_contiguous() and w_up.is_contiguous() and w_down.is_contiguous())
    if strided:
        wstr = (ctypes.c_int64 * 4)(*_strides(w_gate), *_strides(w_down))
        nbytes = L.moe_fused_ex_workspace_bytes(T, H, I, E, top_k, bm, int(shared_expert is not None),
                                                int(router_weight is not None))
    elif shared_expert is not None:
        nbytes = L.moe_fused_shared_workspace_bytes(T, H, I, E, top_k, bm)
    elif router_weight is not None:
        nbytes = L.moe_fused_hidden_workspace_bytes(T, H, I, E, top_k, bm)
    else:
        nbytes = L.moe_fused_workspace_bytes(T, H, I, E, top_k, bm, 0 if w8a8 is None else (2 if w8a8.fmt == "fp8" else 1))
    ws = _workspace(dev, ("fused", None if w8a8 is None else w8a8.fmt), nbytes)
    ids = torch.empty((T, ncol), dtype=torch.int32, device=dev) if return_routing else None
    wts = torch.empty((T, ncol), dtype=torch.float32, device=dev) if return_routing else None
    with torch.cuda.device(dev):
        if strided:
            sh = shared_expert if shared_expert is not None else (None, None, None)
            rc = L.moe_fused_forward_ex(
                _ptr(x), _ptr(router_logits), _ptr(router_weight), _ptr(expert_bias), _ptr(w_gate), _ptr(w_up),
                _ptr(w_down), _ptr(sh[0]), _ptr(sh[1]), _ptr(sh[2]), wstr, _ptr(out), T, H, I,
                E, top_k, bm, _ptr(ws), ws.numel(), _ptr(ids), _ptr(wts), _stream(dev), None)
        elif shared_expert is not None:
            rc = L.moe_fused_forward_shared(
                _ptr(x), _ptr(router_logits), _ptr(router_weight), _ptr(expert_bias), _ptr(w_gate), _ptr(w_up),
                _ptr(w_down), _ptr(sg_), _ptr(su_), _ptr(sd_), _ptr(out), T, H, I, E, top_k, bm, _ptr(ws),
                ws.numel(), _ptr(ids), _ptr(wts), _stream(dev))
        elif router_weight is not None:
            rc = L.moe_fused_forward_hidden(_ptr(x), _ptr(router_weight), _ptr(expert_bias), _ptr(w_gate),
                                            _ptr(w_up), _ptr(w_down), _ptr(out), T, H, I, E, top_k, bm,
                                            _ptr(ws), ws.numel(), _ptr(ids), _ptr(wts), _stream(dev))
        elif w8a8 is None:
            rc = L.moe_fused_forward(_ptr(x), _ptr(router_logits), _ptr(expert_bias), _ptr(w_gate),
                                     _ptr(w_up), _ptr(w_down), _ptr(out), T, H, I, E, top_k, bm,
                                     _ptr(ws), ws.numel(), _ptr(ids), _ptr(wts), _stream(dev))
        elif w8a8.fmt == "fp8":
            q = w8a8
            rc = L.moe_fused_forward_fp8(
                _ptr(x), _ptr(router_logits), _ptr(expert_bias), _ptr(q.q_gate), _ptr(q.s_gate),
                _ptr(q.q_up), _ptr(q.s_up), _ptr(q.q_down), _ptr(q.s_down), _ptr(out), T, H, I, E,
                top_k, bm, _ptr(ws), ws.numel(), _ptr(ids), _ptr(wts), _stream(dev), None)
        else:
            q = w8a8
            rc = L.moe_fused_forward_w8a8(
                _ptr(x), _ptr(router_logits), _ptr(expert_bias), _ptr(q.q_gate), _ptr(q.s_gate),
                _ptr(q.q_up), _ptr(q.s_up), _ptr(q.q_down), _ptr(q.s_down), _ptr(out), T, H, I, E,
                top_k, bm, _ptr(ws), ws.numel(), _ptr(ids), _ptr(wts), _stream(dev))
    check(rc, "fused_moe")
    if return_routing:
        return out, (ids, wts)
    return out
