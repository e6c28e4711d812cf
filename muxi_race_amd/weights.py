"""On-disk format for pre-quantised expert weights (int8 or fp8 e4m3 codes
with fp32 per-row scales), so a model is quantised once and loaded straight
into HBM afterwards.

One safetensors file per MoE layer (a format that executes nothing on load):

    q_gate  int8 | float8_e4m3fn  [E, I, H]     s_gate  float32 [E, I]
    q_up    int8 | float8_e4m3fn  [E, I, H]     s_up    float32 [E, I]
    q_down  int8 | float8_e4m3fn  [E, H, I]     s_down  float32 [E, H]

metadata: {"format": "muxi_race_amd.w8a8", "version": "1", "fmt": "int8"|"fp8",
"experts": E, "hidden": H, "intermediate": I}.  Codes and scales are exactly
what ``quantize_w8a8_weights`` produces (per output row: scale = amax/127 for
int8, amax/448 for fp8), so a loaded file runs bit-identically to a fresh
quantisation.  The reference quantises at run time only
(xpuoj_data/submission_v321_int8_fixed.py:160-227); it has no stored format.
"""
from __future__ import annotations

import torch

from .moe import W8A8Weights

FORMAT = "muxi_race_amd.w8a8"
VERSION = "1"
_NAMES = ("q_gate", "s_gate", "q_up", "s_up", "q_down", "s_down")


def _shapes(E: int, H: int, I: int) -> dict:
    return {"q_gate": (E, I, H), "s_gate": (E, I), "q_up": (E, I, H), "s_up": (E, I),
            "q_down": (E, H, I), "s_down": (E, H)}


def save_w8a8(path: str, weights: W8A8Weights) -> None:
    """Write ``weights`` (on any device) to ``path`` as safetensors."""
    from safetensors.torch import save_file
    E, I, H = weights.q_gate.shape
    tensors = {n: getattr(weights, n).detach().contiguous().cpu() for n in _NAMES}
    for n, shape in _shapes(E, H, I).items():
        if tuple(tensors[n].shape) != shape:
            raise ValueError(f"{n}: shape {tuple(tensors[n].shape)} != {shape}")
    code_dtype = tensors["q_gate"].dtype
    for n in ("q_up", "q_down"):
        if tensors[n].dtype != code_dtype:
            raise ValueError(f"{n}: dtype {tensors[n].dtype} != q_gate's {code_dtype}")
    meta = {"format": FORMAT, "version": VERSION, "fmt": weights.fmt, "experts": str(E), "hidden": str(H),
            "intermediate": str(I)}
    save_file(tensors, path, metadata=meta)


def load_w8a8(path: str, device="cuda") -> W8A8Weights:
    """Read a file written by ``save_w8a8`` onto ``device`` (tensor by tensor,
    memory-mapped), checking the format tag, shapes and dtypes."""
    from safetensors import safe_open
    with safe_open(path, framework="pt", device=str(device)) as f:
        meta = f.metadata() or {}
        if meta.get("format") != FORMAT or meta.get("version") != VERSION:
            raise ValueError(f"{path}: not a {FORMAT} v{VERSION} file (metadata {meta})")
        fmt = meta.get("fmt")
        code_dtype = {"int8": torch.int8, "fp8": torch.float8_e4m3fn}.get(fmt)
        if code_dtype is None:
            raise ValueError(f"{path}: unknown code format {fmt!r}")
        E, H, I = int(meta["experts"]), int(meta["hidden"]), int(meta["intermediate"])
        missing = set(_NAMES) - set(f.keys())
        if missing:
            raise ValueError(f"{path}: missing tensors {sorted(missing)}")
        out = {n: f.get_tensor(n) for n in _NAMES}
    for n, shape in _shapes(E, H, I).items():
        want = code_dtype if n.startswith("q_") else torch.float32
        if tuple(out[n].shape) != shape or out[n].dtype != want:
            raise ValueError(f"{path}: {n} is {out[n].dtype} {tuple(out[n].shape)}, expected {want} {shape}")
    return W8A8Weights(**out)
