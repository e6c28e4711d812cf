"""Token sampling for the checkers (test infrastructure, like the rest of
this package): which tokens of a routing an oracle comparison must include so
that every work item of the GPU schedule feeds a checked element."""

from __future__ import annotations

import numpy as np


def stratified_tokens(ids, block=128, extra=16, seed=0, max_block_starts=None, experts=None):
    """Tokens whose rows cover the schedule of a routing (ids int [T, k]).

    Pairs are ordered as align orders them (by expert, then pair index).  The
    set holds the token of every touched expert's first and last pair (so
    every expert, and every tail block's last valid row), the token at the
    start of every ``block``-row block of every expert (so every paired,
    single and 256-row item of both stages), and ``extra`` random tokens.
    ``max_block_starts`` caps the block starts (randomly chosen) and
    ``experts`` restricts all of it to those expert ids.  Tokens are
    independent, so an oracle run on these rows is exact for them."""
    ids = np.asarray(ids)
    T, k = ids.shape
    flat = ids.reshape(-1)
    order = np.argsort(flat, kind="stable")
    se = flat[order]
    starts = np.flatnonzero(np.r_[True, se[1:] != se[:-1]])
    ends = np.r_[starts[1:], flat.size]
    rng = np.random.default_rng(seed)
    pick, bstarts = set(), []
    for s, e in zip(starts, ends):
        if experts is not None and int(se[s]) not in experts:
            continue
        pick.add(int(order[s]) // k)
        pick.add(int(order[e - 1]) // k)
        bstarts.extend(int(p) // k for p in order[s:e:block])
    if max_block_starts is not None and len(bstarts) > max_block_starts:
        bstarts = rng.choice(np.asarray(bstarts), max_block_starts, replace=False).tolist()
    pick.update(bstarts)
    if extra:
        pick.update(int(t) for t in rng.choice(T, min(extra, T), replace=False))
    return np.asarray(sorted(pick), dtype=np.int64)
