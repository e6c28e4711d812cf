"""Pins oracle.route_topk by brute force and closed forms (no reference router
exists: problem_detail.json:18/:30)."""
import itertools

import numpy as np
import pytest
import torch
from scipy.special import softmax

from oracle import route_topk, router_logits


def _brute_topk(v, k):
    """Expert i is selected iff fewer than k experts beat it, where j beats i
    when v[j] > v[i] or (v[j] == v[i] and j < i); rank = number beating it."""
    E = v.shape[0]
    ranks = {}
    for i in range(E):
        beat = sum(1 for j in range(E) if v[j] > v[i] or (v[j] == v[i] and j < i))
        if beat < k:
            ranks[beat] = i
    return [ranks[r] for r in range(k)]


@pytest.mark.parametrize("E,k", [(4, 1), (5, 2), (8, 3), (8, 8)])
def test_topk_matches_brute_force(rng, E, k):
    T = 64
    logits = rng.standard_normal((T, E)).astype(np.float32)
    # force ties: quantise half of the rows to a coarse grid
    logits[::2] = np.round(logits[::2] * 2) / 2
    bias = rng.standard_normal(E).astype(np.float32) * 0.5
    ids, w = route_topk(logits, k, bias)
    v = logits + bias
    for t in range(T):
        assert list(ids[t]) == _brute_topk(v[t], k)


def test_topk_exhaustive_small():
    """Every ordering of a 4-expert row with a forced tie."""
    base = np.array([0.5, 0.5, -1.0, 2.0], dtype=np.float32)
    for perm in itertools.permutations(range(4)):
        row = base[list(perm)][None, :]
        ids, _ = route_topk(row, 2)
        assert list(ids[0]) == _brute_topk(row[0], 2)


def test_weights_closed_form(rng):
    """Renormalised softmax over the k selected = exp(v_i) / sum_sel exp(v_j);
    the full-softmax denominator cancels.  Checked against scipy in fp64."""
    T, E, k = 32, 16, 4
    logits = rng.standard_normal((T, E)).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.5).astype(np.float32)
    ids, w = route_topk(logits, k, bias)
    v = (logits + bias).astype(np.float64)
    p = softmax(v, axis=1)
    for t in range(T):
        sel = p[t, ids[t]]
        np.testing.assert_allclose(w[t], sel / sel.sum(), rtol=2e-6)
        e = np.exp(v[t, ids[t]])
        np.testing.assert_allclose(w[t], e / e.sum(), rtol=2e-6)
    assert np.all(np.diff(w, axis=1) <= 0), "weights follow selection order (descending)"
    np.testing.assert_allclose(w.sum(1), 1.0, rtol=1e-6)


def test_bias_changes_selection_not_definition():
    """A large bias on expert 3 forces it into every row; weights use softmax
    of the biased logits (build-defined)."""
    logits = np.zeros((3, 4), dtype=np.float32)
    bias = np.array([0, 0, 0, 10], dtype=np.float32)
    ids, w = route_topk(logits, 2, bias)
    assert (ids[:, 0] == 3).all() and (ids[:, 1] == 0).all()
    np.testing.assert_allclose(w[:, 0], np.exp(10) / (np.exp(10) + 1), rtol=1e-6)


def test_k_equals_one_weight_is_one(rng):
    logits = rng.standard_normal((10, 7)).astype(np.float32)
    ids, w = route_topk(logits, 1)
    assert (ids[:, 0] == logits.argmax(1)).all()
    np.testing.assert_array_equal(w, np.ones_like(w))


def test_router_logits_one_hot_rows_select_weight_columns(rng):
    """x = e_h (one-hot token rows) gives logits[:, e] = w_router[e, h]: a
    transposed operand or a wrong contraction axis fails this."""
    E, H = 5, 128
    w = torch.from_numpy(rng.standard_normal((E, H)).astype(np.float16))
    hs = [0, 7, 127]
    x = torch.zeros((len(hs), H), dtype=torch.float16)
    for t, h in enumerate(hs):
        x[t, h] = 1.0
    got = router_logits(x, w)
    np.testing.assert_array_equal(got, w.float().numpy()[:, hs].T)


def test_router_logits_against_float64(rng):
    T, H, E = 9, 256, 12
    x = rng.standard_normal((T, H)).astype(np.float16)
    w = (rng.standard_normal((E, H)) / 16).astype(np.float16)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    np.testing.assert_allclose(router_logits(torch.from_numpy(x), torch.from_numpy(w)), ref, rtol=1e-5, atol=1e-5)
