"""Pins the oracle's MoE dispatch / gather / combine (crates/backend-cpu/src/
kernels/moe.rs:839-848, 954-957, 1024-1033).

Pins: numpy's stable argsort / bincount for the grouping (the reference's
push order is ascending assignment index within an expert); direct row
indexing for the gather; for the combine, a second restatement that walks
the groups expert by expert and token by token exactly as moe.rs:1024-1033
does (the oracle instead walks tokens and sorts each token's slots by
expert), which must agree bit for bit; and an end-to-end identity: experts
that scale their input by c_e give y = y0 + sum_s w_s c_e(s) x.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle


def random_ids(rng, tokens, k, n_experts):
    return np.stack([rng.choice(n_experts, size=k, replace=False) for _ in range(tokens)]).astype(np.uint32)


@pytest.mark.parametrize("tokens,k,n_experts", [(1, 1, 1), (7, 2, 4), (300, 8, 128), (64, 6, 512), (33, 4, 4)])
def test_dispatch_is_stable_counting_sort(tokens, k, n_experts):
    rng = np.random.default_rng(tokens * 31 + k)
    ids = random_ids(rng, tokens, k, n_experts)
    counts, offsets, order, inv = oracle.moe_dispatch(ids, n_experts)
    flat = ids.ravel()
    assert np.array_equal(counts, np.bincount(flat, minlength=n_experts))
    assert np.array_equal(offsets, np.concatenate([[0], np.cumsum(counts)]).astype(np.uint32))
    assert np.array_equal(order, np.argsort(flat, kind="stable").astype(np.uint32))
    assert np.array_equal(inv[order], np.arange(flat.size, dtype=np.uint32))


def test_dispatch_rejects_out_of_range_ids():
    with pytest.raises(ValueError):
        oracle.moe_dispatch(np.array([[0, 5]], np.uint32), 4)


def test_gather_rows():
    rng = np.random.default_rng(2)
    tokens, k, h, E = 50, 4, 96, 16
    ids = random_ids(rng, tokens, k, E)
    _, _, order, _ = oracle.moe_dispatch(ids, E)
    x = rng.normal(size=(tokens, h)).astype(np.float32)
    g = oracle.moe_gather(x, k, order)
    assert np.array_equal(g, x[order // k])


def combine_by_groups(y0, expert_out, ids, weights, offsets, order, n_experts):
    """moe.rs:1024-1033 shape: for each expert's group, for each (token, weight) in push order."""
    y = y0.astype(np.float32).copy()
    k = ids.shape[1]
    for e in range(n_experts):
        for pos in range(offsets[e], offsets[e + 1]):
            a = order[pos]
            t = a // k
            y[t] = (y[t] + np.float32(weights.ravel()[a]) * expert_out[pos]).astype(np.float32)
    return y


@pytest.mark.parametrize("tokens,k,n_experts,h", [(40, 8, 128, 64), (9, 2, 4, 17), (128, 6, 64, 256)])
def test_combine_matches_group_walk_bitwise(tokens, k, n_experts, h):
    rng = np.random.default_rng(tokens + h)
    ids = random_ids(rng, tokens, k, n_experts)
    w = rng.random(size=(tokens, k)).astype(np.float32)
    _, offsets, order, inv = oracle.moe_dispatch(ids, n_experts)
    eo = rng.normal(size=(tokens * k, h)).astype(np.float32)
    y0 = rng.normal(size=(tokens, h)).astype(np.float32)
    got = oracle.moe_combine(y0, eo, ids, w, inv)
    ref = combine_by_groups(y0, eo, ids, w, offsets, order, n_experts)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_dispatch_gather_combine_identity_experts():
    rng = np.random.default_rng(5)
    tokens, k, E, h = 30, 4, 8, 32
    ids = random_ids(rng, tokens, k, E)
    w = rng.random(size=(tokens, k)).astype(np.float32)
    c = rng.uniform(0.5, 2.0, size=E).astype(np.float32)
    _, offsets, order, inv = oracle.moe_dispatch(ids, E)
    x = rng.normal(size=(tokens, h)).astype(np.float32)
    g = oracle.moe_gather(x, k, order)
    expert_of_pos = ids.ravel()[order]
    eo = (g * c[expert_of_pos][:, None]).astype(np.float32)
    y = oracle.moe_combine(np.zeros((tokens, h), np.float32), eo, ids, w, inv)
    ref = (w.astype(np.float64)[:, :, None] * c[ids].astype(np.float64)[:, :, None] * x.astype(np.float64)[:, None, :]).sum(1)
    assert np.abs(y - ref).max() < 1e-5 * np.abs(ref).max()


def test_combine_repeated_expert_in_a_token():
    """Drawn with replacement: a token may route twice to one expert; the
    group walk then meets its two slots in slot order."""
    rng = np.random.default_rng(8)
    tokens, k, E, h = 20, 4, 3, 8
    ids = rng.integers(0, E, size=(tokens, k)).astype(np.uint32)
    w = rng.random(size=(tokens, k)).astype(np.float32)
    _, offsets, order, inv = oracle.moe_dispatch(ids, E)
    eo = rng.normal(size=(tokens * k, h)).astype(np.float32)
    y0 = rng.normal(size=(tokens, h)).astype(np.float32)
    got = oracle.moe_combine(y0, eo, ids, w, inv)
    ref = combine_by_groups(y0, eo, ids, w, offsets, order, E)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_weighted_reduce_closed_forms():
    rng = np.random.default_rng(12)
    tokens, k, h = 16, 4, 24
    w = rng.random(size=(tokens, k)).astype(np.float32)
    eo = rng.normal(size=(tokens * k, h)).astype(np.float32)
    # one slot: exactly w * e
    got = oracle.moe_weighted_reduce(None, eo[::k], w[:, :1])
    assert np.array_equal(got, (w[:, :1] * eo[::k]).astype(np.float32))
    # slot order matters only through rounding: close to the f64 sum
    got = oracle.moe_weighted_reduce(None, eo, w)
    ref = (w.astype(np.float64)[:, :, None] * eo.reshape(tokens, k, h)).sum(1)
    assert np.abs(got - ref).max() < 1e-5
    # grouped rows in slot order: the group walk with one expert per slot index
    ids = np.tile(np.arange(k, dtype=np.uint32), (tokens, 1))
    _, _, order, inv = oracle.moe_dispatch(ids, k)
    grouped = eo[order]
    assert np.array_equal(oracle.moe_combine(np.zeros((tokens, h), np.float32), grouped, ids, w, inv), got)
