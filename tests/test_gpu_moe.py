"""GPU parity of MoE dispatch / gather / combine against the oracle.

Bar: bit-exact everywhere.  Dispatch and gather are integer / byte work; the
combine rounds w * v and the add separately in f32 in the same order as the
oracle (ascending expert id over grouped rows, or slot order over
per-assignment rows), so its f32 bits must match too.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def ops():
    from fellm_amd import ops as _ops

    return _ops


def route_ids(rng, tokens, k, n_experts, replace=False):
    if replace:
        return rng.integers(0, n_experts, size=(tokens, k)).astype(np.uint32)
    # top-k style: distinct experts per token, skewed popularity
    p = rng.dirichlet(np.full(n_experts, 0.3))
    return np.stack([rng.choice(n_experts, size=k, replace=False, p=p) for _ in range(tokens)]).astype(np.uint32)


def to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).to(dev)


def u32(t):
    return t.cpu().numpy().view(np.uint32)


DISPATCH = [(1, 1, 1), (3, 2, 4), (64, 8, 128), (65, 8, 128), (256, 8, 128), (257, 8, 128), (1000, 8, 128),
            (16384, 8, 128), (700, 6, 4096), (300, 64, 300), (4096, 4, 2), (2000, 8, 256), (70001, 8, 64),
            (1 << 17, 8, 128)]


@pytest.mark.parametrize("tokens,k,n_experts", DISPATCH)
def test_dispatch_matches_oracle(ops, dev, tokens, k, n_experts):
    rng = np.random.default_rng(tokens * 7 + k * 3 + n_experts)
    ids = route_ids(rng, tokens, k, n_experts, replace=k > n_experts)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    d = ops.moe_dispatch(to_dev(ids, dev), n_experts, err_flag=err)
    counts, offsets, order, inv = oracle.moe_dispatch(ids, n_experts)
    assert np.array_equal(u32(d.counts), counts)
    assert np.array_equal(u32(d.offsets), offsets)
    assert np.array_equal(u32(d.order), order)
    assert np.array_equal(u32(d.inv), inv)
    assert int(err.item()) == 0


def test_dispatch_repeated_calls_are_identical(ops, dev):
    rng = np.random.default_rng(4)
    ids = to_dev(route_ids(rng, 5000, 8, 64), dev)
    a = ops.moe_dispatch(ids, 64)
    b = ops.moe_dispatch(ids, 64)
    for _ in range(3):
        b.order.fill_(7)
        b.inv.fill_(7)
        ops.moe_dispatch(ids, 64, out=b)
        assert torch.equal(a.order, b.order) and torch.equal(a.inv, b.inv)
        assert torch.equal(a.counts, b.counts) and torch.equal(a.offsets, b.offsets)


@pytest.mark.parametrize("tokens", [10, 3000])
def test_dispatch_invalid_ids(ops, dev, tokens):
    """Ids >= E are left out of every group and raise the error flag."""
    rng = np.random.default_rng(tokens)
    k, E = 4, 16
    ids = route_ids(rng, tokens, k, E)
    bad = rng.random(ids.shape) < 0.05
    bad[0, 0] = True
    ids[bad] = E + rng.integers(0, 1000, size=int(bad.sum()))
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    d = ops.moe_dispatch(to_dev(ids, dev), E, err_flag=err)
    assert int(err.item()) == 1
    flat = ids.ravel()
    valid = flat < E
    assert np.array_equal(u32(d.counts), np.bincount(flat[valid], minlength=E))
    nv = int(valid.sum())
    assert int(u32(d.offsets)[E]) == nv
    exp_order = np.nonzero(valid)[0][np.argsort(flat[valid], kind="stable")]
    order = u32(d.order)
    assert np.array_equal(order[:nv], exp_order)
    assert np.all(order[nv:] == 0xFFFFFFFF)
    inv = u32(d.inv)
    assert np.all(inv[~valid] == 0xFFFFFFFF)
    assert np.array_equal(inv[order[:nv]], np.arange(nv))


def test_dispatch_zero_tokens_and_shape_errors(ops, dev):
    d = ops.moe_dispatch(torch.zeros((0, 8), dtype=torch.int32, device=dev), 16)
    assert d.counts.cpu().numpy().tolist() == [0] * 16
    assert d.offsets.cpu().numpy().tolist() == [0] * 17
    from fellm_amd._lib import FellmRocmError

    ids = torch.zeros((4, 65), dtype=torch.int32, device=dev)
    with pytest.raises(FellmRocmError):
        ops.moe_dispatch(ids, 128)
    with pytest.raises(FellmRocmError):
        ops.moe_dispatch(torch.zeros((4, 2), dtype=torch.int32, device=dev), 4097)


@pytest.mark.parametrize("dtype,hidden", [(torch.float32, 2048), (torch.float16, 256), (torch.bfloat16, 2048),
                                          (torch.float32, 7), (torch.float16, 7), (torch.uint8, 33),
                                          (torch.float32, 8192), (torch.bfloat16, 3000), (torch.uint8, 16)])
@pytest.mark.parametrize("use_inv", [False, True])
def test_gather_rows(ops, dev, dtype, hidden, use_inv):
    rng = np.random.default_rng(hidden)
    tokens, k, E = 300, 8, 64
    ids = route_ids(rng, tokens, k, E)
    _, _, order, inv = oracle.moe_dispatch(ids, E)
    if dtype == torch.uint8:
        x = torch.from_numpy(rng.integers(0, 256, size=(tokens, hidden), dtype=np.uint8))
    else:
        x = torch.from_numpy(rng.normal(size=(tokens, hidden)).astype(np.float32)).to(dtype)
    got = ops.moe_gather(x.to(dev), to_dev(order, dev), k, inv=to_dev(inv, dev) if use_inv else None).cpu()
    ref = x[torch.from_numpy((order // k).astype(np.int64))]
    assert torch.equal(got.view(torch.uint8), ref.contiguous().view(torch.uint8))
    if dtype == torch.float32:
        assert np.array_equal(got.numpy(), oracle.moe_gather(x.numpy(), k, order))


@pytest.mark.parametrize("use_inv", [False, True])
def test_gather_invalid_order_rows_are_zero(ops, dev, use_inv):
    """Ids >= E leave the order tail invalid: those grouped rows come out zero
    (pre-filled with garbage here), every other row is its token's row."""
    tokens, k, E, h = 4, 2, 4, 16
    ids = torch.tensor([[0, 9], [3, 1], [7, 2], [1, 0]], dtype=torch.int32, device=dev)
    d = ops.moe_dispatch(ids, E)
    x = torch.arange(tokens * h, dtype=torch.float32, device=dev).reshape(tokens, h) + 1
    out = torch.full((tokens * k, h), 123.0, device=dev)
    got = ops.moe_gather(x, d.order, k, inv=d.inv if use_inv else None, out=out).cpu()
    order = u32(d.order)
    assert list(order[6:]) == [0xFFFFFFFF, 0xFFFFFFFF]
    assert torch.all(got[6:] == 0)
    assert torch.equal(got[:6], x.cpu()[torch.from_numpy(order[:6].astype(np.int64) // k)])


COMBINE = [(40, 8, 128, 2048), (9, 2, 4, 17), (128, 6, 64, 256), (1, 1, 1, 64), (257, 64, 128, 12), (3000, 8, 16, 100)]


@pytest.mark.parametrize("tokens,k,n_experts,h", COMBINE)
@pytest.mark.parametrize("with_y0", [True, False])
def test_combine_expert_order(ops, dev, tokens, k, n_experts, h, with_y0):
    rng = np.random.default_rng(tokens + h + k)
    ids = route_ids(rng, tokens, k, n_experts, replace=k > n_experts)
    w = rng.random(size=(tokens, k)).astype(np.float32)
    _, _, _, inv = oracle.moe_dispatch(ids, n_experts)
    eo = rng.normal(size=(tokens * k, h)).astype(np.float32)
    y0 = rng.normal(size=(tokens, h)).astype(np.float32) if with_y0 else np.zeros((tokens, h), np.float32)
    ref = oracle.moe_combine(y0, eo, ids, w, inv)
    got = ops.moe_combine(torch.from_numpy(eo).to(dev), torch.from_numpy(w).to(dev), ids=to_dev(ids, dev),
                          inv=to_dev(inv, dev), y0=torch.from_numpy(y0).to(dev) if with_y0 else None)
    assert np.array_equal(got.cpu().numpy().view(np.uint32), ref.view(np.uint32))


def test_combine_repeated_experts_and_in_place(ops, dev):
    rng = np.random.default_rng(21)
    tokens, k, E, h = 200, 8, 3, 64
    ids = route_ids(rng, tokens, k, E, replace=True)
    w = rng.random(size=(tokens, k)).astype(np.float32)
    _, _, _, inv = oracle.moe_dispatch(ids, E)
    eo = rng.normal(size=(tokens * k, h)).astype(np.float32)
    y0 = rng.normal(size=(tokens, h)).astype(np.float32)
    ref = oracle.moe_combine(y0, eo, ids, w, inv)
    y = torch.from_numpy(y0).to(dev)
    ops.moe_combine(torch.from_numpy(eo).to(dev), torch.from_numpy(w).to(dev), ids=to_dev(ids, dev),
                    inv=to_dev(inv, dev), y0=y, out=y)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("tokens,k,h", [(40, 8, 2048), (9, 2, 17), (1000, 6, 256)])
@pytest.mark.parametrize("with_y0", [True, False])
def test_combine_slot_order(ops, dev, tokens, k, h, with_y0):
    rng = np.random.default_rng(tokens * h)
    w = rng.random(size=(tokens, k)).astype(np.float32)
    eo = rng.normal(size=(tokens * k, h)).astype(np.float32)
    y0 = rng.normal(size=(tokens, h)).astype(np.float32) if with_y0 else None
    ref = oracle.moe_weighted_reduce(y0, eo, w)
    got = ops.moe_combine(torch.from_numpy(eo).to(dev), torch.from_numpy(w).to(dev),
                          y0=torch.from_numpy(y0).to(dev) if with_y0 else None)
    assert np.array_equal(got.cpu().numpy().view(np.uint32), ref.view(np.uint32))


def test_dispatch_gather_combine_chain_at_headline_size(ops, dev):
    """16384 tokens, top-8 of 128 experts, H 2048 (the c5 shape): dispatch,
    gather, per-expert scaling as a stand-in expert FFN, combine; every stage
    bit-exact with the oracle."""
    rng = np.random.default_rng(99)
    tokens, k, E, h = 16384, 8, 128, 2048
    ids = route_ids(rng, tokens, k, E)
    w = rng.random(size=(tokens, k)).astype(np.float32)
    x = rng.normal(size=(tokens, h)).astype(np.float32)
    c = rng.uniform(0.5, 2.0, size=E).astype(np.float32)
    d = ops.moe_dispatch(to_dev(ids, dev), E)
    counts, offsets, order, inv = oracle.moe_dispatch(ids, E)
    assert np.array_equal(u32(d.order), order) and np.array_equal(u32(d.inv), inv)
    xd = torch.from_numpy(x).to(dev)
    g = ops.moe_gather(xd, d.order, k, inv=d.inv)
    scale = torch.from_numpy(c[ids.ravel()[order]]).to(dev)
    eo = g * scale[:, None]
    y0 = torch.from_numpy(x).to(dev)
    y = ops.moe_combine(eo, torch.from_numpy(w).to(dev), ids=to_dev(ids, dev), inv=d.inv, y0=y0)
    g_ref = oracle.moe_gather(x, k, order)
    assert torch.equal(g.cpu(), torch.from_numpy(g_ref))
    eo_ref = (g_ref * c[ids.ravel()[order]][:, None]).astype(np.float32)
    ref = oracle.moe_combine(x, eo_ref, ids, w, inv)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), ref.view(np.uint32))
