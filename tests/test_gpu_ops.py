"""GPU parity: every kernel through the device-pointer C ABI against the CPU oracle.

Seeded inputs at sizes the oracle finishes in well under a second; the
tolerances are stated in parity_util.py.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from parity_util import (KINDS, assert_close, assert_exact, from_dev,
                         random_stored, to_dev)

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def ops():
    from fellm_amd import ops as _ops

    return _ops


def sync():
    torch.cuda.synchronize()


# ---- expf --------------------------------------------------------------------
def test_device_expf_matches_glibc(ops, dev):
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, size=1 << 22, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    special = np.array([0.0, -0.0, 1.0, -1.0, 88.0, 88.7, float.fromhex('0x1.62e42ep6'), 89.0, -103.0, -103.97, -104.0,
                        float.fromhex('-0x1.9fe368p6'),
                        np.inf, -np.inf, np.nan, 1e-45, -1e-45], np.float32)
    dense = np.linspace(-110.0, 90.0, 1 << 20, dtype=np.float32)
    x = np.concatenate([x, special, dense])
    got = from_dev(ops.expf(torch.from_numpy(x).to(dev)))
    ref = oracle.expf(x)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert_exact(got[~nan], ref[~nan], "expf")


def test_device_logf_matches_glibc(ops, dev):
    rng = np.random.default_rng(3)
    bits = rng.integers(0, 2**32, size=1 << 22, dtype=np.uint64).astype(np.uint32)
    special = np.array([0.0, -0.0, 1.0, -1.0, 1e-45, 1e-38, 1.17549435e-38, 3.4e38, np.inf, -np.inf, np.nan, 2.0,
                        0.5, 1.0000001, 0.99999994], np.float32)
    dense = np.linspace(0.5, 4.0, 1 << 20, dtype=np.float32)
    x = np.concatenate([bits.view(np.float32), special, dense])
    got = from_dev(ops.logf(torch.from_numpy(x).to(dev)))
    ref = oracle.logf(x)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert_exact(got[~nan], ref[~nan], "logf")


def test_device_sincosf_matches_glibc(ops, dev):
    """RoPE's sin/cos table entries: every reduction path (|x| < 2^-12, < pi/4,
    < 120, Payne-Hanek) and the RoPE angle range, bit for bit."""
    rng = np.random.default_rng(2)
    bits = rng.integers(0, 2**32, size=1 << 22, dtype=np.uint64).astype(np.uint32)
    special = np.array([0.0, -0.0, 2.0 ** -12, -(2.0 ** -12), 0.785398, 0.7853982, 119.99999, 120.0, -120.0, 1e30,
                        3.4e38, np.inf, -np.inf, np.nan, 1e-45], np.float32)
    dense = np.linspace(-40000.0, 40000.0, 1 << 21, dtype=np.float32)
    pos = np.arange(32768, dtype=np.float32)
    inv = oracle.rope_inv_freqs(500000.0, 128)
    angles = (pos[:, None] * inv[None, :]).astype(np.float32).ravel()
    x = np.concatenate([bits.view(np.float32), special, dense, angles])
    s, c = ops.sincosf(torch.from_numpy(x).to(dev))
    rs, rc = oracle.sincosf(x)
    for got, ref, what in ((from_dev(s), rs, "sinf"), (from_dev(c), rc, "cosf")):
        nan = np.isnan(ref)
        assert np.array_equal(np.isnan(got), nan), what
        assert_exact(got[~nan], ref[~nan], what)


# ---- SwiGLU --------------------------------------------------------------------
@pytest.mark.parametrize("kind", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("n", [1, 7, 8, 4096 * 3 + 5, 64 * 8192])
def test_silu_gate(ops, dev, kind, n):
    rng = np.random.default_rng(n)
    g = random_stored(rng, n, kind)
    u = random_stored(rng, n, kind)
    ref = oracle.narrow(oracle.silu_gate(oracle.widen(g, kind), oracle.widen(u, kind)), kind)
    got = from_dev(ops.silu_gate(to_dev(g, kind, dev), to_dev(u, kind, dev)))
    assert_exact(got, ref, f"silu_gate {kind} n={n}")


@pytest.mark.parametrize("kind", ["f16", "bf16"])
def test_silu_gate_16bit_in_f32_out(ops, dev, kind):
    """16-bit gate/up with an f32 output: the exact silu path (the interval
    test only decides 16-bit outputs), bit-exact against the oracle."""
    rng = np.random.default_rng(31)
    n = 65536 + 3
    g = random_stored(rng, n, kind, sigma=4.0)
    u = random_stored(rng, n, kind)
    ref = oracle.silu_gate(oracle.widen(g, kind), oracle.widen(u, kind))
    got = from_dev(ops.silu_gate(to_dev(g, kind, dev), to_dev(u, kind, dev), out_dtype=torch.float32))
    assert_exact(got, ref, f"silu_gate {kind} -> f32")


def test_silu_fast_bound_covers_every_gate(ops, dev):
    """The 16-bit SwiGLU outputs skip the exact silu when an interval of
    +-D bit steps around a fast f32 silu fixes the rounded result.  That is
    bit-exact iff the exact silu lies within D steps of the fast one for every
    gate of the fast domain: the device sweep over all 2^32 f32 patterns
    measures the largest distance."""
    measured, assumed = ops.silu_fast_bound()
    assert 0 < measured <= assumed, (measured, assumed)


@pytest.mark.parametrize("kind", ["f16", "bf16"])
def test_silu_gate_rounding_boundaries(ops, dev, kind):
    """Pairs whose f32 product lies within 64 f32 steps of a 16-bit rounding
    midpoint, where the fast interval cannot decide and the exact silu runs,
    mixed with random pairs decided by the interval alone."""
    rng = np.random.default_rng(29)
    n = 1 << 23
    g = random_stored(rng, n, kind)
    u = random_stored(rng, n, kind)
    p = oracle.silu_gate(oracle.widen(g, kind), oracle.widen(u, kind))
    low = 13 if kind == "f16" else 16
    r = (p.view(np.uint32) & ((1 << low) - 1)).astype(np.int64)
    near = np.abs(r - (1 << (low - 1))) <= 64
    keep = near | (rng.random(n) < 0.01)
    assert near.sum() > 1000
    g, u, p = g[keep], u[keep], p[keep]
    got = from_dev(ops.silu_gate(to_dev(g, kind, dev), to_dev(u, kind, dev)))
    assert_exact(got, oracle.narrow(p, kind), f"silu_gate {kind} near rounding midpoints")


@pytest.mark.parametrize("kind", ["f16", "bf16"])
def test_silu_gate_16bit_specials(ops, dev, kind):
    """16-bit SwiGLU over every pair of special gates and ups: signed zeros,
    tiny and boundary gates of the fast domain (|g| in [2^-100, 64)), +-inf,
    NaN, and ups that are NaN, infinite or large enough to overflow the
    product.  The fast interval decides only non-NaN ups; everything else
    takes the exact path.  Bit-exact against the oracle, NaN bits included."""
    gs = np.array([0.0, -0.0, 1e-30, -1e-30, 2.0 ** -99, -(2.0 ** -99), 1.0, -1.0, 3.5, -3.5, 63.9, -63.9,
                   64.0, -64.0, 100.0, -100.0, np.inf, -np.inf, np.nan], np.float32)
    big = 60000.0 if kind == "f16" else 3e38
    us = np.array([0.0, -0.0, 1.5, -1.5, big, -big, np.inf, -np.inf, np.nan], np.float32)
    g32, u32 = (a.ravel() for a in np.meshgrid(gs, us, indexing="ij"))
    g, u = oracle.narrow(g32, kind), oracle.narrow(u32, kind)
    ref = oracle.narrow(oracle.silu_gate(oracle.widen(g, kind), oracle.widen(u, kind)), kind)
    got = from_dev(ops.silu_gate(to_dev(g, kind, dev), to_dev(u, kind, dev)))
    assert_exact(got, ref, f"silu_gate {kind} specials")


def test_silu_gate_unaligned_and_extremes(ops, dev):
    g = np.array([0.0, -0.0, 100.0, -100.0, 20.0, -20.0, 88.0, -88.0, 1e-30, np.inf, -np.inf, 3.5], np.float32)
    u = np.full_like(g, 1.5)
    ref = oracle.silu_gate(g, u)
    gd = torch.from_numpy(np.concatenate([[0.0], g]).astype(np.float32)).to(dev)[1:]
    ud = torch.from_numpy(np.concatenate([[0.0], u]).astype(np.float32)).to(dev)[1:]
    got = from_dev(ops.silu_gate(gd, ud))
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert_exact(got[~nan], ref[~nan], "silu extremes")
    assert got[0] == 0.0


# ---- Add + RMSNorm -------------------------------------------------------------
@pytest.mark.parametrize("kind", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("rows,group", [(1, 2048), (3, 4096), (64, 2048), (1500, 4096), (7, 8192), (5, 3584),
                                        (9, 100), (2, 65536), (33, 16)])
def test_add_rmsnorm(ops, dev, kind, rows, group):
    rng = np.random.default_rng(rows * 7919 + group)
    x = random_stored(rng, (rows, group), kind)
    r = random_stored(rng, (rows, group), kind, sigma=2.0)
    w = rng.normal(1.0, 0.1, size=group).astype(np.float32)
    eps = 1e-5
    h_ref, y_ref = oracle.add_rmsnorm(x, r, w, eps, kind)
    h, y = ops.add_rmsnorm(to_dev(x, kind, dev), to_dev(r, kind, dev), torch.from_numpy(w).to(dev), eps)
    assert_exact(from_dev(h), h_ref, f"h {kind}")
    assert_close(from_dev(y), y_ref, kind, what=f"y {kind} {rows}x{group}")


@pytest.mark.parametrize("kind", ["f16", "bf16"])
@pytest.mark.parametrize("rows,group", [(6, 2048), (6, 8192), (1030, 4096)])
def test_add_rmsnorm_specials(ops, dev, kind, rows, group):
    """16-bit rows holding NaNs with payloads, infinities, sums that overflow
    the 16-bit type and signed zeros, beside ordinary rows (the row layouts of
    every size class).  h bit-exact (a lane with a NaN rounds element by
    element), y NaN exactly where the oracle's is and within tolerance
    elsewhere."""
    rng = np.random.default_rng(rows + group)
    x = random_stored(rng, (rows, group), kind)
    r = random_stored(rng, (rows, group), kind, sigma=2.0)
    nan_a, nan_b = (0x7E01, 0xFE07) if kind == "f16" else (0x7FC1, 0xFFC7)
    inf, big = (0x7C00, 0x7BFF) if kind == "f16" else (0x7F80, 0x7F7F)
    x[1, 3], x[1, 100], r[2, 7] = nan_a, nan_b, nan_a
    x[3, 0], r[3, 1] = inf, inf | 0x8000
    x[4, 5], r[4, 5] = big, big
    x[5, :], r[5, :] = 0x8000, 0
    w = rng.normal(1.0, 0.1, size=group).astype(np.float32)
    h_ref, y_ref = oracle.add_rmsnorm(x, r, w, 1e-5, kind)
    h, y = ops.add_rmsnorm(to_dev(x, kind, dev), to_dev(r, kind, dev), torch.from_numpy(w).to(dev), 1e-5)
    assert_exact(from_dev(h), h_ref, f"h {kind} specials")
    yg, yr = from_dev(y), y_ref
    wide = lambda a: oracle.widen(a, kind)
    assert np.array_equal(np.isnan(wide(yg)), np.isnan(wide(yr)))
    ok = ~np.isnan(wide(yr))
    assert_close(yg[ok], yr[ok], kind, what=f"y {kind} specials")


@pytest.mark.parametrize("kind", ["f32", "bf16"])
def test_rmsnorm_plain_and_no_h(ops, dev, kind):
    rng = np.random.default_rng(5)
    x = random_stored(rng, (256, 8192), kind)
    w = rng.normal(1.0, 0.1, size=8192).astype(np.float32)
    y_ref = oracle.narrow(oracle.rmsnorm(oracle.widen(x, kind), w, 1e-6), kind)
    y = ops.rmsnorm(to_dev(x, kind, dev), torch.from_numpy(w).to(dev), 1e-6)
    assert_close(from_dev(y), y_ref, kind, what="plain rmsnorm")
    r = random_stored(rng, (256, 8192), kind)
    _, y_ref2 = oracle.add_rmsnorm(x, r, w, 1e-6, kind)
    h, y2 = ops.add_rmsnorm(to_dev(x, kind, dev), to_dev(r, kind, dev), torch.from_numpy(w).to(dev), 1e-6,
                            store_h=False)
    assert h is None
    assert_close(from_dev(y2), y_ref2, kind, what="no-h rmsnorm")


def test_add_rmsnorm_inplace_residual(ops, dev):
    rng = np.random.default_rng(11)
    kind = "f16"
    for group in (4096, 100, 65536):
        x = random_stored(rng, (4, group), kind)
        r = random_stored(rng, (4, group), kind)
        w = rng.normal(1.0, 0.1, size=group).astype(np.float32)
        h_ref, y_ref = oracle.add_rmsnorm(x, r, w, 1e-5, kind)
        xd = to_dev(x, kind, dev)
        h, y = ops.add_rmsnorm(xd, to_dev(r, kind, dev), torch.from_numpy(w).to(dev), 1e-5, h_out=xd)
        assert_exact(from_dev(xd), h_ref, "in-place h")
        assert_close(from_dev(y), y_ref, kind, what="in-place y")


# ---- Embedding -----------------------------------------------------------------
def _dense_table(rng, vocab, dim, kind):
    return random_stored(rng, (vocab, dim), kind, sigma=0.02)


@pytest.mark.parametrize("table_kind", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("out_kind", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("dim", [2048, 100])
def test_embedding_dense(ops, dev, table_kind, out_kind, dim):
    rng = np.random.default_rng(dim)
    vocab = 1000
    t = _dense_table(rng, vocab, dim, table_kind)
    ids = rng.integers(0, vocab, size=77, dtype=np.uint32)
    code = {"f32": 0, "f16": 1, "bf16": 30}[table_kind]
    ref = oracle.narrow(oracle.embedding(t.view(np.uint8), code, vocab, dim, ids), out_kind)
    got = ops.embedding(to_dev(t, table_kind, dev), torch.from_numpy(ids.view(np.int32)).to(dev),
                        out_dtype=KINDS[out_kind])
    assert_exact(from_dev(got), ref, f"embedding {table_kind}->{out_kind}")


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
@pytest.mark.parametrize("out_kind", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("dim", [256, 3584, 4096, 1280])
def test_embedding_quant(ops, dev, qtype, out_kind, dim):
    from fellm_amd import synth

    rng = np.random.default_rng(dim + len(qtype))
    vocab = 300
    table = synth.q4k_table(rng, vocab, dim) if qtype == "q4k" else synth.q6k_table(rng, vocab, dim)
    ids = synth.zipf_ids(rng, 200, vocab)
    code = 12 if qtype == "q4k" else 14
    ref = oracle.narrow(oracle.embedding(table, code, vocab, dim, ids), out_kind)
    got = ops.embedding(torch.from_numpy(table).to(dev), torch.from_numpy(ids.view(np.int32)).to(dev), dim=dim,
                        qtype=qtype, out_dtype=KINDS[out_kind])
    assert_exact(from_dev(got), ref, f"embedding {qtype} dim={dim} -> {out_kind}")


@pytest.mark.parametrize("src", ["q4k", "q6k", "f16", "f32"])
def test_embedding_rmsnorm_fused(ops, dev, src):
    from fellm_amd import synth

    rng = np.random.default_rng(3)
    vocab, dim = 500, 3584
    out_kind = "f32" if src == "f32" else "f16"
    if src == "q4k":
        table, code = synth.q4k_table(rng, vocab, dim), 12
        td = torch.from_numpy(table).to(dev)
    elif src == "q6k":
        table, code = synth.q6k_table(rng, vocab, dim), 14
        td = torch.from_numpy(table).to(dev)
    else:
        st = _dense_table(rng, vocab, dim, src)
        table, code = st.view(np.uint8), {"f16": 1, "f32": 0}[src]
        td = to_dev(st, src, dev)
    ids = synth.zipf_ids(rng, 300, vocab)
    w = rng.normal(1.0, 0.1, size=dim).astype(np.float32)
    e = oracle.embedding(table, code, vocab, dim, ids)
    h_ref = oracle.narrow(e, out_kind)
    y_ref = oracle.narrow(oracle.rmsnorm(e, w, 1e-6), out_kind)
    h, y = ops.embedding_rmsnorm(td, torch.from_numpy(ids.view(np.int32)).to(dev), torch.from_numpy(w).to(dev),
                                 1e-6, dim=dim, qtype=src if src.startswith("q") else None,
                                 out_dtype=KINDS[out_kind])
    assert_exact(from_dev(h), h_ref, "fused h")
    assert_close(from_dev(y), y_ref, out_kind, what="fused y")


@pytest.mark.parametrize("table_kind,out_kind,dim", [("f16", "f16", 4096), ("f32", "f32", 4096), ("bf16", "f32", 2048),
                                                      ("f16", "bf16", 100), ("f32", "f16", 1024)])
@pytest.mark.parametrize("n_rows", [4099, 6144, 2051])
def test_embedding_dense_many_rows(ops, dev, table_kind, out_kind, dim, n_rows):
    """Thousands of rows take the persistent gather (each workgroup walks
    rows b, b + grid, ...): rows counts that end on either half of its two
    register sets, and out-of-range ids spread through the batch."""
    rng = np.random.default_rng(n_rows + dim)
    vocab = 3000
    t = _dense_table(rng, vocab, dim, table_kind)
    ids = rng.integers(0, vocab, size=n_rows, dtype=np.uint32)
    bad = rng.choice(n_rows, size=5, replace=False)
    ids[bad] = vocab + np.arange(5, dtype=np.uint32) * 1000
    code = {"f32": 0, "f16": 1, "bf16": 30}[table_kind]
    ok = ids < vocab
    ref = np.zeros((n_rows, dim), np.float32)
    ref[ok] = oracle.embedding(t.view(np.uint8), code, vocab, dim, ids[ok])
    ref = oracle.narrow(ref, out_kind)
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    got = ops.embedding(to_dev(t, table_kind, dev), torch.from_numpy(ids.view(np.int32)).to(dev),
                        out_dtype=KINDS[out_kind], err_flag=flag)
    assert int(flag.item()) == 1
    assert_exact(from_dev(got), ref, f"embedding {n_rows} rows {table_kind}->{out_kind} dim {dim}")


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
@pytest.mark.parametrize("out_kind,dim,n_rows", [("f16", 3584, 8195), ("bf16", 4096, 4099), ("f32", 256, 6000),
                                                 ("f16", 16384, 4097)])
def test_embedding_quant_many_rows(ops, dev, qtype, out_kind, dim, n_rows):
    """Thousands of K-quant rows (one workgroup per row, 1-2 parts per thread
    or the looping layout at dim 16384); Zipf ids with out-of-range ids spread
    through the batch; bit-exact against the oracle."""
    from fellm_amd import synth

    rng = np.random.default_rng(n_rows + dim + len(qtype))
    vocab = 700
    table = synth.q4k_table(rng, vocab, dim) if qtype == "q4k" else synth.q6k_table(rng, vocab, dim)
    ids = synth.zipf_ids(rng, n_rows, vocab)
    bad = rng.choice(n_rows, size=4, replace=False)
    ids[bad] = vocab + np.arange(4, dtype=np.uint32)
    code = 12 if qtype == "q4k" else 14
    ok = ids < vocab
    ref = np.zeros((n_rows, dim), np.float32)
    ref[ok] = oracle.embedding(table, code, vocab, dim, ids[ok])
    ref = oracle.narrow(ref, out_kind)
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    got = ops.embedding(torch.from_numpy(table).to(dev), torch.from_numpy(ids.view(np.int32)).to(dev), dim=dim,
                        qtype=qtype, out_dtype=KINDS[out_kind], err_flag=flag)
    assert int(flag.item()) == 1
    assert_exact(from_dev(got), ref, f"embedding {qtype} {n_rows} rows dim={dim} -> {out_kind}")


def test_embedding_bad_id_sets_flag(ops, dev):
    rng = np.random.default_rng(0)
    t = _dense_table(rng, 10, 64, "f32")
    ids = np.array([1, 10, 3], np.uint32)
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    got = from_dev(ops.embedding(to_dev(t, "f32", dev), torch.from_numpy(ids.view(np.int32)).to(dev),
                                 err_flag=flag))
    assert int(flag.item()) == 1
    assert_exact(got[0], t[1], "row 0")
    assert np.all(got[1] == 0)
    assert_exact(got[2], t[3], "row 2")


# ---- RoPE ----------------------------------------------------------------------
@pytest.mark.parametrize("kind", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("pairing", [0, 1, 2])
@pytest.mark.parametrize("head_dim,rope_dim", [(128, 128), (64, 64), (128, 64), (6, 4)])
def test_rope_qk(ops, dev, kind, pairing, head_dim, rope_dim):
    rng = np.random.default_rng(head_dim * 10 + rope_dim + pairing)
    rows, nq, nk = 37, 8, 2
    theta = 500000.0
    inv = oracle.rope_inv_freqs(theta, rope_dim)
    q = random_stored(rng, (rows, nq * head_dim), kind)
    k = random_stored(rng, (rows, nk * head_dim), kind)
    pos = rng.integers(0, 32768, size=rows, dtype=np.uint32)
    qr = oracle.narrow(oracle.rope(oracle.widen(q, kind), nq, head_dim, rope_dim, pairing, inv, pos), kind)
    kr = oracle.narrow(oracle.rope(oracle.widen(k, kind), nk, head_dim, rope_dim, pairing, inv, pos), kind)
    qo, ko = ops.rope(to_dev(q, kind, dev), torch.from_numpy(inv).to(dev), head_dim=head_dim, rope_dim=rope_dim,
                      pairing=pairing, positions=torch.from_numpy(pos.view(np.int32)).to(dev),
                      x2=to_dev(k, kind, dev))
    assert_exact(from_dev(qo), qr, "q")
    assert_exact(from_dev(ko), kr, "k")
    # passthrough dims are copied exactly
    if rope_dim < head_dim:
        qv, rv = from_dev(qo).reshape(rows, nq, head_dim), q.reshape(rows, nq, head_dim)
        sl = slice(0, head_dim - rope_dim) if pairing == 2 else slice(rope_dim, head_dim)
        assert_exact(qv[..., sl], rv[..., sl], "passthrough")


def test_rope_position0_inplace(ops, dev):
    rng = np.random.default_rng(9)
    rows, nh, hd = 64, 32, 64
    inv = oracle.rope_inv_freqs(500000.0, hd)
    x = rng.normal(size=(rows, nh * hd)).astype(np.float32)
    ref = oracle.rope(x, nh, hd, hd, 0, inv, None, position0=100)
    xd = torch.from_numpy(x).to(dev)
    ops.rope(xd, torch.from_numpy(inv).to(dev), head_dim=hd, position0=100, inplace=True)
    assert_exact(from_dev(xd), ref, "in-place pos0")
    # position 0 is the identity (rope.rs:69-77)
    x0 = rng.normal(size=(1, nh * hd)).astype(np.float32)
    got = from_dev(ops.rope(torch.from_numpy(x0).to(dev), torch.from_numpy(inv).to(dev), head_dim=hd))
    assert_exact(got, x0, "pos 0 identity")


# ---- Paged KV ------------------------------------------------------------------
def _cache(dev, n_blocks, block_size, stride, kv_kind):
    from fellm_amd.ops import PagedKvCache

    bb = PagedKvCache.block_bytes_for(stride, block_size)
    arena = torch.zeros(n_blocks * bb, dtype=torch.uint8, device=dev)
    return bb, arena


@pytest.mark.parametrize("kv_kind", ["f16", "bf16"])
@pytest.mark.parametrize("act", ["f32", "bf16"])
def test_kv_write_paged(ops, dev, kv_kind, act):
    from fellm_amd import synth
    from fellm_amd.ops import PagedKvCache

    rng = np.random.default_rng(21)
    batch, nkv, hd, bs, n_blocks, n_layers = 19, 2, 64, 16, 64, 2
    stride = nkv * hd
    pos, table, n_logical = synth.paged_layout(rng, batch, n_blocks, bs, 512, n_layers)
    bb, arena = _cache(dev, n_blocks, bs, stride, kv_kind)
    rows = random_stored(rng, (batch, stride), act)
    cache = PagedKvCache(arena, torch.from_numpy(table.view(np.int32)).to(dev), n_layers, n_logical, bs, bb, stride,
                         KINDS[kv_kind])
    ref = np.zeros(arena.numel(), np.uint8)
    for is_v in (False, True):
        ops.kv_write(to_dev(rows, act, dev), torch.from_numpy(pos.view(np.int32)).to(dev), cache, layer=1,
                     is_v=is_v)
        oracle.kv_write_paged(oracle.widen(rows, act), stride, pos, table, n_logical, n_layers, 1, bs, bb, ref,
                              is_v, kv_kind)
    sync()
    assert_exact(arena.cpu().numpy(), ref, "arena")


@pytest.mark.parametrize("kind,kv_kind,specials", [("bf16", "bf16", False), ("bf16", "bf16", True),
                                                   ("f32", "f16", False), ("f16", "f16", False)])
@pytest.mark.parametrize("pairing", [0, 1])
def test_rope_kv_write_fused(ops, dev, kind, kv_kind, specials, pairing):
    """specials: NaNs with payloads in V (stored unrotated, so their bits must
    survive the cache store: bf16 stores take the integer path for a lane
    holding a NaN) and infinities in rotated q and k elements."""
    from fellm_amd import synth
    from fellm_amd.ops import PagedKvCache

    rng = np.random.default_rng(31 + pairing)
    batch, nq, nkv, hd, bs, n_blocks = 33, 16, 2, 128, 16, 128
    stride = nkv * hd
    kv_pos, table, n_logical = synth.paged_layout(rng, batch, n_blocks, bs, 2048)
    rope_pos = kv_pos + 7
    inv = oracle.rope_inv_freqs(500000.0, hd)
    q = random_stored(rng, (batch, nq * hd), kind)
    k = random_stored(rng, (batch, stride), kind)
    v = random_stored(rng, (batch, stride), kind)
    if specials:
        v[3, 5], v[4, 9], v[4, 200] = 0x7FE1, 0xFFC3, 0x7FC0
        k[2, 0], q[1, 2], q[6, 77] = 0x7F80, 0xFF80, 0x7F80
    bb, arena = _cache(dev, n_blocks, bs, stride, kv_kind)
    cache = PagedKvCache(arena, torch.from_numpy(table.view(np.int32)).to(dev), 1, n_logical, bs, bb, stride,
                         KINDS[kv_kind])
    k_out = to_dev(np.zeros_like(k), kind, dev)
    qo = ops.rope_kv_write(to_dev(q, kind, dev), to_dev(k, kind, dev), to_dev(v, kind, dev),
                           torch.from_numpy(inv).to(dev), torch.from_numpy(kv_pos.view(np.int32)).to(dev), cache,
                           head_dim=hd, pairing=pairing,
                           rope_positions=torch.from_numpy(rope_pos.view(np.int32)).to(dev), k_out=k_out)
    sync()
    qf, kf = oracle.widen(q, kind), oracle.widen(k, kind)
    q_ref = oracle.rope(qf, nq, hd, hd, pairing, inv, rope_pos)
    k_ref = oracle.rope(kf, nkv, hd, hd, pairing, inv, rope_pos)
    assert_exact(from_dev(qo), oracle.narrow(q_ref, kind), "q")
    assert_exact(from_dev(k_out), oracle.narrow(k_ref, kind), "k_out")
    # V slots and K slots (the rotated K rounded once to the cache dtype): bit-exact.
    ref = np.zeros(arena.numel(), np.uint8)
    oracle.kv_write_paged(k_ref, stride, kv_pos, table, n_logical, 1, 0, bs, bb, ref, False, kv_kind)
    oracle.kv_write_paged(oracle.widen(v, kind), stride, kv_pos, table, n_logical, 1, 0, bs, bb, ref, True, kv_kind)
    got = arena.cpu().numpy()
    row_bytes = stride * 2
    for b in range(batch):
        phys = table[kv_pos[b] // bs]
        base = phys * bb + (kv_pos[b] % bs) * row_bytes
        vbase = base + bs * row_bytes
        assert_exact(got[vbase:vbase + row_bytes], ref[vbase:vbase + row_bytes], f"V row {b}")
        gk = got[base:base + row_bytes].view(np.uint16)
        rk = ref[base:base + row_bytes].view(np.uint16)
        assert_exact(gk, rk, f"K row {b}")
        got[base:base + row_bytes] = ref[base:base + row_bytes]
        got[vbase:vbase + row_bytes] = ref[vbase:vbase + row_bytes]
    assert_exact(got, ref, "untouched arena bytes")


def test_kv_write_out_of_range_flags(ops, dev):
    from fellm_amd.ops import PagedKvCache

    stride, bs = 64, 16
    bb, arena = _cache(dev, 4, bs, stride, "f16")
    # row 1, logical block 3 -> physical block 9, outside the 4-block arena
    table = np.array([0, 1, 2, 3, 0, 1, 2, 9], np.uint32)
    cache = PagedKvCache(arena, torch.from_numpy(table.view(np.int32)).to(dev), 1, 4, bs, bb, stride, torch.float16)
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    rows = torch.ones((2, stride), dtype=torch.float32, device=dev)
    pos = torch.tensor([5, 3 * bs + 1], dtype=torch.int32, device=dev)
    ops.kv_write(rows, pos, cache, err_flag=flag)
    sync()
    assert int(flag.item()) == 1
    a = arena.cpu().numpy()
    assert (a[5 * stride * 2: 6 * stride * 2].view(np.uint16) == 0x3C00).all()  # f16 1.0 in block 0 slot 5


# ---- Router --------------------------------------------------------------------
@pytest.mark.parametrize("n_exp,k", [(128, 8), (64, 6), (256, 8), (512, 32), (60, 1), (128, 128)])
@pytest.mark.parametrize("gating,norm,rsf", [(1, True, 0.0), (2, False, 2.5), (1, False, 1.0), (4, True, 0.0),
                                             (4, False, 2.5)])
def test_router_topk(ops, dev, n_exp, k, gating, norm, rsf):
    rng = np.random.default_rng(n_exp * 100 + k)
    tokens = 1023
    logits = rng.normal(size=(tokens, n_exp)).astype(np.float32)
    # constructed ties: equal logits in a few rows, and logits that differ by one ulp
    logits[0, :] = 0.5
    logits[1, : n_exp // 2] = logits[1, n_exp // 2 - 1]
    logits[2, 1] = np.nextafter(logits[2, 0], np.float32(np.inf))
    ids_ref, w_ref = oracle.router(logits, k, gating, norm, rsf)
    ids, w = ops.router_topk(torch.from_numpy(logits).to(dev), k, gating_func=gating, norm_topk_prob=norm,
                             routed_scaling_factor=rsf)
    assert_exact(from_dev(ids), ids_ref, "ids")
    assert_exact(from_dev(w), w_ref, "weights")


@pytest.mark.parametrize("gating", [1, 2])
@pytest.mark.parametrize("n_exp,k", [(128, 8), (128, 5), (256, 8), (64, 4)])
def test_router_near_ties_and_specials(ops, dev, gating, n_exp, k):
    """Rows built against the ranking's shortcut (unique 32-bit keys of
    truncated scores, checked for near-ties): logits one ulp apart at the
    rank k-1 / k boundary and inside the top k, exact duplicates of the k-th
    logit at a lower expert id, all-equal rows, -inf / +inf / NaN logits, and
    logits spread far enough that exp(l - max) falls under 2^-100 (the
    division's IEEE fallback).  Ids and weights bit-exact against the oracle
    on every row."""
    rng = np.random.default_rng(n_exp * 10 + k + gating)
    tokens = 4099
    logits = rng.normal(size=(tokens, n_exp)).astype(np.float32)
    order = np.argsort(-logits, axis=1, kind="stable")
    for r in range(0, 600, 3):  # one ulp above/below the k-th logit at another expert
        j_k, j_o = order[r, k - 1], order[r, k + 2]
        logits[r, j_o] = np.nextafter(logits[r, j_k], np.float32(np.inf if r % 2 else -np.inf))
    for r in range(1, 600, 3):  # an exact duplicate of the k-th logit
        logits[r, order[r, k + 1]] = logits[r, order[r, k - 1]]
    for r in range(2, 600, 3):  # a near-tie inside the top k
        logits[r, order[r, 1]] = np.nextafter(logits[r, order[r, 0]], np.float32(-np.inf))
    logits[700] = 1.25
    logits[701, :5] = -np.inf
    logits[702, 3] = np.inf
    logits[703, 7] = np.nan
    logits[704] *= 80.0  # e down to exp(-600): zero, and below 2^-100
    logits[705] = np.linspace(-90.0, 0.0, n_exp, dtype=np.float32)
    logits[706] = -12.0 * np.arange(n_exp, dtype=np.float32)  # selected e down to exp(-84), subnormal
    logits[707] = -np.float32(60.0) - np.arange(n_exp, dtype=np.float32) / 4  # e around 2^-87 .. 2^-133
    logits[707, 0] = 0.0
    ids_ref, w_ref = oracle.router(logits, k, gating, True, 0.0)
    ids, w = ops.router_topk(torch.from_numpy(logits).to(dev), k, gating_func=gating)
    got_ids, got_w = from_dev(ids), from_dev(w)
    assert_exact(got_ids, ids_ref, "ids")
    nan = np.isnan(w_ref) & np.isnan(got_w)
    assert_exact(np.where(nan, 0, got_w), np.where(nan, 0, w_ref), "weights")


@pytest.mark.parametrize("kind", ["f16", "bf16"])
@pytest.mark.parametrize("rows", [2051, 8193, 16385])
def test_rope_many_rows(ops, dev, kind, rows):
    """configs[4]'s RoPE shape (head_dim 128, 32 q / 4 kv heads, theta 1e6,
    positions 0..rows-1) at row counts on either side of the launcher's
    switch from one to two rows per workgroup (8192 rows; the row-group walk
    reads non-temporally), each with a ragged last workgroup; bit-exact
    against the oracle."""
    rng = np.random.default_rng(rows)
    nq, nk, hd = 32, 4, 128
    inv = oracle.rope_inv_freqs(1.0e6, hd)
    q = random_stored(rng, (rows, nq * hd), kind)
    k = random_stored(rng, (rows, nk * hd), kind)
    qr = oracle.narrow(oracle.rope(oracle.widen(q, kind), nq, hd, hd, 0, inv, None, position0=0), kind)
    kr = oracle.narrow(oracle.rope(oracle.widen(k, kind), nk, hd, hd, 0, inv, None, position0=0), kind)
    pos = torch.arange(rows, dtype=torch.int32, device=dev)
    qo, ko = ops.rope(to_dev(q, kind, dev), torch.from_numpy(inv).to(dev), head_dim=hd, pairing=0,
                      positions=pos, x2=to_dev(k, kind, dev))
    assert_exact(from_dev(qo), qr, f"q {rows} rows")
    assert_exact(from_dev(ko), kr, f"k {rows} rows")
    # split-half pairing and the position0 form through the same variants
    q1 = random_stored(rng, (rows, 2 * 64), "f32")
    r1 = oracle.rope(q1, 2, 64, 64, 1, oracle.rope_inv_freqs(10000.0, 64), None, position0=3)
    g1 = ops.rope(torch.from_numpy(q1).to(dev), torch.from_numpy(oracle.rope_inv_freqs(10000.0, 64)).to(dev),
                  head_dim=64, pairing=1, position0=3)
    assert_exact(from_dev(g1), r1, f"split-half {rows} rows")


@pytest.mark.parametrize("kind,nq,nk,hd,rd,pairing,inplace,rows", [
    ("f16", 32, 8, 128, 128, 0, False, 4099),
    ("bf16", 48, 16, 128, 64, 2, False, 6000),  # partial rotary
    ("f32", 8, 0, 64, 32, 1, True, 5000),       # in place, q only
    ("f16", 16, 4, 64, 64, 1, False, 4500),
    ("bf16", 24, 8, 256, 256, 0, True, 4097),   # head_dim 256, in place
    ("f16", 64, 16, 128, 128, 0, False, 4500),
])
def test_rope_many_rows_shapes(ops, dev, kind, nq, nk, hd, rd, pairing, inplace, rows):
    """Thousands of rows at other shapes: 1 to 5 (head) slots per thread per
    row, partial rotary, every pairing, in-place rotation, q alone, head_dim
    64 and 256; random positions; bit-exact against the oracle."""
    rng = np.random.default_rng(rows + hd + nq)
    inv = oracle.rope_inv_freqs(500000.0, rd)
    pos = rng.integers(0, 1 << 17, size=rows, dtype=np.uint32)
    q = random_stored(rng, (rows, nq * hd), kind)
    qr = oracle.narrow(oracle.rope(oracle.widen(q, kind), nq, hd, rd, pairing, inv, pos), kind)
    posd = torch.from_numpy(pos.view(np.int32)).to(dev)
    invd = torch.from_numpy(inv).to(dev)
    qd = to_dev(q, kind, dev)
    if nk:
        k = random_stored(rng, (rows, nk * hd), kind)
        kr = oracle.narrow(oracle.rope(oracle.widen(k, kind), nk, hd, rd, pairing, inv, pos), kind)
        kd = to_dev(k, kind, dev)
        qo, ko = ops.rope(qd, invd, head_dim=hd, rope_dim=rd, pairing=pairing, positions=posd, x2=kd,
                          inplace=inplace)
        assert_exact(from_dev(ko), kr, f"k {rows} rows")
    else:
        qo = ops.rope(qd, invd, head_dim=hd, rope_dim=rd, pairing=pairing, positions=posd, inplace=inplace)
    assert_exact(from_dev(qo), qr, f"q {rows} rows")


@pytest.mark.parametrize("kind,group,residual,inplace", [("bf16", 2048, False, False), ("f16", 1024, True, False),
                                                          ("bf16", 512, True, True), ("f32", 1024, True, False)])
@pytest.mark.parametrize("rows", [16384, 20011])
def test_add_rmsnorm_wavefront_rows(ops, dev, kind, group, residual, inplace, rows):
    """Tens of thousands of rows of at most 4 KB (one wavefront per row):
    plain RMSNorm and the residual form, h written in place over x; bit-exact
    h, y within the RMSNorm tolerance."""
    rng = np.random.default_rng(rows + group)
    x = random_stored(rng, (rows, group), kind)
    w = rng.normal(1.0, 0.1, size=group).astype(np.float32)
    xw = oracle.widen(x, kind)
    if residual:
        r = random_stored(rng, (rows, group), kind, sigma=4.0)
        h_ref, y_ref = oracle.add_rmsnorm(x, r, w, 1e-5, kind)
        xd = to_dev(x, kind, dev)
        h_out = xd if inplace else None
        h, y = ops.add_rmsnorm(xd, to_dev(r, kind, dev), torch.from_numpy(w).to(dev), 1e-5, h_out=h_out)
        assert_exact(from_dev(h), h_ref, f"h {rows}x{group}")
    else:
        y_ref = oracle.narrow(oracle.rmsnorm(xw, w, 1e-5), kind)
        y = ops.rmsnorm(to_dev(x, kind, dev), torch.from_numpy(w).to(dev), 1e-5)
    assert_close(from_dev(y), y_ref, kind, what=f"y {rows}x{group}")


@pytest.mark.parametrize("kind", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("rows,group", [(1024, 2048), (1031, 1000), (1024, 8192), (1029, 16384), (1024, 12288)])
def test_add_rmsnorm_many_rows(ops, dev, kind, rows, group):
    """>= 1024 rows select the 256-thread layouts: NCHUNK = 1 (group <= 2048),
    4 (<= 8192) and 8 (<= 16384) chunks of 8 elements per thread, plus the
    two-pass fallback for a group that is not a multiple of 8."""
    rng = np.random.default_rng(rows * 31 + group)
    x = random_stored(rng, (rows, group), kind)
    r = random_stored(rng, (rows, group), kind, sigma=2.0)
    w = rng.normal(1.0, 0.1, size=group).astype(np.float32)
    h_ref, y_ref = oracle.add_rmsnorm(x, r, w, 1e-6, kind)
    h, y = ops.add_rmsnorm(to_dev(x, kind, dev), to_dev(r, kind, dev), torch.from_numpy(w).to(dev), 1e-6)
    assert_exact(from_dev(h), h_ref, f"h {kind}")
    assert_close(from_dev(y), y_ref, kind, what=f"y {kind} {rows}x{group}")
    y_plain = ops.rmsnorm(to_dev(x, kind, dev), torch.from_numpy(w).to(dev), 1e-6)
    assert_close(from_dev(y_plain), oracle.narrow(oracle.rmsnorm(oracle.widen(x, kind), w, 1e-6), kind), kind,
                 what=f"plain {kind} {rows}x{group}")


def test_rmsnorm_c5_shape(ops, dev):
    """configs[4]'s RMSNorm as the bench times it: 16384 x 2048 bf16, eps 1e-6."""
    rng = np.random.default_rng(16384)
    x = random_stored(rng, (16384, 2048), "bf16")
    w = rng.normal(1.0, 0.1, size=2048).astype(np.float32)
    y = ops.rmsnorm(to_dev(x, "bf16", dev), torch.from_numpy(w).to(dev), 1e-6)
    ref = oracle.narrow(oracle.rmsnorm(oracle.widen(x, "bf16"), w, 1e-6), "bf16")
    assert_close(from_dev(y), ref, "bf16", what="c5 rmsnorm")


# ---- Cast (backend.rs:1603-1667) ---------------------------------------------------
def _cast(ops, src, sdt, ddt, n, out_np_dtype, dev):
    from fellm_amd import _lib

    s = torch.from_numpy(np.ascontiguousarray(src)).to(dev)
    out = torch.empty(n * np.dtype(out_np_dtype).itemsize, dtype=torch.uint8, device=dev)
    _lib.call("fellm_rocm_cast", s.data_ptr(), int(sdt), out.data_ptr(), int(ddt), n,
              torch.cuda.current_stream().cuda_stream)
    return out.cpu().numpy().view(out_np_dtype)


@pytest.mark.parametrize("n", [1, 7, 4096, 3 * 4096 + 8, 1 << 20])
def test_cast_dense_pairs(ops, dev, n):
    """f16/bf16 -> f32 widen exactly, f32 -> f16 rounds to nearest even,
    f32 -> bf16 truncates (the CPU backend's Cast, unlike the RNE used for
    kernel outputs); includes ties, subnormals, infinities and NaN."""
    from fellm_amd.abi import DType

    rng = np.random.default_rng(n)
    x = (rng.normal(size=n) * np.exp(rng.uniform(-30, 30, size=n))).astype(np.float32)
    specials = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11, 65520.0, 1e-8,
                         1.0 + 2.0 ** -8, 3.0e38], np.float32)
    x[: min(n, specials.size)] = specials[: min(n, specials.size)]
    h = oracle.f32_to_f16_bits(x)
    b = oracle.f32_to_bf16_bits(x)
    assert np.array_equal(_cast(ops, x, DType.F32, DType.F32, n, np.uint32, dev), x.view(np.uint32))
    assert np.array_equal(_cast(ops, x, DType.F32, DType.F16, n, np.uint16, dev), h)
    assert np.array_equal(_cast(ops, x, DType.F32, DType.BF16, n, np.uint16, dev),
                          oracle.f32_to_bf16_bits(x, truncate=True))
    assert np.array_equal(_cast(ops, h, DType.F16, DType.F32, n, np.uint32, dev),
                          oracle.widen(h, "f16").view(np.uint32))
    assert np.array_equal(_cast(ops, b, DType.BF16, DType.F32, n, np.uint32, dev),
                          oracle.widen(b, "bf16").view(np.uint32))


@pytest.mark.parametrize("dtype,blocks", [(12, 1), (12, 37), (14, 16), (14, 129)])
def test_cast_kquant_to_f32(ops, dev, dtype, blocks):
    from fellm_amd import synth

    rng = np.random.default_rng(dtype * blocks)
    w = synth.KQUANT_TABLES[dtype](rng, blocks, 256).ravel()
    got = _cast(ops, w, dtype, 0, blocks * 256, np.float32, dev)  # 0 = F32
    assert np.array_equal(got.view(np.uint32), oracle.dequantize_row(dtype, w, blocks * 256).view(np.uint32))


def test_cast_rejects_other_pairs(ops, dev):
    from fellm_amd import _lib
    from fellm_amd.abi import DType

    a = torch.zeros(64, dtype=torch.float16, device=dev)
    b = torch.zeros(64, dtype=torch.bfloat16, device=dev)
    rc = _lib.lib().fellm_rocm_cast(a.data_ptr(), int(DType.F16), b.data_ptr(), int(DType.BF16), 64,
                                    torch.cuda.current_stream().cuda_stream)
    assert rc == -10


def test_zero_rows_are_noops(ops, dev):
    """Empty inputs succeed and write nothing, as the CPU backend's loops run
    zero times (backend.rs:1026-1046, 1104-1133, 1135-1172, 1174-1184;
    moe.rs:820-855)."""
    H, hd = 256, 64
    f16 = torch.float16
    e = torch.empty(0, H, dtype=f16, device=dev)
    w = torch.ones(H, device=dev)
    assert ops.silu_gate(e.view(-1), e.view(-1)).numel() == 0
    ops.add_rmsnorm(e, e, w, 1e-5, h_out=torch.empty_like(e), y_out=torch.empty_like(e))
    ops.rmsnorm(e, w, 1e-5, out=torch.empty_like(e))
    table = torch.randn(16, H, device=dev).half()
    assert ops.embedding(table, torch.empty(0, dtype=torch.int32, device=dev)).numel() == 0
    inv = ops.rope_inv_freqs(10000.0, hd).to(dev)
    assert ops.rope(e, inv, head_dim=hd).numel() == 0
    ids, wts = ops.router_topk(torch.empty(0, 8, device=dev), 2)
    assert ids.numel() == 0 and wts.numel() == 0
    torch.cuda.synchronize()



@pytest.mark.parametrize("offset", [2, 6, 10, 14])
@pytest.mark.parametrize("dim", [256, 3584, 16384])
def test_embedding_q6k_unaligned_table(ops, dev, offset, dim):
    """Q6_K tables need only 2-byte alignment (210-byte blocks): a table that
    starts `offset` bytes past a 16-byte boundary shifts every row's span
    against the 16-byte loads that copy it; bit-exact against the oracle."""
    from fellm_amd import synth

    rng = np.random.default_rng(offset * 1000 + dim)
    vocab = 97
    table = synth.q6k_table(rng, vocab, dim)
    ids = synth.zipf_ids(rng, 300, vocab)
    ref = oracle.narrow(oracle.embedding(table, 14, vocab, dim, ids), "f16")
    buf = torch.zeros(table.size + 16, dtype=torch.uint8, device=dev)
    buf[offset:offset + table.size] = torch.from_numpy(table.reshape(-1)).to(dev)
    got = ops.embedding(buf[offset:offset + table.size].view(table.shape), torch.from_numpy(ids.view(np.int32)).to(dev), dim=dim,
                        qtype="q6k", out_dtype=KINDS["f16"])
    assert_exact(from_dev(got), ref, f"embedding q6k table offset {offset} dim={dim}")


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
@pytest.mark.parametrize("dim,store_h", [(256, True), (2048, False), (3584, True), (4096, True), (6144, False)])
def test_embedding_kquant_rmsnorm_rows(ops, dev, qtype, dim, store_h):
    """Fused Q4_K / Q6_K gather + RMSNorm over thousands of Zipf rows with
    out-of-range ids (zero rows, flag set), with and without the h output;
    rows of up to 4096 elements take the one-wavefront LDS layout, longer
    ones the staged layout.  h bit-exact, y within the RMSNorm tolerance."""
    from fellm_amd import synth

    rng = np.random.default_rng(dim + store_h + len(qtype))
    vocab, n_rows = 400, 2051
    code = 12 if qtype == "q4k" else 14
    table = synth.q4k_table(rng, vocab, dim) if qtype == "q4k" else synth.q6k_table(rng, vocab, dim)
    ids = synth.zipf_ids(rng, n_rows, vocab)
    bad = rng.choice(n_rows, size=3, replace=False)
    ids[bad] = vocab + np.arange(3, dtype=np.uint32)
    ok = ids < vocab
    e = np.zeros((n_rows, dim), np.float32)
    e[ok] = oracle.embedding(table, code, vocab, dim, ids[ok])
    w = rng.normal(1.0, 0.1, size=dim).astype(np.float32)
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    h, y = ops.embedding_rmsnorm(torch.from_numpy(table).to(dev), torch.from_numpy(ids.view(np.int32)).to(dev),
                                 torch.from_numpy(w).to(dev), 1e-6, dim=dim, qtype=qtype,
                                 out_dtype=KINDS["bf16"], store_h=store_h, err_flag=flag)
    assert int(flag.item()) == 1
    if store_h:
        assert_exact(from_dev(h), oracle.narrow(e, "bf16"), f"{qtype} fused h dim {dim}")
    assert_close(from_dev(y), oracle.narrow(oracle.rmsnorm(e, w, 1e-6), "bf16"), "bf16",
                 what=f"{qtype} fused y dim {dim}")
