"""Pins the oracle's paged decode attention (reference_attention_paged_f32,
crates/fellm-plugin-abi/src/attention_provider.rs:391-459, driven per batch
row as crates/backend-cpu/src/backend.rs:1286-1323).

Pins: float64 softmax attention recomputed from the f16 cache values (a wrong
KV-head mapping, scale, window or block address fails it); closed forms (one
key gives v exactly, q = 0 gives the mean of v); storage invariance (a
scrambled block table over the same logical rows gives identical bits); the
reference's own decode test inputs (attention_provider.rs:494-549).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle


def build_cache(rng, k, v, block_size=16, n_layers=1, layer=0, kind="f16", scramble=True):
    """k, v: f32 [B][seq_b, stride] lists -> (arena u8, table u32, n_logical, block_bytes, k16, v16)."""
    B = len(k)
    stride = k[0].shape[1]
    max_seq = max(max(x.shape[0] for x in k), 1)
    n_logical = (max_seq + block_size - 1) // block_size
    block_bytes = ((2 * block_size * stride * 2) + 63) // 64 * 64
    n_blocks = B * n_layers * n_logical
    perm = rng.permutation(n_blocks) if scramble else np.arange(n_blocks)
    table = perm.astype(np.uint32)
    arena = np.zeros(n_blocks * block_bytes, np.uint8)
    k16, v16 = [], []
    for r in range(B):
        kb = oracle.narrow(k[r], kind) if k[r].size else np.zeros((0, stride), np.uint16)
        vb = oracle.narrow(v[r], kind) if v[r].size else np.zeros((0, stride), np.uint16)
        k16.append(oracle.widen(kb, kind).reshape(-1, stride))
        v16.append(oracle.widen(vb, kind).reshape(-1, stride))
        for t in range(k[r].shape[0]):
            phys = table[(r * n_layers + layer) * n_logical + t // block_size]
            base = phys * block_bytes + (t % block_size) * stride * 2
            arena[base:base + stride * 2] = kb[t].view(np.uint8)
            vbase = base + block_size * stride * 2
            arena[vbase:vbase + stride * 2] = vb[t].view(np.uint8)
    return arena, table, n_logical, block_bytes, k16, v16


def attention_f64(q, k16, v16, n_heads, n_kv, hd, scale, window=0):
    B = q.shape[0]
    out = np.zeros((B, n_heads * hd))
    group = n_heads // n_kv
    for r in range(B):
        seq = k16[r].shape[0]
        lo = max(0, seq - window) if window else 0
        for h in range(n_heads):
            g = h // group
            if seq - lo <= 0:
                continue
            kk = k16[r][lo:, g * hd:(g + 1) * hd].astype(np.float64)
            vv = v16[r][lo:, g * hd:(g + 1) * hd].astype(np.float64)
            s = kk @ q[r, h * hd:(h + 1) * hd].astype(np.float64) * np.float64(np.float32(scale))
            p = np.exp(s - s.max())
            out[r, h * hd:(h + 1) * hd] = (p[:, None] * vv).sum(0) / p.sum()
    return out


def run(q, k, v, n_heads, n_kv, hd, scale, window=0, kind="f16", seed=0, scramble=True):
    rng = np.random.default_rng(seed)
    arena, table, n_logical, bb, k16, v16 = build_cache(rng, k, v, kind=kind, scramble=scramble)
    lengths = np.array([x.shape[0] for x in k], np.uint32)
    got = oracle.paged_attention(q, n_heads, n_kv, hd, lengths, scale, arena, table, n_logical, 1, 0, 16, bb,
                                 causal=True, window=window, kind=kind)
    return got, attention_f64(q, k16, v16, n_heads, n_kv, hd, scale, window), v16


def check_close(got, ref, v16, n_heads, n_kv, hd, tol=2e-6):
    group = n_heads // n_kv
    for r in range(got.shape[0]):
        vmax = np.abs(v16[r]).max() if v16[r].size else 0.0
        err = np.abs(got[r] - ref[r])
        assert err.max() <= tol * max(vmax, 1e-30) + 1e-30, (r, err.max(), vmax)


@pytest.mark.parametrize("n_heads,n_kv,hd", [(4, 2, 8), (8, 1, 64), (64, 8, 128), (32, 4, 128)])
@pytest.mark.parametrize("kind", ["f16", "bf16"])
def test_paged_attention_matches_f64(n_heads, n_kv, hd, kind):
    rng = np.random.default_rng(n_heads + hd)
    lengths = [1, 17, 40, 5]
    q = rng.normal(size=(len(lengths), n_heads * hd)).astype(np.float32)
    k = [rng.normal(size=(n, n_kv * hd)).astype(np.float32) for n in lengths]
    v = [rng.normal(size=(n, n_kv * hd)).astype(np.float32) for n in lengths]
    scale = 1.0 / np.sqrt(hd)
    got, ref, v16 = run(q, k, v, n_heads, n_kv, hd, scale, kind=kind)
    check_close(got, ref, v16, n_heads, n_kv, hd)


@pytest.mark.parametrize("window", [1, 7, 16, 100])
def test_paged_attention_window(window):
    rng = np.random.default_rng(window)
    n_heads, n_kv, hd = 8, 2, 32
    lengths = [50, 3, 17]
    q = rng.normal(size=(3, n_heads * hd)).astype(np.float32)
    k = [rng.normal(size=(n, n_kv * hd)).astype(np.float32) for n in lengths]
    v = [rng.normal(size=(n, n_kv * hd)).astype(np.float32) for n in lengths]
    got, ref, v16 = run(q, k, v, n_heads, n_kv, hd, 0.2, window=window)
    check_close(got, ref, v16, n_heads, n_kv, hd)


def test_paged_attention_closed_forms():
    rng = np.random.default_rng(3)
    n_heads, n_kv, hd = 4, 2, 16
    # one key: p = 1, l = 1 -> out = v exactly
    k = [rng.normal(size=(1, n_kv * hd)).astype(np.float32)]
    v = [rng.normal(size=(1, n_kv * hd)).astype(np.float32)]
    q = rng.normal(size=(1, n_heads * hd)).astype(np.float32)
    got, _, v16 = run(q, k, v, n_heads, n_kv, hd, 0.25)
    for h in range(n_heads):
        g = h // 2
        assert np.array_equal(got[0, h * hd:(h + 1) * hd], v16[0][0, g * hd:(g + 1) * hd])
    # q = 0: every score 0, uniform softmax -> mean of v
    n = 37
    k = [rng.normal(size=(n, n_kv * hd)).astype(np.float32)]
    v = [rng.normal(size=(n, n_kv * hd)).astype(np.float32)]
    got, _, v16 = run(np.zeros((1, n_heads * hd), np.float32), k, v, n_heads, n_kv, hd, 0.25)
    for h in range(n_heads):
        g = h // 2
        mean = v16[0][:, g * hd:(g + 1) * hd].astype(np.float64).mean(0)
        assert np.abs(got[0, h * hd:(h + 1) * hd] - mean).max() < 1e-6
    # empty sequence -> zeros
    got, _, _ = run(q, [np.zeros((0, n_kv * hd), np.float32)], [np.zeros((0, n_kv * hd), np.float32)], n_heads,
                    n_kv, hd, 0.25)
    assert np.all(got == 0.0)


def test_paged_attention_storage_invariance():
    rng = np.random.default_rng(9)
    n_heads, n_kv, hd = 8, 2, 64
    lengths = [33, 70]
    q = rng.normal(size=(2, n_heads * hd)).astype(np.float32)
    k = [rng.normal(size=(n, n_kv * hd)).astype(np.float32) for n in lengths]
    v = [rng.normal(size=(n, n_kv * hd)).astype(np.float32) for n in lengths]
    a, _, _ = run(q, k, v, n_heads, n_kv, hd, 0.125, scramble=True, seed=1)
    b, _, _ = run(q, k, v, n_heads, n_kv, hd, 0.125, scramble=False, seed=2)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_reference_decode_inputs():
    """attention_provider.rs:494-549 inputs (4 heads, 2 kv heads, hd 8, 17 keys,
    scale 1/sqrt(8)); the reference asserts its FA2 path within 1e-4 of the
    serial reference.  Here: the oracle (serial reference over the f16 cache)
    against float64 on the same cache values."""
    n_heads, n_kv, hd, kv_len = 4, 2, 8, 17
    q = ((np.arange(n_heads * hd) * 17) % 13).astype(np.float32) * np.float32(0.1) - np.float32(0.5)
    kf = ((np.arange(n_kv * kv_len * hd) * 7) % 11).astype(np.float32) * np.float32(0.1) - np.float32(0.3)
    vf = ((np.arange(n_kv * kv_len * hd) * 3) % 9).astype(np.float32) * np.float32(0.05)
    # the reference's contiguous layout is (kj * n_kv + kv_h) * hd: token-major rows of stride n_kv*hd
    k = [kf.reshape(kv_len, n_kv * hd)]
    v = [vf.reshape(kv_len, n_kv * hd)]
    got, ref, v16 = run(q.reshape(1, -1), k, v, n_heads, n_kv, hd, float(np.float32(1.0 / np.sqrt(8.0))))
    assert np.abs(got - ref).max() < 1e-6


# ---- non-paged attention (contiguous decode, canvas) ------------------------------
def _f64_attention(q, n_heads, n_kv, hd, keys, vals, scale):
    """float64 softmax attention of every query row over the key list."""
    rows = q.shape[0]
    out = np.zeros((rows, n_heads * hd))
    g = n_heads // n_kv
    for r in range(rows):
        for h in range(n_heads):
            kh = h // g
            qh = q[r, h * hd:(h + 1) * hd].astype(np.float64)
            if len(keys) == 0:
                continue
            K = keys[:, kh * hd:(kh + 1) * hd].astype(np.float64)
            V = vals[:, kh * hd:(kh + 1) * hd].astype(np.float64)
            s = K @ qh * scale
            p = np.exp(s - s.max())
            out[r, h * hd:(h + 1) * hd] = (p / p.sum()) @ V
    return out


@pytest.mark.parametrize("n_heads,n_kv,hd,seq", [(8, 2, 64, 37), (32, 8, 128, 300), (4, 4, 80, 5), (16, 1, 128, 1)])
def test_attention_f32kv_matches_f64(n_heads, n_kv, hd, seq):
    rng = np.random.default_rng(seq + hd)
    q = rng.normal(size=(1, n_heads * hd)).astype(np.float32)
    k = rng.normal(size=(seq, n_kv * hd)).astype(np.float32)
    v = rng.normal(size=(seq, n_kv * hd)).astype(np.float32)
    scale = float(np.float32(1) / np.sqrt(np.float32(hd)))
    got = oracle.attention_f32kv(q, n_heads, n_kv, hd, k, v, 0, seq)
    ref = _f64_attention(q, n_heads, n_kv, hd, k, v, scale)
    assert np.abs(got - ref).max() <= 2e-6 * max(1.0, np.abs(v).max())


def test_attention_f32kv_closed_forms_and_segments():
    rng = np.random.default_rng(21)
    nh, nkv, hd = 4, 2, 64
    q = rng.normal(size=(3, nh * hd)).astype(np.float32)
    k = rng.normal(size=(20, nkv * hd)).astype(np.float32)
    v = rng.normal(size=(20, nkv * hd)).astype(np.float32)
    # one key: the output is that key's V row, exactly
    one = oracle.attention_f32kv(q[:1], nh, nkv, hd, k, v, 7, 8)
    for h in range(nh):
        assert np.array_equal(one[0, h * hd:(h + 1) * hd], v[7, (h // 2) * hd:(h // 2 + 1) * hd])
    # q = 0: uniform weights, the mean of V
    z = oracle.attention_f32kv(np.zeros((1, nh * hd), np.float32), nh, nkv, hd, k, v, 0, 20)
    assert np.allclose(z[0, :hd], v[:, :hd].mean(axis=0), atol=1e-6)
    # no keys: zero rows
    assert not oracle.attention_f32kv(q, nh, nkv, hd, k, v, 5, 5).any()
    # two segments == one concatenated segment (canvas = prefix keys then canvas keys)
    two = oracle.attention_f32kv(q, nh, nkv, hd, k[:12], v[:12], 4, 12, k[12:], v[12:], 8)
    cat = oracle.attention_f32kv(q, nh, nkv, hd, k[4:], v[4:], 0, 16)
    assert np.array_equal(two, cat)
    scale = float(np.float32(1) / np.sqrt(np.float32(hd)))
    assert np.abs(two - _f64_attention(q, nh, nkv, hd, k[4:], v[4:], scale)).max() < 2e-6 * np.abs(v).max()


def _masked_softmax_f64(q, k, v, nh, nkv, hd, ql, kvl, scale, causal, window):
    """Dense f64 restatement from the mask rules alone (one explicit mask
    matrix, no tiles or online softmax): q head-major [nh, ql, hd]."""
    qh = q.reshape(nh, ql, hd).astype(np.float64)
    kh = k.reshape(kvl, nkv, hd).astype(np.float64)
    vh = v.reshape(kvl, nkv, hd).astype(np.float64)
    qi = np.arange(ql)[:, None]
    kj = np.arange(kvl)[None, :]
    if causal:
        bound = kvl - ql + qi
        allow = kj <= bound
        if window:
            allow &= (bound - kj) < window
    elif window:
        allow = np.abs(qi - kj) < window
    else:
        allow = np.ones((ql, kvl), bool)
    out = np.zeros((nh, ql, hd))
    g = nh // nkv
    for h in range(nh):
        s = qh[h] @ kh[:, h // g].T * scale
        s = np.where(allow, s, -np.inf)
        mx = s.max(axis=1, keepdims=True)
        e = np.where(allow, np.exp(s - np.where(np.isfinite(mx), mx, 0)), 0.0)
        den = e.sum(axis=1, keepdims=True)
        out[h] = np.where(den > 0, (e / np.where(den > 0, den, 1)) @ vh[:, h // g], 0.0)
    return out.reshape(-1)


@pytest.mark.parametrize("ql,kvl,causal,window", [(1, 37, True, 0), (5, 37, True, 0), (16, 16, True, 0),
                                                  (20, 70, True, 8), (7, 33, False, 0), (9, 40, False, 5),
                                                  (33, 33, True, 1)])
def test_fa2_attention_matches_masked_f64(ql, kvl, causal, window):
    """The host FA2 restatement against a dense f64 softmax built from the
    mask rules alone (attention_provider.rs:306-318): causal bound
    kv_len - query_len + qi with its window, the non-causal |qi - kj| window.
    A dropped mask term, a wrong offset or a transposed head/row index fails."""
    rng = np.random.default_rng(ql * 100 + kvl + window)
    nh, nkv, hd = 8, 2, 32
    q = rng.normal(size=nh * ql * hd).astype(np.float32)
    k = rng.normal(size=(kvl, nkv * hd)).astype(np.float32)
    v = rng.normal(size=(kvl, nkv * hd)).astype(np.float32)
    scale = float(np.float32(1 / np.sqrt(hd)))
    got = oracle.fa2_attention(q, k, v, nh, nkv, hd, ql, kvl, scale, causal, window)
    ref = _masked_softmax_f64(q, k, v, nh, nkv, hd, ql, kvl, scale, causal, window)
    assert np.abs(got - ref).max() <= 2e-5 * np.abs(v).max()
    # Tiles of other sizes reorder the online softmax only.
    alt = oracle.fa2_attention(q, k, v, nh, nkv, hd, ql, kvl, scale, causal, window, q_tile=4, kv_tile=64)
    assert np.abs(alt - got).max() <= 2e-5 * np.abs(v).max()


def test_fa2_attention_one_row_equals_decode_oracle():
    """query_len 1, causal: the decode form (keys 0..kv_len) of the two-pass oracle."""
    rng = np.random.default_rng(5)
    nh, nkv, hd, kvl = 16, 4, 64, 90
    q = rng.normal(size=nh * hd).astype(np.float32)
    k = rng.normal(size=(kvl, nkv * hd)).astype(np.float32)
    v = rng.normal(size=(kvl, nkv * hd)).astype(np.float32)
    scale = float(np.float32(1 / np.sqrt(hd)))
    got = oracle.fa2_attention(q, k, v, nh, nkv, hd, 1, kvl, scale, True)
    ref = oracle.attention_f32kv(q[None], nh, nkv, hd, k, v, 0, kvl, scale=scale)[0]
    assert np.abs(got - ref).max() <= 2e-5 * np.abs(v).max()
