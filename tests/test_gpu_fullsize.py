"""Parity at the BASELINE configs' full sizes, on the kernels the bench times.

Each config's chain is built exactly as bench.py builds it (same shapes,
seeds and launch paths), run once, and 64-128 seeded sample rows of every
op's output are compared with the oracle on the same input rows:
  * configs[0] (Llama-3.2-1B, 64 tokens, f32; every row): embedding gather
    from the full 128256 x 2048 table, RMSNorm (alone and fused with a
    residual add), RoPE q+k 32/8 heads at positions 0..63, SwiGLU 64 x 8192;
  * configs[1] (Llama-3-8B prefill, T 4096, f16): embedding gather, residual
    add + RMSNorm, RoPE q+k, SwiGLU;
  * configs[2] (Qwen2-7B, Q4_K / Q6_K tables 152064 x 3584, Zipf ids): both
    gathers and the fused gather + RMSNorm; Q5_K and Q8_0 tables of the same
    shape;
  * configs[3] (Llama-3-70B decode, 256 sequences, 4.29 GB bf16 paged arena):
    RoPE + K/V append (q rows and the K/V slot bytes), add + RMSNorm, SwiGLU;
  * configs[4] (Qwen3-30B-A3B, 16384 tokens): router top-8 (every row),
    routed SwiGLU, RMSNorm, RoPE q+k.
Bars: bit-exact for gathers, residual sums, RoPE, K/V slots, SwiGLU and the
router; RMSNorm y within 1 ulp of the 16-bit output.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from parity_util import assert_close, assert_exact

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

SAMPLES = 64


@pytest.fixture(scope="module")
def ops():
    from fellm_amd import ops as _ops

    return _ops


def _rows(t: torch.Tensor, idx: np.ndarray) -> np.ndarray:
    """Host copy of rows `idx` of a 2-D device tensor, as f32 values or 16-bit bits."""
    sel = t[torch.from_numpy(idx.astype(np.int64)).to(t.device)].cpu()
    if sel.dtype == torch.float32:
        return sel.numpy()
    return sel.view(torch.int16).numpy().view(np.uint16)


def _kind(t: torch.Tensor) -> str:
    return {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}[t.dtype]


def _sample(rng, n, k=SAMPLES):
    idx = rng.choice(n, size=min(k, n), replace=False)
    return np.sort(np.concatenate([idx, [0, n - 1]])).astype(np.int64)


def _run(chain, s):
    for op in chain:
        op.fn(s)
    torch.cuda.synchronize()


def test_c1_chain_full_size(ops, dev):
    """configs[0] as stated: one seed; table ~N(0, 0.02) of 128256 x 2048 f32,
    64 uniform ids, RMSNorm weight ~N(1, 0.1) at eps 1e-5, RoPE hd 64 with 32 Q
    and 8 KV heads at theta 5e5 and positions 0..63, gate and up ~N(0, 1) of
    64 x 8192.  The gathered rows feed the RMSNorm, as in the model."""
    V, H, T, nq, nkv, hd, I = 128256, 2048, 64, 32, 8, 64, 8192
    rng = np.random.default_rng(100)
    table = np.empty((V, H), np.float32)
    for i in range(0, V, 16384):  # f32 draws, in slices to bound host memory
        n = min(16384, V - i)
        table[i:i + n] = rng.standard_normal(size=(n, H), dtype=np.float32) * np.float32(0.02)
    ids = rng.integers(0, V, size=T, dtype=np.uint32)
    w = (1.0 + 0.1 * rng.standard_normal(size=H)).astype(np.float32)
    r = (2.0 * rng.standard_normal(size=(T, H))).astype(np.float32)
    q = rng.standard_normal(size=(T, nq * hd)).astype(np.float32)
    k = rng.standard_normal(size=(T, nkv * hd)).astype(np.float32)
    g = rng.standard_normal(size=(T, I)).astype(np.float32)
    u = rng.standard_normal(size=(T, I)).astype(np.float32)

    def d(a):
        return torch.from_numpy(a).to(dev)

    tab_d = d(table)
    del table
    emb = ops.embedding(tab_d, d(ids.view(np.int32)), out_dtype=torch.float32)
    w_d = d(w)
    y = ops.rmsnorm(emb, w_d, 1e-5)
    h2, y2 = ops.add_rmsnorm(emb, d(r), w_d, 1e-5)
    inv = ops.rope_inv_freqs(500000.0, hd).to(dev)
    qo, ko = ops.rope(d(q), inv, head_dim=hd, x2=d(k))
    act = ops.silu_gate(d(g), d(u))
    torch.cuda.synchronize()
    rows = tab_d[torch.from_numpy(ids.astype(np.int64)).to(dev)].cpu().numpy()
    e_ref = oracle.embedding(rows.view(np.uint8), 0, T, H, np.arange(T, dtype=np.uint32))
    assert_exact(emb.cpu().numpy(), e_ref, "c1 embedding")
    assert_close(y.cpu().numpy(), oracle.rmsnorm(e_ref, w, 1e-5), "f32", what="c1 rmsnorm")
    h_ref, y2_ref = oracle.add_rmsnorm(e_ref, r, w, 1e-5, "f32")
    assert_exact(h2.cpu().numpy(), h_ref, "c1 h")
    assert_close(y2.cpu().numpy(), y2_ref, "f32", what="c1 add + rmsnorm")
    inv_ref = oracle.rope_inv_freqs(500000.0, hd)
    pos = np.arange(T, dtype=np.uint32)
    assert_exact(qo.cpu().numpy(), oracle.rope(q, nq, hd, hd, 0, inv_ref, pos), "c1 rope q")
    assert_exact(ko.cpu().numpy(), oracle.rope(k, nkv, hd, hd, 0, inv_ref, pos), "c1 rope k")
    assert_exact(act.cpu().numpy(), oracle.silu_gate(g, u), "c1 swiglu")


def test_c2_chain_full_size(ops, dev):
    import bench

    chain, sets, T = bench.c2_ops(torch, ops, dev, 1)
    s = sets[0]
    _run(chain, s)
    rng = np.random.default_rng(401)
    idx = _sample(rng, T)
    # embedding: out[t] = table[ids[t]] (f16 copy)
    ids = s["ids"].cpu().numpy().view(np.uint32)
    tab_rows = _rows(bench_table(chain), ids[idx])
    assert_exact(_rows(s["emb"], idx), tab_rows, "c2 embedding rows")
    # add + RMSNorm
    w = bench_norm_weight(chain)
    h_ref, y_ref = oracle.add_rmsnorm(_rows(s["x"], idx), _rows(s["r"], idx), w, 1e-5, "f16")
    assert_exact(_rows(s["h"], idx), h_ref, "c2 h")
    assert_close(_rows(s["y"], idx), y_ref, "f16", what="c2 y")
    # RoPE q + k at positions 0..T-1
    inv = oracle.rope_inv_freqs(500000.0, 128)
    pos = idx.astype(np.uint32)
    for src, dst, nh in (("q", "qo", 32), ("k", "ko", 8)):
        ref = oracle.narrow(oracle.rope(oracle.widen(_rows(s[src], idx), "f16"), nh, 128, 128, 0, inv, pos), "f16")
        assert_exact(_rows(s[dst], idx), ref, f"c2 rope {src}")
    # SwiGLU
    g, u = oracle.widen(_rows(s["gate"], idx), "f16"), oracle.widen(_rows(s["up"], idx), "f16")
    assert_exact(_rows(s["act"], idx), oracle.narrow(oracle.silu_gate(g, u), "f16"), "c2 swiglu")


def bench_table(chain):
    """The embedding table tensor the c2 embedding op closes over."""
    return _closure(chain[0].fn, "table")


def bench_norm_weight(chain):
    return _closure(chain[1].fn, "w_norm").cpu().numpy()


def _closure(fn, name):
    for var, cell in zip(fn.__code__.co_freevars, fn.__closure__ or ()):
        if var == name:
            return cell.cell_contents
    raise KeyError(name)


def test_c3_quantized_gathers_full_size(ops, dev):
    import bench
    chain, sets, T = bench.c3_ops(torch, ops, dev, 1)
    s = sets[0]
    D = 3584
    rng = np.random.default_rng(402)
    idx = _sample(rng, T)
    ids = s["ids"].cpu().numpy().view(np.uint32)
    q4 = _closure(chain[0].fn, "q4").cpu().numpy()
    q6 = _closure(chain[1].fn, "q6").cpu().numpy()
    w = _closure(chain[2].fn, "w").cpu().numpy()
    for op, tab, code in ((chain[0], q4, 12), (chain[1], q6, 14)):
        op.fn(s)
        torch.cuda.synchronize()
        ref = oracle.narrow(oracle.embedding(tab, code, tab.shape[0], D, ids[idx]), "f16")
        assert_exact(_rows(s["out"], idx), ref, f"c3 {op.name}")
    for op, tab, code in ((chain[2], q4, 12), (chain[3], q6, 14)):
        op.fn(s)
        torch.cuda.synchronize()
        rows = oracle.embedding(tab, code, tab.shape[0], D, ids[idx])
        assert_exact(_rows(s["out"], idx), oracle.narrow(rows, "f16"), f"c3 {op.name} h")
        assert_close(_rows(s["y"], idx), oracle.narrow(oracle.rmsnorm(rows, w, 1e-6), "f16"), "f16",
                     what=f"c3 {op.name} y")
    for op, name, code in ((chain[4], "q5", 13), (chain[5], "q8", 8)):
        tab = _closure(op.fn, name).cpu().numpy()
        op.fn(s)
        torch.cuda.synchronize()
        ref = oracle.narrow(oracle.embedding(tab, code, tab.shape[0], D, ids[idx]), "f16")
        assert_exact(_rows(s["out"], idx), ref, f"c3 {op.name}")


def test_c4_decode_step_full_size(ops, dev):
    import bench

    chain, sets, B = bench.c4_ops(torch, ops, dev, 1)
    s = sets[0]
    _run(chain, s)
    nq, nkv, hd, bs = 64, 8, 128, 16
    stride = nkv * hd
    inv = oracle.rope_inv_freqs(500000.0, hd)
    idx = np.arange(B)  # every row of the batch
    pos = s["pos"].cpu().numpy().view(np.uint32)
    qr = oracle.narrow(oracle.rope(oracle.widen(_rows(s["q"], idx), "bf16"), nq, hd, hd, 0, inv, pos), "bf16")
    assert_exact(_rows(s["qo"], idx), qr, "c4 rope q")
    kr = oracle.narrow(oracle.rope(oracle.widen(_rows(s["k"], idx), "bf16"), nkv, hd, hd, 0, inv, pos), "bf16")
    vr = _rows(s["v"], idx)
    cache = s["cache"]
    table = cache.block_table.cpu().numpy().view(np.uint32)
    bb = cache.block_bytes
    arena = cache.arena
    for b in range(B):
        base = int(table[b * cache.n_logical_blocks + pos[b] // bs]) * bb + int(pos[b] % bs) * stride * 2
        kslot = arena[base:base + stride * 2].cpu().numpy().view(np.uint16)
        vbase = base + bs * stride * 2
        vslot = arena[vbase:vbase + stride * 2].cpu().numpy().view(np.uint16)
        assert_exact(kslot, kr[b], f"c4 K slot row {b}")
        assert_exact(vslot, vr[b], f"c4 V slot row {b}")
    w = _closure(chain[1].fn, "w").cpu().numpy()
    h_ref, y_ref = oracle.add_rmsnorm(_rows(s["x"], idx), _rows(s["r"], idx), w, 1e-5, "bf16")
    assert_exact(_rows(s["h"], idx), h_ref, "c4 h")
    assert_close(_rows(s["y"], idx), y_ref, "bf16", what="c4 y")
    g, u = oracle.widen(_rows(s["gate"], idx), "bf16"), oracle.widen(_rows(s["up"], idx), "bf16")
    assert_exact(_rows(s["act"], idx), oracle.narrow(oracle.silu_gate(g, u), "bf16"), "c4 swiglu")


def test_c5_moe_layer_ops_full_size(ops, dev):
    import bench

    chain, sets, T = bench.c5_ops(torch, ops, dev, 1)
    s = sets[0]
    _run(chain, s)
    ids_ref, w_ref = oracle.router(s["logits"].cpu().numpy(), 8)
    assert_exact(s["ids"].cpu().numpy().view(np.uint32), ids_ref, "c5 router ids (all rows)")
    assert_exact(s["wts"].cpu().numpy(), w_ref, "c5 router weights (all rows)")
    rng = np.random.default_rng(405)
    ridx = _sample(rng, T * 8, 128)
    g, u = oracle.widen(_rows(s["gate"], ridx), "bf16"), oracle.widen(_rows(s["up"], ridx), "bf16")
    assert_exact(_rows(s["act"], ridx), oracle.narrow(oracle.silu_gate(g, u), "bf16"), "c5 routed swiglu")
    idx = _sample(rng, T)
    w = _closure(chain[2].fn, "w").cpu().numpy()
    y_ref = oracle.narrow(oracle.rmsnorm(oracle.widen(_rows(s["x"], idx), "bf16"), w, 1e-6), "bf16")
    assert_close(_rows(s["y"], idx), y_ref, "bf16", what="c5 rmsnorm")
    inv = oracle.rope_inv_freqs(1.0e6, 128)
    for src, dst, nh in (("q", "qo", 32), ("k", "ko", 4)):
        ref = oracle.narrow(oracle.rope(oracle.widen(_rows(s[src], idx), "bf16"), nh, 128, 128, 0, inv,
                                        idx.astype(np.uint32)), "bf16")
        assert_exact(_rows(s[dst], idx), ref, f"c5 rope {src}")
