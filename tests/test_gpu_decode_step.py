"""fellm_rocm_decode_step (one launch for a decode step's RoPE + paged K/V
append, residual add + RMSNorm and SwiGLU) against the three standalone
launches on the same inputs, and against the oracle.

Bars: rotated q, K/V slot bytes, h and the SwiGLU output bit-exact with the
standalone launches (and with the oracle); y within 1 ulp of the 16-bit
output or 1e-5 relative in f32 (the fused row reduces its sum of squares in
another order)."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from parity_util import KINDS, assert_close, assert_exact, from_dev, random_stored, to_dev

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def ops():
    from fellm_amd import ops as _ops

    return _ops


CASES = [
    # act, kv, batch, nq, nkv, hd, H, I
    ("bf16", "bf16", 256, 64, 8, 128, 8192, 28672),  # configs[3]
    ("f16", "f16", 7, 8, 2, 128, 4096, 1000),
    ("f32", "f16", 33, 16, 4, 64, 2560, 512),
    ("bf16", "bf16", 5, 8, 2, 64, 2048, 256),  # rows of 2048: the standalone-launch path
]


@pytest.mark.parametrize("act,kvk,batch,nq,nkv,hd,H,I", CASES)
def test_decode_step_matches_standalone(ops, dev, act, kvk, batch, nq, nkv, hd, H, I):
    from fellm_amd import synth

    rng = np.random.default_rng(batch * 7 + H)
    stride = nkv * hd
    n_blocks = max(64, batch * 4)
    kv_pos, table, n_logical = synth.paged_layout(rng, batch, n_blocks, 16, 32768 if batch > 64 else 2048)
    inv = oracle.rope_inv_freqs(500000.0, hd)
    q = random_stored(rng, (batch, nq * hd), act)
    k = random_stored(rng, (batch, stride), act)
    v = random_stored(rng, (batch, stride), act)
    x = random_stored(rng, (batch, H), act)
    r = random_stored(rng, (batch, H), act, sigma=2.0)
    w = rng.normal(1.0, 0.1, size=H).astype(np.float32)
    g = random_stored(rng, (batch, I), act)
    u = random_stored(rng, (batch, I), act)
    bb = ops.PagedKvCache.block_bytes_for(stride)
    d = lambda a: to_dev(a, act, dev)
    tab = torch.from_numpy(table.view(np.int32)).to(dev)
    pos = torch.from_numpy(kv_pos.view(np.int32)).to(dev)
    invd = torch.from_numpy(inv).to(dev)
    wd = torch.from_numpy(w).to(dev)

    def cache():
        arena = torch.zeros(n_blocks * bb, dtype=torch.uint8, device=dev)
        return ops.PagedKvCache(arena, tab, 1, n_logical, 16, bb, stride, KINDS[kvk])

    # standalone launches
    c1 = cache()
    q1 = ops.rope_kv_write(d(q), d(k), d(v), invd, pos, c1, head_dim=hd)
    h1, y1 = ops.add_rmsnorm(d(x), d(r), wd, 1e-5)
    a1 = ops.silu_gate(d(g), d(u))
    # one launch
    c2 = cache()
    q2, h2, y2, a2 = ops.decode_step(d(q), d(k), d(v), invd, pos, c2, d(x), d(r), wd, 1e-5, d(g), d(u), head_dim=hd)
    torch.cuda.synchronize()
    assert_exact(from_dev(q2), from_dev(q1), "q")
    assert_exact(c2.arena.cpu().numpy(), c1.arena.cpu().numpy(), "K/V arena")
    assert_exact(from_dev(h2), from_dev(h1), "h")
    assert_exact(from_dev(a2), from_dev(a1), "swiglu")
    assert_close(from_dev(y2), from_dev(y1), act, what="y vs standalone")
    # and the oracle
    h_ref, y_ref = oracle.add_rmsnorm(x, r, w, 1e-5, act)
    assert_exact(from_dev(h2), h_ref, "h vs oracle")
    assert_close(from_dev(y2), y_ref, act, what="y vs oracle")
    q_ref = oracle.narrow(oracle.rope(oracle.widen(q, act), nq, hd, hd, 0, inv, kv_pos), act)
    assert_exact(from_dev(q2), q_ref, "q vs oracle")
    a_ref = oracle.narrow(oracle.silu_gate(oracle.widen(g, act), oracle.widen(u, act)), act)
    assert_exact(from_dev(a2), a_ref, "swiglu vs oracle")
