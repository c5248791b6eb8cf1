"""HIP graph capture / replay of decode chains through the device-pointer API
(fellm_rocm_graph_*, the hipGraph counterpart of crates/backend-cuda/src/
graph.rs), with per-step values in device memory: position / length arrays,
and the DeviceStepParams block (crates/fellm-plugin-abi/src/
physical_plan.rs:103-128) read by single-sequence launches.

Every replay is checked bit for bit against the same launches run eagerly on
a twin set of buffers, with eager work and synchronisations between replays;
the eager kernels themselves are pinned against the oracle by the op tests.
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


@pytest.fixture(scope="module")
def graph():
    from fellm_amd import graph as _graph

    return _graph


def make_cache(ops, dev, n_seqs, n_logical, stride, dtype=torch.float16, seed=0):
    bb = ops.PagedKvCache.block_bytes_for(stride)
    n_blocks = n_seqs * n_logical
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    table = torch.randperm(n_blocks, generator=g).to(torch.int32).to(dev)
    arena = torch.zeros(n_blocks * bb, dtype=torch.uint8, device=dev)
    return ops.PagedKvCache(arena=arena, block_table=table, n_layers=1, n_logical_blocks=n_logical, block_size=16,
                            block_bytes=bb, stride=stride, kv_dtype=dtype)


def twin(ops, cache):
    return ops.PagedKvCache(arena=cache.arena.clone(), block_table=cache.block_table, n_layers=cache.n_layers,
                            n_logical_blocks=cache.n_logical_blocks, block_size=cache.block_size,
                            block_bytes=cache.block_bytes, stride=cache.stride, kv_dtype=cache.kv_dtype)


def same_bits(a, b, what):
    assert a.dtype == b.dtype and a.shape == b.shape, what
    ua = a.contiguous().view(torch.uint8)
    ub = b.contiguous().view(torch.uint8)
    if not torch.equal(ua, ub):
        bad = (ua != ub).nonzero()
        raise AssertionError(f"{what}: {bad.numel()} bytes differ, first at {bad[:4].flatten().tolist()}")


def test_batch_decode_chain_replay(ops, graph, dev):
    """configs[3]-style decode step for 8 sequences (RoPE + paged K/V append,
    residual + RMSNorm, SwiGLU, paged attention) captured once and replayed
    over 12 steps: positions advance in device memory, inputs are refilled in
    place; each replay must equal the eager run of the same step."""
    B, nq, nkv, hd, H, I = 8, 8, 2, 128, 1024, 2816
    n_logical = 4  # 64 keys per sequence
    stride = nkv * hd
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    inv = ops.rope_inv_freqs(500000.0, hd).to(dev)
    w = (1.0 + 0.1 * torch.randn(H, generator=g, device=dev)).float()
    cache_g = make_cache(ops, dev, B, n_logical, stride, torch.bfloat16)
    cache_e = twin(ops, cache_g)
    max_seq = n_logical * 16
    start = torch.randint(0, 40, (B,), generator=g, device=dev, dtype=torch.int32)

    def buffers():
        return {
            "q": torch.empty(B, nq * hd, dtype=torch.bfloat16, device=dev),
            "k": torch.empty(B, stride, dtype=torch.bfloat16, device=dev),
            "v": torch.empty(B, stride, dtype=torch.bfloat16, device=dev),
            "x": torch.empty(B, H, dtype=torch.bfloat16, device=dev),
            "r": torch.empty(B, H, dtype=torch.bfloat16, device=dev),
            "gate": torch.empty(B, I, dtype=torch.bfloat16, device=dev),
            "up": torch.empty(B, I, dtype=torch.bfloat16, device=dev),
            "pos": torch.empty(B, dtype=torch.int32, device=dev),
            "lens": torch.empty(B, dtype=torch.int32, device=dev),
            "qo": torch.empty(B, nq * hd, dtype=torch.bfloat16, device=dev),
            "h": torch.empty(B, H, dtype=torch.bfloat16, device=dev),
            "y": torch.empty(B, H, dtype=torch.bfloat16, device=dev),
            "act": torch.empty(B, I, dtype=torch.bfloat16, device=dev),
            "att": torch.empty(B, nq * hd, dtype=torch.float32, device=dev),
            "ws": torch.empty(max(ops._lib.lib().fellm_rocm_paged_attention_workspace(B, nq, nkv, hd, max_seq) // 4,
                                  1), dtype=torch.float32, device=dev),
        }

    def step(bf, cache):
        ops.rope_kv_write(bf["q"], bf["k"], bf["v"], inv, bf["pos"], cache, head_dim=hd, rope_positions=bf["pos"],
                          q_out=bf["qo"])
        ops.add_rmsnorm(bf["x"], bf["r"], w, 1e-5, h_out=bf["h"], y_out=bf["y"])
        ops.silu_gate(bf["gate"], bf["up"], out=bf["act"])
        ops.paged_attention(bf["qo"], bf["lens"], cache, n_heads=nq, n_kv_heads=nkv, head_dim=hd, max_seq=max_seq,
                            out=bf["att"], workspace=bf["ws"])

    G, E = buffers(), buffers()

    def fill(s):
        gg = torch.Generator(device=dev)
        gg.manual_seed(100 + s)
        for name in ("q", "k", "v", "x", "r", "gate", "up"):
            src = torch.randn(G[name].shape, generator=gg, device=dev).to(G[name].dtype)
            G[name].copy_(src)
            E[name].copy_(src)
        G["pos"].copy_(start + s)
        E["pos"].copy_(start + s)
        G["lens"].copy_(start + s + 1)
        E["lens"].copy_(start + s + 1)

    stream = torch.cuda.Stream()
    fill(0)
    torch.cuda.synchronize()
    with graph.GraphCapture(stream) as cap:
        step(G, cache_g)
    exe = cap.graph
    for s in range(12):
        fill(s)
        torch.cuda.synchronize()
        step(E, cache_e)          # eager twin on the default stream
        torch.cuda.synchronize()
        exe.launch(stream)
        stream.synchronize()
        for name in ("qo", "h", "y", "act", "att"):
            same_bits(G[name], E[name], f"step {s} {name}")
        same_bits(cache_g.arena, cache_e.arena, f"step {s} arena")
    exe.close()


def test_single_sequence_step_params_replay(ops, graph, dev):
    """One sequence driven by a device DeviceStepParams block: q/k/v rows are
    gathered at token_id, rotated at position, appended at the KV slot that
    fellm_rocm_step_kv_position derives from (sequence_length, kv_write_slot),
    and attention reads sequence_length keys.  One capture, 40 replays
    crossing two cache blocks, each equal to the eager run and the last one
    checked against the oracle."""
    from fellm_amd.abi import DeviceStepParams

    nq, nkv, hd, vocab = 8, 2, 64, 97
    stride = nkv * hd
    n_logical = 64  # 1024-key capacity: attention splits the key range and combines
    g = torch.Generator(device=dev)
    g.manual_seed(2)
    tq = torch.randn(vocab, nq * hd, generator=g, device=dev)
    tk = torch.randn(vocab, stride, generator=g, device=dev)
    tv = torch.randn(vocab, stride, generator=g, device=dev)
    inv = ops.rope_inv_freqs(10000.0, hd).to(dev)
    cache_g = make_cache(ops, dev, 1, n_logical, stride, seed=3)
    cache_e = twin(ops, cache_g)
    max_seq = n_logical * 16
    tokens = np.random.default_rng(4).integers(0, vocab, size=40)

    def buffers():
        b = {"params": torch.zeros(48, dtype=torch.uint8, device=dev),
             "q": torch.empty(1, nq * hd, device=dev), "k": torch.empty(1, stride, device=dev),
             "v": torch.empty(1, stride, device=dev), "qo": torch.empty(1, nq * hd, device=dev),
             "kvpos": torch.empty(1, dtype=torch.int32, device=dev), "att": torch.empty(1, nq * hd, device=dev),
             "ws": torch.empty(max(ops._lib.lib().fellm_rocm_paged_attention_workspace(1, nq, nkv, hd, max_seq) // 4,
                                   1), dtype=torch.float32, device=dev)}
        return b

    def step(b, cache):
        tok = ops.step_field(b["params"], "token_id")
        ops.embedding(tq, tok, out=b["q"])
        ops.embedding(tk, tok, out=b["k"])
        ops.embedding(tv, tok, out=b["v"])
        ops.step_kv_position(b["params"], 16, out=b["kvpos"])
        ops.rope_kv_write(b["q"], b["k"], b["v"], inv, b["kvpos"], cache, head_dim=hd,
                          rope_positions=ops.step_field(b["params"], "position"), q_out=b["qo"])
        ops.paged_attention(b["qo"], ops.step_field(b["params"], "sequence_length"), cache, n_heads=nq,
                            n_kv_heads=nkv, head_dim=hd, max_seq=max_seq, out=b["att"], workspace=b["ws"])

    def set_params(b, s):
        p = DeviceStepParams(token_id=int(tokens[s]), position=s, sequence_length=s + 1, active_batch=1,
                             kv_write_slot=s % 16)
        host = torch.frombuffer(bytearray(bytes(p)), dtype=torch.uint8)
        b["params"].copy_(host)

    G, E = buffers(), buffers()
    stream = torch.cuda.Stream()
    set_params(G, 0)
    torch.cuda.synchronize()
    with graph.GraphCapture(stream) as cap:
        step(G, cache_g)
    exe = cap.graph
    for s in range(40):
        set_params(G, s)
        set_params(E, s)
        torch.cuda.synchronize()
        step(E, cache_e)
        torch.cuda.synchronize()
        exe.launch(stream)
        stream.synchronize()
        for name in ("q", "k", "v", "qo", "kvpos", "att"):
            same_bits(G[name], E[name], f"step {s} {name}")
        same_bits(cache_g.arena, cache_e.arena, f"step {s} arena")
        assert int(G["kvpos"].item()) == s
    exe.close()

    # the last step against the oracle over the cache the replays built
    arena = cache_g.arena.cpu().numpy()
    table = cache_g.block_table.cpu().numpy().astype(np.uint32)
    q = G["qo"].cpu().numpy()
    ref = oracle.paged_attention(q, nq, nkv, hd, np.array([40]), float(np.float32(1 / np.sqrt(hd))), arena, table,
                                 n_logical, 1, 0, 16, cache_g.block_bytes)
    got = G["att"].cpu().numpy()
    assert np.abs(got - ref).max() <= 2e-5 * 5.0 + np.abs(ref).max() * 2.0 ** -23


def test_moe_chain_replay(ops, graph, dev):
    """Router top-k, dispatch, gather through inv and expert-order combine,
    captured once and replayed with new logits and activations."""
    T, E, K, H = 700, 64, 6, 256
    g = torch.Generator(device=dev)

    def buffers():
        return {"logits": torch.empty(T, E, device=dev), "x": torch.empty(T, H, device=dev),
                "ids": torch.empty(T, K, dtype=torch.int32, device=dev), "w": torch.empty(T, K, device=dev),
                "d": ops.moe_dispatch(torch.zeros(T, K, dtype=torch.int32, device=dev), E),
                "ws": torch.empty(ops._lib.lib().fellm_rocm_moe_dispatch_workspace(T, K, E), dtype=torch.uint8,
                                  device=dev),
                "grouped": torch.empty(T * K, H, device=dev), "y": torch.empty(T, H, device=dev)}

    def step(b):
        ops.router_topk(b["logits"], K, ids=b["ids"], weights=b["w"])
        ops.moe_dispatch(b["ids"], E, workspace=b["ws"], out=b["d"])
        ops.moe_gather(b["x"], b["d"].order, K, inv=b["d"].inv, out=b["grouped"])
        ops.moe_combine(b["grouped"], b["w"], ids=b["ids"], inv=b["d"].inv, y0=b["x"], out=b["y"])

    G, Ebuf = buffers(), buffers()
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    with graph.GraphCapture(stream) as cap:
        step(G)
    exe = cap.graph
    for s in range(5):
        g.manual_seed(50 + s)
        logits = torch.randn(T, E, generator=g, device=dev)
        x = torch.randn(T, H, generator=g, device=dev)
        for b in (G, Ebuf):
            b["logits"].copy_(logits)
            b["x"].copy_(x)
        torch.cuda.synchronize()
        step(Ebuf)
        torch.cuda.synchronize()
        exe.launch(stream)
        stream.synchronize()
        for name in ("ids", "w", "grouped", "y"):
            same_bits(G[name], Ebuf[name], f"replay {s} {name}")
        for f in ("counts", "offsets", "order", "inv"):
            same_bits(getattr(G["d"], f), getattr(Ebuf["d"], f), f"replay {s} {f}")
    exe.close()


def test_capture_abort_leaves_stream_usable(ops, graph, dev):
    """A capture abandoned half way (an exception inside the block) ends
    capture mode; the stream then runs eager work normally."""
    stream = torch.cuda.Stream()
    a = torch.randn(1024, device=dev)
    b = torch.randn(1024, device=dev)
    out = torch.empty_like(a)
    with pytest.raises(RuntimeError, match="boom"):
        with graph.GraphCapture(stream):
            ops.add(a, b, out=out)
            raise RuntimeError("boom")
    assert not graph.is_capturing(stream)
    with torch.cuda.stream(stream):
        ops.add(a, b, out=out)
    stream.synchronize()
    assert torch.equal(out, a + b)
