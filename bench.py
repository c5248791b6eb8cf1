"""Benchmark of FeLLM's per-layer memory-bound op chain on one MI355X.

Default workload: BASELINE configs[1], Llama-3-8B-shaped prefill, T = 4096
tokens, f16 activations with f32 arithmetic:
  embedding gather  128256 x 4096 f16 table -> f16 rows
  residual add + RMSNorm  H = 4096, eps 1e-5 (reads x, r; writes h, y)
  RoPE q + k  head_dim 128, 32 Q / 8 KV heads, theta 5e5, positions 0..4095
  SwiGLU  I = 14336
One step = one pass of the four kernels over one batch of synthetic inputs
already resident in HBM.  Three input sets rotate between steps (> 1.8 GB
touched per rotation) so the 256 MB MALL cannot serve repeated reads.

`value` = tokens per second over K uninstrumented steps (wall clock between
two synchronisations).  Per-op kernel time comes from a second pass of K steps
with HIP events recorded around each launch on the stream the kernels run on;
achieved GB/s = algorithmic bytes / kernel time (bytes each op must read and
write once).  The CPU baseline times the C restatement of
backend-cpu (oracle/, 1 thread) on a bounded sample of the same chain.

--suite measures every BASELINE config's ops (per-op GB/s table) instead, plus the
decode gate/up K-quant GEMV + SwiGLU (next_gemv) and paged decode attention
(next_attention).
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0
METRIC = "achieved HBM GB/s (% of peak) per fused op; tokens/s for op chain at 8B shape"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # The GPU idles at ~110 MHz and its clock ramps up under load: a short
    # warm-up leaves part of the timed steps on the ramp (configs[1] chain:
    # 35.3 M tokens/s at 5 warm-up / 50 timed steps, 37.2-37.6 M from 200
    # warm-up steps on, flat to 2000 / 2000).
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--sets", type=int, default=3, help="rotating input sets")
    ap.add_argument("--only", default=None, help="with --suite: comma-separated suite entries to run")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline time budget")
    ap.add_argument("--suite", action="store_true", help="per-op table for every config")
    ap.add_argument("--reps", type=int, default=0, help="per-op timing reps (default max(steps, 50))")
    ap.add_argument("--no-ceiling", action="store_true", help="skip the same-run copy-ceiling probes")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a plain 512 MiB device copy (PMC byte-counter calibration)")
    return ap.parse_args()


# --------------------------------------------------------------------------- #
# Workloads
# --------------------------------------------------------------------------- #
class Op:
    """One timed op: algorithmic bytes per launch, the launch, and the
    streaming pattern of its ceiling probe: (read streams, bytes read per
    stream, bytes written) (None: no probe)."""

    def __init__(self, name, nbytes, fn, probe=None):
        self.name, self.nbytes, self.fn, self.probe = name, nbytes, fn, probe


def c2_ops(torch, ops, dev, n_sets, seed=1):
    """Llama-3-8B prefill chain."""
    T, H, I, V = 4096, 4096, 14336, 128256
    nq, nkv, hd, theta = 32, 8, 128, 500000.0
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    f16 = torch.float16

    def randn(*shape, std=1.0):
        return (torch.randn(*shape, generator=g, device=dev, dtype=torch.float32) * std).to(f16)

    table = randn(V, H, std=0.02)
    w_norm = (1.0 + 0.1 * torch.randn(H, generator=g, device=dev)).float()
    inv = ops.rope_inv_freqs(theta, hd).to(dev)
    pos = torch.arange(T, dtype=torch.int32, device=dev)
    sets = []
    for _ in range(n_sets):
        s = {
            "ids": torch.randint(0, V, (T,), generator=g, device=dev, dtype=torch.int32),
            "emb": torch.empty(T, H, dtype=f16, device=dev),
            "x": randn(T, H), "r": randn(T, H, std=2.0),
            "h": torch.empty(T, H, dtype=f16, device=dev), "y": torch.empty(T, H, dtype=f16, device=dev),
            "q": randn(T, nq * hd), "k": randn(T, nkv * hd),
            "qo": torch.empty(T, nq * hd, dtype=f16, device=dev), "ko": torch.empty(T, nkv * hd, dtype=f16, device=dev),
            "gate": randn(T, I), "up": randn(T, I), "act": torch.empty(T, I, dtype=f16, device=dev),
        }
        sets.append(s)
    e = 2  # bytes per f16
    bytes_emb = T * H * e * 2 + T * 4
    bytes_norm = T * H * e * 4
    bytes_rope = T * (nq + nkv) * hd * e * 2 + T * 4
    bytes_swiglu = T * I * e * 3

    def op_emb(s):
        ops.embedding(table, s["ids"], out=s["emb"])

    def op_norm(s):
        ops.add_rmsnorm(s["x"], s["r"], w_norm, 1e-5, h_out=s["h"], y_out=s["y"])

    def op_rope(s):
        ops.rope(s["q"], inv, head_dim=hd, pairing=0, positions=pos, x2=s["k"], out1=s["qo"], out2=s["ko"])

    def op_swiglu(s):
        ops.silu_gate(s["gate"], s["up"], out=s["act"])

    chain = [Op("embedding_f16", bytes_emb, op_emb, (1, T * H * e, T * H * e)),
             Op("add_rmsnorm", bytes_norm, op_norm, (2, T * H * e, 2 * T * H * e)),
             Op("rope_qk", bytes_rope, op_rope, (1, T * (nq + nkv) * hd * e, T * (nq + nkv) * hd * e)),
             Op("swiglu", bytes_swiglu, op_swiglu, (2, T * I * e, T * I * e))]
    return chain, sets, T


def c3_ops(torch, ops, dev, n_sets, seed=3):
    """Qwen2-7B quantized embedding gather, Zipf ids."""
    import numpy as np

    from fellm_amd import synth

    V, D, T = 152064, 3584, 8192
    rng = np.random.default_rng(seed)
    q4 = torch.from_numpy(synth.q4k_table(rng, V, D)).to(dev)
    q6 = torch.from_numpy(synth.q6k_table(rng, V, D)).to(dev)
    w = torch.from_numpy(rng.normal(1.0, 0.1, size=D).astype(np.float32)).to(dev)
    sets = [{"ids": torch.from_numpy(synth.zipf_ids(rng, T, V).view(np.int32)).to(dev),
             "out": torch.empty(T, D, dtype=torch.float16, device=dev),
             "y": torch.empty(T, D, dtype=torch.float16, device=dev)} for _ in range(n_sets)]
    out_b = T * D * 2
    chain = [
        Op("q4k_gather", T * 2016 + out_b + T * 4, lambda s: ops.embedding(q4, s["ids"], dim=D, qtype="q4k",
                                                                           out=s["out"]), (1, T * 2016, out_b)),
        Op("q6k_gather", T * 2940 + out_b + T * 4, lambda s: ops.embedding(q6, s["ids"], dim=D, qtype="q6k",
                                                                           out=s["out"]), (1, T * 2940, out_b)),
        Op("q4k_gather_rmsnorm", T * 2016 + 2 * out_b + T * 4,
           lambda s: ops.embedding_rmsnorm(q4, s["ids"], w, 1e-6, dim=D, qtype="q4k", h_out=s["out"],
                                           y_out=s["y"]), (1, T * 2016, 2 * out_b)),
        Op("q6k_gather_rmsnorm", T * 2940 + 2 * out_b + T * 4,
           lambda s: ops.embedding_rmsnorm(q6, s["ids"], w, 1e-6, dim=D, qtype="q6k", h_out=s["out"],
                                           y_out=s["y"]), (1, T * 2940, 2 * out_b)),
    ]
    # The CUDA plugin's other quantized embedding keys (Q5_K, Q8_0) at the same
    # shape; drawn after the ids so the four ops above see the same inputs.
    q5 = torch.from_numpy(synth.q5k_table(rng, V, D)).to(dev)
    q8 = torch.from_numpy(synth.q8_0_table(rng, V, D)).to(dev)
    chain += [
        Op("q5k_gather", T * 2464 + out_b + T * 4, lambda s: ops.embedding(q5, s["ids"], dim=D, qtype="q5k",
                                                                           out=s["out"]), (1, T * 2464, out_b)),
        Op("q8_0_gather", T * 3808 + out_b + T * 4, lambda s: ops.embedding(q8, s["ids"], dim=D, qtype="q8_0",
                                                                            out=s["out"]), (1, T * 3808, out_b)),
    ]
    return chain, sets, T


def c4_ops(torch, ops, dev, n_sets, seed=4):
    """Llama-3-70B continuous-batching decode step, 256 sequences."""
    import numpy as np

    from fellm_amd import synth

    B, nq, nkv, hd, bs, n_blocks = 256, 64, 8, 128, 16, 65536
    H, I = 8192, 28672
    stride = nkv * hd
    bf = torch.bfloat16
    rng = np.random.default_rng(seed)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    bb = ops.PagedKvCache.block_bytes_for(stride, bs)
    arena = torch.zeros(n_blocks * bb, dtype=torch.uint8, device=dev)
    inv = ops.rope_inv_freqs(500000.0, hd).to(dev)
    w = (1.0 + 0.1 * torch.randn(H, generator=g, device=dev)).float()
    sets = []
    for _ in range(n_sets):
        pos, table, n_logical = synth.paged_layout(rng, B, n_blocks, bs, 32768)
        cache = ops.PagedKvCache(arena, torch.from_numpy(table.view(np.int32)).to(dev), 1, n_logical, bs, bb, stride,
                                 bf)
        sets.append({
            "pos": torch.from_numpy(pos.view(np.int32)).to(dev), "cache": cache,
            "q": torch.randn(B, nq * hd, generator=g, device=dev).to(bf),
            "k": torch.randn(B, stride, generator=g, device=dev).to(bf),
            "v": torch.randn(B, stride, generator=g, device=dev).to(bf),
            "qo": torch.empty(B, nq * hd, dtype=bf, device=dev),
            "x": torch.randn(B, H, generator=g, device=dev).to(bf),
            "r": (2 * torch.randn(B, H, generator=g, device=dev)).to(bf),
            "h": torch.empty(B, H, dtype=bf, device=dev), "y": torch.empty(B, H, dtype=bf, device=dev),
            "gate": torch.randn(B, I, generator=g, device=dev).to(bf),
            "up": torch.randn(B, I, generator=g, device=dev).to(bf),
            "act": torch.empty(B, I, dtype=bf, device=dev),
        })
    chain = [
        Op("rope_kv_write", B * (nq * hd * 2 + 2 * stride) * 2 + B * 2 * stride * 2 + B * 4,
           lambda s: ops.rope_kv_write(s["q"], s["k"], s["v"], inv, s["pos"], s["cache"], head_dim=hd,
                                       q_out=s["qo"]), (1, B * (nq * hd + 2 * stride) * 2, B * (nq * hd + 2 * stride) * 2)),
        Op("add_rmsnorm", B * H * 2 * 4, lambda s: ops.add_rmsnorm(s["x"], s["r"], w, 1e-5, h_out=s["h"],
                                                                   y_out=s["y"]), (2, B * H * 2, 2 * B * H * 2)),
        Op("swiglu", B * I * 2 * 3, lambda s: ops.silu_gate(s["gate"], s["up"], out=s["act"]), (2, B * I * 2, B * I * 2)),
    ]
    # The same three ops in one launch (fellm_rocm_decode_step).
    chain.append(Op("decode_step_fused", sum(op.nbytes for op in chain),
                    lambda s: ops.decode_step(s["q"], s["k"], s["v"], inv, s["pos"], s["cache"], s["x"], s["r"], w, 1e-5,
                                              s["gate"], s["up"], head_dim=hd, q_out=s["qo"], h_out=s["h"],
                                              y_out=s["y"], act_out=s["act"])))
    return chain, sets, B


def c5_ops(torch, ops, dev, n_sets, seed=5):
    """Qwen3-30B-A3B MoE layer ops, 16384 tokens."""
    T, E, K, H, Iexp = 16384, 128, 8, 2048, 768
    nq, nkv, hd = 32, 4, 128
    bf = torch.bfloat16
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    inv = ops.rope_inv_freqs(1.0e6, hd).to(dev)
    pos = torch.arange(T, dtype=torch.int32, device=dev)
    w = (1.0 + 0.1 * torch.randn(H, generator=g, device=dev)).float()
    sets = []
    for _ in range(n_sets):
        sets.append({
            "logits": torch.randn(T, E, generator=g, device=dev),
            "ids": torch.empty(T, K, dtype=torch.int32, device=dev),
            "wts": torch.empty(T, K, dtype=torch.float32, device=dev),
            "gate": torch.randn(T * K, Iexp, generator=g, device=dev).to(bf),
            "up": torch.randn(T * K, Iexp, generator=g, device=dev).to(bf),
            "act": torch.empty(T * K, Iexp, dtype=bf, device=dev),
            "x": torch.randn(T, H, generator=g, device=dev).to(bf),
            "y": torch.empty(T, H, dtype=bf, device=dev),
            "q": torch.randn(T, nq * hd, generator=g, device=dev).to(bf),
            "k": torch.randn(T, nkv * hd, generator=g, device=dev).to(bf),
            "qo": torch.empty(T, nq * hd, dtype=bf, device=dev),
            "ko": torch.empty(T, nkv * hd, dtype=bf, device=dev),
        })
    chain = [
        Op("router_topk", T * E * 4 + T * K * 8, lambda s: ops.router_topk(s["logits"], K, ids=s["ids"],
                                                                          weights=s["wts"]), (1, T * E * 4, T * K * 8)),
        Op("swiglu_routed", T * K * Iexp * 2 * 3, lambda s: ops.silu_gate(s["gate"], s["up"], out=s["act"]),
           (2, T * K * Iexp * 2, T * K * Iexp * 2)),
        Op("rmsnorm", T * H * 2 * 2, lambda s: ops.rmsnorm(s["x"], w, 1e-6, out=s["y"]), (1, T * H * 2, T * H * 2)),
        Op("rope_qk", T * (nq + nkv) * hd * 2 * 2 + T * 4,
           lambda s: ops.rope(s["q"], inv, head_dim=hd, positions=pos, x2=s["k"], out1=s["qo"], out2=s["ko"]),
           (1, T * (nq + nkv) * hd * 2, T * (nq + nkv) * hd * 2)),
    ]
    return chain, sets, T


def gemv_ops(torch, ops, dev, n_sets, seed=6):
    """Decode FFN gate/up GEMV + SwiGLU (GateUpSwiGlu) on GGUF K-quant weights:
    Llama-3-8B (14336 x 4096) as Q4_K and Q6_K, Llama-3-70B (28672 x 8192) as
    Q4_K; each also as quantize_q8k + the _q8k GEMV (x quantized once per
    call instead of once per workgroup, both launches timed).  One activation vector; weights rotate over enough copies (device
    rolls of one synthetic matrix) that every launch streams them from HBM."""
    import numpy as np

    from fellm_amd import synth

    rng = np.random.default_rng(seed)
    chain, sets = [], []
    cases = (("gate_up_q4k_8b", "q4k", 12, 14336, 4096, max(n_sets, 8)),
             ("gate_up_q6k_8b", "q6k", 14, 14336, 4096, max(n_sets, 6)),
             ("gate_up_q4k_70b", "q4k", 12, 28672, 8192, max(n_sets, 3)))
    per_case = []
    for name, qt, code, rows, cols, nset in cases:
        g0 = torch.from_numpy(synth.KQUANT_TABLES[code](rng, rows, cols)).to(dev)
        u0 = torch.from_numpy(synth.KQUANT_TABLES[code](rng, rows, cols)).to(dev)
        mats = [(g0.roll(7 * i, 0).contiguous(), u0.roll(5 * i, 0).contiguous()) for i in range(nset)]
        x = torch.randn(cols, device=dev)
        out = torch.empty(rows, device=dev)
        per_case.append((mats, x, out))
        nbytes = 2 * g0.numel() + cols * 4 + rows * 4

        def fn(s, mats=mats, x=x, out=out, qt=qt, key=name):
            i = s["i"][key] = (s["i"][key] + 1) % len(mats)
            ops.gate_up_swiglu(mats[i][0], mats[i][1], x, qtype=qt, out=out)

        xq = torch.empty(ops._lib.lib().fellm_rocm_q8k_bytes(cols), dtype=torch.uint8, device=dev)

        def fn_q8k(s, mats=mats, x=x, out=out, qt=qt, key=name, xq=xq):
            i = s["i"][key] = (s["i"][key] + 1) % len(mats)
            ops.quantize_q8k(x, out=xq)
            ops.gate_up_swiglu_q8k(mats[i][0], mats[i][1], xq, qtype=qt, out=out)

        chain.append(Op(name, nbytes, fn))
        chain.append(Op(name + "_q8k", nbytes, fn_q8k))
    # Plain K-quant GEMVs of a Llama-3-8B decode layer: QKV (6144 x 4096) and
    # down (4096 x 14336, rows longer than one 32-block pass).
    mv_cases = (("matvec_q4k_8b_qkv", 6144, 4096, max(n_sets, 16)), ("matvec_q4k_8b_down", 4096, 14336, max(n_sets, 8)))
    for name, rows, cols, nset in mv_cases:
        w0 = torch.from_numpy(synth.KQUANT_TABLES[12](rng, rows, cols)).to(dev)
        mats = [w0.roll(3 * i, 0).contiguous() for i in range(nset)]
        x = torch.randn(cols, device=dev)
        out = torch.empty(rows, device=dev)
        nbytes = w0.numel() + cols * 4 + rows * 4

        def fn(s, mats=mats, x=x, out=out, key=name):
            i = s["i"][key] = (s["i"][key] + 1) % len(mats)
            ops.matvec_kquant(mats[i], x, qtype="q4k", out=out)

        xq = torch.empty(ops._lib.lib().fellm_rocm_q8k_bytes(cols), dtype=torch.uint8, device=dev)

        def fn_q8k(s, mats=mats, x=x, out=out, key=name, xq=xq):
            i = s["i"][key] = (s["i"][key] + 1) % len(mats)
            ops.quantize_q8k(x, out=xq)
            ops.matvec_kquant_q8k(mats[i], xq, qtype="q4k", out=out)

        chain.append(Op(name, nbytes, fn))
        chain.append(Op(name + "_q8k", nbytes, fn_q8k))
    state = {"i": {c[0]: 0 for c in cases + tuple((m[0], 0, 0, 0, 0, 0) for m in mv_cases)}}
    sets = [state]
    return chain, sets, 1


def attention_ops(torch, ops, dev, n_sets, seed=7):
    """Paged decode attention over an f16 cache in FeLLM's layout:
    configs[3]-shaped (Llama-3-70B heads 64/8/128, 256 sequences x 4096 keys,
    the whole 4.29 GB arena) and one Llama-3-8B sequence of 32768 or 2048 keys
    (the split-key path).  Physical blocks are a random permutation."""
    chain = []
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    for name, B, seq, nh, nkv, hd in (("attn_decode_70b_b256_s4096", 256, 4096, 64, 8, 128),
                                      ("attn_decode_8b_b1_s32768", 1, 32768, 32, 8, 128),
                                      ("attn_decode_8b_b1_s2048", 1, 2048, 32, 8, 128)):
        stride = nkv * hd
        bb = ops.PagedKvCache.block_bytes_for(stride)
        n_logical = (seq + 15) // 16
        nblk = B * n_logical
        arena = torch.empty(nblk * bb, dtype=torch.uint8, device=dev)
        arena.view(torch.float16).copy_((torch.randn(arena.numel() // 2, device=dev) * 0.5).half())
        table = torch.randperm(nblk, generator=g).to(torch.int32).to(dev)
        cache = ops.PagedKvCache(arena=arena, block_table=table, n_layers=1, n_logical_blocks=n_logical,
                                 block_size=16, block_bytes=bb, stride=stride)
        q = torch.randn(B, nh * hd, device=dev).half()
        lens = torch.full((B,), seq, dtype=torch.int32, device=dev)
        out = torch.empty(B, nh * hd, device=dev, dtype=torch.half)
        ws_bytes = ops._lib.lib().fellm_rocm_paged_attention_workspace(B, nh, nkv, hd, seq)
        ws = torch.empty(max(ws_bytes // 4, 1), dtype=torch.float32, device=dev)
        nbytes = B * seq * stride * 2 * 2 + 2 * B * nh * hd * 2 + B * 4

        def fn(s, q=q, lens=lens, cache=cache, out=out, ws=ws, nh=nh, nkv=nkv, hd=hd, seq=seq):
            ops.paged_attention(q, lens, cache, n_heads=nh, n_kv_heads=nkv, head_dim=hd, max_seq=seq, out=out,
                                workspace=ws)

        chain.append(Op(name, nbytes, fn))
    return chain, [{}], 1


def moe_ops(torch, ops, dev, n_sets, seed=8):
    """MoE dispatch around the expert FFNs at the configs[4] shape (Qwen3-30B-A3B:
    16384 tokens, top-8 of 128 experts, H 2048): stable per-expert grouping,
    bf16 row gather into grouped order (scatter form through inv, and the
    read-by-order form), f32 weighted combine in expert order
    (CPU backend) and slot order (CUDA plugin); plus the grouping of one
    64-token decode batch (launch-latency bound)."""
    T, E, K, H = 16384, 128, 8, 2048
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    sets = []
    for _ in range(n_sets):
        ids = torch.argsort(torch.rand(T, E, generator=g, device=dev), dim=1)[:, :K].to(torch.int32).contiguous()
        d = ops.moe_dispatch(ids, E)
        sets.append({
            "ids": ids, "d": d,
            "d2": ops.moe_dispatch(ids, E),
            "ids64": ids[:64].contiguous(),
            "d64": ops.moe_dispatch(ids[:64].contiguous(), E),
            "ws": torch.empty(ops._lib.lib().fellm_rocm_moe_dispatch_workspace(T, K, E), dtype=torch.uint8,
                              device=dev),
            "wts": torch.rand(T, K, generator=g, device=dev),
            "x": torch.randn(T, H, generator=g, device=dev).to(torch.bfloat16),
            "grouped": torch.empty(T * K, H, dtype=torch.bfloat16, device=dev),
            "eo": torch.randn(T * K, H, generator=g, device=dev),
            "y0": torch.randn(T, H, generator=g, device=dev),
            "y": torch.empty(T, H, device=dev),
        })
    A = T * K
    chain = [
        Op("moe_dispatch_t16384", A * 4 + 2 * A * 4 + (2 * E + 1) * 4,
           lambda s: ops.moe_dispatch(s["ids"], E, workspace=s["ws"], out=s["d2"])),
        Op("moe_dispatch_t64", 64 * K * 4 * 3 + (2 * E + 1) * 4, lambda s: ops.moe_dispatch(s["ids64"], E, out=s["d64"])),
        Op("moe_gather_bf16", 2 * A * 4 + T * H * 2 + A * H * 2,
           lambda s: ops.moe_gather(s["x"], s["d"].order, K, inv=s["d"].inv, out=s["grouped"])),
        Op("moe_gather_bf16_by_order", A * 4 + T * H * 2 + A * H * 2,
           lambda s: ops.moe_gather(s["x"], s["d"].order, K, out=s["grouped"])),
        Op("moe_combine_expert_order", A * H * 4 + 2 * T * H * 4 + A * 12,
           lambda s: ops.moe_combine(s["eo"], s["wts"], ids=s["ids"], inv=s["d"].inv, y0=s["y0"], out=s["y"])),
        Op("moe_combine_slot_order", A * H * 4 + T * H * 4 + A * 4,
           lambda s: ops.moe_combine(s["eo"], s["wts"], out=s["y"])),
    ]
    return chain, sets, T


def time_eager_vs_graph(torch, fn, steps, warmup):
    """Wall time per step of `fn` launched eagerly (every launch from the
    host) and of one captured replay of it (fellm_rocm_graph_*), both on a
    side stream, synchronised before and after the timed steps."""
    import time

    from fellm_amd import graph

    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            fn()
    stream.synchronize()
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        for _ in range(steps):
            fn()
    stream.synchronize()
    eager = (time.perf_counter() - t0) / steps
    with graph.GraphCapture(stream) as cap:
        fn()
    exe = cap.graph
    for _ in range(warmup):
        exe.launch(stream)
    stream.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        exe.launch(stream)
    stream.synchronize()
    replay = (time.perf_counter() - t0) / steps
    exe.close()
    return {"eager_us_per_step": round(eager * 1e6, 2), "graph_us_per_step": round(replay * 1e6, 2),
            "speedup": round(eager / replay, 2)}


def decode_graph_report(torch, ops, dev, steps, warmup):
    """Launch-latency floor of decode steps, eager against HIP graph replay.

    * configs[3]'s decode step (RoPE + paged K/V append, residual + RMSNorm,
      SwiGLU for 256 sequences at Llama-3-70B shape);
    * one Llama-3-8B decode layer for one sequence with Q4_K weights and f32
      activations, driven by a device DeviceStepParams block: RMSNorm, QKV
      GEMV, RoPE + K/V append at the step position, paged attention over the
      step's sequence length (2048 keys of a 4096-key table), O GEMV,
      residual + RMSNorm, gate/up GEMV + SwiGLU, down GEMV, residual add."""
    import numpy as np

    from fellm_amd import synth
    from fellm_amd.abi import DeviceStepParams

    out = {}
    chain, sets, _ = c4_ops(torch, ops, dev, 1)
    st = sets[0]
    sep = [op for op in chain if op.name != "decode_step_fused"]
    fused = [op for op in chain if op.name == "decode_step_fused"][0]
    out["c4_decode_step_b256"] = time_eager_vs_graph(torch, lambda: [op.fn(st) for op in sep], steps, warmup)
    out["c4_decode_step_b256_one_launch"] = time_eager_vs_graph(torch, lambda: fused.fn(st), steps, warmup)
    del chain, sets, st
    torch.cuda.empty_cache()

    H, I, nq, nkv, hd, n_logical = 4096, 14336, 32, 8, 128, 256
    stride = nkv * hd
    rng = np.random.default_rng(9)
    q4k = synth.KQUANT_TABLES[12]
    w_qkv = torch.from_numpy(q4k(rng, H + 2 * stride, H)).to(dev)
    w_o = torch.from_numpy(q4k(rng, H, H)).to(dev)
    w_g = torch.from_numpy(q4k(rng, I, H)).to(dev)
    w_u = torch.from_numpy(q4k(rng, I, H)).to(dev)
    w_d = torch.from_numpy(q4k(rng, H, I)).to(dev)
    g = torch.Generator(device=dev)
    g.manual_seed(9)
    n1 = (1.0 + 0.1 * torch.randn(H, generator=g, device=dev)).float()
    n2 = (1.0 + 0.1 * torch.randn(H, generator=g, device=dev)).float()
    inv = ops.rope_inv_freqs(500000.0, hd).to(dev)
    bb = ops.PagedKvCache.block_bytes_for(stride)
    arena = torch.zeros(n_logical * bb, dtype=torch.uint8, device=dev)
    arena.view(torch.float16).copy_((0.5 * torch.randn(arena.numel() // 2, generator=g, device=dev)).half())
    table = torch.from_numpy(rng.permutation(n_logical).astype(np.int32)).to(dev)
    cache = ops.PagedKvCache(arena=arena, block_table=table, n_layers=1, n_logical_blocks=n_logical, block_size=16,
                             block_bytes=bb, stride=stride)
    seq = 2048
    params = torch.frombuffer(bytearray(bytes(DeviceStepParams(token_id=0, position=seq - 1, sequence_length=seq,
                                                               active_batch=1, kv_write_slot=(seq - 1) % 16))),
                              dtype=torch.uint8).to(dev)
    max_seq = n_logical * 16
    b = {"x": torch.randn(1, H, generator=g, device=dev), "h": torch.empty(1, H, device=dev),
         "y": torch.empty(1, H, device=dev), "qkv": torch.empty(H + 2 * stride, device=dev),
         "qo": torch.empty(1, H, device=dev), "kvpos": torch.empty(1, dtype=torch.int32, device=dev),
         "att": torch.empty(1, H, device=dev), "o": torch.empty(H, device=dev), "h2": torch.empty(1, H, device=dev),
         "y2": torch.empty(1, H, device=dev), "act": torch.empty(I, device=dev), "down": torch.empty(H, device=dev),
         "out": torch.empty(1, H, device=dev),
         "ws": torch.empty(max(ops._lib.lib().fellm_rocm_paged_attention_workspace(1, nq, nkv, hd, max_seq) // 4, 1),
                           dtype=torch.float32, device=dev)}
    qkv = b["qkv"]
    q, k, v = qkv[:H].view(1, H), qkv[H:H + stride].view(1, stride), qkv[H + stride:].view(1, stride)

    def layer():
        ops.rmsnorm(b["x"], n1, 1e-5, out=b["y"])
        ops.matvec_kquant(w_qkv, b["y"].view(-1), qtype="q4k", out=qkv)
        ops.step_kv_position(params, 16, out=b["kvpos"])
        ops.rope_kv_write(q, k, v, inv, b["kvpos"], cache, head_dim=hd,
                          rope_positions=ops.step_field(params, "position"), q_out=b["qo"])
        ops.paged_attention(b["qo"], ops.step_field(params, "sequence_length"), cache, n_heads=nq, n_kv_heads=nkv,
                            head_dim=hd, max_seq=max_seq, out=b["att"], workspace=b["ws"])
        ops.matvec_kquant(w_o, b["att"].view(-1), qtype="q4k", out=b["o"])
        ops.add_rmsnorm(b["o"].view(1, H), b["x"], n2, 1e-5, h_out=b["h2"], y_out=b["y2"])
        ops.gate_up_swiglu(w_g, w_u, b["y2"].view(-1), qtype="q4k", out=b["act"])
        ops.matvec_kquant(w_d, b["act"].view(-1), qtype="q4k", out=b["down"])
        ops.add(b["down"].view(1, H), b["h2"], out=b["out"])

    out["llama8b_decode_layer_q4k"] = time_eager_vs_graph(torch, layer, steps, warmup)
    out["llama8b_decode_layer_q4k"]["weight_bytes"] = int(sum(t.numel() for t in (w_qkv, w_o, w_g, w_u, w_d)))
    out["llama8b_decode_layer_plugin"] = plugin_decode_graph(torch, dev, steps, warmup)
    return out


def plugin_decode_graph(torch, dev, steps, warmup):
    """The same decode layer minus the projections, driven through the plugin
    ABI with host buffers as FeLLM's host drives it (RmsNorm, rope_kv_write,
    Attention, add_rmsnorm, GateUpSwiGlu on Q4_K, Add; positions and lengths
    from the step block, device-resident block table): eager launches (host
    mirror bookkeeping, snapshot callbacks and error-word reads per launch)
    against one replay of the captured plugin stream."""
    import time

    import numpy as np

    from fellm_amd import abi, synth
    from fellm_amd.plugin_host import PagedKvContext, PluginHost

    D = abi.DType
    H, I, nq, nkv, hd, n_logical, bs = 4096, 14336, 32, 8, 128, 256, 16
    stride = nkv * hd
    rng = np.random.default_rng(10)
    keep = []

    def tref(a, dt, dims=None, logical_id=0):
        keep.append(a)
        return abi.tensor_ref(a.ctypes.data, a.nbytes, dt, dims or [a.size], logical_id)

    def tmut(a, dt, dims=None):
        keep.append(a)
        return abi.tensor_mut(a.ctypes.data, a.nbytes, dt, dims or [a.size])

    host = PluginHost()
    bb = (2 * bs * stride * 2 + 63) // 64 * 64
    arena = torch.zeros(n_logical * bb, dtype=torch.uint8, device=dev)
    table = rng.permutation(n_logical).astype(np.uint32)
    table_dev = torch.from_numpy(table.view(np.int32)).to(dev)
    host_arena = np.zeros(8, np.uint8)
    zero = np.zeros(1, np.uint32)
    ctx = PagedKvContext(arena_ptr=host_arena.ctypes.data, arena_len=8, block_table=table, n_logical_blocks=n_logical,
                         n_layers=1, tokens_stride=stride, block_bytes=bb, block_size=bs, row_positions=zero,
                         row_rope_positions=zero, row_lengths=zero + 1, device_arena_ptr=arena.data_ptr(),
                         device_arena_len=arena.numel(), device_block_table_ptr=table_dev.data_ptr(),
                         n_device_block_table=table.size, device_logical_stride=n_logical)
    seq = 2048
    x = rng.normal(size=H).astype(np.float32)
    n1 = (1 + 0.1 * rng.normal(size=H)).astype(np.float32)
    n2 = (1 + 0.1 * rng.normal(size=H)).astype(np.float32)
    q = rng.normal(size=H).astype(np.float32)
    k = rng.normal(size=stride).astype(np.float32)
    v = rng.normal(size=stride).astype(np.float32)
    inv = (1.0 / (500000.0 ** (np.arange(0, hd, 2) / hd))).astype(np.float32)
    wg = synth.KQUANT_TABLES[12](rng, I, H)
    wu = synth.KQUANT_TABLES[12](rng, I, H)
    y = np.zeros(H, np.float32)
    qo = np.zeros(H, np.float32)
    att = np.zeros(H, np.float32)
    h2 = np.zeros(H, np.float32)
    y2 = np.zeros(H, np.float32)
    act = np.zeros(I, np.float32)
    o = np.zeros(I, np.float32)
    dummy = np.zeros(1, np.float32)
    lk = lambda op, i, od: host.lookup(op, i, od)  # noqa: E731
    h_rms = lk(abi.OpKind.RMSNORM, [D.F32, D.F32], D.F32)
    h_rkv = lk(abi.OP_ROPE_KV_WRITE, [D.F32, D.F32, D.F32, D.F32], D.F32)
    h_att = lk(abi.OpKind.ATTENTION, [D.F32, D.F32, D.F32], D.F32)
    h_arn = lk(abi.OP_ADD_RMSNORM, [D.F32, D.F32, D.F32], D.F32)
    h_gu = lk(abi.OpKind.GATE_UP_SWIGLU, [D.Q4K, D.Q4K, D.F32], D.F32)
    h_add = lk(abi.OpKind.ADD, [D.F32, D.F32], D.F32)

    def layer():
        host.launch(h_rms, abi.OpAttrs(eps=1e-5), [tref(x, D.F32), tref(n1, D.F32)], [tmut(y, D.F32)])
        host.launch(h_rkv, abi.OpAttrs(n_heads=nq, n_kv_heads=nkv, head_dim=hd, rope_dim=hd, block_size=bs),
                    [tref(q, D.F32), tref(k, D.F32), tref(v, D.F32), tref(inv, D.F32)], [tmut(qo, D.F32)])
        host.launch(h_att, abi.OpAttrs(n_heads=nq, n_kv_heads=nkv, head_dim=hd, block_size=bs),
                    [tref(qo, D.F32), tref(dummy, D.F32), tref(dummy, D.F32)], [tmut(att, D.F32)])
        host.launch(h_arn, abi.OpAttrs(eps=1e-5), [tref(att, D.F32), tref(x, D.F32), tref(n2, D.F32)],
                    [tmut(h2, D.F32), tmut(y2, D.F32)])
        host.launch(h_gu, abi.OpAttrs(), [tref(wg, D.Q4K, [I, H], 91), tref(wu, D.Q4K, [I, H], 92),
                                          tref(y2, D.F32)], [tmut(act, D.F32)])
        host.launch(h_add, abi.OpAttrs(), [tref(act, D.F32), tref(act, D.F32)], [tmut(o, D.F32)])

    host.set_paged_context(ctx)
    try:
        host.update_step_params(abi.DeviceStepParams(position=seq - 1, sequence_length=seq, active_batch=1,
                                                     kv_write_slot=(seq - 1) % bs))
        stream = host.stream()
        for _ in range(warmup):
            layer()
        stream.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            layer()
        stream.synchronize()
        eager = (time.perf_counter() - t0) / steps
        cap = host.begin_graph_capture()
        try:
            layer()
        except Exception:
            cap.abort()
            raise
        exe = cap.finish()
        for _ in range(warmup):
            exe.launch(stream)
        stream.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            exe.launch(stream)
        stream.synchronize()
        replay = (time.perf_counter() - t0) / steps
        exe.close()
    finally:
        host.set_paged_context(None)
    return {"eager_us_per_step": round(eager * 1e6, 2), "graph_us_per_step": round(replay * 1e6, 2),
            "speedup": round(eager / replay, 2)}


# --------------------------------------------------------------------------- #
# Timing
# --------------------------------------------------------------------------- #
class DeviceEvent:
    """A HIP event recorded with a device-scope release (hipEventReleaseToDevice).

    torch's events record with a system-scope release, which writes dirty
    cache lines back at every record; between the kernels of a chain that
    perturbs the very kernels being timed (a traced SwiGLU took 62.5 us
    without events in between and 68-85 us with them).  A device-scope
    release leaves the caches alone."""

    _hip = None
    RELEASE_TO_DEVICE = 0x40000000

    def __init__(self):
        import ctypes

        if DeviceEvent._hip is None:
            hip = ctypes.CDLL("libamdhip64.so")
            hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
            hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
            hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
            hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
            DeviceEvent._hip = hip
        self._ctypes = ctypes
        self.h = ctypes.c_void_p()
        if DeviceEvent._hip.hipEventCreateWithFlags(ctypes.byref(self.h), self.RELEASE_TO_DEVICE) != 0:
            raise RuntimeError("hipEventCreateWithFlags failed")

    def record(self, stream):
        if DeviceEvent._hip.hipEventRecord(self.h, stream.cuda_stream) != 0:
            raise RuntimeError("hipEventRecord failed")

    def elapsed_time(self, end) -> float:
        ms = self._ctypes.c_float()
        if DeviceEvent._hip.hipEventElapsedTime(self._ctypes.byref(ms), self.h, end.h) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value

    def __del__(self):
        try:
            if self.h:
                DeviceEvent._hip.hipEventDestroy(self.h)
        except Exception:
            pass


def run_chain(torch, chain, sets, steps, warmup, reps=None):
    """Two timed passes.

    Pass 1 (whole job): `steps` steps of the chain with no instrumentation,
    wall clock between two device synchronisations -> elapsed seconds.
    Pass 2 (per op): `reps` (>= 50) more steps of the chain in the same order
    and input rotation, every op armed with its own event pair through
    fellm_rocm_timing_arm: the events are attached to the op's kernels
    (hipExtLaunchKernel), so each pair measures the kernels' device time with
    nothing inserted between launches.  Per-op time = median over the reps.
    """
    from fellm_amd import _lib

    lib = _lib.lib()
    reps = max(steps, 50) if reps is None else reps
    for i in range(warmup):
        for op in chain:
            op.fn(sets[i % len(sets)])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        s = sets[i % len(sets)]
        for op in chain:
            op.fn(s)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ev = [[(DeviceEvent(), DeviceEvent()) for _ in chain] for _ in range(reps)]
    for i in range(reps):
        s = sets[i % len(sets)]
        for j, op in enumerate(chain):
            a, b = ev[i][j]
            if lib.fellm_rocm_timing_arm(a.h, b.h) != 0:
                raise RuntimeError("fellm_rocm_timing_arm failed")
            try:
                op.fn(s)
            finally:
                lib.fellm_rocm_timing_disarm()
    torch.cuda.synchronize()
    per_op = []
    for j, op in enumerate(chain):
        ms = sorted(ev[i][j][0].elapsed_time(ev[i][j][1]) for i in range(reps))
        per_op.append({"op": op.name, "bytes": op.nbytes, "ms_median": ms[len(ms) // 2],
                       "ms_mean": sum(ms) / len(ms), "ms_min": ms[0], "reps": reps})
    return (t1 - t0), per_op


PROBE_VARIANTS = {0: "U1", 2: "U2", 3: "U4", 4: "U1 nt", 6: "U2 nt", 7: "U4 nt"}


def measure_ceilings(torch, chain, reps, min_rotation_bytes=768 << 20):
    """Same-run copy ceiling of each op: fellm_rocm_stream_probe moving the
    op's read and write bytes (its `probe` pattern) with no arithmetic, every
    variant (16-byte units per thread 1/2/4, regular or non-temporal), each
    timed like the ops (kernel-attached events, median of `reps`), buffers
    rotating over enough sets (>= 3, together >= min_rotation_bytes, three
    times the 256 MB MALL) that no launch finds its inputs cached.  The
    ceiling is the fastest variant."""
    from fellm_amd import _lib

    lib = _lib.lib()
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    out = {}
    for op in chain:
        if op.probe is None:
            continue
        nr, rlen, wlen = op.probe
        moved = nr * rlen + wlen
        n_sets = max(3, -(-min_rotation_bytes // moved))
        bufs = [[torch.empty(rlen, dtype=torch.uint8, device=dev) for _ in range(nr)] +
                [torch.empty(wlen, dtype=torch.uint8, device=dev)] for _ in range(n_sets)]
        for b in bufs:
            for t in b[:nr]:
                t.random_(0, 255)
        best = None
        for var, vname in PROBE_VARIANTS.items():
            ev = [(DeviceEvent(), DeviceEvent()) for _ in range(reps)]
            for i in range(reps + 3):
                b = bufs[i % n_sets]
                args = (b[0].data_ptr(), b[1].data_ptr() if nr == 2 else None, rlen, b[nr].data_ptr(), wlen, var,
                        stream.cuda_stream)
                if i < 3:
                    lib.fellm_rocm_stream_probe(*args)
                    continue
                e0, e1 = ev[i - 3]
                lib.fellm_rocm_timing_arm(e0.h, e1.h)
                try:
                    if lib.fellm_rocm_stream_probe(*args) != 0:
                        raise RuntimeError("stream probe failed")
                finally:
                    lib.fellm_rocm_timing_disarm()
            torch.cuda.synchronize()
            ms = sorted(a.elapsed_time(b) for a, b in ev)[reps // 2]
            if best is None or ms < best[0]:
                best = (ms, vname)
        out[op.name] = {"probe_bytes": moved, "probe_us": round(best[0] * 1e3, 2), "probe_variant": best[1],
                        "probe_GBps": round(moved / (best[0] * 1e-3) / 1e9, 1),
                        "probe_frac_of_peak": round(moved / (best[0] * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}
        del bufs
    return out


def op_report(per_op):
    """Per-op GB/s from the median kernel time (algorithmic bytes / time)."""
    out = {}
    for r in per_op:
        gbps = r["bytes"] / (r["ms_median"] * 1e-3) / 1e9
        out[r["op"]] = {"bytes": r["bytes"], "us_median": round(r["ms_median"] * 1e3, 2),
                        "us_mean": round(r["ms_mean"] * 1e3, 2), "us_min": round(r["ms_min"] * 1e3, 2),
                        "reps": r["reps"], "GBps": round(gbps, 1), "frac_of_peak": round(gbps / HBM_PEAK_GBPS, 4)}
    return out


# --------------------------------------------------------------------------- #
# CPU baseline: the oracle (C restatement of backend-cpu), 1 thread
# --------------------------------------------------------------------------- #
def host_cpu_info(flags: str) -> dict:
    """CPU model, logical CPUs available to this process, and the vector ISA
    the -march=native build targets (from gcc's resolved target options)."""
    import re
    import subprocess

    info = {"cpu": platform.processor() or "unknown", "host_logical_cpus": len(os.sched_getaffinity(0))}
    try:
        cpuinfo = Path("/proc/cpuinfo").read_text()
        info["cpu"] = next((l.split(":", 1)[1].strip() for l in cpuinfo.splitlines() if l.startswith("model name")),
                           info["cpu"])
    except OSError:
        pass
    try:
        q = subprocess.run(["gcc", *flags.split(), "-Q", "--help=target"], capture_output=True, text=True,
                           check=True).stdout
        enabled = set(re.findall(r"^\s+-m(\S+)\s+\[enabled\]", q, re.M))
        march = re.search(r"^\s+-march=\s+(\S+)", q, re.M)
        isa = "AVX-512" if "avx512f" in enabled else ("AVX2" if "avx2" in enabled else "SSE2")
        info["isa"] = (f"{isa} (gcc {' '.join(flags.split()[1:3])} resolved to -march={march.group(1) if march else '?'}"
                       f"; fma {'on' if 'fma' in enabled else 'off'}, f16c {'on' if 'f16c' in enabled else 'off'})")
    except (OSError, subprocess.CalledProcessError):
        info["isa"] = "unknown"
    return info


def cpu_baseline(budget_s: float, threads: int = 1, _native=None):
    """CPU baseline: the oracle's restatement of backend-cpu's c2 chain
    (f32 ops, as the CPU backend computes them) on 64-token samples, compiled
    for this host with -march=native the way the reference is built
    (.cargo/config.toml:1-7): RMSNorm's sum of squares in 8-lane f32
    vectors (norm.rs:12-19), add at the widest width, silu/RoPE through
    libm expf/sinf/cosf, scalar as in the reference.  threads > 1: that many
    workers each run their own samples concurrently (the C code releases the
    GIL), i.e. rows spread over cores; the reference's own launchers are
    serial, so threads = 1 is the faithful figure."""
    import tempfile

    import numpy as np

    import oracle

    if _native is None:
        path, flags = oracle.build_native(Path(tempfile.mkdtemp(prefix="oracle_native_")))
        oracle.use_library(path)
        _native = flags
    if threads > 1:
        from concurrent.futures import ThreadPoolExecutor

        with ThreadPoolExecutor(max_workers=threads) as ex:
            parts = list(ex.map(lambda _: cpu_baseline(budget_s, 1, _native), range(threads)))
        out = dict(parts[0])
        out["value"] = round(sum(p["value"] for p in parts), 1)
        out["cores"] = threads
        out["sample"] = (f"{threads} threads, each repeating 64-token c2 chains for {budget_s:.0f}s "
                         "(rows spread over cores; f32 ops as backend-cpu)")
        return out

    T, H, I, V = 64, 4096, 14336, 4096  # sample: 64 tokens of the c2 chain
    nq, nkv, hd = 32, 8, 128
    rng = np.random.default_rng(7)
    # The reference's op boundary is f32: the CPU path gathers f16 rows into f32.
    table = (rng.normal(0, 0.02, size=(V, H))).astype(np.float16)
    ids = rng.integers(0, V, size=T, dtype=np.uint32)
    x = rng.normal(size=(T, H)).astype(np.float32)
    r = (2 * rng.normal(size=(T, H))).astype(np.float32)
    w = rng.normal(1.0, 0.1, size=H).astype(np.float32)
    q = rng.normal(size=(T, nq * hd)).astype(np.float32)
    k = rng.normal(size=(T, nkv * hd)).astype(np.float32)
    inv = oracle.rope_inv_freqs(500000.0, hd)
    pos = np.arange(T, dtype=np.uint32)
    gt = rng.normal(size=(T, I)).astype(np.float32)
    up = rng.normal(size=(T, I)).astype(np.float32)
    iters, t0 = 0, time.perf_counter()
    while True:
        oracle.embedding(table.view(np.uint8), 1, V, H, ids)
        h = oracle.add(x, r)
        oracle.rmsnorm(h, w, 1e-5)
        oracle.rope(q, nq, hd, hd, 0, inv, pos)
        oracle.rope(k, nkv, hd, hd, 0, inv, pos)
        oracle.silu_gate(gt, up)
        iters += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    out = {"value": round(T * iters / el, 1), "unit": "tokens/s", "cores": 1, "kind": "port",
           "sample": f"{iters} x 64-token c2 chain (embedding f16->f32, add, rmsnorm, rope q+k, swiglu) in "
                     f"{el:.1f}s, f32 ops as backend-cpu, 1 thread",
           "code": "oracle/fellm_oracle.c, a C restatement of backend-cpu in its operation order, "
                   f"compiled on this host: gcc {_native}"}
    out.update(host_cpu_info(_native))
    return out


def cpu_suite_ops(cfg: str):
    """Per-op CPU samples of a config: (op name as the GPU suite names it,
    rows of that op in the config, rows in the sample, callable).  The
    oracle computes every op as backend-cpu does, in f32 at the op boundary
    (gathers widen or dequantize to f32 rows); tables are 4096-row slices of
    the config's table shape (a gather's cost per row does not depend on the
    vocabulary), the paged arena 512 blocks."""
    import numpy as np

    import oracle
    from fellm_amd import synth

    rng = np.random.default_rng(11)
    f32 = np.float32

    def randn(*shape, std=1.0):
        return (std * rng.normal(size=shape)).astype(f32)

    ops = []

    def chain(T_cfg, T, H, nq, nkv, hd, theta, I, eps, table_kind, with_add=True):
        V = 4096
        if table_kind == "f16":
            table = rng.normal(0, 0.02, size=(V, H)).astype(np.float16).view(np.uint8)
            code = 1
        else:
            table = rng.normal(0, 0.02, size=(V, H)).astype(f32).view(np.uint8)
            code = 0
        ids = rng.integers(0, V, size=T, dtype=np.uint32)
        x, r, w = randn(T, H), randn(T, H, std=2.0), (1.0 + 0.1 * rng.normal(size=H)).astype(f32)
        q, k = randn(T, nq * hd), randn(T, nkv * hd)
        inv = oracle.rope_inv_freqs(theta, hd)
        pos = np.arange(T, dtype=np.uint32)
        g, u = randn(T, I), randn(T, I)
        emb = "embedding_f16" if table_kind == "f16" else "embedding_f32"
        ops.append((emb, T_cfg, T, lambda: oracle.embedding(table, code, V, H, ids)))
        if with_add:
            ops.append(("add_rmsnorm", T_cfg, T, lambda: oracle.rmsnorm(oracle.add(x, r), w, eps)))
        else:
            ops.append(("rmsnorm", T_cfg, T, lambda: oracle.rmsnorm(x, w, eps)))
        ops.append(("rope_qk", T_cfg, T, lambda: (oracle.rope(q, nq, hd, hd, 0, inv, pos),
                                                  oracle.rope(k, nkv, hd, hd, 0, inv, pos))))
        ops.append(("swiglu", T_cfg, T, lambda: oracle.silu_gate(g, u)))

    if cfg == "c1":
        chain(64, 64, 2048, 32, 8, 64, 500000.0, 8192, 1e-5, "f32")
    elif cfg == "c2":
        chain(4096, 64, 4096, 32, 8, 128, 500000.0, 14336, 1e-5, "f16")
    elif cfg == "c3":
        V, D, T = 4096, 3584, 256
        q4, q6 = synth.q4k_table(rng, V, D), synth.q6k_table(rng, V, D)
        ids = synth.zipf_ids(rng, T, V)
        w = (1.0 + 0.1 * rng.normal(size=D)).astype(f32)
        ops.append(("q4k_gather", 8192, T, lambda: oracle.embedding(q4, 12, V, D, ids)))
        ops.append(("q6k_gather", 8192, T, lambda: oracle.embedding(q6, 14, V, D, ids)))
        ops.append(("q4k_gather_rmsnorm", 8192, T, lambda: oracle.rmsnorm(oracle.embedding(q4, 12, V, D, ids), w, 1e-6)))
        ops.append(("q6k_gather_rmsnorm", 8192, T, lambda: oracle.rmsnorm(oracle.embedding(q6, 14, V, D, ids), w, 1e-6)))
        q5, q8 = synth.q5k_table(rng, V, D), synth.q8_0_table(rng, V, D)
        ops.append(("q5k_gather", 8192, T, lambda: oracle.embedding(q5, 13, V, D, ids)))
        ops.append(("q8_0_gather", 8192, T, lambda: oracle.embedding(q8, 8, V, D, ids)))
    elif cfg == "c4":
        B, nq, nkv, hd, bs, nblk, H, I = 256, 64, 8, 128, 16, 512, 8192, 28672
        stride = nkv * hd
        bb = 2 * bs * stride * 2
        pos, table, n_logical = synth.paged_layout(rng, B, nblk, bs, 32768)
        arena = np.zeros(nblk * bb, np.uint8)
        inv = oracle.rope_inv_freqs(500000.0, hd)
        q, k, v = randn(B, nq * hd), randn(B, stride), randn(B, stride)
        x, r, w = randn(B, H), randn(B, H, std=2.0), (1.0 + 0.1 * rng.normal(size=H)).astype(f32)
        g, u = randn(B, I), randn(B, I)

        def rope_kv():
            oracle.rope(q, nq, hd, hd, 0, inv, pos)
            kr = oracle.rope(k, nkv, hd, hd, 0, inv, pos)
            oracle.kv_write_paged(kr, stride, pos, table, n_logical, 1, 0, bs, bb, arena, False, "bf16")
            oracle.kv_write_paged(v, stride, pos, table, n_logical, 1, 0, bs, bb, arena, True, "bf16")

        ops.append(("rope_kv_write", B, B, rope_kv))
        ops.append(("add_rmsnorm", B, B, lambda: oracle.rmsnorm(oracle.add(x, r), w, 1e-5)))
        ops.append(("swiglu", B, 32, lambda: oracle.silu_gate(g[:32], u[:32])))
    elif cfg == "c5":
        T, E, H, I, hd = 16384, 128, 2048, 768, 128
        logits = randn(T, E)
        ops.append(("router_topk", T, T, lambda: oracle.router(logits, 8)))
        g, u = randn(1024, I), randn(1024, I)
        ops.append(("swiglu_routed", T * 8, 1024, lambda: oracle.silu_gate(g, u)))
        x, w = randn(512, H), (1.0 + 0.1 * rng.normal(size=H)).astype(f32)
        ops.append(("rmsnorm", T, 512, lambda: oracle.rmsnorm(x, w, 1e-6)))
        q, k = randn(256, 32 * hd), randn(256, 4 * hd)
        inv = oracle.rope_inv_freqs(1e6, hd)
        pos = np.arange(8000, 8256, dtype=np.uint32)
        ops.append(("rope_qk", T, 256, lambda: (oracle.rope(q, 32, hd, hd, 0, inv, pos),
                                                oracle.rope(k, 4, hd, hd, 0, inv, pos))))
    return ops


def cpu_suite(cfg: str, gpu_ops: dict | None, budget_s: float = 0.5) -> dict:
    """Times each of the config's ops on the CPU (1 thread, the native oracle
    build) for about budget_s each; reports rows/s, the full-config time
    extrapolated per row, and the GPU's speedup over it where the GPU suite
    timed the same op."""
    out = {}
    for name, rows_cfg, rows, fn in cpu_suite_ops(cfg):
        fn()
        n, t0 = 0, time.perf_counter()
        while True:
            fn()
            n += 1
            el = time.perf_counter() - t0
            if el >= budget_s and n >= 3:
                break
        per_row_us = el / n / rows * 1e6
        rec = {"sample_rows": rows, "config_rows": rows_cfg, "us_per_sample": round(el / n * 1e6, 1),
               "rows_per_s": round(rows / (el / n), 1), "us_full_config_est": round(per_row_us * rows_cfg, 1)}
        if gpu_ops and name in gpu_ops and "us_median" in gpu_ops[name]:
            rec["gpu_speedup"] = round(per_row_us * rows_cfg / gpu_ops[name]["us_median"], 1)
        out[name] = rec
    return out


# --------------------------------------------------------------------------- #
def read_traffic():
    """HBM bytes per SwiGLU launch from the committed rocprofv3 PMC summary, if present."""
    p = ROOT / "profiles" / "swiglu_c2_pmc_traffic.txt"
    if not p.exists():
        return None
    for line in p.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (every op shards by tokens "
              "or rows with no exchange between GPUs).  Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch

    from fellm_amd import ops

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.calibrate_copy:
        n = 512 << 20
        a = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()

    if args.suite:
        result = {}
        for name, make in (("c2", c2_ops), ("c3", c3_ops), ("c4", c4_ops), ("c5", c5_ops),
                           ("next_gemv", gemv_ops), ("next_attention", attention_ops),
                           ("next_moe", moe_ops)):
            if args.only and name not in args.only.split(","):
                continue
            chain, sets, _ = make(torch, ops, dev, args.sets)
            _, per_op = run_chain(torch, chain, sets, args.steps, args.warmup, args.reps or None)
            result[name] = op_report(per_op)
            del sets
            torch.cuda.empty_cache()
            ceilings = {} if args.no_ceiling else measure_ceilings(torch, chain, args.reps or max(args.steps, 50))
            for op_name, c in ceilings.items():
                result[name][op_name].update(c)
                result[name][op_name]["frac_of_probe"] = round(result[name][op_name]["GBps"] / c["probe_GBps"], 4)
            del chain
            torch.cuda.empty_cache()
        if not args.only or "next_graph" in args.only.split(","):
            result["next_graph"] = decode_graph_report(torch, ops, dev, max(args.steps, 50), args.warmup)
        if not args.no_cpu_baseline:
            # The same ops on the host (1 thread, the oracle built -march=native
            # as the reference is built), per op, after the GPU work.
            import tempfile

            import oracle

            path, flags = oracle.build_native(Path(tempfile.mkdtemp(prefix="oracle_native_")))
            oracle.use_library(path)
            cpu = {"info": host_cpu_info(flags), "threads": 1,
                   "method": "oracle/fellm_oracle.c (backend-cpu's operation order, f32 at the op boundary) on a "
                             "sample of each op's rows for ~0.5 s; us_full_config_est = per-row time x the "
                             "config's rows; gpu_speedup = that / the GPU median above"}
            for cfg in ("c1", "c2", "c3", "c4", "c5"):
                if args.only and cfg not in args.only.split(",") and "cpu" not in args.only.split(","):
                    continue
                cpu[cfg] = cpu_suite(cfg, result.get(cfg))
                if cfg == "c4" and all(k in cpu[cfg] for k in ("rope_kv_write", "add_rmsnorm", "swiglu")):
                    est = sum(cpu[cfg][k]["us_full_config_est"] for k in ("rope_kv_write", "add_rmsnorm", "swiglu"))
                    rec = {"us_full_config_est": round(est, 1), "of": "the three ops above"}
                    if result.get("c4", {}).get("decode_step_fused"):
                        rec["gpu_speedup"] = round(est / result["c4"]["decode_step_fused"]["us_median"], 1)
                    cpu[cfg]["decode_step_fused"] = rec
            result["cpu"] = cpu
        print(json.dumps({"suite": result}, indent=1))
        return

    chain, sets, T = c2_ops(torch, ops, dev, args.sets)
    elapsed, per_op = run_chain(torch, chain, sets, args.steps, args.warmup, args.reps or None)
    rep = op_report(per_op)
    del sets
    torch.cuda.empty_cache()
    ceilings = {} if args.no_ceiling else measure_ceilings(torch, chain, args.reps or max(args.steps, 50))
    for name, c in ceilings.items():
        rep[name].update(c)
        rep[name]["frac_of_probe"] = round(rep[name]["GBps"] / c["probe_GBps"], 4)
    ms_step = elapsed / args.steps * 1e3
    kernel_sum_ms = sum(r["ms_median"] for r in per_op)
    dom = max(per_op, key=lambda r: r["bytes"])
    achieved = dom["bytes"] / (dom["ms_median"] * 1e-3) / 1e9
    traffic = read_traffic()
    line = {
        "metric": METRIC,
        "value": round(T * args.steps / elapsed, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded; table ~N(0,0.02), x ~N(0,1), r ~N(0,4), ids uniform)",
        "config": {"workload": "configs[1] Llama-3-8B prefill op chain: embedding f16 gather + add/RMSNorm "
                               "H4096 + RoPE q+k hd128 32/8 + SwiGLU I14336", "tokens": T,
                   "rotating_input_sets": args.sets},
        "roofline": {"bound": "hbm", "kernel": dom["op"], "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": traffic,
                     "traffic_source": "committed constant, not measured in this run: HBM bytes per SwiGLU "
                                       "launch from profiles/swiglu_c2_pmc_traffic.txt (rocprofv3 --pmc "
                                       "FETCH_SIZE and WRITE_SIZE, calibrated on a plain device copy)",
                     "time_source": "median of the per-op pass's kernel-attached HIP events "
                                    "(fellm_rocm_timing_arm)",
                     "same_run_probe_frac": rep[dom["op"]].get("frac_of_probe")},
        "ops": rep,
        "chain_tokens_per_s_kernel_sum": round(T / (kernel_sum_ms * 1e-3), 1),
        "chain_GBps_kernel_sum": round(sum(r["bytes"] for r in per_op) / (kernel_sum_ms * 1e-3) / 1e9, 1),
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
        n_par = min(16, os.cpu_count() or 1)
        if n_par > 1:
            line["cpu_baseline_parallel"] = cpu_baseline(min(args.cpu_seconds, 5.0), n_par)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
