"""GPU tests through the plugin C ABI with host buffers, as FeLLM's plugin host
drives it (crates/fellm-plugin-host/tests/load_cuda_kernels.rs pattern):
dlopen + ABI check + registration, then registry launches with TensorRef /
TensorMut over host memory.  Outputs stay device-valid; a same-dtype Cast
launch materialises them into host memory (launchers.rs:140-170).
"""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")  # load torch's HIP runtime before the plugin

import oracle  # noqa: E402
from fellm_amd import abi, synth  # noqa: E402
from fellm_amd.plugin_host import PagedKvContext, PluginHost  # noqa: E402
from parity_util import assert_close, assert_exact, ordered16  # noqa: E402

pytestmark = pytest.mark.gpu
D = abi.DType


@pytest.fixture(scope="module")
def host():
    torch.cuda.init()
    h = PluginHost()
    yield h
    h.set_paged_context(None)


# The plugin keys device mirrors by (host pointer, byte length), like the
# reference (plugins/cuda_kernels/src/buffers.rs:341-394): a freed host buffer
# whose address numpy hands out again would alias a stale mirror.  FeLLM's host
# owns long-lived buffers and invalidates after CPU writes; these tests keep
# every host buffer alive for the module instead.
_KEEP = []


def tref(a: np.ndarray, dt, dims=None, logical_id=0):
    _KEEP.append(a)
    return abi.tensor_ref(a.ctypes.data, a.nbytes, dt, dims or [a.size], logical_id)


def tmut(a: np.ndarray, dt, dims=None):
    _KEEP.append(a)
    return abi.tensor_mut(a.ctypes.data, a.nbytes, dt, dims or [a.size])


def run(host, op, ins_dt, out_dt, attrs, ins, outs):
    h = host.lookup(op, ins_dt, out_dt)
    assert h is not None, (op, ins_dt, out_dt)
    host.launch(h, attrs, ins, outs)


def materialize(host, buf: np.ndarray, dt):
    """Cast launch: copy buf's device mirror into a fresh host array."""
    out = np.empty_like(buf)
    run(host, abi.OpKind.CAST, [dt], dt, abi.OpAttrs(), [tref(buf, dt)], [tmut(out, dt)])
    return out


def test_rmsnorm_f32(host):
    rng = np.random.default_rng(0)
    x = rng.normal(size=(64, 2048)).astype(np.float32)
    w = rng.normal(1, 0.1, 2048).astype(np.float32)
    y = np.zeros_like(x)
    run(host, abi.OpKind.RMSNORM, [D.F32, D.F32], D.F32, abi.OpAttrs(eps=1e-5),
        [tref(x, D.F32, [64, 2048]), tref(w, D.F32, logical_id=101)], [tmut(y, D.F32, [64, 2048])])
    got = materialize(host, y, D.F32)
    assert_close(got, oracle.rmsnorm(x, w, 1e-5), "f32", what="plugin rmsnorm")


def test_silu_gate_f16_and_chain_stays_on_device(host):
    rng = np.random.default_rng(1)
    g = rng.normal(size=4096).astype(np.float16)
    u = rng.normal(size=4096).astype(np.float16)
    a = np.zeros(4096, np.float16)
    b = np.zeros(4096, np.float16)
    sg = (abi.OpKind.SILU_GATE, [D.F16, D.F16], D.F16)
    run(host, *sg, abi.OpAttrs(), [tref(g, D.F16), tref(u, D.F16)], [tmut(a, D.F16)])
    # `a` is only device-valid: feeding it back must use the device copy, not the zero host bytes
    run(host, *sg, abi.OpAttrs(), [tref(a, D.F16), tref(u, D.F16)], [tmut(b, D.F16)])
    ref_a = oracle.narrow(oracle.silu_gate(g.astype(np.float32), u.astype(np.float32)), "f16")
    ref_b = oracle.narrow(oracle.silu_gate(oracle.widen(ref_a, "f16"), u.astype(np.float32)), "f16")
    assert np.all(a == 0), "host copy of a device-valid output must not be written without a Cast"
    assert_exact(materialize(host, b, D.F16).view(np.uint16), ref_b, "chained silu")


def test_invalidate_refreshes_mirror(host):
    x = np.ones(1024, np.float32)
    z = np.zeros(1024, np.float32)
    out = np.zeros(1024, np.float32)
    add = (abi.OpKind.ADD, [D.F32, D.F32], D.F32)
    run(host, *add, abi.OpAttrs(), [tref(x, D.F32), tref(z, D.F32)], [tmut(out, D.F32)])
    x[:] = 5.0  # host write; the device mirror is now stale
    run(host, *add, abi.OpAttrs(), [tref(x, D.F32), tref(z, D.F32)], [tmut(out, D.F32)])
    assert np.all(materialize(host, out, D.F32) == 1.0)  # mirror reused, as in the reference cache
    host.invalidate(x.ctypes.data, x.nbytes)
    run(host, *add, abi.OpAttrs(), [tref(x, D.F32), tref(z, D.F32)], [tmut(out, D.F32)])
    assert np.all(materialize(host, out, D.F32) == 5.0)


def test_register_device_tensor(host):
    dev = torch.arange(256, dtype=torch.float32, device="cuda")
    shadow = np.zeros(256, np.float32)  # host view that is never read
    _KEEP.append((dev, shadow))  # the binding lives as long as the plugin
    assert host.register_device_tensor(shadow.ctypes.data, shadow.nbytes, dev.data_ptr()) == 0
    ones = np.ones(256, np.float32)
    out = np.zeros(256, np.float32)
    run(host, abi.OpKind.ADD, [D.F32, D.F32], D.F32, abi.OpAttrs(), [tref(shadow, D.F32), tref(ones, D.F32)],
        [tmut(out, D.F32)])
    assert np.array_equal(materialize(host, out, D.F32), np.arange(256, dtype=np.float32) + 1)


_QTABLE = {D.Q4K: synth.q4k_table, D.Q5K: synth.q5k_table, D.Q6K: synth.q6k_table, D.Q8_0: synth.q8_0_table}


@pytest.mark.parametrize("qt,out_dt", [(D.Q4K, D.F32), (D.Q6K, D.F16), (D.Q4K, D.F16), (D.Q5K, D.F32), (D.Q5K, D.F16),
                                       (D.Q8_0, D.F32), (D.Q8_0, D.F16)])
def test_embedding_quant(host, qt, out_dt):
    rng = np.random.default_rng(int(qt) + int(out_dt))
    vocab, dim = 200, 1024
    table = _QTABLE[qt](rng, vocab, dim)
    ids = rng.integers(0, vocab, size=50, dtype=np.uint32)
    out = np.zeros((50, dim), np.float32 if out_dt == D.F32 else np.float16)
    run(host, abi.OpKind.EMBEDDING, [qt, D.U32], out_dt, abi.OpAttrs(),
        [tref(table, qt, [vocab, dim], logical_id=2000 + int(qt) * 10 + int(out_dt)), tref(ids, D.U32)],
        [tmut(out, out_dt, [50, dim])])
    got = materialize(host, out, out_dt)
    ref = oracle.embedding(table, int(qt), vocab, dim, ids)
    if out_dt == D.F32:
        assert_exact(got, ref, "plugin q-embedding")
    else:
        assert_exact(got.view(np.uint16), oracle.narrow(ref, "f16"), "plugin q-embedding f16")


def test_embedding_q8_0_reference_block(host):
    """The Q8_0 block of the reference's CUDA test (load_cuda_kernels.rs:131-140: d = 1.0, values
    1..=32) as a one-row table, gathered through the registry's Embedding [Q8_0, U32] -> F32 key."""
    table = np.zeros(34, np.uint8)
    table[0:2] = [0x00, 0x3C]
    table[2:] = np.arange(1, 33)
    ids = np.zeros(3, np.uint32)
    out = np.zeros((3, 32), np.float32)
    run(host, abi.OpKind.EMBEDDING, [D.Q8_0, D.U32], D.F32, abi.OpAttrs(),
        [tref(table, D.Q8_0, [1, 32], logical_id=2999), tref(ids, D.U32)], [tmut(out, D.F32, [3, 32])])
    got = materialize(host, out, D.F32)
    assert np.array_equal(got, np.tile(np.arange(1, 33, dtype=np.float32), (3, 1)))


def test_embedding_weight_cached_by_logical_id(host):
    vocab, dim = 16, 64
    t = np.full((vocab, dim), 2.0, np.float32)
    ids = np.array([3], np.uint32)
    out = np.zeros((1, dim), np.float32)
    key = (abi.OpKind.EMBEDDING, [D.F32, D.U32], D.F32)
    run(host, *key, abi.OpAttrs(), [tref(t, D.F32, [vocab, dim], logical_id=777), tref(ids, D.U32)],
        [tmut(out, D.F32, [1, dim])])
    t[:] = 9.0  # weights are immutable per logical id: no re-upload
    run(host, *key, abi.OpAttrs(), [tref(t, D.F32, [vocab, dim], logical_id=777), tref(ids, D.U32)],
        [tmut(out, D.F32, [1, dim])])
    assert np.all(materialize(host, out, D.F32) == 2.0)


def _paged(rng, batch, nkv, hd, n_blocks, bs, max_pos, kv_dtype):
    stride = nkv * hd
    kv_pos, table, n_logical = synth.paged_layout(rng, batch, n_blocks, bs, max_pos)
    bb = (2 * bs * stride * 2 + 63) // 64 * 64
    arena = torch.zeros(n_blocks * bb, dtype=torch.uint8, device="cuda")
    host_arena = np.zeros(8, np.uint8)  # host mirror unused by the ROCm path
    rope_pos = (kv_pos + 3).astype(np.uint32)
    ctx = PagedKvContext(arena_ptr=host_arena.ctypes.data, arena_len=host_arena.size, block_table=table,
                         n_logical_blocks=n_logical, n_layers=1, tokens_stride=stride, block_bytes=bb,
                         block_size=bs, row_positions=kv_pos, row_rope_positions=rope_pos,
                         device_arena_ptr=arena.data_ptr(), device_arena_len=arena.numel())
    ctx._keep = (host_arena,)
    return ctx, arena, kv_pos, rope_pos, table, n_logical, bb, stride


def test_rope_uses_paged_row_positions(host):
    rng = np.random.default_rng(3)
    batch, nh, hd = 6, 4, 64
    ctx, arena, kv_pos, rope_pos, *_ = _paged(rng, batch, 1, hd, 16, 16, 256, "f16")
    host.set_paged_context(ctx)
    try:
        x = rng.normal(size=(batch, nh * hd)).astype(np.float32)
        inv = oracle.rope_inv_freqs(500000.0, hd)
        y = np.zeros_like(x)
        run(host, abi.OpKind.ROPE, [D.F32, D.F32], D.F32,
            abi.OpAttrs(n_heads=nh, head_dim=hd, rope_dim=hd, rope_pairing=0, position=99),
            [tref(x, D.F32), tref(inv, D.F32)], [tmut(y, D.F32)])
        got = materialize(host, y, D.F32)
        ref = oracle.rope(x, nh, hd, hd, 0, inv, rope_pos)
        assert_exact(got, ref, "plugin rope paged")
    finally:
        host.set_paged_context(None)
    # without a paged context: attrs.position + row
    x = rng.normal(size=(3, nh * hd)).astype(np.float32)
    y = np.zeros_like(x)
    run(host, abi.OpKind.ROPE, [D.F32, D.F32], D.F32, abi.OpAttrs(n_heads=nh, head_dim=hd, rope_dim=hd, position=40),
        [tref(x, D.F32), tref(inv, D.F32)], [tmut(y, D.F32)])
    assert_exact(materialize(host, y, D.F32), oracle.rope(x, nh, hd, hd, 0, inv, None, position0=40), "plugin rope pos0")


def test_rope_pre_rope_write_request_rotates(host):
    """custom_op_id 1 (backend.rs:1152-1158) asks for the pre-rotation rows to
    be captured; the plugin has no channel to the host's store (neither has the
    CUDA plugin), so the launch must still rotate exactly as without it."""
    rng = np.random.default_rng(13)
    nh, hd = 4, 64
    x = rng.normal(size=(5, nh * hd)).astype(np.float32)
    inv = oracle.rope_inv_freqs(500000.0, hd)
    y = np.zeros_like(x)
    run(host, abi.OpKind.ROPE, [D.F32, D.F32], D.F32,
        abi.OpAttrs(n_heads=nh, head_dim=hd, rope_dim=hd, position=7, custom_op_id=1, layer_ord=2),
        [tref(x, D.F32), tref(inv, D.F32)], [tmut(y, D.F32)])
    assert_exact(materialize(host, y, D.F32), oracle.rope(x, nh, hd, hd, 0, inv, None, position0=7), "pre-rope")


def test_rejected_launch_keeps_output_mirror(host):
    """An output that is valid only on the device stays valid when a later
    launch writing it is rejected before its kernel runs."""
    from fellm_amd.plugin_host import PluginError

    rng = np.random.default_rng(14)
    g = rng.normal(size=512).astype(np.float32)
    u = rng.normal(size=512).astype(np.float32)
    y = np.zeros(512, np.float32)
    run(host, abi.OpKind.SILU_GATE, [D.F32, D.F32], D.F32, abi.OpAttrs(), [tref(g, D.F32), tref(u, D.F32)],
        [tmut(y, D.F32)])
    inv = oracle.rope_inv_freqs(10000.0, 128)  # enough frequencies for rope_dim 128
    h = host.lookup(abi.OpKind.ROPE, [D.F32, D.F32], D.F32)
    with pytest.raises(PluginError) as e:  # rope_dim > head_dim: rejected by the kernel's shape check
        host.launch(h, abi.OpAttrs(n_heads=8, head_dim=64, rope_dim=128), [tref(g, D.F32), tref(inv, D.F32)],
                    [tmut(y, D.F32)])
    assert e.value.code == -2
    assert np.all(y == 0)
    assert_exact(materialize(host, y, D.F32), oracle.silu_gate(g, u), "device copy kept")


def test_kv_write_paged(host):
    rng = np.random.default_rng(4)
    batch, nkv, hd, bs, n_blocks = 9, 2, 64, 16, 32
    ctx, arena, kv_pos, _, table, n_logical, bb, stride = _paged(rng, batch, nkv, hd, n_blocks, bs, 500, "f16")
    host.set_paged_context(ctx)
    try:
        rows = rng.normal(size=(batch, stride)).astype(np.float32)
        cache_view = np.zeros(4, np.float32)
        for slot in (0, 1):
            run(host, abi.OpKind.KV_WRITE, [D.F32, D.F32], D.F32,
                abi.OpAttrs(block_size=bs, kv_slot=slot, layer_ord=0), [tref(rows, D.F32)],
                [tmut(cache_view, D.F32)])
        torch.cuda.synchronize()
        ref = np.zeros(arena.numel(), np.uint8)
        for slot in (0, 1):
            oracle.kv_write_paged(rows, stride, kv_pos, table, n_logical, 1, 0, bs, bb, ref, bool(slot))
        assert_exact(arena.cpu().numpy(), ref, "plugin paged kv")
    finally:
        host.set_paged_context(None)


def test_kv_write_paged_rejects_out_of_range_slot(host):
    """A row whose position lies past the sequence's logical blocks is refused
    before anything is enqueued (launchers.rs:3913-3945): the launch fails
    with the paged-range code and the arena is untouched."""
    from fellm_amd.plugin_host import PluginError
    rng = np.random.default_rng(5)
    batch, nkv, hd, bs, n_blocks = 4, 2, 64, 16, 16
    ctx, arena, kv_pos, *_ = _paged(rng, batch, nkv, hd, n_blocks, bs, 200, "f16")
    n_logical = ctx.n_logical_blocks
    bad = kv_pos.copy()
    bad[2] = n_logical * bs  # first position past the last logical block
    ctx.row_positions = bad
    host.set_paged_context(ctx)
    try:
        rows = rng.normal(size=(batch, nkv * hd)).astype(np.float32)
        with pytest.raises(PluginError) as e:
            run(host, abi.OpKind.KV_WRITE, [D.F32, D.F32], D.F32,
                abi.OpAttrs(block_size=bs, kv_slot=0, layer_ord=0), [tref(rows, D.F32)],
                [tmut(np.zeros(4, np.float32), D.F32)])
        assert e.value.code == abi.ERR_PAGED_RANGE
        torch.cuda.synchronize()
        assert not arena.cpu().numpy().any()
    finally:
        host.set_paged_context(None)


def test_kv_write_contiguous(host):
    row = np.arange(32, dtype=np.float32)
    cache = np.full((8, 32), -1.0, np.float32)
    run(host, abi.OpKind.KV_WRITE, [D.F32, D.F32], D.F32, abi.OpAttrs(position=5),
        [tref(row, D.F32)], [tmut(cache, D.F32, [8, 32])])
    got = materialize(host, cache, D.F32)
    want = np.full((8, 32), -1.0, np.float32)
    want[5] = row
    assert np.array_equal(got, want)


def test_custom_add_rmsnorm_f16(host):
    rng = np.random.default_rng(5)
    x = rng.normal(size=(33, 4096)).astype(np.float16)
    r = (2 * rng.normal(size=(33, 4096))).astype(np.float16)
    w = rng.normal(1, 0.1, 4096).astype(np.float32)
    h = np.zeros_like(x)
    y = np.zeros_like(x)
    run(host, abi.OP_ADD_RMSNORM, [D.F16, D.F16, D.F32], D.F16, abi.OpAttrs(eps=1e-5),
        [tref(x, D.F16), tref(r, D.F16), tref(w, D.F32)], [tmut(h, D.F16), tmut(y, D.F16)])
    h_ref, y_ref = oracle.add_rmsnorm(x.view(np.uint16), r.view(np.uint16), w, 1e-5, "f16")
    assert_exact(materialize(host, h, D.F16).view(np.uint16), h_ref, "plugin h")
    assert_close(materialize(host, y, D.F16).view(np.uint16), y_ref, "f16", what="plugin y")


def test_custom_router(host):
    rng = np.random.default_rng(6)
    logits = rng.normal(size=(300, 128)).astype(np.float32)
    ids = np.zeros((300, 8), np.uint32)
    w = np.zeros((300, 8), np.float32)
    run(host, abi.OP_ROUTER_TOPK, [D.F32], D.U32,
        abi.OpAttrs(n_experts=128, n_expert_used=8, expert_gating_func=1, norm_topk_prob=1),
        [tref(logits, D.F32)], [tmut(ids, D.U32), tmut(w, D.F32)])
    ids_r, w_r = oracle.router(logits, 8, 1, True, 0.0)
    assert_exact(materialize(host, ids, D.U32), ids_r, "plugin router ids")
    assert_exact(materialize(host, w, D.F32), w_r, "plugin router weights")


def test_custom_rope_kv_write_bf16(host):
    rng = np.random.default_rng(7)
    batch, nq, nkv, hd, bs, n_blocks = 12, 8, 2, 128, 16, 64
    ctx, arena, kv_pos, rope_pos, table, n_logical, bb, stride = _paged(rng, batch, nkv, hd, n_blocks, bs, 900,
                                                                         "bf16")
    host.set_paged_context(ctx)
    try:
        bits = lambda a: oracle.f32_to_bf16_bits(a)
        q = bits(rng.normal(size=(batch, nq * hd)).astype(np.float32))
        k = bits(rng.normal(size=(batch, stride)).astype(np.float32))
        v = bits(rng.normal(size=(batch, stride)).astype(np.float32))
        inv = oracle.rope_inv_freqs(500000.0, hd)
        qo = np.zeros_like(q)
        run(host, abi.OP_ROPE_KV_WRITE, [D.BF16, D.BF16, D.BF16, D.F32], D.BF16,
            abi.OpAttrs(n_heads=nq, n_kv_heads=nkv, head_dim=hd, rope_dim=hd, rope_pairing=0, layer_ord=0,
                        cast_to=int(D.BF16), block_size=bs),
            [tref(q, D.BF16), tref(k, D.BF16), tref(v, D.BF16), tref(inv, D.F32)], [tmut(qo, D.BF16)])
        qf = oracle.widen(q, "bf16")
        q_ref = oracle.narrow(oracle.rope(qf, nq, hd, hd, 0, inv, rope_pos), "bf16")
        assert_exact(materialize(host, qo, D.BF16), q_ref, "q")
        torch.cuda.synchronize()
        ref = np.zeros(arena.numel(), np.uint8)
        oracle.kv_write_paged(oracle.widen(v, "bf16"), stride, kv_pos, table, n_logical, 1, 0, bs, bb, ref, True,
                              "bf16")
        got = arena.cpu().numpy()
        for b in range(batch):
            vb = table[kv_pos[b] // bs] * bb + bs * stride * 2 + (kv_pos[b] % bs) * stride * 2
            assert_exact(got[vb:vb + stride * 2], ref[vb:vb + stride * 2], f"V row {b}")
    finally:
        host.set_paged_context(None)


def test_custom_embedding_rmsnorm(host):
    rng = np.random.default_rng(8)
    vocab, dim = 100, 3584
    table = synth.q4k_table(rng, vocab, dim)
    ids = synth.zipf_ids(rng, 64, vocab)
    w = rng.normal(1, 0.1, dim).astype(np.float32)
    h = np.zeros((64, dim), np.float16)
    y = np.zeros((64, dim), np.float16)
    run(host, abi.OP_EMBEDDING_RMSNORM, [D.Q4K, D.U32, D.F32], D.F16, abi.OpAttrs(eps=1e-6),
        [tref(table, D.Q4K, [vocab, dim], logical_id=4242), tref(ids, D.U32), tref(w, D.F32)],
        [tmut(h, D.F16, [64, dim]), tmut(y, D.F16, [64, dim])])
    e = oracle.embedding(table, 12, vocab, dim, ids)
    assert_exact(materialize(host, h, D.F16).view(np.uint16), oracle.narrow(e, "f16"), "fused h")
    assert_close(materialize(host, y, D.F16).view(np.uint16), oracle.narrow(oracle.rmsnorm(e, w, 1e-6), "f16"),
                 "f16", what="fused y")


@pytest.mark.parametrize("gt,ut", [(D.Q4K, D.Q4K), (D.Q5K, D.Q5K), (D.Q6K, D.Q6K), (D.Q4K, D.Q6K)])
def test_gate_up_swiglu(host, gt, ut):
    """GateUpSwiGlu [gate_w, up_w, x] -> out (backend.rs:944-1002), keyed like
    the CUDA plugin's registration (lib.rs:467-496), bit-exact with the oracle."""
    rng = np.random.default_rng(int(gt) * 31 + int(ut))
    rows, cols = 512, 2048
    g = synth.KQUANT_TABLES[int(gt)](rng, rows, cols)
    u = synth.KQUANT_TABLES[int(ut)](rng, rows, cols)
    x = rng.normal(size=cols).astype(np.float32)
    out = np.zeros(rows, np.float32)
    run(host, abi.OpKind.GATE_UP_SWIGLU, [gt, ut, D.F32], D.F32, abi.OpAttrs(),
        [tref(g, gt, [rows, cols], logical_id=7000 + 100 * int(gt) + int(ut)),
         tref(u, ut, [rows, cols], logical_id=8000 + 100 * int(gt) + int(ut)),
         tref(x, D.F32)], [tmut(out, D.F32)])
    ref = oracle.gate_up_swiglu(int(gt), g, int(ut), u, rows, cols, x)
    assert_exact(materialize(host, out, D.F32), ref, "plugin gate_up_swiglu")


def test_gate_up_swiglu_shape_errors(host):
    rows, cols = 8, 512
    g = np.zeros((rows, cols // 256 * 144), np.uint8)
    x = np.zeros(cols - 256, np.float32)  # wrong length
    out = np.zeros(rows, np.float32)
    h = host.lookup(abi.OpKind.GATE_UP_SWIGLU, [D.Q4K, D.Q4K, D.F32], D.F32)
    rc = host.launch_raw(h, abi.OpAttrs(), [tref(g, D.Q4K, [rows, cols], logical_id=901),
                                            tref(g, D.Q4K, [rows, cols], logical_id=901), tref(x, D.F32)],
                         [tmut(out, D.F32)])
    assert rc == abi.ERR_SHAPE


def test_attention_paged_batch(host):
    """Attention [q, k, v] -> out through the paged snapshot (backend.rs:1286-1323
    batch path): row r attends to row_lengths[r] keys of the device arena."""
    from test_oracle_attention import build_cache

    rng = np.random.default_rng(41)
    nh, nkv, hd = 16, 4, 128
    lengths = [3, 40, 17, 200]
    k = [rng.normal(size=(n, nkv * hd)).astype(np.float32) for n in lengths]
    v = [rng.normal(size=(n, nkv * hd)).astype(np.float32) for n in lengths]
    arena_np, table, n_logical, bb, _, v16 = build_cache(rng, k, v)
    arena = torch.from_numpy(arena_np).to("cuda")
    _KEEP.append(arena)
    q = rng.normal(size=(len(lengths), nh * hd)).astype(np.float32)
    lens = np.array(lengths, np.uint32)
    ctx = PagedKvContext(arena_ptr=arena_np.ctypes.data, arena_len=arena_np.size, block_table=table,
                         n_logical_blocks=n_logical, n_layers=1, tokens_stride=nkv * hd, block_bytes=bb,
                         block_size=16, row_positions=lens - 1, row_rope_positions=lens - 1, row_lengths=lens,
                         device_arena_ptr=arena.data_ptr(), device_arena_len=arena.numel())
    ctx._keep = (arena_np,)
    host.set_paged_context(ctx)
    try:
        out = np.zeros_like(q)
        dummy = np.zeros(1, np.float32)
        run(host, abi.OpKind.ATTENTION, [D.F32, D.F32, D.F32], D.F32,
            abi.OpAttrs(n_heads=nh, n_kv_heads=nkv, head_dim=hd, block_size=16, attention_window=0),
            [tref(q, D.F32), tref(dummy, D.F32), tref(dummy, D.F32)], [tmut(out, D.F32)])
        got = materialize(host, out, D.F32)
    finally:
        host.set_paged_context(None)
    ref = oracle.paged_attention(q, nh, nkv, hd, lens, float(np.float32(1 / np.sqrt(hd))), arena_np, table,
                                 n_logical, 1, 0, 16, bb)
    for r in range(len(lengths)):
        tol = 2e-5 * np.abs(v16[r]).max() + np.abs(ref[r]) * 2.0 ** -23
        assert np.all(np.abs(got[r] - ref[r]) <= tol), (r, np.abs(got[r] - ref[r]).max())


@pytest.mark.parametrize("window,mode", [(0, 0), (16, 0), (16, 1)])
def test_attention_contiguous_decode(host, window, mode):
    """Attention [F32, F32, F32] with block_size 0: one query row against keys
    0..past_len of host K/V (backend.rs:1371-1397); a window keeps the last
    `window` keys when causal, the first ones otherwise (attention_provider.rs:
    305-318 for one query row)."""
    rng = np.random.default_rng(31 + window + mode)
    nh, nkv, hd, past = 32, 8, 128, 200
    q = rng.normal(size=nh * hd).astype(np.float32)
    k = rng.normal(size=(256, nkv * hd)).astype(np.float32)  # capacity 256 rows, past + 1 used
    v = rng.normal(size=(256, nkv * hd)).astype(np.float32)
    out = np.zeros_like(q)
    run(host, abi.OpKind.ATTENTION, [D.F32, D.F32, D.F32], D.F32,
        abi.OpAttrs(n_heads=nh, n_kv_heads=nkv, head_dim=hd, past_len=past, block_size=0, attention_window=window,
                    attention_mode=mode),
        [tref(q, D.F32), tref(k, D.F32), tref(v, D.F32)], [tmut(out, D.F32)])
    seq = past + 1
    b, e = 0, seq
    if window:
        b, e = (seq - window, seq) if mode == 0 else (0, window)
    ref = oracle.attention_f32kv(q[None], nh, nkv, hd, k, v, b, e)[0]
    got = materialize(host, out, D.F32)
    assert np.abs(got - ref).max() <= 2e-5 * np.abs(v).max() + np.abs(ref).max() * 2.0 ** -23


def _contiguous_decode(host, q, k, v, nh, nkv, hd, past):
    out = np.zeros_like(q)
    run(host, abi.OpKind.ATTENTION, [D.F32, D.F32, D.F32], D.F32,
        abi.OpAttrs(n_heads=nh, n_kv_heads=nkv, head_dim=hd, past_len=past, block_size=0),
        [tref(q, D.F32), tref(k, D.F32), tref(v, D.F32)], [tmut(out, D.F32)])
    ref = oracle.attention_f32kv(q[None], nh, nkv, hd, k, v, 0, past + 1)[0]
    got = materialize(host, out, D.F32)
    assert np.abs(got - ref).max() <= 2e-5 * np.abs(v).max() + np.abs(ref).max() * 2.0 ** -23


def test_attention_contiguous_decode_follows_host_kv(host):
    """The K/V mirrors of contiguous decode are keyed by the whole tensors:
    rows appended by the host between steps are uploaded as the key range
    grows, and after a host rewrite of rows already read,
    _fellm_plugin_invalidate_f32 over the tensor makes the next launch read
    the new values (the same past_len twice, with the rewrite in between)."""
    rng = np.random.default_rng(77)
    nh, nkv, hd, cap = 8, 2, 64, 64
    q = rng.normal(size=nh * hd).astype(np.float32)
    k = np.zeros((cap, nkv * hd), np.float32)
    v = np.zeros((cap, nkv * hd), np.float32)
    for past in range(0, 12):  # decode steps: the host appends row `past`, then attends 0..past
        k[past] = rng.normal(size=nkv * hd)
        v[past] = rng.normal(size=nkv * hd)
        _contiguous_decode(host, q, k, v, nh, nkv, hd, past)
    k[:12] = rng.normal(size=(12, nkv * hd))
    v[3] = 10.0 * rng.normal(size=nkv * hd)
    host.invalidate(k.ctypes.data, k.nbytes)
    host.invalidate(v.ctypes.data + 3 * v.itemsize * nkv * hd, v.itemsize * nkv * hd)  # one row of v
    _contiguous_decode(host, q, k, v, nh, nkv, hd, 11)


@pytest.mark.parametrize("ql,mode,window", [(6, 0, 0), (6, 0, 4), (5, 1, 3)])
def test_attention_contiguous_query_rows(host, ql, mode, window):
    """Contiguous Attention with query_len > 1 rows: q and out head-major, the
    causal mask offset by kv_len - query_len (backend.rs:1385-1391 ->
    attention_provider.rs:251-385)."""
    rng = np.random.default_rng(50 + ql + mode + window)
    nh, nkv, hd, past = 8, 2, 64, 40
    q = rng.normal(size=nh * ql * hd).astype(np.float32)
    k = rng.normal(size=(48, nkv * hd)).astype(np.float32)
    v = rng.normal(size=(48, nkv * hd)).astype(np.float32)
    out = np.zeros_like(q)
    run(host, abi.OpKind.ATTENTION, [D.F32, D.F32, D.F32], D.F32,
        abi.OpAttrs(n_heads=nh, n_kv_heads=nkv, head_dim=hd, past_len=past, block_size=0, attention_window=window,
                    attention_mode=mode, query_len=ql),
        [tref(q, D.F32), tref(k, D.F32), tref(v, D.F32)], [tmut(out, D.F32)])
    ref = oracle.fa2_attention(q, k[:past + 1], v[:past + 1], nh, nkv, hd, ql, past + 1,
                               float(np.float32(1 / np.sqrt(hd))), mode == 0, window)
    got = materialize(host, out, D.F32)
    assert np.abs(got - ref).max() <= 2e-5 * np.abs(v).max() + np.abs(ref).max() * 2.0 ** -23


def test_attention_canvas(host):
    """Attention [F32 x 5] in canvas mode (attention_mode 1): query_len rows,
    each attending the prefix keys [past - window, past) of inputs 1, 2 and
    every canvas key of inputs 3, 4 (backend.rs:1412-1535)."""
    rng = np.random.default_rng(41)
    nh, nkv, hd, rows, past, window = 8, 2, 64, 12, 50, 20
    q = rng.normal(size=(rows, nh * hd)).astype(np.float32)
    pk = rng.normal(size=(past, nkv * hd)).astype(np.float32)
    pv = rng.normal(size=(past, nkv * hd)).astype(np.float32)
    ck = rng.normal(size=(rows, nkv * hd)).astype(np.float32)
    cv = rng.normal(size=(rows, nkv * hd)).astype(np.float32)
    out = np.zeros_like(q)
    attrs = abi.OpAttrs(n_heads=nh, n_kv_heads=nkv, head_dim=hd, past_len=past, attention_mode=1, query_len=rows,
                        attention_window=window)
    run(host, abi.OpKind.ATTENTION, [D.F32] * 5, D.F32, attrs,
        [tref(q, D.F32), tref(pk, D.F32), tref(pv, D.F32), tref(ck, D.F32), tref(cv, D.F32)], [tmut(out, D.F32)])
    ref = oracle.attention_f32kv(q, nh, nkv, hd, pk, pv, past - window, past, ck, cv, rows)
    got = materialize(host, out, D.F32)
    assert np.abs(got - ref).max() <= 2e-5 * max(np.abs(pv).max(), np.abs(cv).max()) + np.abs(ref).max() * 2.0 ** -23


def test_cast_converts_on_device(host):
    """Cast F32 -> BF16 (truncation) and Q4_K -> F32 (dequantization) through
    the plugin; the converted outputs are materialised with a same-dtype Cast."""
    rng = np.random.default_rng(77)
    x = rng.normal(size=1000).astype(np.float32) * np.float32(3.7)
    y = np.zeros(1000, np.uint16)
    run(host, abi.OpKind.CAST, [D.F32], D.BF16, abi.OpAttrs(cast_to=int(D.BF16)), [tref(x, D.F32)],
        [tmut(y, D.BF16)])
    assert_exact(materialize(host, y, D.BF16), oracle.f32_to_bf16_bits(x, truncate=True), "f32 -> bf16")
    w = synth.KQUANT_TABLES[12](rng, 3, 512).ravel()
    z = np.zeros(3 * 512, np.float32)
    run(host, abi.OpKind.CAST, [D.Q4K], D.F32, abi.OpAttrs(cast_to=int(D.F32)), [tref(w, D.Q4K)],
        [tmut(z, D.F32)])
    assert_exact(materialize(host, z, D.F32), oracle.dequantize_row(12, w, 3 * 512), "q4k -> f32")
