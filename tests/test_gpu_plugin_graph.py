"""Graph capture and replay through the plugin ABI, with the device-resident
step block (`_fellm_plugin_update_step_params`, c_abi.rs:196-198;
fellm-plugin-host loader.rs:212-224).

Restates the reference's live check crates/backend-cuda/examples/
graph_smoke.rs: an Add captured and replayed; a single-row RoPE captured at
one position and replayed after the step block moves to another.  Then a
single-sequence decode step (embedding at token_id, RoPE + paged K/V append,
paged attention) captured once and replayed for 40 tokens, every replay bit
for bit equal to the eager launches of the same step.

Once a step block has been uploaded, the plugin's single-row decode launches
read it for the rest of the process (as the CUDA plugin's do), so this file
runs after the other plugin tests (pytest collects it after
test_gpu_plugin.py).
"""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import oracle  # noqa: E402
from fellm_amd import abi  # noqa: E402
from fellm_amd.plugin_host import PagedKvContext, PluginError, PluginHost  # noqa: E402
from parity_util import assert_exact  # noqa: E402

pytestmark = pytest.mark.gpu
D = abi.DType
_KEEP = []


@pytest.fixture(scope="module")
def host():
    torch.cuda.init()
    h = PluginHost()
    yield h
    h.set_paged_context(None)


def tref(a, dt, dims=None):
    _KEEP.append(a)
    return abi.tensor_ref(a.ctypes.data, a.nbytes, dt, dims or [a.size], 0)


def tmut(a, dt, dims=None):
    _KEEP.append(a)
    return abi.tensor_mut(a.ctypes.data, a.nbytes, dt, dims or [a.size])


def handle(host, op, ins_dt, out_dt):
    h = host.lookup(op, ins_dt, out_dt)
    assert h is not None, (op, ins_dt, out_dt)
    return h


def materialize(host, buf, dt):
    out = np.empty_like(buf)
    host.launch(handle(host, abi.OpKind.CAST, [dt], dt), abi.OpAttrs(), [tref(buf, dt)], [tmut(out, dt)])
    return out


def sync(host):
    host.stream().synchronize()


def test_graph_smoke_add_and_controlled_rope(host):
    """crates/backend-cuda/examples/graph_smoke.rs, restated."""
    add = handle(host, abi.OpKind.ADD, [D.F32, D.F32], D.F32)
    lhs = np.array([1, 2, 3, 4], np.float32)
    rhs = np.array([10, 20, 30, 40], np.float32)
    out = np.zeros(4, np.float32)
    ins = [tref(lhs, D.F32), tref(rhs, D.F32)]
    host.launch(add, abi.OpAttrs(), ins, [tmut(out, D.F32)])  # warm-up: resident inputs and output
    sync(host)
    cap = host.begin_graph_capture()
    host.launch(add, abi.OpAttrs(), ins, [tmut(out, D.F32)])
    g = cap.finish()
    for _ in range(3):
        g.launch(host.stream())
        sync(host)
        assert materialize(host, out, D.F32).tolist() == [11, 22, 33, 44]
    g.close()

    rope = handle(host, abi.OpKind.ROPE, [D.F32, D.F32], D.F32)
    x = np.array([1, 0, 1, 0], np.float32)
    inv = np.array([1.0, 0.1], np.float32)
    y = np.zeros(4, np.float32)
    attrs = abi.OpAttrs(n_heads=1, head_dim=4, rope_dim=4, position=999)
    rins = [tref(x, D.F32), tref(inv, D.F32)]
    host.update_step_params(abi.DeviceStepParams(position=1))
    host.launch(rope, attrs, rins, [tmut(y, D.F32)])
    sync(host)
    got1 = materialize(host, y, D.F32)
    assert_exact(got1, oracle.rope(x, 1, 4, 4, 0, inv, np.array([1], np.uint32)), "eager rope at the step position")
    cap = host.begin_graph_capture()
    host.launch(rope, attrs, rins, [tmut(y, D.F32)])
    g = cap.finish()
    for pos in (2, 7, 2, 31000):
        host.update_step_params(abi.DeviceStepParams(position=pos))
        g.launch(host.stream())
        sync(host)
        got = materialize(host, y, D.F32)
        ref = oracle.rope(x, 1, 4, 4, 0, inv, np.array([pos], np.uint32))
        assert_exact(got, ref, f"replay at position {pos}")
    exp2 = np.array([np.cos(2.0), np.sin(2.0), np.cos(0.2), np.sin(0.2)], np.float32)
    host.update_step_params(abi.DeviceStepParams(position=2))
    g.launch(host.stream())
    sync(host)
    assert np.abs(materialize(host, y, D.F32) - exp2).max() < 1e-5  # graph_smoke.rs's own check
    g.close()


def test_capture_refuses_uploads(host):
    """A launch whose input is not resident cannot be recorded (the upload
    would replay stale host memory): it fails with -4 and enqueues nothing;
    the capture is then abandoned and the stream works eagerly again."""
    add = handle(host, abi.OpKind.ADD, [D.F32, D.F32], D.F32)
    a = np.arange(64, dtype=np.float32)
    b = np.ones(64, np.float32)
    out = np.zeros(64, np.float32)
    cap = host.begin_graph_capture()
    try:
        with pytest.raises(PluginError) as e:
            host.launch(add, abi.OpAttrs(), [tref(a, D.F32), tref(b, D.F32)], [tmut(out, D.F32)])
        assert e.value.code == abi.ERR_LAUNCH
    finally:
        cap.abort()
    host.launch(add, abi.OpAttrs(), [tref(a, D.F32), tref(b, D.F32)], [tmut(out, D.F32)])
    assert np.array_equal(materialize(host, out, D.F32), a + 1)


def test_decode_step_replay_through_plugin(host):
    """Embedding (token_id) -> rope_kv_write (position, kv slot) -> paged
    attention (sequence_length) for one sequence, all reading the step block;
    the block table is device-resident (the snapshot's device table).  Eager
    launches over 40 tokens, then the arena is cleared and one captured step
    is replayed 40 times: outputs and the arena match the eager run bit for
    bit, and the last output matches the oracle."""
    rng = np.random.default_rng(17)
    nq, nkv, hd, vocab, bs, n_logical = 8, 2, 64, 61, 16, 64
    stride = nkv * hd
    bb = (2 * bs * stride * 2 + 63) // 64 * 64
    tq = rng.normal(size=(vocab, nq * hd)).astype(np.float32)
    tk = rng.normal(size=(vocab, stride)).astype(np.float32)
    tv = rng.normal(size=(vocab, stride)).astype(np.float32)
    inv = oracle.rope_inv_freqs(10000.0, hd)
    table = rng.permutation(n_logical).astype(np.uint32)
    arena = torch.zeros(n_logical * bb, dtype=torch.uint8, device="cuda")
    table_dev = torch.from_numpy(table.view(np.int32)).to("cuda")
    host_arena = np.zeros(8, np.uint8)
    zero = np.zeros(1, np.uint32)
    ctx = PagedKvContext(arena_ptr=host_arena.ctypes.data, arena_len=host_arena.size, block_table=table,
                         n_logical_blocks=n_logical, n_layers=1, tokens_stride=stride, block_bytes=bb,
                         block_size=bs, row_positions=zero, row_rope_positions=zero, row_lengths=zero + 1,
                         device_arena_ptr=arena.data_ptr(), device_arena_len=arena.numel(),
                         device_block_table_ptr=table_dev.data_ptr(), n_device_block_table=table.size,
                         device_logical_stride=n_logical)
    _KEEP.extend([host_arena, table_dev, arena])
    tokens = rng.integers(0, vocab, size=40)
    ids = np.zeros(1, np.uint32)
    q = np.zeros(nq * hd, np.float32)
    k = np.zeros(stride, np.float32)
    v = np.zeros(stride, np.float32)
    qo = np.zeros(nq * hd, np.float32)
    att = np.zeros(nq * hd, np.float32)
    dummy = np.zeros(1, np.float32)
    emb = handle(host, abi.OpKind.EMBEDDING, [D.F32, D.U32], D.F32)
    rkv = handle(host, abi.OP_ROPE_KV_WRITE, [D.F32, D.F32, D.F32, D.F32], D.F32)
    attn = handle(host, abi.OpKind.ATTENTION, [D.F32, D.F32, D.F32], D.F32)
    rkv_attrs = abi.OpAttrs(n_heads=nq, n_kv_heads=nkv, head_dim=hd, rope_dim=hd, rope_pairing=0, layer_ord=0,
                            block_size=bs)
    att_attrs = abi.OpAttrs(n_heads=nq, n_kv_heads=nkv, head_dim=hd, block_size=bs, attention_mode=0, past_len=0)

    def launch_step():
        for table_np, out_np, d in ((tq, q, nq * hd), (tk, k, stride), (tv, v, stride)):
            host.launch(emb, abi.OpAttrs(), [tref(table_np, D.F32, [vocab, d]), tref(ids, D.U32)],
                        [tmut(out_np, D.F32)])
        host.launch(rkv, rkv_attrs, [tref(q, D.F32), tref(k, D.F32), tref(v, D.F32), tref(inv, D.F32)],
                    [tmut(qo, D.F32)])
        host.launch(attn, att_attrs, [tref(qo, D.F32), tref(dummy, D.F32), tref(dummy, D.F32)],
                    [tmut(att, D.F32)])

    def params(s):
        return abi.DeviceStepParams(token_id=int(tokens[s]), position=s, sequence_length=s + 1, active_batch=1,
                                    kv_write_slot=s % bs)

    host.set_paged_context(ctx)
    try:
        eager = []
        for s in range(40):
            host.update_step_params(params(s))
            launch_step()
            eager.append(materialize(host, att, D.F32))
        sync(host)
        eager_arena = arena.cpu()
        arena.zero_()
        torch.cuda.synchronize()
        host.update_step_params(params(0))
        cap = host.begin_graph_capture()
        try:
            launch_step()
        except Exception:
            cap.abort()
            raise
        g = cap.finish()
        for s in range(40):
            host.update_step_params(params(s))
            g.launch(host.stream())
            sync(host)
            got = materialize(host, att, D.F32)
            assert np.array_equal(got.view(np.uint32), eager[s].view(np.uint32)), f"replay {s}"
        g.close()
        sync(host)
        assert torch.equal(arena.cpu(), eager_arena)
        q_last = materialize(host, qo, D.F32)
    finally:
        host.set_paged_context(None)
    ref = oracle.paged_attention(q_last.reshape(1, -1), nq, nkv, hd, np.array([40]),
                                 float(np.float32(1 / np.sqrt(hd))), eager_arena.numpy(), table, n_logical, 1, 0, bs,
                                 bb)
    assert np.abs(eager[-1] - ref[0]).max() <= 2e-5 * 5.0 + np.abs(ref).max() * 2.0 ** -23
