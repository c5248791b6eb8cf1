"""GPU parity for the Q5_K and Q8_0 embedding gathers (the CUDA plugin's
Embedding [Q5K, U32] and [Q8_0, U32] keys, plugins/cuda_kernels/src/lib.rs:637-661;
dequant.rs:59-107 and :172-192) through the device-pointer C ABI: plain
gathers, the fused gather + RMSNorm, long rows split into segments, tables at
the minimum alignment, and Cast to f32.  Gathered rows are bit-exact against
the oracle; the normalised rows are held to the RMSNorm tolerance.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from parity_util import KINDS, assert_close, assert_exact, from_dev

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

Q8_0, Q5K = 8, 13


@pytest.fixture(scope="module")
def ops():
    from fellm_amd import ops as _ops

    return _ops


def _table(qtype, rng, vocab, dim):
    from fellm_amd import synth

    return synth.q5k_table(rng, vocab, dim) if qtype == "q5k" else synth.q8_0_table(rng, vocab, dim)


def _code(qtype):
    return Q5K if qtype == "q5k" else Q8_0


def _ids_with_bad(rng, n, vocab, n_bad):
    from fellm_amd import synth

    ids = synth.zipf_ids(rng, n, vocab)
    if n_bad:
        bad = rng.choice(n, size=n_bad, replace=False)
        ids[bad] = vocab + np.arange(n_bad, dtype=np.uint32) * 7
    return ids


def _ref_rows(table, code, vocab, dim, ids):
    ok = ids < vocab
    e = np.zeros((ids.size, dim), np.float32)
    if ok.any():
        e[ok] = oracle.embedding(table, code, vocab, dim, ids[ok])
    return e


@pytest.mark.parametrize("qtype", ["q5k", "q8_0"])
@pytest.mark.parametrize("out_kind", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("dim", [256, 1280, 3584, 4096])
def test_embedding_q5k_q8_0(ops, dev, qtype, out_kind, dim):
    rng = np.random.default_rng(dim + len(qtype) + len(out_kind))
    vocab = 300
    table = _table(qtype, rng, vocab, dim)
    ids = _ids_with_bad(rng, 517, vocab, 3)
    ref = oracle.narrow(_ref_rows(table, _code(qtype), vocab, dim, ids), out_kind)
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    got = ops.embedding(torch.from_numpy(table).to(dev), torch.from_numpy(ids.view(np.int32)).to(dev), dim=dim,
                        qtype=qtype, out_dtype=KINDS[out_kind], err_flag=flag)
    assert int(flag.item()) == 1
    assert_exact(from_dev(got), ref, f"embedding {qtype} dim={dim} -> {out_kind}")


@pytest.mark.parametrize("dim", [32, 96, 4128, 7200])
def test_embedding_q8_0_dims_not_multiple_of_256(ops, dev, dim):
    """Q8_0 rows need only dim % 32 == 0 (34-byte blocks of 32)."""
    rng = np.random.default_rng(dim)
    vocab = 150
    table = _table("q8_0", rng, vocab, dim)
    ids = _ids_with_bad(rng, 301, vocab, 0)
    ref = oracle.narrow(_ref_rows(table, Q8_0, vocab, dim, ids), "f16")
    got = ops.embedding(torch.from_numpy(table).to(dev), torch.from_numpy(ids.view(np.int32)).to(dev), dim=dim,
                        qtype="q8_0", out_dtype=torch.float16)
    assert_exact(from_dev(got), ref, f"embedding q8_0 dim={dim}")


@pytest.mark.parametrize("qtype", ["q5k", "q8_0"])
@pytest.mark.parametrize("dim", [16384, 32768])
def test_embedding_long_rows_split_into_segments(ops, dev, qtype, dim):
    """Rows longer than one workgroup's LDS copy are gathered as segments of
    blocks, one workgroup each (dim 32768 does not fit one 64-thread copy)."""
    rng = np.random.default_rng(dim + len(qtype))
    vocab = 40
    table = _table(qtype, rng, vocab, dim)
    ids = _ids_with_bad(rng, 67, vocab, 2)
    ref = oracle.narrow(_ref_rows(table, _code(qtype), vocab, dim, ids), "f32")
    got = ops.embedding(torch.from_numpy(table).to(dev), torch.from_numpy(ids.view(np.int32)).to(dev), dim=dim,
                        qtype=qtype, out_dtype=torch.float32)
    assert_exact(from_dev(got), ref, f"embedding {qtype} long rows dim={dim}")


@pytest.mark.parametrize("qtype,offset", [("q5k", 4), ("q5k", 12), ("q8_0", 2), ("q8_0", 6), ("q8_0", 14)])
@pytest.mark.parametrize("dim", [256, 3584])
def test_embedding_unaligned_table(ops, dev, qtype, offset, dim):
    """Q5_K tables need 4-byte alignment, Q8_0 tables 2-byte alignment: a table
    starting `offset` bytes past a 16-byte boundary shifts every row's span
    against the 16-byte loads that copy it."""
    rng = np.random.default_rng(offset * 1000 + dim)
    vocab = 97
    table = _table(qtype, rng, vocab, dim)
    ids = _ids_with_bad(rng, 300, vocab, 0)
    ref = oracle.narrow(_ref_rows(table, _code(qtype), vocab, dim, ids), "f16")
    buf = torch.zeros(table.size + 16, dtype=torch.uint8, device=dev)
    buf[offset:offset + table.size] = torch.from_numpy(table.reshape(-1)).to(dev)
    got = ops.embedding(buf[offset:offset + table.size].view(table.shape),
                        torch.from_numpy(ids.view(np.int32)).to(dev), dim=dim, qtype=qtype, out_dtype=torch.float16)
    assert_exact(from_dev(got), ref, f"embedding {qtype} table offset {offset} dim={dim}")


@pytest.mark.parametrize("qtype", ["q5k", "q8_0"])
@pytest.mark.parametrize("dim,store_h", [(256, True), (3584, False), (4096, True), (8192, True), (16384, False)])
def test_embedding_rmsnorm_q5k_q8_0(ops, dev, qtype, dim, store_h):
    """Fused gather + RMSNorm: rows of up to 4096 elements in 64-thread
    workgroups, longer ones in 256-thread workgroups; out-of-range ids give
    zero rows and set the flag.  h bit-exact, y within the RMSNorm tolerance."""
    rng = np.random.default_rng(dim + store_h + len(qtype))
    vocab, n_rows = 200, 1031 if dim <= 4096 else 130
    table = _table(qtype, rng, vocab, dim)
    ids = _ids_with_bad(rng, n_rows, vocab, 3)
    e = _ref_rows(table, _code(qtype), vocab, dim, ids)
    w = rng.normal(1.0, 0.1, size=dim).astype(np.float32)
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    h, y = ops.embedding_rmsnorm(torch.from_numpy(table).to(dev), torch.from_numpy(ids.view(np.int32)).to(dev),
                                 torch.from_numpy(w).to(dev), 1e-6, dim=dim, qtype=qtype, out_dtype=torch.float16,
                                 store_h=store_h, err_flag=flag)
    assert int(flag.item()) == 1
    if store_h:
        assert_exact(from_dev(h), oracle.narrow(e, "f16"), f"{qtype} fused h dim {dim}")
    assert_close(from_dev(y), oracle.narrow(oracle.rmsnorm(e, w, 1e-6), "f16"), "f16",
                 what=f"{qtype} fused y dim {dim}")


@pytest.mark.parametrize("qtype,n", [("q5k", 256), ("q5k", 37 * 256), ("q8_0", 32), ("q8_0", 96), ("q8_0", 129 * 32)])
def test_cast_q5k_q8_0_to_f32(ops, dev, qtype, n):
    """Cast of the block stream to f32 (backend.rs:1657-1661 dequantizes through dequantize_row)."""
    from fellm_amd import _lib

    rng = np.random.default_rng(n)
    blk = 256 if qtype == "q5k" else 32
    src = _table(qtype, rng, n // blk, blk).ravel()
    s = torch.from_numpy(src).to(dev)
    out = torch.empty(n, dtype=torch.float32, device=dev)
    _lib.call("fellm_rocm_cast", s.data_ptr(), _code(qtype), out.data_ptr(), 0, n,
              torch.cuda.current_stream().cuda_stream)
    ref = oracle.dequantize_row(_code(qtype), src, n)
    assert_exact(from_dev(out), ref, f"cast {qtype} -> f32 n={n}")


def test_reject_misaligned_shapes(ops, dev):
    """Q5_K needs dim % 256 == 0 and a 4-byte-aligned table; Q8_0 dim % 32 == 0."""
    from fellm_amd import _lib

    ids = torch.zeros(4, dtype=torch.int32, device=dev)
    out = torch.empty(4 * 512, dtype=torch.float32, device=dev)
    t = torch.zeros(4096, dtype=torch.uint8, device=dev)
    lib = _lib.lib()
    st = torch.cuda.current_stream().cuda_stream
    assert lib.fellm_rocm_embedding(t.data_ptr(), Q5K, 4, 300, ids.data_ptr(), 4, out.data_ptr(), 0, None, st) == -2
    assert lib.fellm_rocm_embedding(t.data_ptr() + 2, Q5K, 4, 256, ids.data_ptr(), 4, out.data_ptr(), 0, None,
                                    st) == -2
    assert lib.fellm_rocm_embedding(t.data_ptr(), Q8_0, 4, 48, ids.data_ptr(), 4, out.data_ptr(), 0, None, st) == -2
    assert lib.fellm_rocm_embedding(t.data_ptr() + 1, Q8_0, 4, 64, ids.data_ptr(), 4, out.data_ptr(), 0, None,
                                    st) == -2
