"""GPU parity of paged decode attention against the oracle
(reference_attention_paged_f32 over the same paged cache).

Tolerance (floating point, different summation order and exp):
|got - ref| <= 2e-5 * max|V| of the row's keys + one ulp of the output
dtype at |ref|.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from test_oracle_attention import build_cache

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

TORCH = {"f32": None, "f16": None, "bf16": None}


@pytest.fixture(scope="module")
def ops():
    from fellm_amd import ops as _ops

    return _ops


def tdtype(kind):
    return {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[kind]


def make_case(rng, lengths, n_heads, n_kv, hd, kv_kind):
    q = rng.normal(size=(len(lengths), n_heads * hd)).astype(np.float32)
    k = [rng.normal(size=(n, n_kv * hd)).astype(np.float32) for n in lengths]
    v = [rng.normal(size=(n, n_kv * hd)).astype(np.float32) for n in lengths]
    arena, table, n_logical, bb, k16, v16 = build_cache(rng, k, v, kind=kv_kind)
    return q, arena, table, n_logical, bb, v16


def run_gpu(ops, dev, q, q_kind, out_kind, arena, table, n_logical, bb, lengths, n_heads, n_kv, hd, kv_kind,
            window=0, scale=0.0, workspace="auto"):
    cache = ops.PagedKvCache(arena=torch.from_numpy(arena).to(dev),
                             block_table=torch.from_numpy(table.astype(np.int32)).to(dev), n_layers=1,
                             n_logical_blocks=n_logical, block_size=16, block_bytes=bb, stride=n_kv * hd,
                             kv_dtype=tdtype(kv_kind))
    qt = torch.from_numpy(q).to(dev).to(tdtype(q_kind))
    lens = torch.tensor(lengths, dtype=torch.int32, device=dev)
    kw = {}
    if workspace is None:
        kw["workspace"] = torch.empty(0, dtype=torch.float32, device=dev)
    out = ops.paged_attention(qt, lens, cache, n_heads=n_heads, n_kv_heads=n_kv, head_dim=hd,
                              max_seq=max(max(lengths), 1), scale=scale, window=window,
                              out_dtype=tdtype(out_kind), **kw)
    return out.float().cpu().numpy(), qt.float().cpu().numpy()


def check(got, ref, v16, out_kind, what):
    ulp_bits = {"f32": 23, "f16": 10, "bf16": 7}[out_kind]
    for r in range(got.shape[0]):
        vmax = float(np.abs(v16[r]).max()) if v16[r].size else 0.0
        tol = 2e-5 * vmax + np.abs(ref[r]) * 2.0 ** -ulp_bits + 1e-30
        err = np.abs(got[r] - ref[r])
        bad = err > tol
        assert not bad.any(), f"{what} row {r}: max err {err.max()} (tol {tol[bad][:3]}) got {got[r][bad][:3]} ref {ref[r][bad][:3]}"


SHAPES = [(32, 8, 128), (64, 8, 128), (32, 4, 128), (8, 1, 64), (4, 4, 128), (16, 1, 256), (32, 2, 256),
          (16, 1, 64), (64, 4, 128), (48, 4, 128)]  # the last three: 12-16 query heads per K/V head


@pytest.mark.parametrize("n_heads,n_kv,hd", SHAPES)
@pytest.mark.parametrize("kv_kind", ["f16", "bf16"])
def test_paged_attention_shapes(ops, dev, n_heads, n_kv, hd, kv_kind):
    rng = np.random.default_rng(n_heads * 1000 + hd + (kv_kind == "bf16"))
    lengths = [1, 15, 16, 17, 100, 333]
    q, arena, table, n_logical, bb, v16 = make_case(rng, lengths, n_heads, n_kv, hd, kv_kind)
    got, _ = run_gpu(ops, dev, q, "f32", "f32", arena, table, n_logical, bb, lengths, n_heads, n_kv, hd, kv_kind)
    ref = oracle.paged_attention(q, n_heads, n_kv, hd, np.array(lengths), float(np.float32(1 / np.sqrt(hd))), arena,
                                 table, n_logical, 1, 0, 16, bb, kind=kv_kind)
    check(got, ref, v16, "f32", f"{n_heads}/{n_kv}/{hd} {kv_kind}")


@pytest.mark.parametrize("q_kind,out_kind", [("f16", "f16"), ("bf16", "bf16"), ("f16", "f32"), ("bf16", "f32")])
def test_paged_attention_16bit_activations(ops, dev, q_kind, out_kind):
    rng = np.random.default_rng(7)
    n_heads, n_kv, hd = 32, 8, 128
    lengths = [5, 64, 250]
    q, arena, table, n_logical, bb, v16 = make_case(rng, lengths, n_heads, n_kv, hd, "f16")
    got, qw = run_gpu(ops, dev, q, q_kind, out_kind, arena, table, n_logical, bb, lengths, n_heads, n_kv, hd, "f16")
    ref = oracle.paged_attention(qw, n_heads, n_kv, hd, np.array(lengths), float(np.float32(1 / np.sqrt(hd))), arena,
                                 table, n_logical, 1, 0, 16, bb)
    check(got, ref, v16, out_kind, f"q {q_kind} out {out_kind}")


@pytest.mark.parametrize("window", [1, 16, 50])
def test_paged_attention_window_and_scale(ops, dev, window):
    rng = np.random.default_rng(window)
    n_heads, n_kv, hd = 16, 4, 64
    lengths = [1, 40, 200]
    q, arena, table, n_logical, bb, v16 = make_case(rng, lengths, n_heads, n_kv, hd, "f16")
    got, _ = run_gpu(ops, dev, q, "f32", "f32", arena, table, n_logical, bb, lengths, n_heads, n_kv, hd, "f16",
                     window=window, scale=0.3)
    ref = oracle.paged_attention(q, n_heads, n_kv, hd, np.array(lengths), 0.3, arena, table, n_logical, 1, 0, 16, bb,
                                 window=window)
    check(got, ref, v16, "f32", f"window {window}")


@pytest.mark.parametrize("workspace", ["auto", None])
def test_paged_attention_long_single_row_splits(ops, dev, workspace):
    """One row of 3000 keys: with a workspace the keys are split across
    wavefronts and combined; without one a single wavefront walks them."""
    rng = np.random.default_rng(11)
    n_heads, n_kv, hd = 32, 8, 128
    lengths = [3000]
    q, arena, table, n_logical, bb, v16 = make_case(rng, lengths, n_heads, n_kv, hd, "f16")
    got, _ = run_gpu(ops, dev, q, "f32", "f32", arena, table, n_logical, bb, lengths, n_heads, n_kv, hd, "f16",
                     workspace=workspace)
    ref = oracle.paged_attention(q, n_heads, n_kv, hd, np.array(lengths), float(np.float32(1 / np.sqrt(hd))), arena,
                                 table, n_logical, 1, 0, 16, bb)
    check(got, ref, v16, "f32", f"split workspace={workspace}")


def test_paged_attention_empty_rows_and_zero_batch(ops, dev):
    rng = np.random.default_rng(2)
    n_heads, n_kv, hd = 8, 2, 128
    lengths = [0, 20, 0]
    q, arena, table, n_logical, bb, v16 = make_case(rng, lengths, n_heads, n_kv, hd, "f16")
    got, _ = run_gpu(ops, dev, q, "f32", "f32", arena, table, n_logical, bb, lengths, n_heads, n_kv, hd, "f16")
    assert np.all(got[0] == 0.0) and np.all(got[2] == 0.0)
    ref = oracle.paged_attention(q, n_heads, n_kv, hd, np.array(lengths), float(np.float32(1 / np.sqrt(hd))), arena,
                                 table, n_logical, 1, 0, 16, bb)
    check(got, ref, v16, "f32", "empty rows")


# ---- non-paged attention: f32 K/V rows (contiguous decode, canvas) -----------------
def _f32kv(ops, q, n_heads, n_kv, hd, k1, v1, b1, e1, k2=None, v2=None, n2=0, scale=0.0):
    from fellm_amd import _lib

    dev = torch.device("cuda:0")
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev) if a is not None else None
    qd, k1d, v1d, k2d, v2d = t(q), t(k1), t(v1), t(k2), t(v2)
    out = torch.full_like(qd, float("nan"))
    p = lambda x: x.data_ptr() if x is not None else None
    rc = _lib.lib().fellm_rocm_attention_f32kv(p(qd), p(out), q.shape[0], n_heads, n_kv, hd, p(k1d), p(v1d), b1, e1,
                                               p(k2d), p(v2d), n2, scale, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, rc
    return out.cpu().numpy()


@pytest.mark.parametrize("n_heads,n_kv,hd,seq,b1", [(32, 8, 128, 4096, 0), (8, 2, 64, 37, 0), (32, 8, 128, 300, 44),
                                                    (16, 1, 128, 129, 0), (4, 4, 80, 5, 0), (8, 1, 256, 1000, 10),
                                                    (2, 2, 96, 64, 0), (12, 4, 64, 1, 0)])
def test_attention_f32kv_decode(ops, n_heads, n_kv, hd, seq, b1):
    rng = np.random.default_rng(seq * 7 + hd)
    q = rng.normal(size=(1, n_heads * hd)).astype(np.float32)
    k = rng.normal(size=(seq, n_kv * hd)).astype(np.float32)
    v = rng.normal(size=(seq, n_kv * hd)).astype(np.float32)
    got = _f32kv(ops, q, n_heads, n_kv, hd, k, v, b1, seq)
    ref = oracle.attention_f32kv(q, n_heads, n_kv, hd, k, v, b1, seq)
    assert np.abs(got - ref).max() <= 2e-5 * np.abs(v).max() + np.abs(ref).max() * 2.0 ** -23


@pytest.mark.parametrize("rows,past", [(4, 100), (1, 0), (17, 3), (32, 513)])
def test_attention_f32kv_canvas(ops, rows, past):
    rng = np.random.default_rng(rows * 100 + past)
    nh, nkv, hd = 16, 4, 128
    q = rng.normal(size=(rows, nh * hd)).astype(np.float32)
    pk = rng.normal(size=(max(past, 1), nkv * hd)).astype(np.float32)
    pv = rng.normal(size=(max(past, 1), nkv * hd)).astype(np.float32)
    ck = rng.normal(size=(rows, nkv * hd)).astype(np.float32)
    cv = rng.normal(size=(rows, nkv * hd)).astype(np.float32)
    got = _f32kv(ops, q, nh, nkv, hd, pk, pv, 0, past, ck, cv, rows, 0.07)
    ref = oracle.attention_f32kv(q, nh, nkv, hd, pk, pv, 0, past, ck, cv, rows, 0.07)
    assert np.abs(got - ref).max() <= 2e-5 * max(np.abs(pv).max(), np.abs(cv).max()) + np.abs(ref).max() * 2.0 ** -23


def test_attention_f32kv_empty_and_errors(ops):
    from fellm_amd import _lib

    rng = np.random.default_rng(5)
    q = rng.normal(size=(2, 4 * 64)).astype(np.float32)
    k = rng.normal(size=(8, 2 * 64)).astype(np.float32)
    assert not _f32kv(ops, q, 4, 2, 64, k, k, 3, 3).any()  # no keys: zero rows
    lib = _lib.lib()
    x = torch.zeros(4096, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    assert lib.fellm_rocm_attention_f32kv(x.data_ptr(), x.data_ptr(), 1, 4, 3, 64, x.data_ptr(), x.data_ptr(), 0, 1,
                                          None, None, 0, 0.0, s) == -2  # heads not a multiple of KV heads
    assert lib.fellm_rocm_attention_f32kv(x.data_ptr(), x.data_ptr(), 1, 32, 1, 128, x.data_ptr(), x.data_ptr(), 0,
                                          1, None, None, 0, 0.0, s) == -2  # 32 heads per KV head


@pytest.mark.parametrize("ql,kvl,causal,window", [(1, 37, True, 0), (5, 37, True, 0), (16, 16, True, 0),
                                                  (20, 300, True, 8), (7, 33, False, 0), (9, 40, False, 5),
                                                  (33, 33, True, 1), (64, 1000, True, 0), (3, 2, False, 4)])
def test_attention_f32kv_rows(ops, ql, kvl, causal, window):
    """query_len rows over contiguous f32 K/V (the CPU backend's host FA2 path,
    attention_provider.rs:251-385): head-major q and out, the causal bound
    kv_len - query_len + row and its window, or the non-causal row window;
    against the oracle's restatement of that path."""
    from fellm_amd import _lib

    rng = np.random.default_rng(ql * 1000 + kvl + window)
    nh, nkv, hd = 16, 4, 128
    q = rng.normal(size=nh * ql * hd).astype(np.float32)
    k = rng.normal(size=(kvl, nkv * hd)).astype(np.float32)
    v = rng.normal(size=(kvl, nkv * hd)).astype(np.float32)
    scale = float(np.float32(1 / np.sqrt(hd)))
    dev = torch.device("cuda:0")
    qd, kd, vd = (torch.from_numpy(a).to(dev) for a in (q, k, v))
    out = torch.full_like(qd, float("nan"))
    rc = _lib.lib().fellm_rocm_attention_f32kv_rows(qd.data_ptr(), out.data_ptr(), ql, nh, nkv, hd, kd.data_ptr(),
                                                    vd.data_ptr(), kvl, 0.0, int(causal), window,
                                                    torch.cuda.current_stream().cuda_stream)
    assert rc == 0, rc
    got = out.cpu().numpy()
    ref = oracle.fa2_attention(q, k, v, nh, nkv, hd, ql, kvl, scale, causal, window)
    assert np.abs(got - ref).max() <= 2e-5 * np.abs(v).max() + np.abs(ref).max() * 2.0 ** -23


def test_attention_f32kv_rows_rejects_more_rows_than_keys(ops):
    from fellm_amd import _lib

    x = torch.zeros(4096, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    assert _lib.lib().fellm_rocm_attention_f32kv_rows(x.data_ptr(), x.data_ptr(), 4, 4, 2, 64, x.data_ptr(),
                                                      x.data_ptr(), 3, 0.0, 1, 0, s) == -2
