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


SHAPES = [(32, 8, 128), (64, 8, 128), (32, 4, 128), (8, 1, 64), (4, 4, 128), (16, 1, 256), (32, 2, 256)]


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
