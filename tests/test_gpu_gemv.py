"""GPU parity of the K-quant GEMV and the fused gate/up SwiGLU GEMV.

Both are bit-exact against the oracle (oracle/fellm_oracle.c: Q8_K
quantization of x as quantize_row_q8_k_avx2, block dots as the CPU's portable
path, serial f32 row sums, glibc-exact silu): integer parts are exact by
construction and the f32 combine follows the same operation order.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from fellm_amd import synth
from parity_util import assert_exact

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

NAMES = {12: "q4k", 13: "q5k", 14: "q6k"}


@pytest.fixture(scope="module")
def ops():
    from fellm_amd import ops as _ops

    return _ops


def weights(rng, dtype, rows, cols):
    return synth.KQUANT_TABLES[dtype](rng, rows, cols)


def to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("gt", [12, 13, 14])
@pytest.mark.parametrize("ut", [12, 13, 14])
def test_gate_up_swiglu_pairs(ops, dev, gt, ut):
    rng = np.random.default_rng(gt * 100 + ut)
    rows, cols = 300, 4096
    g, u = weights(rng, gt, rows, cols), weights(rng, ut, rows, cols)
    x = rng.normal(size=cols).astype(np.float32)
    ref = oracle.gate_up_swiglu(gt, g, ut, u, rows, cols, x)
    got = ops.gate_up_swiglu(to_dev(g, dev), to_dev(u, dev), to_dev(x, dev), qtype=NAMES[gt],
                             up_qtype=NAMES[ut]).cpu().numpy()
    assert_exact(got, ref, f"gate_up_swiglu {NAMES[gt]}/{NAMES[ut]}")


# nb = cols/256 blocks per row: 1, 14 (partial pass), 16, 17, 32 (two passes), 65 (ragged third pass)
@pytest.mark.parametrize("dtype", [12, 13, 14])
@pytest.mark.parametrize("cols", [256, 3584, 4096, 4352, 8192, 16640])
def test_matvec_kquant_shapes(ops, dev, dtype, cols):
    rng = np.random.default_rng(dtype * 7 + cols)
    rows = 129
    w = weights(rng, dtype, rows, cols)
    x = (rng.normal(size=cols) * rng.uniform(0.01, 20.0, size=cols)).astype(np.float32)
    ref = oracle.matvec_kquant(dtype, w, rows, cols, x)
    got = ops.matvec_kquant(to_dev(w, dev), to_dev(x, dev), qtype=NAMES[dtype]).cpu().numpy()
    assert_exact(got, ref, f"matvec {NAMES[dtype]} cols={cols}")


@pytest.mark.parametrize("gt,ut", [(12, 12), (13, 13), (14, 14), (14, 12)])
@pytest.mark.parametrize("cols", [16640, 49152])
def test_gate_up_swiglu_long_rows(ops, dev, gt, ut, cols):
    """Multi-pass rows (more than 32 blocks) of the fused GEMV up to the
    longest accepted row: 8-wavefront workgroups where their LDS stages fit,
    4 where they do not (fused Q5_K / Q6_K at 49152 columns)."""
    rng = np.random.default_rng(gt * 1000 + ut * 10 + cols)
    rows = 37
    g, u = weights(rng, gt, rows, cols), weights(rng, ut, rows, cols)
    x = rng.normal(size=cols).astype(np.float32)
    ref = oracle.gate_up_swiglu(gt, g, ut, u, rows, cols, x)
    got = ops.gate_up_swiglu(to_dev(g, dev), to_dev(u, dev), to_dev(x, dev), qtype=NAMES[gt],
                             up_qtype=NAMES[ut]).cpu().numpy()
    assert_exact(got, ref, f"gate_up_swiglu {NAMES[gt]}/{NAMES[ut]} cols={cols}")


@pytest.mark.parametrize("dtype", [12, 13, 14])
def test_matvec_kquant_longest_rows(ops, dev, dtype):
    """The plain GEMV at the longest accepted row (192 blocks, six passes)."""
    rng = np.random.default_rng(dtype + 49152)
    rows, cols = 41, 49152
    w = weights(rng, dtype, rows, cols)
    x = (rng.normal(size=cols) * rng.uniform(0.01, 20.0, size=cols)).astype(np.float32)
    ref = oracle.matvec_kquant(dtype, w, rows, cols, x)
    got = ops.matvec_kquant(to_dev(w, dev), to_dev(x, dev), qtype=NAMES[dtype]).cpu().numpy()
    assert_exact(got, ref, f"matvec {NAMES[dtype]} cols={cols}")


@pytest.mark.parametrize("dtype", [12, 13, 14])
def test_matvec_q8k_edges(ops, dev, dtype):
    """Zero blocks, round-half-even ties (amax 127 makes iscale 1), a block
    whose amax is a denormal, and huge magnitudes."""
    rng = np.random.default_rng(99 + dtype)
    cols, rows = 2048, 70
    x = rng.normal(size=cols).astype(np.float32)
    x[0:256] = 0.0
    x[256:512] = rng.integers(-127, 128, size=256).astype(np.float32) + np.float32(0.5)
    x[256] = 127.0
    x[512:768] = np.float32(1e-40) * rng.integers(-3, 4, size=256)
    x[768] = np.float32(3e-40)
    x[1024:1280] *= np.float32(1e30)
    w = weights(rng, dtype, rows, cols)
    ref = oracle.matvec_kquant(dtype, w, rows, cols, x)
    got = ops.matvec_kquant(to_dev(w, dev), to_dev(x, dev), qtype=NAMES[dtype]).cpu().numpy()
    assert_exact(got, ref, f"matvec edges {NAMES[dtype]}")


@pytest.mark.parametrize("dtype", [12, 14])
def test_gate_up_swiglu_llama3_8b_decode(ops, dev, dtype):
    """Llama-3-8B FFN shape: 14336 rows, 4096 columns."""
    rng = np.random.default_rng(8000 + dtype)
    rows, cols = 14336, 4096
    g, u = weights(rng, dtype, rows, cols), weights(rng, dtype, rows, cols)
    x = rng.normal(size=cols).astype(np.float32)
    ref = oracle.gate_up_swiglu(dtype, g, dtype, u, rows, cols, x)
    got = ops.gate_up_swiglu(to_dev(g, dev), to_dev(u, dev), to_dev(x, dev), qtype=NAMES[dtype]).cpu().numpy()
    assert_exact(got, ref, f"gate_up 8B {NAMES[dtype]}")


def test_gate_up_zero_x_and_empty(ops, dev):
    rng = np.random.default_rng(5)
    rows, cols = 64, 1024
    g, u = weights(rng, 12, rows, cols), weights(rng, 12, rows, cols)
    got = ops.gate_up_swiglu(to_dev(g, dev), to_dev(u, dev), torch.zeros(cols, device=dev)).cpu().numpy()
    assert np.all(got == 0.0)
    empty = torch.empty((0, cols // 256 * 144), dtype=torch.uint8, device=dev)
    out = ops.gate_up_swiglu(empty, empty, torch.zeros(cols, device=dev))
    assert out.numel() == 0


def test_gemv_rejects_bad_shapes(ops, dev):
    from fellm_amd._lib import FellmRocmError

    w = torch.zeros((4, 144), dtype=torch.uint8, device=dev)
    with pytest.raises(ValueError):
        ops.matvec_kquant(w, torch.zeros(200, device=dev))  # cols % 256 != 0
    with pytest.raises(FellmRocmError):
        ops.matvec_kquant(torch.zeros((4, 2 * 144), dtype=torch.uint8, device=dev),
                          torch.zeros(513, device=dev)[1:])  # x not 16-byte aligned


# ---- x quantized once: fellm_rocm_quantize_q8k + the _q8k GEMVs ------------------


def split_blob(blob: np.ndarray, cols: int):
    nb = cols // 256
    qs = blob[: nb * 256].view(np.int8)
    bs = blob[nb * 256: nb * 288].view(np.int16)
    d = blob[nb * 288: nb * 292].view(np.float32)
    return qs, bs, d


@pytest.mark.parametrize("cols", [256, 4096, 14336, 49152])
def test_quantize_q8k_blob(ops, dev, cols):
    """The blob equals the oracle's Q8_K quantization (qs, bsums, d), with
    the edge blocks of test_matvec_q8k_edges in it."""
    rng = np.random.default_rng(cols)
    x = (rng.normal(size=cols) * rng.uniform(0.01, 20.0, size=cols)).astype(np.float32)
    if cols >= 1024:
        x[0:256] = 0.0
        x[256:512] = rng.integers(-127, 128, size=256).astype(np.float32) + np.float32(0.5)
        x[256] = 127.0
        x[512:768] = np.float32(1e-40) * rng.integers(-3, 4, size=256)
    blob = ops.quantize_q8k(to_dev(x, dev)).cpu().numpy()
    assert blob.size == cols // 256 * 292
    qs, bs, d = split_blob(blob, cols)
    rq, rb, rd = oracle.quantize_q8k(x)
    assert np.array_equal(qs, rq) and np.array_equal(bs, rb) and np.array_equal(d.view(np.uint32), rd.view(np.uint32))


@pytest.mark.parametrize("dtype", [12, 13, 14])
@pytest.mark.parametrize("cols", [256, 3584, 4096, 4352, 8192, 14336, 16640])
def test_matvec_kquant_q8k_matches(ops, dev, dtype, cols):
    """Same bits as matvec_kquant (and the oracle), including two- and
    three-pass rows and the Q6_K rows finished by the direct kernel."""
    rng = np.random.default_rng(dtype * 11 + cols)
    rows = 131
    w = weights(rng, dtype, rows, cols)
    x = (rng.normal(size=cols) * rng.uniform(0.01, 20.0, size=cols)).astype(np.float32)
    wd, xd = to_dev(w, dev), to_dev(x, dev)
    got = ops.matvec_kquant_q8k(wd, ops.quantize_q8k(xd), qtype=NAMES[dtype]).cpu().numpy()
    assert_exact(got, ops.matvec_kquant(wd, xd, qtype=NAMES[dtype]).cpu().numpy(), "q8k vs in-kernel quantization")
    assert_exact(got, oracle.matvec_kquant(dtype, w, rows, cols, x), f"matvec_q8k {NAMES[dtype]} cols={cols}")


@pytest.mark.parametrize("gt,ut", [(12, 12), (13, 14), (14, 14), (14, 12)])
def test_gate_up_swiglu_q8k_matches(ops, dev, gt, ut):
    rng = np.random.default_rng(gt * 17 + ut)
    rows, cols = 1000, 4096
    g, u = weights(rng, gt, rows, cols), weights(rng, ut, rows, cols)
    x = rng.normal(size=cols).astype(np.float32)
    xq = ops.quantize_q8k(to_dev(x, dev))
    got = ops.gate_up_swiglu_q8k(to_dev(g, dev), to_dev(u, dev), xq, qtype=NAMES[gt], up_qtype=NAMES[ut])
    assert_exact(got.cpu().numpy(), oracle.gate_up_swiglu(gt, g, ut, u, rows, cols, x),
                 f"gate_up_q8k {NAMES[gt]}/{NAMES[ut]}")


@pytest.mark.parametrize("dtype", [12, 13])
def test_gemv_distance_from_avx2_order(ops, dev, dtype):
    """The device GEMV is bit-exact with the CPU's portable order; an x86 host
    with AVX2 + FMA (or AVX-512) combines the same integers in another f32
    order (vec_dot_q4k.rs:381-451, vec_dot_q5k.rs:229-312).  This measures the
    device result's distance from that order at the Llama-3-8B gate shape
    (14336 x 4096) and bounds it by 4e-6 of each row's magnitude; the printed
    ulp distances are the figures quoted for it."""
    rng = np.random.default_rng(8 + dtype)
    rows, cols = 14336, 4096
    w = weights(rng, dtype, rows, cols)
    x = rng.normal(size=cols).astype(np.float32)
    got = ops.matvec_kquant(to_dev(w, dev), to_dev(x, dev), qtype=NAMES[dtype]).cpu().numpy()
    qs, bs, d = oracle.quantize_q8k(x)
    avx = np.array([oracle.kquant_row_dot_avx2(dtype, w[r], cols, qs, bs, d) for r in range(rows)], np.float32)
    port = oracle.matvec_kquant(dtype, w, rows, cols, x)
    assert_exact(got, port, "device vs portable order")
    gi, ai = got.view(np.int32).astype(np.int64), avx.view(np.int32).astype(np.int64)
    gi = np.where(gi < 0, -(gi & 0x7FFFFFFF), gi)
    ai = np.where(ai < 0, -(ai & 0x7FFFFFFF), ai)
    ulps = np.abs(gi - ai)
    xq = (qs.astype(np.float64).reshape(-1, 256) * d[:, None].astype(np.float64)).ravel()
    mags = np.array([float(np.dot(np.abs(oracle.dequantize_row(dtype, w[r], cols).astype(np.float64)), np.abs(xq)))
                     for r in range(0, rows, 97)])
    dev_rel = np.abs(got[::97].astype(np.float64) - avx[::97].astype(np.float64)) / mags
    print(f"\n{NAMES[dtype]} {rows}x{cols}: device vs AVX2-order: equal {int((ulps == 0).sum())}/{rows}, "
          f"ulp distance max {int(ulps.max())} median {float(np.median(ulps))} p99 {float(np.percentile(ulps, 99))}; "
          f"max |diff| / row magnitude {dev_rel.max():.2e}")
    assert dev_rel.max() <= 4e-6
