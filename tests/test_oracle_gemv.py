"""Pins the oracle's K-quant GEMV path (Q8_K activations, Q4_K/Q5_K/Q6_K row
dots, gate/up SwiGLU) before it checks the GPU.

Pins, chosen so that a swapped nibble/bit index, a dropped min term or a
wrong rounding mode fails:
  * the reference's own tests, restated with their inputs
    (vec_dot_q4k.rs:788-857, vec_dot_q5k.rs:587-640): block dot within the
    stated tolerance of the dot of the dequantized block;
  * exact integer identities: with d = dmin = 1 (f16-exact) the dequantized
    weights (dequant already pinned by golden vectors) are integers, and with
    x integral and max |x| = 127 Q8_K is the identity (d = 1), so the row dot
    must equal the int64 dot exactly; d = 0 / dmin = 0 isolate sumi and
    sumi_min;
  * Q8_K closed forms (constant rows, zero rows, round-to-nearest-even ties,
    the |x - d q| <= d/2 bound, bsums = sums of qs);
  * float64 recomputation of the per-block combine for random blocks.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from fellm_amd import synth

Q4K, Q5K, Q6K = 12, 13, 14
BB = {Q4K: 144, Q5K: 176, Q6K: 210}


def f16_bytes(v: float) -> bytes:
    return np.array([v], np.float16).view(np.uint8).tobytes()


# ---- reference test inputs --------------------------------------------------------
def make_k45_block(dtype: int) -> np.ndarray:
    """Block of vec_dot_q4k.rs:788-811 / vec_dot_q5k.rs:587-612: d = 1, dmin = 0.1,
    scales j+1 / j+5, mins j+2 / j+3, byte patterns i*17 (qs) and i*13 (qh)."""
    out = np.zeros(BB[dtype], np.uint8)
    out[0:2] = np.frombuffer(f16_bytes(1.0), np.uint8)
    out[2:4] = np.frombuffer(f16_bytes(0.1), np.uint8)
    for j in range(4):
        out[4 + j] = (j + 1) & 63
        out[8 + j] = (j + 2) & 63
    for j in range(4):
        ls, lm = (j + 5) & 63, (j + 3) & 63
        out[12 + j] = (ls & 0x0F) | ((lm & 0x0F) << 4)
        out[4 + j] |= (ls >> 4) << 6
        out[8 + j] |= (lm >> 4) << 6
    qs_off = 48 if dtype == Q5K else 16
    out[qs_off:qs_off + 128] = (np.arange(128) * 17) & 0xFF
    if dtype == Q5K:
        out[16:48] = (np.arange(32) * 13) & 0xFF
    return out


def lcg_x(seed: int, n: int) -> np.ndarray:
    """x of vec_dot_q4k.rs:830-834: 64-bit LCG, (state >> 33) as f32 / u32::MAX as f32 * 2 - 1."""
    out = np.empty(n, np.float32)
    s = seed
    for i in range(n):
        s = (s * 6364136223846793005 + 1) & (2**64 - 1)
        out[i] = np.float32(s >> 33) / np.float32(4294967295.0) * np.float32(2.0) - np.float32(1.0)
    return out


def test_reference_q4k_block_matches_dequant_dot():
    # vec_dot_q4k.rs:826-857
    block = make_k45_block(Q4K)
    x = lcg_x(42, 256)
    qs, bs, d = oracle.quantize_q8k(x)
    got = np.float32(oracle.kquant_row_dot(Q4K, block, 256, qs, bs, d))
    w = oracle.dequantize_row(Q4K, block, 256)
    ref = np.float32(0.0)
    for i in range(256):
        ref = np.float32(ref + w[i] * np.float32(d[0] * np.float32(qs[i])))
    err = abs(float(got) - float(ref))
    assert err < 1e-3 * max(abs(float(ref)), 1.0) + 1e-3, (got, ref)


def test_reference_q5k_block_matches_dequant_dot():
    # vec_dot_q5k.rs:615-640
    block = make_k45_block(Q5K)
    x = (np.arange(256, dtype=np.float32) * np.float32(0.01) - np.float32(1.2)).astype(np.float32)
    qs, bs, d = oracle.quantize_q8k(x)
    got = oracle.kquant_row_dot(Q5K, block, 256, qs, bs, d)
    w = oracle.dequantize_row(Q5K, block, 256)
    acc = np.float32(0.0)
    for i in range(256):
        acc = np.float32(acc + w[i] * np.float32(qs[i]))
    expected = float(np.float32(acc * d[0]))
    assert abs(got - expected) < 1e-4 * max(abs(expected), 1.0), (got, expected)


def test_reference_row_is_sum_of_blocks():
    # vec_dot_q4k.rs:859-881: a two-block row equals the sum of its block dots
    b1 = make_k45_block(Q4K)
    b2 = make_k45_block(Q4K)
    b2[16] = 0xAB
    row = np.concatenate([b1, b2])
    x = lcg_x(7, 512)
    qs, bs, d = oracle.quantize_q8k(x)
    total = oracle.kquant_row_dot(Q4K, row, 512, qs, bs, d)
    s0 = oracle.kquant_row_dot(Q4K, b1, 256, qs[:256], bs[:16], d[:1])
    s1 = oracle.kquant_row_dot(Q4K, b2, 256, qs[256:], bs[16:], d[1:])
    assert total == float(np.float32(np.float32(s0) + np.float32(s1)))


# ---- Q8_K closed forms ------------------------------------------------------------
def test_q8k_constant_and_zero_rows():
    x = np.concatenate([np.full(256, 0.37, np.float32), np.zeros(256, np.float32),
                        np.full(256, -2.5, np.float32)])
    qs, bs, d = oracle.quantize_q8k(x)
    assert np.all(qs[:256] == 127) and np.all(bs[:16] == 16 * 127)
    assert d[0] == np.float32(np.float32(0.37) / np.float32(127.0))
    assert np.all(qs[256:512] == 0) and np.all(bs[16:32] == 0) and d[1] == 0.0
    assert np.all(qs[512:] == -127) and np.all(bs[32:] == -16 * 127)


def test_q8k_rounds_ties_to_even():
    # amax = 127 gives iscale = 1 exactly, so x*iscale = x: ties at k + 0.5.
    x = np.zeros(256, np.float32)
    x[0] = 127.0
    x[1:9] = [2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 1.5, 126.5]
    qs, _, d = oracle.quantize_q8k(x)
    assert d[0] == 1.0
    assert list(qs[1:9]) == [2, 4, -2, -4, 0, 0, 2, 126]


def test_q8k_tiny_amax_follows_cvtps_integer_indefinite():
    # amax = 3e-40 makes iscale = 127/amax overflow to inf; x*iscale is +-inf
    # (or NaN for x = 0), which cvtps_epi32 maps to INT32_MIN -> -128.
    x = np.zeros(256, np.float32)
    x[:3] = [np.float32(3e-40), np.float32(-1e-40), np.float32(2e-40)]
    qs, bs, d = oracle.quantize_q8k(x)
    assert np.all(qs == -128) and np.all(bs == -16 * 128)
    assert d[0] == np.float32(np.float32(3e-40) / np.float32(127.0))


def test_q8k_random_bounds():
    rng = np.random.default_rng(3)
    x = (rng.normal(size=4096) * rng.uniform(0.01, 10, size=4096)).astype(np.float32)
    qs, bs, d = oracle.quantize_q8k(x)
    xb = x.reshape(16, 256)
    amax = np.abs(xb).max(axis=1)
    assert np.array_equal(d, (amax / np.float32(127.0)).astype(np.float32))
    q = qs.reshape(16, 256).astype(np.int32)
    assert np.all(np.abs(q).max(axis=1) == 127)
    err = np.abs(xb.astype(np.float64) - d[:, None].astype(np.float64) * q)
    assert np.all(err <= d[:, None] * 0.5 * (1 + 1e-5))
    assert np.array_equal(bs, q.reshape(-1, 16).sum(axis=1).astype(np.int16))


# ---- exact integer identities ------------------------------------------------------
def _integral_x(rng, n):
    x = rng.integers(-127, 128, size=n).astype(np.float32)
    x[::256] = 127.0  # every Q8_K block has amax 127, so d = 1 and qs = x
    return x


@pytest.mark.parametrize("dtype", [Q4K, Q5K])
@pytest.mark.parametrize("d,dmin", [(1.0, 1.0), (1.0, 0.0), (0.0, 1.0)])
def test_k45_row_dot_exact_integers(dtype, d, dmin):
    rng = np.random.default_rng(dtype * 10 + int(d) * 2 + int(dmin))
    cols = 1024
    row = synth.KQUANT_TABLES[dtype](rng, 1, cols)[0].reshape(-1, BB[dtype])
    row[:, 0:2] = np.frombuffer(f16_bytes(d), np.uint8)
    row[:, 2:4] = np.frombuffer(f16_bytes(dmin), np.uint8)
    ls = rng.integers(0, 16, size=(row.shape[0], 8))
    lm = rng.integers(0, 64, size=(row.shape[0], 8))
    row[:, 4:16] = synth.pack_scale_min_k4(ls, lm)
    row = row.ravel()
    x = _integral_x(rng, cols)
    qs, bs, dq = oracle.quantize_q8k(x)
    assert np.all(dq == 1.0) and np.array_equal(qs.astype(np.float32), x)
    w = oracle.dequantize_row(dtype, row, cols)
    assert np.array_equal(w, np.round(w))  # integral weights
    exact = int(np.dot(w.astype(np.int64), x.astype(np.int64)))
    assert abs(exact) < 2**24
    assert oracle.kquant_row_dot(dtype, row, cols, qs, bs, dq) == float(exact)
    # the x86 AVX2/FMA combine partitions the same integers differently: exact too
    assert oracle.kquant_row_dot_avx2(dtype, row, cols, qs, bs, dq) == float(exact)


def test_q6k_row_dot_exact_integers():
    rng = np.random.default_rng(66)
    cols = 1024
    row = synth.q6k_table(rng, 1, cols)[0].reshape(-1, 210)
    row[:, 192:208] = rng.integers(-3, 4, size=(row.shape[0], 16)).astype(np.int8).view(np.uint8)
    row[:, 208:210] = np.frombuffer(f16_bytes(1.0), np.uint8)
    row = row.ravel()
    x = _integral_x(rng, cols)
    qs, bs, dq = oracle.quantize_q8k(x)
    w = oracle.dequantize_row(Q6K, row, cols)
    exact = int(np.dot(w.astype(np.int64), x.astype(np.int64)))
    assert abs(exact) < 2**24
    assert oracle.kquant_row_dot(Q6K, row, cols, qs, bs, dq) == float(exact)


@pytest.mark.parametrize("dtype", [Q4K, Q5K])
def test_k45_ints_against_dequant(dtype):
    """sumi and sumi_min from the unit-scale dequant: with d=1, dmin=0 the
    dequantized block is sc*q; with d=0, dmin=1 it is -m."""
    rng = np.random.default_rng(5 + dtype)
    for _ in range(20):
        blk = synth.KQUANT_TABLES[dtype](rng, 1, 256)[0]
        x = rng.normal(size=256).astype(np.float32)
        qs, bs, _ = oracle.quantize_q8k(x)
        sumi, sumi_min = oracle.kquant45_ints(dtype, blk, qs, bs)
        b1 = blk.copy()
        b1[0:2] = np.frombuffer(f16_bytes(1.0), np.uint8)
        b1[2:4] = 0
        b2 = blk.copy()
        b2[0:2] = 0
        b2[2:4] = np.frombuffer(f16_bytes(1.0), np.uint8)
        scq = oracle.dequantize_row(dtype, b1, 256).astype(np.int64)
        negm = oracle.dequantize_row(dtype, b2, 256).astype(np.int64)
        assert sumi == int(np.dot(scq, qs.astype(np.int64)))
        assert sumi_min == -int(np.dot(negm, qs.astype(np.int64)))


@pytest.mark.parametrize("dtype", [Q4K, Q5K, Q6K])
def test_row_dot_close_to_exact(dtype):
    """float64 dot of the dequantized weights with d*q: the f32 combine stays
    within a few ulps of the sum of the magnitudes of the terms."""
    rng = np.random.default_rng(11 + dtype)
    cols, rows = 4096, 64
    w = synth.KQUANT_TABLES[dtype](rng, rows, cols)
    x = rng.normal(size=cols).astype(np.float32)
    qs, bs, d = oracle.quantize_q8k(x)
    xq = (qs.astype(np.float64).reshape(-1, 256) * d[:, None].astype(np.float64)).ravel()
    y = oracle.matvec_kquant(dtype, w, rows, cols, x)
    for r in range(rows):
        wr = oracle.dequantize_row(dtype, w[r], cols).astype(np.float64)
        ref = float(np.dot(wr, xq))
        mag = float(np.dot(np.abs(wr), np.abs(xq)))
        assert abs(float(y[r]) - ref) <= 2e-5 * mag, (r, y[r], ref, mag)


@pytest.mark.parametrize("dtype", [Q4K, Q5K])
def test_avx2_combine_close_to_exact(dtype):
    """The AVX2/FMA-order restatement (vec_dot_q4k.rs:381-451,
    vec_dot_q5k.rs:229-312) stays within the same bound of the float64 dot,
    and differs from the portable order by at most a few ulps of the row's
    magnitude (the two orders are what an AVX2 host and the device compute)."""
    rng = np.random.default_rng(31 + dtype)
    cols, rows = 4096, 64
    w = synth.KQUANT_TABLES[dtype](rng, rows, cols)
    x = rng.normal(size=cols).astype(np.float32)
    qs, bs, d = oracle.quantize_q8k(x)
    xq = (qs.astype(np.float64).reshape(-1, 256) * d[:, None].astype(np.float64)).ravel()
    diffs = 0
    for r in range(rows):
        a = oracle.kquant_row_dot_avx2(dtype, w[r], cols, qs, bs, d)
        p = oracle.kquant_row_dot(dtype, w[r], cols, qs, bs, d)
        wr = oracle.dequantize_row(dtype, w[r], cols).astype(np.float64)
        ref, mag = float(np.dot(wr, xq)), float(np.dot(np.abs(wr), np.abs(xq)))
        assert abs(a - ref) <= 2e-5 * mag
        assert abs(a - p) <= 4e-6 * mag
        diffs += a != p
    assert diffs > 0  # the orders do differ in the last bits


def test_gate_up_swiglu_composes():
    rng = np.random.default_rng(21)
    rows, cols = 96, 2048
    g = synth.q4k_table(rng, rows, cols)
    u = synth.q6k_table(rng, rows, cols)
    x = rng.normal(size=cols).astype(np.float32)
    out = oracle.gate_up_swiglu(Q4K, g, Q6K, u, rows, cols, x)
    ref = oracle.silu_gate(oracle.matvec_kquant(Q4K, g, rows, cols, x), oracle.matvec_kquant(Q6K, u, rows, cols, x))
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    z = oracle.gate_up_swiglu(Q4K, g, Q6K, u, rows, cols, np.zeros(cols, np.float32))
    assert np.all(z == 0.0)
