"""Pins the CPU oracle (oracle/fellm_oracle.c) before it is trusted as the checker.

Each function is checked against the reference's own known-answer tests
(tests/golden/reference_known_answers.json, transcribed with file:line), and
where those leave gaps against an independent formulation (per-element
decodes written from the CUDA plugin's indexing, numpy's IEEE binary16,
float64 recomputation, brute-force sorting) chosen so that a dropped term,
a swapped index or a wrong rounding mode fails a test.
"""
from __future__ import annotations

import json
import math
from decimal import Decimal, getcontext
from pathlib import Path

import numpy as np
import pytest

import oracle
from fellm_amd import synth

GOLD = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())
F32, F16, Q8_0, Q4K, Q5K, Q6K, BF16 = 0, 1, 8, 12, 13, 14, 30


# ---- dtype edges ----------------------------------------------------------------
def test_f16_widening_all_patterns():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_bits_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_rne_matches_ieee():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.normal(size=1 << 20).astype(np.float32) * np.float32(4.0),
        (rng.random(1 << 18) * 70000).astype(np.float32),
        (rng.random(1 << 18) * 1e-4).astype(np.float32),  # subnormal f16 range
        np.array([65504, 65519.99, 65520, 1e30, -1e30, 0.0, -0.0, np.inf, -np.inf, 5.96e-8, 2.98e-8, 2.99e-8],
                 np.float32),
    ])
    got = oracle.f32_to_f16_bits(x)
    ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_f32_to_f16_ties_round_to_even():
    # 1 + 2^-11 is exactly halfway between 1 and the next f16: RNE keeps 1.0;
    # 1 + 3*2^-11 is halfway between two odd/even neighbours and rounds up to
    # the even one.  A round-half-up conversion fails the first case.
    x = np.array([1 + 2**-11, 1 + 3 * 2**-11, -(1 + 2**-11), 2048 + 1], np.float32)
    got = oracle.f32_to_f16_bits(x)
    assert got.tolist() == [0x3C00, 0x3C02, 0xBC00, 0x6800]


def test_bf16_edges():
    x = np.array([1.0, 1.0 + 2**-8, 1.0 + 3 * 2**-8, -2.5, np.inf], np.float32)
    assert oracle.f32_to_bf16_bits(x).tolist() == [0x3F80, 0x3F80, 0x3F82, 0xC020, 0x7F80]
    assert oracle.f32_to_bf16_bits(x, truncate=True).tolist() == [0x3F80, 0x3F80, 0x3F81, 0xC020, 0x7F80]
    bits = np.arange(0, 65536, 97, dtype=np.uint32).astype(np.uint16)
    w = oracle.bf16_bits_to_f32(bits)
    assert np.array_equal(w.view(np.uint32), bits.astype(np.uint32) << 16)


# ---- dequant known answers --------------------------------------------------------
def test_q5k_reference_fixture():
    g = GOLD["q5k_fixture"]
    src = np.array([(i * 37 + 11) % 256 for i in range(g["block_bytes"])], np.uint8)
    out = oracle.dequantize_row(Q5K, src, 256)
    assert out[:8].tolist() == g["first8"]
    assert float(out.astype(np.float64).sum()) == g["sum_f64"]


def test_q4k_nibble_layout():
    g = GOLD["q4k_nibble_layout"]
    block = np.zeros(144, np.uint8)
    block[0:2] = np.array([g["d_f16_bits"]], np.uint16).view(np.uint8)
    block[4:16] = g["scale_bytes_4_to_16"]
    block[16:48] = g["qs_first_chunk_byte"]
    out = oracle.dequantize_row(Q4K, block, 256)
    for rng_s, val in g["expect"].items():
        a, b = map(int, rng_s.split(":"))
        assert np.all(np.abs(out[a:b] - val) < g["tolerance"]), rng_s


def test_get_scale_min_k4_roundtrip():
    g = GOLD["get_scale_min_k4"]
    packed = synth.pack_scale_min_k4(np.array(g["scales"]), np.array(g["mins"]))
    for j in range(8):
        assert oracle.get_scale_min_k4(j, packed.tobytes()) == (g["scales"][j], g["mins"][j])


def test_closed_form_blocks():
    q4 = np.zeros(144, np.uint8)
    q4[0:2] = [0x00, 0x3C]
    q4[4:8] = 1
    q4[12:16] = 1
    q4[16:] = 0x11
    v = oracle.dequantize_row(Q4K, q4, 256)
    assert np.all(v == GOLD["q4k_all_ones_block"]["every_value"])
    assert float(v.sum()) == GOLD["q4k_all_ones_block"]["dot_ones"]
    q6 = np.zeros(210, np.uint8)
    q6[192:208] = 1
    q6[208:210] = [0x00, 0x3C]
    v = oracle.dequantize_row(Q6K, q6, 256)
    assert np.all(v == GOLD["q6k_all_minus32_block"]["every_value"])
    assert float(v.sum()) == GOLD["q6k_all_minus32_block"]["dot_ones"]


def _scales_mins_masked(sb: np.ndarray):
    """Scale/min unpack in the 32-bit mask form of the CUDA plugin
    (plugins/cuda_kernels/src/oxide_kernels.rs:5298-5331), vectorised."""
    u = sb.reshape(-1, 12).view("<u4").astype(np.uint32)  # [n, 3]
    k1, k2, k3 = np.uint32(0x3F3F3F3F), np.uint32(0x0F0F0F0F), np.uint32(0x03030303)
    u0, u1, u2 = u[:, 0], u[:, 1], u[:, 2]
    u3 = ((u2 >> 4) & k2) | (((u1 >> 6) & k3) << 4)
    uaux = u1 & k1
    u1n = (u2 & k2) | (((u0 >> 6) & k3) << 4)
    u0n = u0 & k1
    sc = np.stack([u0n, u1n], 1).astype("<u4").view(np.uint8).reshape(-1, 8)
    mn = np.stack([uaux, u3], 1).astype("<u4").view(np.uint8).reshape(-1, 8)
    return sc, mn


def _q4k_per_element(block: np.ndarray) -> np.ndarray:
    """Per-element Q4_K decode with the CUDA plugin's indexing (oxide_kernels.rs:3638-3685)."""
    nb = block.size // 144
    b = block.reshape(nb, 144)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    dmin = b[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]
    sc, mn = _scales_mins_masked(b[:, 4:16].copy())
    j = np.arange(256)
    group, lane = j // 32, j % 32
    qbase = 16 + (j // 64) * 32
    raw = b[:, qbase + lane]
    q = np.where(j % 64 < 32, raw & 15, raw >> 4).astype(np.float32)
    d_sc = (d[:, None] * sc[:, group].astype(np.float32)).astype(np.float32)
    m = (dmin[:, None] * mn[:, group].astype(np.float32)).astype(np.float32)
    return (d_sc * q - m).astype(np.float32).reshape(-1)


def _q6k_per_element(block: np.ndarray) -> np.ndarray:
    """Per-element Q6_K decode with the CUDA plugin's indexing (oxide_kernels.rs:3830-3876)."""
    nb = block.size // 210
    b = block.reshape(nb, 210)
    d = b[:, 208:210].copy().view(np.float16).astype(np.float32)[:, 0]
    j = np.arange(256)
    half, local = j // 128, j % 128
    lane, quad = local % 32, local // 32
    shift = quad * 2
    qi = np.where((quad == 0) | (quad == 2), lane, lane + 32)
    qlv = b[:, half * 64 + qi]
    nib = np.where(quad < 2, qlv & 15, qlv >> 4).astype(np.int32)
    qh = b[:, 128 + half * 32 + lane].astype(np.int32)
    q = (nib | (((qh >> shift) & 3) << 4)) - 32
    sc = b[:, 192 + half * 8 + lane // 16 + quad * 2].view(np.int8).astype(np.float32)
    return ((d[:, None] * sc).astype(np.float32) * q.astype(np.float32)).astype(np.float32).reshape(-1)


def _q5k_per_element(block: np.ndarray) -> np.ndarray:
    """Per-element Q5_K decode with the CUDA plugin's indexing (oxide_kernels.rs:3687-3719,
    q5k_dequant_at): group j / 32, qs chunk j / 64 at byte 48, high bit (1 or 2) << 2 * chunk of
    qh[j % 32] at byte 16; y = d * sc * q - dmin * m, evaluated left to right."""
    nb = block.size // 176
    b = block.reshape(nb, 176)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    dmin = b[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]
    sc, mn = _scales_mins_masked(b[:, 4:16].copy())
    j = np.arange(256)
    group, lane, chunk = j // 32, j % 32, j // 64
    low = j % 64 < 32
    raw = b[:, 48 + chunk * 32 + lane]
    bit = np.where(low, 1, 2) << (chunk * 2)
    hi = (b[:, 16 + lane] & bit) != 0
    q = (np.where(low, raw & 15, raw >> 4) + np.where(hi, 16, 0)).astype(np.float32)
    d_sc = (d[:, None] * sc[:, group].astype(np.float32)).astype(np.float32)
    m = (dmin[:, None] * mn[:, group].astype(np.float32)).astype(np.float32)
    return ((d_sc * q).astype(np.float32) - m).astype(np.float32).reshape(-1)


def _q8_0_per_element(row: np.ndarray) -> np.ndarray:
    """Per-element Q8_0 decode with the CUDA plugin's indexing (oxide_kernels.rs:2559-2581,
    embedding_q8_0_rows): d at the 34-byte block's start, int8 value at 2 + lane."""
    b = row.reshape(-1, 34)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    q = b[:, 2:].view(np.int8).astype(np.float32)
    return (d[:, None] * q).astype(np.float32).reshape(-1)


_PER_ELEMENT = {"q4k": (Q4K, _q4k_per_element), "q5k": (Q5K, _q5k_per_element), "q6k": (Q6K, _q6k_per_element),
                "q8_0": (Q8_0, _q8_0_per_element)}


@pytest.mark.parametrize("kind", ["q4k", "q5k", "q6k", "q8_0"])
def test_quant_decode_matches_per_element_restatement(kind):
    rng = np.random.default_rng(17)
    dim = 2048
    code, per_element = _PER_ELEMENT[kind]
    table = {"q4k": synth.q4k_table, "q5k": synth.q5k_table, "q6k": synth.q6k_table,
             "q8_0": synth.q8_0_table}[kind](rng, 64, dim)
    for row in range(64):
        got = oracle.dequantize_row(code, table[row], dim)
        ref = per_element(table[row])
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"row {row}"


def test_q8_0_reference_block():
    """The Q8_0 block of the reference's CUDA matmul test: d = 1.0, values 1..=32; its dots with
    rows of ones and twos are the test's expected 528 and 1056."""
    g = GOLD["q8_0_one_to_32_block"]
    block = np.zeros(34, np.uint8)
    block[0:2] = [0x00, 0x3C]
    block[2:] = np.arange(1, 33)
    v = oracle.dequantize_row(Q8_0, block, 32)
    assert v.tolist() == g["values"]
    assert float(v.sum()) == g["dot_ones"] and float((2 * v).sum()) == g["dot_twos"]
    # Negative values are two's-complement int8 (`as i8`, dequant.rs:187).
    block[2:] = np.arange(0x80, 0xA0)
    assert oracle.dequantize_row(Q8_0, block, 32).tolist() == list(range(-128, -96))
    assert oracle.row_bytes(Q8_0, 96) == 102 and oracle.row_bytes(Q8_0, 100) == 0


def test_embedding_gathers_rows_exactly():
    rng = np.random.default_rng(2)
    t16 = rng.normal(0, 0.02, size=(50, 96)).astype(np.float16)
    ids = np.array([0, 49, 7, 7, 13], np.uint32)
    got = oracle.embedding(t16.view(np.uint8), F16, 50, 96, ids)
    assert np.array_equal(got, t16[ids].astype(np.float32))
    t32 = rng.normal(size=(50, 96)).astype(np.float32)
    assert np.array_equal(oracle.embedding(t32.view(np.uint8), F32, 50, 96, ids), t32[ids])
    with pytest.raises(ValueError):
        oracle.embedding(t32.view(np.uint8), F32, 50, 96, np.array([50], np.uint32))


# ---- rmsnorm -----------------------------------------------------------------------
def test_rmsnorm_reference_tests():
    g = GOLD["rmsnorm_identity_scale"]
    y = oracle.rmsnorm(np.array(g["x"], np.float32), np.array(g["w"], np.float32), g["eps"])
    assert abs(math.sqrt(float((y.astype(np.float64) ** 2).mean())) - g["expect_rms"]) < g["tolerance"]
    g = GOLD["rmsnorm_groups"]
    y = oracle.rmsnorm(np.array(g["x"], np.float32), np.array(g["w"], np.float32), g["eps"]).astype(np.float64)
    for k, want in enumerate(g["expect_group_rms"]):
        assert abs(math.sqrt(float((y[2 * k:2 * k + 2] ** 2).mean())) - want) < g["tolerance"]


def test_rmsnorm_closed_form_and_f64():
    c = np.float32(3.0)
    x = np.full(4096, c, np.float32)
    w = np.random.default_rng(0).normal(1, 0.1, 4096).astype(np.float32)
    y = oracle.rmsnorm(x, w, 1e-5)
    expect = (c / np.sqrt(np.float64(c) ** 2 + 1e-5)) * w.astype(np.float64)
    assert np.allclose(y, expect, rtol=1e-6, atol=0)
    rng = np.random.default_rng(3)
    for n in (8, 100, 2048, 4099):
        x = rng.normal(size=(5, n)).astype(np.float32)
        w = rng.normal(1, 0.1, n).astype(np.float32)
        y = oracle.rmsnorm(x, w, 1e-6).astype(np.float64)
        xd = x.astype(np.float64)
        ref = xd / np.sqrt((xd ** 2).mean(axis=1, keepdims=True) + 1e-6) * w
        assert np.all(np.abs(y - ref) <= 1e-6 * np.abs(ref) + 1e-30), n
    with pytest.raises(ValueError):
        oracle.rmsnorm(np.ones(10, np.float32), np.ones(3, np.float32), 1e-5)


# ---- rope --------------------------------------------------------------------------
def test_rope_zero_position_identity():
    g = GOLD["rope_zero_position_identity"]
    x = np.array(g["x"], np.float32)
    y = oracle.rope(x, g["n_heads"], g["head_dim"], g["rope_dim"], 0, np.array(g["inv_freqs"], np.float32),
                    np.array([g["pos"]], np.uint32))
    assert np.all(np.abs(y - x) < g["tolerance"])


def test_rope_inv_freqs_match_theta_power():
    getcontext().prec = 40
    for theta, d in ((500000.0, 128), (1e6, 128), (500000.0, 64)):
        f = oracle.rope_inv_freqs(theta, d)
        for i in range(d // 2):
            e = -np.float32(2 * i) / np.float32(d)  # the reference's f32 exponent
            exact = float(Decimal(theta) ** Decimal(float(e)))
            assert abs(float(f[i]) - exact) <= 2 * float(np.spacing(np.float32(exact))), (theta, d, i)


@pytest.mark.parametrize("pairing", [0, 1, 2])
def test_rope_against_f64_rotation(pairing):
    rng = np.random.default_rng(pairing)
    rows, nh, hd, rd = 9, 3, 16, 12 if pairing != 1 else 16
    inv = oracle.rope_inv_freqs(10000.0, rd)
    x = rng.normal(size=(rows, nh * hd)).astype(np.float32)
    pos = rng.integers(0, 32768, size=rows).astype(np.uint32)
    y = oracle.rope(x, nh, hd, rd, pairing, inv, pos).astype(np.float64)
    xr = x.reshape(rows, nh, hd).astype(np.float64)
    ref = xr.copy()
    start = hd - rd if pairing == 2 else 0
    for i in range(rd // 2):
        a_i, b_i = (i, i + rd // 2) if pairing == 1 else (start + 2 * i, start + 2 * i + 1)
        th = (pos.astype(np.float32) * inv[i]).astype(np.float64)[:, None]
        a, b = xr[..., a_i], xr[..., b_i]
        ref[..., a_i] = a * np.cos(th) - b * np.sin(th)
        ref[..., b_i] = a * np.sin(th) + b * np.cos(th)
    mag = np.abs(xr).sum(axis=2, keepdims=True)
    assert np.all(np.abs(y.reshape(rows, nh, hd) - ref) <= 1e-6 * mag)
    # rotation preserves each pair's norm; a dropped or sign-flipped term does not
    yr = y.reshape(rows, nh, hd)
    for i in range(rd // 2):
        a_i, b_i = (i, i + rd // 2) if pairing == 1 else (start + 2 * i, start + 2 * i + 1)
        n0 = np.hypot(xr[..., a_i], xr[..., b_i])
        n1 = np.hypot(yr[..., a_i], yr[..., b_i])
        assert np.allclose(n0, n1, rtol=1e-6)


def test_rope_quarter_turn():
    # theta = pi/2 (up to f32 rounding): (a, b) -> (-b, a)
    inv = np.array([np.float32(np.pi / 2)], np.float32)
    x = np.array([1.5, -2.0], np.float32)
    y = oracle.rope(x, 1, 2, 2, 0, inv, np.array([1], np.uint32))
    assert np.allclose(y, [2.0, 1.5], atol=1e-6)


def test_rope_positions_default_to_position0_plus_row():
    rng = np.random.default_rng(4)
    inv = oracle.rope_inv_freqs(10000.0, 8)
    x = rng.normal(size=(4, 8)).astype(np.float32)
    a = oracle.rope(x, 1, 8, 8, 0, inv, None, position0=10)
    b = oracle.rope(x, 1, 8, 8, 0, inv, np.array([10, 11, 12, 13], np.uint32))
    assert np.array_equal(a, b)


# ---- silu --------------------------------------------------------------------------
def test_silu_gate():
    assert abs(float(oracle.silu_gate(np.zeros(1, np.float32), np.ones(1, np.float32))[0])) < \
        GOLD["silu_at_zero"]["expect_abs_below"]
    rng = np.random.default_rng(5)
    g = (rng.normal(size=100000) * 6).astype(np.float32)
    u = rng.normal(size=100000).astype(np.float32)
    y = oracle.silu_gate(g, u).astype(np.float64)
    gd = g.astype(np.float64)
    ref = gd / (1 + np.exp(-gd)) * u
    assert np.all(np.abs(y - ref) <= 4e-7 * np.abs(ref) + 1e-38)
    big = oracle.silu_gate(np.array([30.0, -30.0], np.float32), np.ones(2, np.float32))
    assert big[0] == np.float32(30.0) and abs(big[1]) < 1e-11


def test_oracle_expf_is_libm():
    import ctypes
    import ctypes.util

    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    libm.expf.restype = ctypes.c_float
    libm.expf.argtypes = [ctypes.c_float]
    x = np.linspace(-100, 80, 997, dtype=np.float32)
    got = oracle.expf(x)
    assert all(got[i] == np.float32(libm.expf(float(x[i]))) for i in range(x.size))


def test_oracle_sincosf_is_libm():
    import ctypes
    import ctypes.util

    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    for fn in (libm.sinf, libm.cosf):
        fn.restype = ctypes.c_float
        fn.argtypes = [ctypes.c_float]
    x = np.concatenate([np.linspace(-3e4, 3e4, 997), [0.0, 1e-5, 100.0, 1e20]]).astype(np.float32)
    s, c = oracle.sincosf(x)
    assert all(s[i] == np.float32(libm.sinf(float(x[i]))) for i in range(x.size))
    assert all(c[i] == np.float32(libm.cosf(float(x[i]))) for i in range(x.size))


def test_device_inv_pio4_table_is_4_over_pi():
    """The Payne-Hanek table of the device sinf/cosf (common.hpp kInvPio4):
    entry i = floor(4/pi * 2^(8i+7)) mod 2^32, recomputed here from pi by
    Machin's formula in integer arithmetic (300 decimal digits)."""
    import re
    from pathlib import Path

    src = (Path(__file__).resolve().parents[1] / "fellm_amd" / "csrc" / "common.hpp").read_text()
    body = re.search(r"kInvPio4\[24\] = \{(.*?)\};", src, re.S).group(1)
    table = [int(v.rstrip("u"), 16) for v in re.findall(r"0x[0-9a-fA-F]+u", body)]

    def arctan_inv(x, one):
        total, term, n, sign = 0, one // x, 1, 1
        while term:
            total += sign * (term // n)
            term //= x * x
            n += 2
            sign = -sign
        return total

    one = 10 ** 300
    pi = 4 * (4 * arctan_inv(5, one) - arctan_inv(239, one))  # pi * 10^300
    want = [((4 * one) << (8 * i + 7)) // pi & 0xFFFFFFFF for i in range(24)]
    assert table == want


# ---- paged kv write -------------------------------------------------------------------
@pytest.mark.parametrize("elem", ["f16", "bf16"])
def test_kv_write_addressing(elem):
    """Independent restatement of paged_ctx.rs:341-360: row r, position t ->
    block table[(r * n_layers + layer) * n_logical + t // bs], slot t % bs."""
    rng = np.random.default_rng(6)
    batch, stride, bs, n_blocks, n_layers, layer = 7, 24, 16, 20, 3, 2
    pos, table, n_logical = synth.paged_layout(rng, batch, n_blocks, bs, 200, n_layers)
    bb = (2 * bs * stride * 2 + 63) // 64 * 64
    rows = rng.normal(size=(batch, stride)).astype(np.float32)
    arena = np.zeros(n_blocks * bb, np.uint8)
    oracle.kv_write_paged(rows, stride, pos, table, n_logical, n_layers, layer, bs, bb, arena, True, elem)
    expect = np.zeros_like(arena)
    conv = (lambda v: v.astype(np.float16).view(np.uint8)) if elem == "f16" else \
        (lambda v: oracle.f32_to_bf16_bits(v).view(np.uint8))
    for r in range(batch):
        phys = table.reshape(batch, n_layers, n_logical)[r, layer, pos[r] // bs]
        off = phys * bb + bs * stride * 2 + (pos[r] % bs) * stride * 2
        expect[off:off + stride * 2] = conv(rows[r])
    assert np.array_equal(arena, expect)


def test_kv_write_rejects_out_of_table():
    arena = np.zeros(4 * 128, np.uint8)
    with pytest.raises(ValueError):
        oracle.kv_write_paged(np.ones((1, 2), np.float32), 2, np.array([5 * 16], np.uint32),
                              np.zeros(4, np.uint32), 4, 1, 0, 16, 128, arena, False)


# ---- router --------------------------------------------------------------------------
def _brute_router(logits, k, gating, norm, rsf):
    t, e = logits.shape
    ids = np.zeros((t, min(k, e)), np.uint32)
    w = np.zeros((t, min(k, e)), np.float32)
    for i in range(t):
        l = logits[i]
        if gating == 2:
            s = (np.float32(1) / (np.float32(1) + oracle.expf(-l))).astype(np.float32)
        elif gating == 4:  # moe.rs:68-77
            sp = np.where(l > 20, l, np.where(l < -20, oracle.expf(l),
                                               oracle.logf((np.float32(1) + oracle.expf(l)).astype(np.float32))))
            s = np.sqrt(np.maximum(sp.astype(np.float32), np.float32(0))).astype(np.float32)
        else:
            m = np.float32(max(l))
            ex = oracle.expf((l - m).astype(np.float32))
            den = np.float32(0)
            for v in ex:  # expert order
                den = np.float32(den + v)
            s = (ex / den).astype(np.float32) if den > 0 else ex
        order = sorted(range(e), key=lambda j: (-float(s[j]), j))[: min(k, e)]
        sel = s[order].astype(np.float32)
        if norm:
            tot = np.float32(0)
            for v in sel:
                tot = np.float32(tot + v)
            if tot > 0:
                sel = (sel / tot).astype(np.float32)
        sel = (sel * np.float32(1.0 if rsf == 0 else rsf)).astype(np.float32)
        ids[i], w[i] = order, sel
    return ids, w


@pytest.mark.parametrize("gating,norm,rsf", [(1, True, 0.0), (2, False, 2.5), (1, False, 1.0), (4, True, 2.5),
                                             (4, False, 0.0)])
def test_router_brute_force(gating, norm, rsf):
    rng = np.random.default_rng(7)
    logits = rng.normal(size=(40, 16)).astype(np.float32)
    logits[0] = 0.25                    # all tied: lower ids win
    logits[1, :8] = logits[1, 7]         # partial ties
    ids, w = oracle.router(logits, 4, gating, norm, rsf)
    ids_b, w_b = _brute_router(logits, 4, gating, norm, rsf)
    assert np.array_equal(ids, ids_b)
    assert np.array_equal(w.view(np.uint32), w_b.view(np.uint32))
    assert ids[0].tolist() == [0, 1, 2, 3]
    if norm and gating == 1:
        assert np.allclose(w.sum(axis=1), 1.0, atol=1e-6)


def test_router_sqrt_softplus_closed_forms():
    """gating 4 (moe.rs:68-77): sqrt(v) above 20, sqrt(exp(v)) below -20,
    sqrt(ln 2) at 0, and a float64 recomputation in between."""
    l = np.array([[25.0, -25.0, 0.0, 3.0, -3.0, 20.0, -20.0, np.nan]], np.float32)
    ids, w = oracle.router(l, 8, 4, False, 0.0)
    s = dict(zip(ids[0].tolist(), w[0].tolist()))
    assert s[0] == np.float32(np.sqrt(np.float32(25.0)))
    assert s[1] == np.float32(np.sqrt(oracle.expf(np.array([-25.0], np.float32))[0]))
    assert abs(s[2] - np.sqrt(np.log(2.0))) < 1e-7
    for e, v in ((3, 3.0), (4, -3.0), (5, 20.0), (6, -20.0)):
        # the f32 sum 1 + exp(v) is rounded before the log, as in the reference
        one_plus = float(np.float32(1) + oracle.expf(np.array([v], np.float32))[0])
        want = np.sqrt(np.log(one_plus))
        assert abs(s[e] - want) <= 3e-7 * want
    assert s[7] == 0.0  # NaN: max(NaN, 0) is 0, as f32::max
    assert ids[0][0] == 0


def test_oracle_logf_is_libm():
    import ctypes
    import ctypes.util

    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    libm.logf.restype = ctypes.c_float
    libm.logf.argtypes = [ctypes.c_float]
    x = np.concatenate([np.geomspace(1e-40, 1e38, 997), [1.0, 0.0, 2.0]]).astype(np.float32)
    got = oracle.logf(x)
    assert all(got[i] == np.float32(libm.logf(float(x[i]))) for i in range(x.size))


def test_router_k_clamped_and_sigmoid_monotone():
    rng = np.random.default_rng(8)
    logits = rng.normal(size=(5, 6)).astype(np.float32)
    ids, w = oracle.router(logits, 10, 2, False, 0.0)
    assert ids.shape == (5, 6)
    for i in range(5):
        assert ids[i].tolist() == sorted(range(6), key=lambda j: (-logits[i, j], j))


def test_native_build_matches_checker(tmp_path):
    """The -march=native build the bench times as the CPU baseline computes the
    same bits as the checker build (vectorisation without reassociation, and
    F16C widening, which is exact)."""
    path, flags = oracle.build_native(tmp_path)
    assert "-march=native" in flags
    rng = np.random.default_rng(17)
    table = rng.normal(0, 0.02, size=(64, 4096)).astype(np.float16)
    ids = rng.integers(0, 64, size=16, dtype=np.uint32)
    x = rng.normal(size=(16, 4096)).astype(np.float32)
    r = (2 * rng.normal(size=(16, 4096))).astype(np.float32)
    w = rng.normal(1, 0.1, size=4096).astype(np.float32)
    q = rng.normal(size=(16, 32 * 128)).astype(np.float32)
    inv = oracle.rope_inv_freqs(500000.0, 128)
    g = rng.normal(size=(16, 14336)).astype(np.float32)

    def run():
        return [oracle.embedding(table.view(np.uint8), 1, 64, 4096, ids), oracle.add(x, r),
                oracle.rmsnorm(x, w, 1e-5), oracle.rope(q, 32, 128, 128, 0, inv, np.arange(16, dtype=np.uint32)),
                oracle.silu_gate(g, g)]

    ref = run()
    try:
        oracle.use_library(path)
        got = run()
    finally:
        oracle.use_library(None)
    for a, b in zip(got, ref):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
