"""CPU oracle for parity tests: numpy wrapper over liboracle.so (fellm_oracle.c).

TEST INFRASTRUCTURE ONLY.  Imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the checker; the product library never uses
it.  Build with ``make -C oracle``.

Also composes the 16-bit activation variants the way the reference's f32 op
boundary implies: widen inputs exactly, run the f32 reference op, round the
f32 result once (f16: IEEE RNE as half::f16::from_f32; bf16: RNE).
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def build_native(out_dir: Path) -> tuple[Path, str]:
    """Compile the restatement for this host (-march=native, as the reference
    is built) into out_dir; returns (library path, compiler flags)."""
    out = Path(out_dir) / "liboracle_native.so"
    subprocess.run(["make", "-s", "-C", str(HERE), "native", f"NATIVE_OUT={out}"], check=True)
    flags = subprocess.run(["make", "-s", "-C", str(HERE), "native-flags"], check=True, capture_output=True,
                           text=True).stdout.strip()
    return out, flags


def use_library(path: Path | None) -> None:
    """Route every wrapper below through the library at `path` (None: the
    default checker build)."""
    global _lib
    _lib = None
    lib(path)


def lib(path: Path | None = None) -> C.CDLL:
    global _lib
    if _lib is None:
        if path is None and not LIB_PATH.exists():
            build()
        l = C.CDLL(str(path or LIB_PATH))
        P, S, U32, F = C.c_void_p, C.c_size_t, C.c_uint32, C.c_float
        sigs = {
            "oracle_f16_to_f32": (None, [P, P, S]),
            "oracle_f32_to_f16": (None, [P, P, S]),
            "oracle_bf16_to_f32": (None, [P, P, S]),
            "oracle_f32_to_bf16": (None, [P, P, S, C.c_int]),
            "oracle_expf": (None, [P, P, S]),
            "oracle_sincosf": (None, [P, P, P, S]),
            "oracle_logf": (None, [P, P, S]),
            "oracle_attention_f32kv": (None, [P, P, S, S, S, S, P, P, S, S, P, P, S, F]),
            "oracle_fa2_attention_f32": (None, [P, P, P, P, S, S, S, S, S, F, C.c_int, S, S, S]),
            "oracle_get_scale_min_k4": (None, [S, P, P, P]),
            "oracle_row_bytes": (S, [U32, S]),
            "oracle_dequantize_row": (C.c_int, [U32, P, P, S]),
            "oracle_embedding": (C.c_int, [P, U32, S, S, P, S, P]),
            "oracle_add": (None, [P, P, P, S]),
            "oracle_rmsnorm": (C.c_int, [P, P, S, S, F, P]),
            "oracle_silu_gate": (None, [P, P, P, S]),
            "oracle_rope_inv_freqs": (None, [F, U32, P]),
            "oracle_rope": (C.c_int, [P, P, S, S, S, S, U32, P, P, S, U32]),
            "oracle_kv_write_paged": (C.c_int, [P, S, S, P, P, S, S, S, S, S, S, P, S, C.c_int, C.c_int]),
            "oracle_router": (C.c_int, [P, S, S, S, U32, U32, F, P, P]),
            "oracle_quantize_q8k": (None, [P, S, P, P, P]),
            "oracle_kquant45_ints": (None, [U32, P, P, P, P]),
            "oracle_kquant_row_dot": (F, [U32, P, S, P, P, P]),
            "oracle_kquant_row_dot_avx2": (F, [U32, P, S, P, P, P]),
            "oracle_matvec_kquant": (C.c_int, [U32, P, S, S, P, P]),
            "oracle_gate_up_swiglu": (C.c_int, [U32, P, U32, P, S, S, P, P]),
            "oracle_moe_dispatch": (C.c_int, [P, S, S, S, P, P, P, P]),
            "oracle_moe_gather": (None, [P, S, S, S, P, P]),
            "oracle_moe_combine": (None, [P, P, P, P, P, S, S, S, P]),
            "oracle_paged_attention": (C.c_int, [P, P, S, S, S, S, P, F, C.c_int, S, P, S, P, S, S, S, S, S, S,
                                                 C.c_int]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def _c(a: np.ndarray, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


# ---- dtype edges -------------------------------------------------------------
def f16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    b = _c(bits, np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().oracle_f16_to_f32(_p(b), _p(out), b.size)
    return out


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    a = _c(x, np.float32)
    out = np.empty(a.shape, np.uint16)
    lib().oracle_f32_to_f16(_p(a), _p(out), a.size)
    return out


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    b = _c(bits, np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().oracle_bf16_to_f32(_p(b), _p(out), b.size)
    return out


def f32_to_bf16_bits(x: np.ndarray, truncate: bool = False) -> np.ndarray:
    a = _c(x, np.float32)
    out = np.empty(a.shape, np.uint16)
    lib().oracle_f32_to_bf16(_p(a), _p(out), a.size, int(truncate))
    return out


def widen(bits_or_f32: np.ndarray, kind: str) -> np.ndarray:
    """Exact f32 value of stored activations ('f32', 'f16' bits or 'bf16' bits)."""
    if kind == "f32":
        return _c(bits_or_f32, np.float32)
    if kind == "f16":
        return f16_bits_to_f32(bits_or_f32)
    if kind == "bf16":
        return bf16_bits_to_f32(bits_or_f32)
    raise ValueError(kind)


def narrow(x: np.ndarray, kind: str) -> np.ndarray:
    """Store an f32 result as 'f32', or as f16/bf16 bits rounded once (RNE)."""
    if kind == "f32":
        return _c(x, np.float32)
    if kind == "f16":
        return f32_to_f16_bits(x)
    if kind == "bf16":
        return f32_to_bf16_bits(x)
    raise ValueError(kind)


def expf(x: np.ndarray) -> np.ndarray:
    a = _c(x, np.float32)
    out = np.empty_like(a)
    lib().oracle_expf(_p(a), _p(out), a.size)
    return out


def logf(x: np.ndarray) -> np.ndarray:
    a = _c(x, np.float32)
    out = np.empty_like(a)
    lib().oracle_logf(_p(a), _p(out), a.size)
    return out


def sincosf(x: np.ndarray):
    """(sinf(x), cosf(x)) from the host's glibc, as f32::sin_cos gives them."""
    a = _c(x, np.float32)
    s, c = np.empty_like(a), np.empty_like(a)
    lib().oracle_sincosf(_p(a), _p(s), _p(c), a.size)
    return s, c


# ---- ops ---------------------------------------------------------------------
def get_scale_min_k4(j: int, scales: bytes) -> tuple[int, int]:
    q = _c(np.frombuffer(scales, np.uint8), np.uint8)
    d, m = C.c_uint8(), C.c_uint8()
    lib().oracle_get_scale_min_k4(j, _p(q), C.addressof(d), C.addressof(m))
    return d.value, m.value


def row_bytes(dtype: int, dim: int) -> int:
    return lib().oracle_row_bytes(dtype, dim)


def dequantize_row(dtype: int, src: np.ndarray, n: int) -> np.ndarray:
    s = _c(src, np.uint8)
    out = np.empty(n, np.float32)
    rc = lib().oracle_dequantize_row(dtype, _p(s), _p(out), n)
    if rc:
        raise ValueError(f"dequantize_row rc={rc}")
    return out


def embedding(table: np.ndarray, dtype: int, vocab: int, dim: int, ids: np.ndarray) -> np.ndarray:
    t = _c(table, np.uint8).reshape(-1)
    i = _c(ids, np.uint32)
    out = np.empty((i.size, dim), np.float32)
    rc = lib().oracle_embedding(_p(t), dtype, vocab, dim, _p(i), i.size, _p(out))
    if rc:
        raise ValueError(f"embedding rc={rc}")
    return out


def add(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a, b = _c(a, np.float32), _c(b, np.float32)
    out = np.empty_like(a)
    lib().oracle_add(_p(a), _p(b), _p(out), a.size)
    return out


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x, w = _c(x, np.float32), _c(w, np.float32)
    out = np.empty_like(x)
    rc = lib().oracle_rmsnorm(_p(x), _p(w), w.size, x.size, eps, _p(out))
    if rc:
        raise ValueError(f"rmsnorm rc={rc}")
    return out


def add_rmsnorm(x, r, w, eps, kind: str = "f32"):
    """Fused residual add + RMSNorm on stored activations of `kind`.

    h = narrow(widen(x) + widen(r)); y = narrow(rmsnorm(widen(h))).
    Returns (h, y) in storage form (f32 values or 16-bit bits).
    """
    h = narrow(add(widen(x, kind), widen(r, kind)), kind)
    y = narrow(rmsnorm(widen(h, kind), w, eps), kind)
    return h, y


def silu_gate(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g, u = _c(g, np.float32), _c(u, np.float32)
    out = np.empty_like(g)
    lib().oracle_silu_gate(_p(g), _p(u), _p(out), g.size)
    return out


def rope_inv_freqs(theta: float, rope_dim: int) -> np.ndarray:
    out = np.empty(rope_dim // 2, np.float32)
    lib().oracle_rope_inv_freqs(theta, rope_dim, _p(out))
    return out


def rope(x: np.ndarray, n_heads: int, head_dim: int, rope_dim: int, pairing: int, inv_freqs: np.ndarray,
         positions: np.ndarray | None = None, position0: int = 0) -> np.ndarray:
    x = _c(x, np.float32)
    f = _c(inv_freqs, np.float32)
    out = np.empty_like(x)
    pos = _c(positions, np.uint32) if positions is not None else None
    lib().oracle_rope(_p(x), _p(out), x.size, n_heads, head_dim, rope_dim, pairing, _p(f),
                      _p(pos) if pos is not None else None, pos.size if pos is not None else 0, position0)
    return out


def kv_write_paged(rows: np.ndarray, stride: int, row_positions: np.ndarray, table: np.ndarray, n_logical: int,
                   n_layers: int, layer: int, block_size: int, block_bytes: int, arena: np.ndarray, is_v: bool,
                   elem: str = "f16") -> None:
    """In-place write into `arena` (uint8) as backend.rs:1734-1775."""
    rows = _c(rows, np.float32)
    pos = _c(row_positions, np.uint32)
    tab = _c(table, np.uint32)
    assert arena.dtype == np.uint8 and arena.flags.c_contiguous
    rc = lib().oracle_kv_write_paged(_p(rows), pos.size, stride, _p(pos), _p(tab), tab.size, n_logical, n_layers,
                                     layer, block_size, block_bytes, _p(arena), arena.size, int(is_v),
                                     1 if elem == "bf16" else 0)
    if rc:
        raise ValueError(f"kv_write rc={rc}")


def router(logits: np.ndarray, k: int, gating: int = 1, norm: bool = True, rsf: float = 0.0):
    l = _c(logits, np.float32)
    t, e = l.shape
    kk = min(k, e)
    ids = np.empty((t, kk), np.uint32)
    w = np.empty((t, kk), np.float32)
    rc = lib().oracle_router(_p(l), t, e, k, gating, int(norm), rsf, _p(ids), _p(w))
    if rc:
        raise ValueError(f"router rc={rc}")
    return ids, w


# ---- next: K-quant GEMV + SwiGLU epilogue -------------------------------------
def quantize_q8k(x: np.ndarray):
    """Q8_K activations of x (len % 256 == 0): (qs int8[n], bsums int16[n/16], d f32[n/256])."""
    a = _c(x, np.float32).ravel()
    qs = np.empty(a.size, np.int8)
    bs = np.empty(a.size // 16, np.int16)
    d = np.empty(a.size // 256, np.float32)
    lib().oracle_quantize_q8k(_p(a), a.size, _p(qs), _p(bs), _p(d))
    return qs, bs, d


def kquant45_ints(dtype: int, block: np.ndarray, qs: np.ndarray, bsums: np.ndarray) -> tuple[int, int]:
    """(sumi, sumi_min) of one Q4_K/Q5_K block against one Q8_K block."""
    b = _c(block, np.uint8)
    q = _c(qs, np.int8)
    s = _c(bsums, np.int16)
    out = np.zeros(2, np.int32)
    lib().oracle_kquant45_ints(dtype, _p(b), _p(q), _p(s), _p(out))
    return int(out[0]), int(out[1])


def kquant_row_dot(dtype: int, row: np.ndarray, cols: int, qs, bsums, d) -> float:
    r = _c(row, np.uint8)
    q, s, dd = _c(qs, np.int8), _c(bsums, np.int16), _c(d, np.float32)
    return float(np.float32(lib().oracle_kquant_row_dot(dtype, _p(r), cols, _p(q), _p(s), _p(dd))))


def kquant_row_dot_avx2(dtype: int, row: np.ndarray, cols: int, qs, bsums, d) -> float:
    """The x86 AVX2/FMA row dot's f32 combine (Q4_K, Q5_K) on a Q8_K vector."""
    r = _c(row, np.uint8)
    q, s, dd = _c(qs, np.int8), _c(bsums, np.int16), _c(d, np.float32)
    return float(np.float32(lib().oracle_kquant_row_dot_avx2(dtype, _p(r), cols, _p(q), _p(s), _p(dd))))


def matvec_kquant(dtype: int, w: np.ndarray, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    ww = _c(w, np.uint8)
    xx = _c(x, np.float32)
    y = np.empty(rows, np.float32)
    rc = lib().oracle_matvec_kquant(dtype, _p(ww), rows, cols, _p(xx), _p(y))
    if rc:
        raise ValueError(f"oracle_matvec_kquant rc={rc}")
    return y


def gate_up_swiglu(gate_dtype: int, gate_w: np.ndarray, up_dtype: int, up_w: np.ndarray, rows: int, cols: int,
                   x: np.ndarray) -> np.ndarray:
    g, u = _c(gate_w, np.uint8), _c(up_w, np.uint8)
    xx = _c(x, np.float32)
    out = np.empty(rows, np.float32)
    rc = lib().oracle_gate_up_swiglu(gate_dtype, _p(g), up_dtype, _p(u), rows, cols, _p(xx), _p(out))
    if rc:
        raise ValueError(f"oracle_gate_up_swiglu rc={rc}")
    return out


# ---- next: paged decode attention ---------------------------------------------
def paged_attention(q: np.ndarray, n_heads: int, n_kv: int, head_dim: int, row_lengths: np.ndarray, scale: float,
                    arena: np.ndarray, table: np.ndarray, n_logical: int, n_layers: int, layer: int, block_size: int,
                    block_bytes: int, causal: bool = True, window: int = 0, kind: str = "f16") -> np.ndarray:
    """reference_attention_paged_f32 per batch row over the paged arena: q f32 [B, n_heads*head_dim]."""
    qq = _c(q, np.float32)
    B = len(row_lengths)
    out = np.empty((B, n_heads * head_dim), np.float32)
    rl = _c(row_lengths, np.uint32)
    ar = _c(arena, np.uint8)
    tb = _c(table, np.uint32)
    rc = lib().oracle_paged_attention(_p(qq), _p(out), B, n_heads, n_kv, head_dim, _p(rl), scale, int(causal),
                                      window, _p(ar), ar.size, _p(tb), tb.size, n_logical, n_layers, layer,
                                      block_size, block_bytes, 1 if kind == "bf16" else 0)
    if rc:
        raise ValueError(f"oracle_paged_attention rc={rc}")
    return out


# ---- next: MoE dispatch / gather / combine -------------------------------------
def moe_dispatch(ids: np.ndarray, n_experts: int):
    """ids u32 [tokens, k] -> (counts [E], offsets [E+1], order [T*k], inv [T*k])."""
    ii = _c(ids, np.uint32)
    tokens, k = ii.shape
    counts = np.empty(n_experts, np.uint32)
    offsets = np.empty(n_experts + 1, np.uint32)
    order = np.empty(tokens * k, np.uint32)
    inv = np.empty(tokens * k, np.uint32)
    rc = lib().oracle_moe_dispatch(_p(ii), tokens, k, n_experts, _p(counts), _p(offsets), _p(order), _p(inv))
    if rc:
        raise ValueError(f"oracle_moe_dispatch rc={rc}")
    return counts, offsets, order, inv


def moe_gather(x: np.ndarray, k: int, order: np.ndarray) -> np.ndarray:
    xx = _c(x, np.float32)
    tokens, h = xx.shape
    out = np.empty((tokens * k, h), np.float32)
    oo = _c(order, np.uint32)
    lib().oracle_moe_gather(_p(xx), tokens, k, h, _p(oo), _p(out))
    return out


def moe_combine(y0: np.ndarray, expert_out: np.ndarray, ids: np.ndarray, weights: np.ndarray,
                inv: np.ndarray) -> np.ndarray:
    yy = _c(y0, np.float32)
    tokens, h = yy.shape
    k = ids.shape[1]
    eo, ii, ww, iv = _c(expert_out, np.float32), _c(ids, np.uint32), _c(weights, np.float32), _c(inv, np.uint32)
    out = np.empty_like(yy)
    lib().oracle_moe_combine(_p(yy), _p(eo), _p(ii), _p(ww), _p(iv), tokens, k, h, _p(out))
    return out


def moe_weighted_reduce(y0: np.ndarray | None, expert_out: np.ndarray, weights: np.ndarray) -> np.ndarray:
    """Slot-order combine over per-assignment rows, as the CUDA plugin's
    moe_weighted_reduce (plugins/cuda_kernels/src/oxide_kernels.rs:2507-2532):
    value = 0 (here y0 when given); value += score * out for slot 0..k-1.
    numpy evaluates w * e and the add as two f32 roundings (no FMA)."""
    ww = np.asarray(weights, np.float32)
    tokens, k = ww.shape
    eo = np.asarray(expert_out, np.float32).reshape(tokens, k, -1)
    y = np.zeros((tokens, eo.shape[2]), np.float32) if y0 is None else np.array(y0, np.float32)
    for s in range(k):
        y = (y + (ww[:, s:s + 1] * eo[:, s]).astype(np.float32)).astype(np.float32)
    return y


def attention_f32kv(q: np.ndarray, n_heads: int, n_kv: int, head_dim: int, k1, v1, b1: int, e1: int,
                    k2=None, v2=None, n2: int = 0, scale: float = 0.0) -> np.ndarray:
    """Non-paged attention (backend.rs:1371-1397, :1412-1535): q [rows, n_heads * head_dim]."""
    q = _c(q, np.float32)
    rows = q.size // (n_heads * head_dim)
    out = np.zeros_like(q)
    if scale <= 0:
        scale = float(np.float32(1.0) / np.sqrt(np.float32(head_dim)))
    ka = _c(k1, np.float32) if k1 is not None else np.zeros(1, np.float32)
    va = _c(v1, np.float32) if v1 is not None else np.zeros(1, np.float32)
    kb = _c(k2, np.float32) if k2 is not None else np.zeros(1, np.float32)
    vb = _c(v2, np.float32) if v2 is not None else np.zeros(1, np.float32)
    lib().oracle_attention_f32kv(_p(q), _p(out), rows, n_heads, n_kv, head_dim, _p(ka), _p(va), b1, e1, _p(kb),
                                 _p(vb), n2, scale)
    return out


def fa2_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, n_heads: int, n_kv: int, head_dim: int,
                  query_len: int, kv_len: int, scale: float, causal: bool, window: int = 0,
                  q_tile: int = 16, kv_tile: int = 16) -> np.ndarray:
    """The CPU backend's host FA2 attention (attention_provider.rs:251-385): q and the result
    head-major [n_heads, query_len, head_dim]; k, v [kv_len, n_kv * head_dim]."""
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    out = np.zeros(n_heads * query_len * head_dim, np.float32)
    lib().oracle_fa2_attention_f32(_p(q), _p(k), _p(v), _p(out), n_heads, n_kv, head_dim, query_len, kv_len, scale,
                                   int(causal), window, q_tile, kv_tile)
    return out
