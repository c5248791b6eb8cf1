/*
 * fellm_oracle.c — CPU restatement of FeLLM backend-cpu for the per-layer
 * memory-bound ops.  TEST INFRASTRUCTURE ONLY: the parity checker and the
 * CPU baseline.  Nothing in the product library links or calls this file.
 *
 * Each function follows the reference line by line, in the same operation
 * order, compiled with -ffp-contract=off (Rust never contracts a*b+c).
 * Paths are relative to the FeLLM repository root.
 *
 * Parity pins (see tests/test_oracle.py):
 *   dequant Q4_K / Q5_K / Q6_K / Q8_0, get_scale_min_k4 — reference known-answer
 *     tests (dequant.rs:377-398, :435-476, :478-498), closed-form blocks from
 *     crates/fellm-plugin-host/tests/load_cuda_kernels.rs:194-199, :257-263,
 *     the Q8_0 block of load_cuda_kernels.rs:131-140 (d = 1, values 1..=32),
 *     and an independent per-element decode on random blocks.
 *   f16 / bf16 conversions — numpy's IEEE binary16 and exhaustive bit checks.
 *   rmsnorm — norm.rs:60-81 tests, closed forms, f64 recomputation.  The
 *     lane-combine order of wide::f32x8::reduce_add (norm.rs:19) is restated
 *     from the crate's AVX horizontal sum; no reference test pins those bits
 *     (parity unpinned at the last bit; tolerance-checked only).
 *   rope — rope.rs:69-77 (pos 0 identity), rotation closed forms, f64 recomputation.
 *   silu_gate — swiglu.rs:32 (silu(0) = 0), f64 recomputation, limits.
 *   kv_write — independent addressing restatement, f16 tie cases.
 *   router — brute-force full sort on small inputs, constructed ties.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define QK_K 256

/* ---- dtype edges (a8) ---------------------------------------------------- */

/* half::f16::to_f32: exact IEEE binary16 widening (dequant.rs:29-35).  With
 * F16C available (a -march=native build on such a host) the hardware
 * conversion, as the half crate uses under that target feature; both are
 * exact. */
#ifdef __F16C__
#include <immintrin.h>
static float f16_to_f32(uint16_t h) { return _cvtsh_ss(h); }
#else
static float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: normalise */
            int e = -1;
            do {
                ++e;
                man <<= 1;
            } while ((man & 0x400u) == 0);
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
        }
    } else if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}
#endif

/* half::f16::from_f32: IEEE round-to-nearest-even (backend.rs:1645, :1765). */
static uint16_t f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) /* inf or nan */
        return sign | 0x7c00u | (ax > 0x7f800000u ? (uint16_t)(0x200u | ((ax >> 13) & 0x3ffu)) : 0);
    if (ax >= 0x477ff000u) return sign | 0x7c00u; /* rounds to >= 65520 -> inf */
    if (ax < 0x38800000u) {                       /* below the smallest normal: subnormal or zero */
        if (ax < 0x33000000u) return sign;        /* < 2^-25: rounds to zero */
        const uint32_t e = ax >> 23;
        const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126 - e;           /* value = m * 2^(e-150); unit = 2^-24 */
        const uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1);
        const uint32_t halfway = 1u << (shift - 1);
        uint32_t r = q + ((rem > halfway || (rem == halfway && (q & 1))) ? 1 : 0);
        return sign | (uint16_t)r;
    }
    uint32_t r = ax - 0x38000000u; /* rebias exponent 127 -> 15 */
    const uint32_t q = r >> 13, rem = r & 0x1fffu;
    uint32_t out = q + ((rem > 0x1000u || (rem == 0x1000u && (q & 1))) ? 1 : 0);
    return sign | (uint16_t)out;
}

/* bf16 widening: bits << 16 (dequant.rs:36-42, backend.rs:1635). */
static float bf16_to_f32(uint16_t b) {
    uint32_t bits = (uint32_t)b << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* Reference Cast f32 -> bf16 truncates (backend.rs:1654). */
static uint16_t f32_to_bf16_trunc(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    return (uint16_t)(x >> 16);
}

/* Round-to-nearest-even bf16, used for the new bf16 activation outputs. */
static uint16_t f32_to_bf16_rne(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

void oracle_f16_to_f32(const uint16_t *in, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = f16_to_f32(in[i]);
}
void oracle_f32_to_f16(const float *in, uint16_t *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = f32_to_f16(in[i]);
}
void oracle_bf16_to_f32(const uint16_t *in, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = bf16_to_f32(in[i]);
}
void oracle_f32_to_bf16(const float *in, uint16_t *out, size_t n, int truncate) {
    for (size_t i = 0; i < n; ++i) out[i] = truncate ? f32_to_bf16_trunc(in[i]) : f32_to_bf16_rne(in[i]);
}

/* glibc expf: the function Rust's f32::exp resolves to on linux-gnu. */
void oracle_expf(const float *in, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = expf(in[i]);
}

/* f32::ln: glibc logf. */
void oracle_logf(const float *in, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = logf(in[i]);
}

/* f32::sin_cos as rope.rs:46-58 calls it: glibc sinf and cosf. */
void oracle_sincosf(const float *in, float *s, float *c, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        s[i] = sinf(in[i]);
        c[i] = cosf(in[i]);
    }
}

/* ---- a1: dequant + embedding -------------------------------------------- */

/* dequant.rs:295-305 */
static void get_scale_min_k4(size_t j, const uint8_t *q, uint8_t *d, uint8_t *m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

void oracle_get_scale_min_k4(size_t j, const uint8_t *q, uint8_t *d, uint8_t *m) { get_scale_min_k4(j, q, d, m); }

static uint16_t le16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* dequant.rs:251-292 */
static int dequantize_q4_k(const uint8_t *src, float *dst, size_t n) {
    if (n % QK_K) return -1;
    for (size_t b = 0; b < n / QK_K; ++b) {
        const uint8_t *base = src + b * 144;
        const float d = f16_to_f32(le16(base));
        const float dmin = f16_to_f32(le16(base + 2));
        const uint8_t *scales = base + 4;
        const uint8_t *qs = base + 16;
        float *out = dst + b * QK_K;
        size_t is = 0, q_off = 0, y_off = 0;
        for (int g = 0; g < 4; ++g) {
            uint8_t sc0, m0, sc1, m1;
            get_scale_min_k4(is, scales, &sc0, &m0);
            get_scale_min_k4(is + 1, scales, &sc1, &m1);
            const float d1 = d * (float)sc0;
            const float m1f = dmin * (float)m0;
            const float d2 = d * (float)sc1;
            const float m2f = dmin * (float)m1;
            const uint8_t *q = qs + q_off;
            for (int l = 0; l < 32; ++l) out[y_off + l] = d1 * (float)(q[l] & 0x0F) - m1f;
            for (int l = 0; l < 32; ++l) out[y_off + 32 + l] = d2 * (float)(q[l] >> 4) - m2f;
            q_off += 32;
            y_off += 64;
            is += 2;
        }
    }
    return 0;
}

/* dequant.rs:59-107 (Q5_K: block layout d, dmin, 12 scale bytes, qh[32], qs[128]). */
static int dequantize_q5_k(const uint8_t *src, float *dst, size_t n) {
    if (n % QK_K) return -1;
    for (size_t b = 0; b < n / QK_K; ++b) {
        const uint8_t *base = src + b * 176;
        const float d = f16_to_f32(le16(base));
        const float dmin = f16_to_f32(le16(base + 2));
        const uint8_t *scales = base + 4, *qh = base + 16, *qs = base + 48;
        float *out = dst + b * QK_K;
        size_t si = 0, lo = 0, oo = 0;
        uint8_t lbit = 1, hbit = 2;
        for (int g = 0; g < 4; ++g) {
            uint8_t ls, lm, hs, hm;
            get_scale_min_k4(si, scales, &ls, &lm);
            get_scale_min_k4(si + 1, scales, &hs, &hm);
            const uint8_t *low = qs + lo;
            for (int i = 0; i < 32; ++i) {
                const uint8_t quant = (uint8_t)((low[i] & 0x0f) + ((qh[i] & lbit) ? 16 : 0));
                out[oo + i] = d * (float)ls * (float)quant - dmin * (float)lm;
            }
            for (int i = 0; i < 32; ++i) {
                const uint8_t quant = (uint8_t)((low[i] >> 4) + ((qh[i] & hbit) ? 16 : 0));
                out[oo + 32 + i] = d * (float)hs * (float)quant - dmin * (float)hm;
            }
            si += 2;
            lo += 32;
            oo += 64;
            lbit <<= 2;
            hbit <<= 2;
        }
    }
    return 0;
}

/* dequant.rs:335-370 */
static void dequantize_q6_k_block(const uint8_t *block, float *out) {
    const uint8_t *ql_all = block, *qh_all = block + 128;
    const int8_t *scales = (const int8_t *)(block + 192);
    const float d = f16_to_f32(le16(block + 208));
    size_t y_off = 0, ql_off = 0, qh_off = 0, sc_off = 0;
    for (int h = 0; h < 2; ++h) {
        const uint8_t *ql = ql_all + ql_off, *qh = qh_all + qh_off;
        const int8_t *sc = scales + sc_off;
        float *o = out + y_off;
        for (int l = 0; l < 32; ++l) {
            const int is = l / 16;
            const int q1 = ((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
            const int q2 = ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
            const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            o[l] = d * (float)sc[is] * (float)q1;
            o[l + 32] = d * (float)sc[is + 2] * (float)q2;
            o[l + 64] = d * (float)sc[is + 4] * (float)q3;
            o[l + 96] = d * (float)sc[is + 6] * (float)q4;
        }
        y_off += 128;
        ql_off += 64;
        qh_off += 32;
        sc_off += 8;
    }
}

static int dequantize_q6_k(const uint8_t *src, float *dst, size_t n) {
    if (n % QK_K) return -1;
    for (size_t b = 0; b < n / QK_K; ++b) dequantize_q6_k_block(src + b * 210, dst + b * QK_K);
    return 0;
}

/* dequant.rs:172-192 (Q8_0: 34-byte blocks of 32, f16 d then 32 int8,
 * y = d * (q as f32)). */
static int dequantize_q8_0(const uint8_t *src, float *dst, size_t n) {
    if (n % 32) return -1;
    for (size_t b = 0; b < n / 32; ++b) {
        const uint8_t *base = src + b * 34;
        const float d = f16_to_f32(le16(base));
        for (int i = 0; i < 32; ++i) dst[b * 32 + i] = d * (float)(int8_t)base[2 + i];
    }
    return 0;
}

/* Row bytes for `dim` elements of a table dtype (DType::byte_size). */
size_t oracle_row_bytes(uint32_t dtype, size_t dim) {
    switch (dtype) {
        case 0: return dim * 4;
        case 1: case 30: return dim * 2;
        case 8: return dim % 32 ? 0 : dim / 32 * 34;
        case 12: return dim / QK_K * 144;
        case 13: return dim / QK_K * 176;
        case 14: return dim / QK_K * 210;
        default: return 0;
    }
}

/* dequant.rs:19-55 (F32, F16, BF16, Q8_0, Q4_K, Q5_K, Q6_K arms) */
int oracle_dequantize_row(uint32_t dtype, const uint8_t *src, float *dst, size_t n) {
    switch (dtype) {
        case 0: memcpy(dst, src, n * 4); return 0;
        case 1: for (size_t i = 0; i < n; ++i) dst[i] = f16_to_f32(le16(src + 2 * i)); return 0;
        case 30: for (size_t i = 0; i < n; ++i) dst[i] = bf16_to_f32(le16(src + 2 * i)); return 0;
        case 8: return dequantize_q8_0(src, dst, n);
        case 12: return dequantize_q4_k(src, dst, n);
        case 13: return dequantize_q5_k(src, dst, n);
        case 14: return dequantize_q6_k(src, dst, n);
        default: return -10;
    }
}

/* backend.rs:1026-1046 -> embedding.rs:10-23 */
int oracle_embedding(const uint8_t *table, uint32_t dtype, size_t vocab, size_t dim, const uint32_t *ids,
                     size_t n_ids, float *out) {
    const size_t rb = oracle_row_bytes(dtype, dim);
    if (!rb || n_ids == 0) return -2;
    for (size_t t = 0; t < n_ids; ++t) {
        if (ids[t] >= vocab) return -2; /* the CPU slice index panics */
        const int rc = oracle_dequantize_row(dtype, table + (size_t)ids[t] * rb, out + t * dim, dim);
        if (rc) return rc;
    }
    return 0;
}

/* ---- a2/a3: add + rmsnorm ----------------------------------------------- */

/* simd_f32.rs:175-197: elementwise f32 add (exact regardless of width). */
void oracle_add(const float *a, const float *b, float *y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = a[i] + b[i];
}

/* norm.rs:6-39.  f32x8 lanes accumulate v*v over chunks of 8; reduce_add is
 * wide's AVX horizontal sum: (lo4 + hi4), then (+ high pair), then (+ lane 1). */
static void rmsnorm_row(const float *x, const float *w, float eps, size_t n, float *y) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; ++l) acc[l] = acc[l] + x[i + l] * x[i + l];
    float s4[4], s2[2];
    for (int l = 0; l < 4; ++l) s4[l] = acc[l] + acc[l + 4];
    for (int l = 0; l < 2; ++l) s2[l] = s4[l] + s4[l + 2];
    float sumsq = 0.0f;
    sumsq += s2[0] + s2[1];
    for (; i < n; ++i) sumsq += x[i] * x[i];
    const float scale = 1.0f / sqrtf(sumsq / (float)n + eps);
    for (size_t j = 0; j < n; ++j) y[j] = x[j] * scale * w[j];
}

/* backend.rs:1104-1133: rows (or head groups) of w.len() elements. */
int oracle_rmsnorm(const float *x, const float *w, size_t group, size_t n, float eps, float *y) {
    if (group == 0 || n % group) return -2;
    for (size_t r = 0; r < n / group; ++r) rmsnorm_row(x + r * group, w, eps, group, y + r * group);
    return 0;
}

/* ---- a6: swiglu ---------------------------------------------------------- */

/* swiglu.rs:5-16 */
void oracle_silu_gate(const float *g, const float *u, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        const float silu = g[i] / (1.0f + expf(-g[i]));
        out[i] = silu * u[i];
    }
}

/* ---- a4: rope ------------------------------------------------------------ */

/* fellm-model/src/rope.rs:13-40 with RopeScalingType::None. */
void oracle_rope_inv_freqs(float base, uint32_t rope_dim, float *out) {
    for (uint32_t i = 0; i < rope_dim / 2; ++i) {
        const float e = -((float)(2 * i)) / (float)rope_dim;
        out[i] = powf(base, e);
    }
}

/* rope.rs:28-62 (one row of n_heads * head_dim, in place) */
static void rope_row(float *x, size_t n_heads, size_t head_dim, size_t rope_dim, uint32_t pos,
                     const float *inv_freqs, int split_half, int tail) {
    const float pf = (float)pos;
    const size_t start = tail ? head_dim - rope_dim : 0;
    for (size_t h = 0; h < n_heads; ++h) {
        float *rot = x + h * head_dim + start;
        for (size_t i = 0; i < rope_dim / 2; ++i) {
            const float theta = pf * inv_freqs[i];
            const float s = sinf(theta), c = cosf(theta);
            const size_t first = split_half ? i : 2 * i;
            const size_t second = split_half ? i + rope_dim / 2 : 2 * i + 1;
            const float a = rot[first], b = rot[second];
            rot[first] = a * c - b * s;
            rot[second] = a * s + b * c;
        }
    }
}

/* backend.rs:1135-1172: copy then rotate each row; pos = positions[row] if
 * given (row < n_positions), else position0 + row (saturating). */
int oracle_rope(const float *x, float *out, size_t n, size_t n_heads, size_t head_dim, size_t rope_dim,
                uint32_t pairing, const float *inv_freqs, const uint32_t *positions, size_t n_positions,
                uint32_t position0) {
    const size_t width = (n_heads ? n_heads : 1) * (head_dim ? head_dim : 1);
    memcpy(out, x, n * 4);
    if (n % width) return 0; /* reference leaves the copy unrotated */
    for (size_t row = 0; row < n / width; ++row) {
        uint32_t pos;
        if (positions && row < n_positions) {
            pos = positions[row];
        } else {
            const uint64_t p = (uint64_t)position0 + row;
            pos = p > 0xffffffffull ? 0xffffffffu : (uint32_t)p;
        }
        rope_row(out + row * width, n_heads, head_dim, rope_dim, pos, inv_freqs, pairing == 1, pairing == 2);
    }
    return 0;
}

/* ---- a5: paged kv write -------------------------------------------------- */

/* backend.rs:1734-1775 with paged_ctx.rs:341-360 (row_mut_for).
 * elem: 0 = f16 RNE (reference), 1 = bf16 RNE (extension). */
int oracle_kv_write_paged(const float *rows, size_t batch, size_t stride, const uint32_t *row_positions,
                          const uint32_t *table, size_t n_table, size_t n_logical, size_t n_layers, size_t layer,
                          size_t block_size, size_t block_bytes, uint8_t *arena, size_t arena_len, int is_v,
                          int elem) {
    const size_t row_bytes = stride * 2;
    for (size_t r = 0; r < batch; ++r) {
        const size_t t = row_positions[r];
        const size_t logical = t / block_size, slot = t % block_size;
        const size_t idx = (r * n_layers + layer) * n_logical + logical;
        if (logical >= n_logical || idx >= n_table) return -22;
        const size_t phys = table[idx];
        const size_t base = phys * block_bytes + (is_v ? block_size * row_bytes : 0) + slot * row_bytes;
        if (base + row_bytes > arena_len) return -22;
        uint16_t *dst = (uint16_t *)(arena + base);
        for (size_t i = 0; i < stride; ++i)
            dst[i] = elem ? f32_to_bf16_rne(rows[r * stride + i]) : f32_to_f16(rows[r * stride + i]);
    }
    return 0;
}

/* ---- a7: router ---------------------------------------------------------- */

typedef struct {
    size_t e;
    float s;
} Scored;

/* f32::total_cmp key */
static int32_t total_key(float f) {
    int32_t i;
    memcpy(&i, &f, 4);
    i ^= (int32_t)(((uint32_t)(i >> 31)) >> 1);
    return i;
}

/* sort_by(|a, b| b.1.total_cmp(&a.1).then_with(|| a.0.cmp(&b.0))) */
static int rank_cmp(const void *pa, const void *pb) {
    const Scored *a = (const Scored *)pa, *b = (const Scored *)pb;
    const int32_t ka = total_key(a->s), kb = total_key(b->s);
    if (kb != ka) return kb < ka ? -1 : 1;
    return a->e < b->e ? -1 : (a->e > b->e ? 1 : 0);
}

/* moe.rs:68-77 */
static float sqrt_softplus(float v) {
    const float sp = v > 20.0f ? v : (v < -20.0f ? expf(v) : logf(1.0f + expf(v)));
    return sqrtf(fmaxf(sp, 0.0f)); /* f32::max returns the non-NaN operand */
}

/* moe.rs:79-186: gate_scores -> sort -> finish_selected, per token. */
int oracle_router(const float *logits, size_t tokens, size_t n_experts, size_t n_expert_used, uint32_t gating,
                  uint32_t norm_topk_prob, float routed_scaling_factor, uint32_t *ids, float *weights) {
    if (n_experts == 0) return -2;
    Scored *sc = (Scored *)malloc(n_experts * sizeof(Scored));
    if (!sc) return -3;
    const size_t k = n_expert_used < n_experts ? n_expert_used : n_experts;
    for (size_t t = 0; t < tokens; ++t) {
        const float *l = logits + t * n_experts;
        if (gating == 2) {
            for (size_t e = 0; e < n_experts; ++e) sc[e] = (Scored){e, 1.0f / (1.0f + expf(-l[e]))};
        } else if (gating == 4) {
            for (size_t e = 0; e < n_experts; ++e) sc[e] = (Scored){e, sqrt_softplus(l[e])};
        } else {
            float m = -INFINITY;
            for (size_t e = 0; e < n_experts; ++e) m = fmaxf(m, l[e]); /* f32::max ignores NaN */
            float denom = 0.0f;
            for (size_t e = 0; e < n_experts; ++e) {
                const float s = expf(l[e] - m);
                denom += s;
                sc[e] = (Scored){e, s};
            }
            if (denom > 0.0f)
                for (size_t e = 0; e < n_experts; ++e) sc[e].s /= denom;
        }
        qsort(sc, n_experts, sizeof(Scored), rank_cmp);
        float sum = 0.0f;
        if (norm_topk_prob) {
            for (size_t r = 0; r < k; ++r) sum += sc[r].s;
            if (sum > 0.0f)
                for (size_t r = 0; r < k; ++r) sc[r].s /= sum;
        }
        const float scale = routed_scaling_factor == 0.0f ? 1.0f : routed_scaling_factor;
        for (size_t r = 0; r < k; ++r) {
            ids[t * k + r] = (uint32_t)sc[r].e;
            weights[t * k + r] = sc[r].s * scale;
        }
    }
    free(sc);
    return 0;
}

/* ---- f32 K/V attention (non-paged Attention arms) ------------------------
 * backend.rs:1412-1535 (launch_canvas_attention, no paged prefix): per query
 * row and head, scores over keys [b1, e1) of (k1, v1) then [0, n2) of
 * (k2, v2): score = sum_d q*k in dimension order, times scale; max; denom =
 * sum exp(s - max) in key order; out = sum (exp(s - max) / denom) * v in key
 * order.  Contiguous decode (backend.rs:1371-1397) is the one-row case over
 * [max(0, seq - window), seq) of one pair. */
void oracle_attention_f32kv(const float *q, float *out, size_t rows, size_t n_heads, size_t n_kv, size_t hd,
                            const float *k1, const float *v1, size_t b1, size_t e1, const float *k2, const float *v2,
                            size_t n2, float scale) {
    const size_t kvw = n_kv * hd, group = n_heads / (n_kv ? n_kv : 1);
    const size_t n1 = e1 > b1 ? e1 - b1 : 0, n = n1 + n2;
    float *sc = (float *)malloc((n ? n : 1) * sizeof(float));
    for (size_t r = 0; r < rows; ++r)
        for (size_t h = 0; h < n_heads; ++h) {
            const size_t kh = h / (group ? group : 1);
            const float *qh = q + (r * n_heads + h) * hd;
            float *oh = out + (r * n_heads + h) * hd;
            for (size_t j = 0; j < n; ++j) {
                const float *kr = j < n1 ? k1 + (b1 + j) * kvw + kh * hd : k2 + (j - n1) * kvw + kh * hd;
                float s = 0.0f;
                for (size_t d = 0; d < hd; ++d) s += qh[d] * kr[d];
                sc[j] = s * scale;
            }
            float mx = -INFINITY, den = 0.0f;
            for (size_t j = 0; j < n; ++j) mx = fmaxf(mx, sc[j]);
            for (size_t j = 0; j < n; ++j) den += expf(sc[j] - mx);
            for (size_t d = 0; d < hd; ++d) oh[d] = 0.0f;
            if (den > 0.0f)
                for (size_t j = 0; j < n; ++j) {
                    const float w = expf(sc[j] - mx) / den;
                    const float *vr = j < n1 ? v1 + (b1 + j) * kvw + kh * hd : v2 + (j - n1) * kvw + kh * hd;
                    for (size_t d = 0; d < hd; ++d) oh[d] += w * vr[d];
                }
        }
    free(sc);
}

/* Contiguous-K/V attention with query_len rows, the CPU backend's default
 * host path (backend.rs:1385-1391 -> attention_provider.rs:251-385,
 * fa2_style_attention_f32): q and out head-major ([h][qi][d]), K/V rows
 * [kj][kv_h][d]; query blocks of br rows, key tiles of bc keys (the dispatch
 * defaults 16/16 raised to at least 4/16, backend.rs:1278-1279).  Causal:
 * key kj <= kv_len - query_len + qi, and within `window` of that bound when
 * window > 0; not causal with window > 0: |qi - kj| < window.  Per tile: the
 * max of the finite scores, alpha = exp(m - m_new) rescales out and l, then
 * p = exp(s - m_new) accumulates into out (key order) and a tile sum added to l. */
void oracle_fa2_attention_f32(const float *q, const float *k, const float *v, float *out, size_t n_heads,
                              size_t n_kv_heads, size_t hd, size_t query_len, size_t kv_len, float scale, int causal,
                              size_t window, size_t q_tile, size_t kv_tile) {
    const size_t n_kv = n_kv_heads ? n_kv_heads : 1;
    size_t group = n_heads / n_kv;
    if (!group) group = 1;
    const size_t br = q_tile ? q_tile : 1, bc = kv_tile ? kv_tile : 1;
    float *m = (float *)malloc(br * sizeof(float)), *l = (float *)malloc(br * sizeof(float));
    float *scores = (float *)malloc(bc * sizeof(float));
    for (size_t h = 0; h < n_heads; ++h) {
        const size_t kv_h = h / group;
        for (size_t q0 = 0; q0 < query_len; q0 += br) {
            const size_t q1 = q0 + br < query_len ? q0 + br : query_len;
            for (size_t i = 0; i < q1 - q0; ++i) {
                m[i] = -INFINITY;
                l[i] = 0.0f;
                memset(out + (h * query_len + q0 + i) * hd, 0, hd * sizeof(float));
            }
            for (size_t k0 = 0; k0 < kv_len; k0 += bc) {
                const size_t k1 = k0 + bc < kv_len ? k0 + bc : kv_len;
                for (size_t qi = q0; qi < q1; ++qi) {
                    const size_t li = qi - q0;
                    const float *qr = q + (h * query_len + qi) * hd;
                    float *orow = out + (h * query_len + qi) * hd;
                    for (size_t kj = k0; kj < k1; ++kj) {
                        scores[kj - k0] = -INFINITY;
                        if (causal) {
                            const size_t max_k = kv_len - query_len + qi;
                            if (kj > max_k) continue;
                            if (window > 0 && max_k - kj >= window) continue;
                        } else if (window > 0) {
                            const size_t dist = qi > kj ? qi - kj : kj - qi;
                            if (dist >= window) continue;
                        }
                        const float *kr = k + (kj * n_kv + kv_h) * hd;
                        float sc = 0.0f;
                        for (size_t d = 0; d < hd; ++d) sc += qr[d] * kr[d];
                        scores[kj - k0] = sc * scale;
                    }
                    float mt = -INFINITY;
                    for (size_t j = 0; j < k1 - k0; ++j)
                        if (isfinite(scores[j]) && scores[j] > mt) mt = scores[j];
                    if (!isfinite(mt)) continue;
                    const float mn = mt > m[li] ? mt : m[li];
                    const float alpha = isfinite(m[li]) ? expf(m[li] - mn) : 0.0f;
                    if (alpha != 1.0f) {
                        for (size_t d = 0; d < hd; ++d) orow[d] *= alpha;
                        l[li] *= alpha;
                    }
                    float lt = 0.0f;
                    for (size_t kj = k0; kj < k1; ++kj) {
                        const float sc = scores[kj - k0];
                        if (!isfinite(sc)) continue;
                        const float p = expf(sc - mn);
                        lt += p;
                        const float *vr = v + (kj * n_kv + kv_h) * hd;
                        for (size_t d = 0; d < hd; ++d) orow[d] += p * vr[d];
                    }
                    l[li] += lt;
                    m[li] = mn;
                }
            }
            for (size_t qi = q0; qi < q1; ++qi) {
                if (l[qi - q0] > 0.0f) {
                    const float inv = 1.0f / l[qi - q0];
                    float *orow = out + (h * query_len + qi) * hd;
                    for (size_t d = 0; d < hd; ++d) orow[d] *= inv;
                }
            }
        }
    }
    free(m);
    free(l);
    free(scores);
}

/* ---- next: quantized gate/up GEMV with the SwiGLU epilogue ---------------
 * backend.rs:944-1002 (launch_gate_up_swiglu) -> matmul.rs:404-531
 * (matvec_quant_multi: x quantized once to Q8_K, every row of gate then up
 * dotted against it, then swiglu.rs silu_gate(gate, up)).
 *
 * Q8_K (matmul.rs:21-29): per 256 elements one f32 d, 256 int8 qs and 16
 * int16 bsums.  Quantization follows quantize_row_q8_k_avx2
 * (matmul.rs:213-270), the path every AVX2 x86 host takes: amax = max |x|,
 * iscale = 127/amax, q = round-to-nearest-even(x*iscale) saturated to int8,
 * bsums = sums of 16 consecutive q, d = amax/127; amax == 0 gives all zeros.
 *
 * Row dots follow the portable (scalar) paths, whose f32 order is fixed:
 *   Q4_K vec_dot_q4k.rs:296-333, Q5_K vec_dot_q5k.rs:189-218 (per block
 *     sumf = ((-dmin)*xd)*f(sumi_min); sumf += (d*xd)*f(sumi)), row = serial
 *     sum over blocks (vec_dot_q4k.rs:68-77);
 *   Q6_K matmul.rs:1597-1644 (fused_q6_k_block: 16 terms (d*sc)*f(dot) in
 *     (half, is, k) order, times xd), row = serial sum (matmul.rs:516-525).
 * The SIMD Q4_K/Q5_K paths (AVX2 / VNNI / AVX-512) compute the same integer
 * dots and differ only in the f32 combine order. */

void oracle_quantize_q8k(const float *x, size_t n, int8_t *qs, int16_t *bsums, float *d) {
    for (size_t b = 0; b < n / QK_K; ++b) {
        const float *xb = x + b * QK_K;
        int8_t *q = qs + b * QK_K;
        float amax = 0.0f;
        for (int i = 0; i < QK_K; ++i) {
            const float a = fabsf(xb[i]);
            amax = a > amax ? a : amax;
        }
        if (amax == 0.0f) {
            memset(q, 0, QK_K);
            memset(bsums + b * 16, 0, 16 * sizeof(int16_t));
            d[b] = 0.0f;
            continue;
        }
        const float iscale = 127.0f / amax;
        for (int i = 0; i < QK_K; ++i) {
            /* _mm256_cvtps_epi32 (round to nearest even) returns INT32_MIN for
             * NaN and |v| >= 2^31 (iscale overflows to inf when amax < ~3.7e-37);
             * the saturating packs then clamp to [-128, 127]. */
            const float v = xb[i] * iscale;
            if (!(fabsf(v) < 2147483648.0f)) {
                q[i] = -128;
                continue;
            }
            const long r = lrintf(v);
            q[i] = (int8_t)(r < -128 ? -128 : r > 127 ? 127 : r);
        }
        for (int g = 0; g < 16; ++g) {
            int s = 0;
            for (int l = 0; l < 16; ++l) s += q[g * 16 + l];
            bsums[b * 16 + g] = (int16_t)s;
        }
        d[b] = amax / 127.0f;
    }
}

/* Integer parts of one Q4_K / Q5_K block against one Q8_K block:
 * sumi = sum_g sc[g] * dot(aux8[32g..], q[32g..]), sumi_min = sum_j bsums[j] * m[j/2]. */
static void kquant45_ints(uint32_t dtype, const uint8_t *blk, const int8_t *q, const int16_t *bs, int32_t *sumi,
                          int32_t *sumi_min) {
    uint8_t sc[8], mn[8], aux8[QK_K];
    for (int j = 0; j < 8; ++j) get_scale_min_k4((size_t)j, blk + 4, &sc[j], &mn[j]);
    const uint8_t *qs = blk + (dtype == 13 ? 48 : 16), *qh = blk + 16;
    for (int j = 0; j < 4; ++j) /* unpack_q4_k_aux8 / unpack_q5_k_aux8 */
        for (int l = 0; l < 32; ++l) {
            uint8_t lo = qs[32 * j + l] & 0x0F, hi = qs[32 * j + l] >> 4;
            if (dtype == 13) {
                lo = (uint8_t)(lo + ((qh[l] >> (2 * j)) & 1) * 16);
                hi = (uint8_t)(hi + ((qh[l] >> (2 * j + 1)) & 1) * 16);
            }
            aux8[64 * j + l] = lo;
            aux8[64 * j + 32 + l] = hi;
        }
    int32_t smin = 0, s = 0;
    for (int j = 0; j < 16; ++j) smin += (int32_t)bs[j] * (int32_t)mn[j / 2];
    for (int g = 0; g < 8; ++g) {
        int32_t dot = 0;
        for (int l = 0; l < 32; ++l) dot += (int32_t)aux8[32 * g + l] * (int32_t)q[32 * g + l];
        s += (int32_t)sc[g] * dot;
    }
    *sumi = s;
    *sumi_min = smin;
}

void oracle_kquant45_ints(uint32_t dtype, const uint8_t *blk, const int8_t *q, const int16_t *bs, int32_t *out2) {
    kquant45_ints(dtype, blk, q, bs, &out2[0], &out2[1]);
}

static float dot_k45_block(uint32_t dtype, const uint8_t *blk, const int8_t *q, const int16_t *bs, float xd) {
    const float d = f16_to_f32(le16(blk)), dmin = f16_to_f32(le16(blk + 2));
    int32_t sumi, sumi_min;
    kquant45_ints(dtype, blk, q, bs, &sumi, &sumi_min);
    float sumf = -dmin * xd * (float)sumi_min;
    sumf += d * xd * (float)sumi;
    return sumf;
}

/* matmul.rs:1597-1644 */
static float dot_q6k_block(const uint8_t *blk, const int8_t *xq, float xd) {
    const uint8_t *ql_all = blk, *qh_all = blk + 128;
    const int8_t *scales = (const int8_t *)(blk + 192);
    const float d = f16_to_f32(le16(blk + 208));
    float acc = 0.0f;
    for (int h = 0; h < 2; ++h) {
        const uint8_t *ql = ql_all + 64 * h, *qh = qh_all + 32 * h;
        const int8_t *sc = scales + 8 * h, *x = xq + 128 * h;
        int32_t dots[4][2] = {{0}};
        for (int l = 0; l < 32; ++l) {
            const int is = l / 16;
            const int q1 = ((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
            const int q2 = ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
            const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            dots[0][is] += q1 * x[l];
            dots[1][is] += q2 * x[l + 32];
            dots[2][is] += q3 * x[l + 64];
            dots[3][is] += q4 * x[l + 96];
        }
        for (int is = 0; is < 2; ++is)
            for (int k = 0; k < 4; ++k) acc += d * (float)sc[is + 2 * k] * (float)dots[k][is];
    }
    return acc * xd;
}

static size_t kquant_block_bytes(uint32_t dtype) {
    return dtype == 12 ? 144 : dtype == 13 ? 176 : dtype == 14 ? 210 : 0;
}

/* One weight row against quantized activations: serial f32 sum over blocks. */
float oracle_kquant_row_dot(uint32_t dtype, const uint8_t *row, size_t cols, const int8_t *qs, const int16_t *bsums,
                            const float *d) {
    const size_t bb = kquant_block_bytes(dtype);
    float acc = 0.0f;
    for (size_t b = 0; b < cols / QK_K; ++b) {
        if (dtype == 14)
            acc += dot_q6k_block(row + b * bb, qs + b * QK_K, d[b]);
        else
            acc += dot_k45_block(dtype, row + b * bb, qs + b * QK_K, bsums + b * 16, d[b]);
    }
    return acc;
}

/* The x86 AVX2 + FMA row dot's f32 combine for Q4_K / Q5_K
 * (vec_dot_q4k.rs:381-451 vec_dot_q4_k_q8_k_row_avx2; vec_dot_q5k.rs:229-312),
 * which an AVX2/FMA host (and, with the same lane layout, the AVX-512 path at
 * vec_dot_q4k.rs:690-774) runs instead of the portable scalar order above.
 * Per block i: d = y.d * d, dmin = -y.d * dmin (f32); eight int32 lanes
 * sumi[k] = sum over the four 64-element chunks j of
 *   sc[2j] * sum_{b=4k..4k+3} lo_j[b] q8[64j + b] + sc[2j+1] * sum_{b} hi_j[b] q8[64j + 32 + b]
 * (maddubs pairs bytes, madd pairs those with the broadcast scale); four
 * int32 lanes prod[m] = mn[2m] (bs[4m] + bs[4m+1]) + mn[2m+1] (bs[4m+2] + bs[4m+3]);
 * acc[k] = fma(d, sumi[k], acc[k]), acc_m[m] = fma(dmin, prod[m], acc_m[m]).
 * End: hsum_float_8(acc) = ((a0+a4) + (a2+a6)) + ((a1+a5) + (a3+a7)),
 * acc_m folded as (m0 + m2) + (m1 + m3), result hsum + acc_m.
 * Used only to measure how far the device GEMV (which follows the portable
 * order bit for bit) lies from what such a host computes. */
float oracle_kquant_row_dot_avx2(uint32_t dtype, const uint8_t *row, size_t cols, const int8_t *qs,
                                 const int16_t *bsums, const float *xd) {
    const size_t bb = kquant_block_bytes(dtype);
    float acc[8] = {0}, acc_m[4] = {0};
    for (size_t i = 0; i < cols / QK_K; ++i) {
        const uint8_t *blk = row + i * bb;
        const int8_t *q = qs + i * QK_K;
        const int16_t *bs = bsums + i * 16;
        const float d = xd[i] * f16_to_f32(le16(blk));
        const float dmin = -xd[i] * f16_to_f32(le16(blk + 2));
        uint8_t sc[8], mn[8];
        for (int j = 0; j < 8; ++j) get_scale_min_k4((size_t)j, blk + 4, &sc[j], &mn[j]);
        for (int m = 0; m < 4; ++m) {
            const int32_t prod = (int32_t)mn[2 * m] * (int32_t)(int16_t)(bs[4 * m] + bs[4 * m + 1]) +
                                 (int32_t)mn[2 * m + 1] * (int32_t)(int16_t)(bs[4 * m + 2] + bs[4 * m + 3]);
            acc_m[m] = fmaf(dmin, (float)prod, acc_m[m]);
        }
        const uint8_t *qb = blk + (dtype == 13 ? 48 : 16), *qh = blk + 16;
        int32_t sumi[8] = {0};
        for (int j = 0; j < 4; ++j)
            for (int k = 0; k < 8; ++k) {
                int32_t pl = 0, ph = 0;
                for (int b = 4 * k; b < 4 * k + 4; ++b) {
                    int lo = qb[32 * j + b] & 0x0F, hi = qb[32 * j + b] >> 4;
                    if (dtype == 13) {
                        lo += ((qh[b] >> (2 * j)) & 1) << 4;
                        hi += ((qh[b] >> (2 * j + 1)) & 1) << 4;
                    }
                    pl += lo * q[64 * j + b];
                    ph += hi * q[64 * j + 32 + b];
                }
                sumi[k] += (int32_t)sc[2 * j] * pl + (int32_t)sc[2 * j + 1] * ph;
            }
        for (int k = 0; k < 8; ++k) acc[k] = fmaf(d, (float)sumi[k], acc[k]);
    }
    const float s0 = acc[0] + acc[4], s1 = acc[1] + acc[5], s2 = acc[2] + acc[6], s3 = acc[3] + acc[7];
    const float h = (s0 + s2) + (s1 + s3);
    const float m = (acc_m[0] + acc_m[2]) + (acc_m[1] + acc_m[3]);
    return h + m;
}

static int matvec_kquant_q(uint32_t dtype, const uint8_t *w, size_t rows, size_t cols, const int8_t *qs,
                           const int16_t *bs, const float *d, float *y) {
    const size_t bb = kquant_block_bytes(dtype);
    if (!bb || cols % QK_K) return -2;
    const size_t rb = cols / QK_K * bb;
    for (size_t r = 0; r < rows; ++r) y[r] = oracle_kquant_row_dot(dtype, w + r * rb, cols, qs, bs, d);
    return 0;
}

/* matvec_quant (matmul.rs:534-600) for the K-quant dtypes. */
int oracle_matvec_kquant(uint32_t dtype, const uint8_t *w, size_t rows, size_t cols, const float *x, float *y) {
    if (cols % QK_K) return -2;
    int8_t *qs = malloc(cols);
    int16_t *bs = malloc(cols / 16 * sizeof(int16_t));
    float *d = malloc(cols / QK_K * sizeof(float));
    oracle_quantize_q8k(x, cols, qs, bs, d);
    const int rc = matvec_kquant_q(dtype, w, rows, cols, qs, bs, d, y);
    free(qs);
    free(bs);
    free(d);
    return rc;
}

/* backend.rs:944-1002: gate and up rows against one Q8_K copy of x, then
 * out = silu(gate) * up (swiglu.rs:5-16). */
int oracle_gate_up_swiglu(uint32_t gate_dtype, const uint8_t *gate_w, uint32_t up_dtype, const uint8_t *up_w,
                          size_t rows, size_t cols, const float *x, float *out) {
    float *g = malloc(rows * sizeof(float)), *u = malloc(rows * sizeof(float));
    int rc = oracle_matvec_kquant(gate_dtype, gate_w, rows, cols, x, g);
    if (!rc) rc = oracle_matvec_kquant(up_dtype, up_w, rows, cols, x, u);
    if (!rc) oracle_silu_gate(g, u, out, rows);
    free(g);
    free(u);
    return rc;
}

/* ---- next: paged decode attention -----------------------------------------
 * crates/fellm-plugin-abi/src/attention_provider.rs:391-459
 * (reference_attention_paged_f32, the ABI's declared attention oracle): per
 * query head h (kv head h / (n_heads / n_kv)), a serial online softmax over
 * keys t = 0 .. seq-1, skipping t when causal && window > 0 &&
 * seq-1-t >= window; score = (sum_d q[d]*k[d] in d order) * scale;
 * m_new = max(m, score); alpha = m finite ? exp(m - m_new) : 0;
 * p = exp(score - m_new); when alpha != 1 the output row and l are scaled by
 * alpha; out += p * v; l += p; finally out *= 1/l when l > 0.
 * Driven per batch row as backend.rs:1286-1323 does (seq = row_lengths[row],
 * causal, window = attention_window); K/V rows from paged_ctx.rs:138-174
 * (K rows of a block first, then its V rows, stride = n_kv * head_dim
 * elements).  elem: 0 = f16 cache (reference), 1 = bf16 (extension). */
int oracle_paged_attention(const float *q, float *out, size_t batch, size_t n_heads, size_t n_kv, size_t hd,
                           const uint32_t *row_lengths, float scale, int causal, size_t window, const uint8_t *arena,
                           size_t arena_len, const uint32_t *table, size_t n_table, size_t n_logical, size_t n_layers,
                           size_t layer, size_t block_size, size_t block_bytes, int elem) {
    const size_t nk = n_kv ? n_kv : 1, group = n_heads / nk ? n_heads / nk : 1, stride = nk * hd;
    const size_t row_bytes = stride * 2;
    for (size_t r = 0; r < batch; ++r) {
        const size_t seq = row_lengths[r];
        for (size_t h = 0; h < n_heads; ++h) {
            const size_t g = h / group;
            const float *qr = q + (r * n_heads + h) * hd;
            float *o = out + (r * n_heads + h) * hd;
            for (size_t d = 0; d < hd; ++d) o[d] = 0.0f;
            float m = -INFINITY, l = 0.0f;
            for (size_t t = 0; t < seq; ++t) {
                if (causal && window > 0 && (seq - 1 - t) >= window) continue;
                const size_t logical = t / block_size, slot = t % block_size;
                const size_t idx = (r * n_layers + layer) * n_logical + logical;
                if (logical >= n_logical || idx >= n_table) return -22;
                const size_t base = (size_t)table[idx] * block_bytes + slot * row_bytes;
                if (base + block_size * row_bytes + row_bytes > arena_len) return -22;
                const uint16_t *kr = (const uint16_t *)(arena + base) + g * hd;
                const uint16_t *vr = (const uint16_t *)(arena + base + block_size * row_bytes) + g * hd;
                float score = 0.0f;
                for (size_t d = 0; d < hd; ++d) score += qr[d] * (elem ? bf16_to_f32(kr[d]) : f16_to_f32(kr[d]));
                score *= scale;
                const float m_new = score > m ? score : m;
                const float alpha = isfinite(m) ? expf(m - m_new) : 0.0f;
                const float p = expf(score - m_new);
                if (alpha != 1.0f) {
                    for (size_t d = 0; d < hd; ++d) o[d] *= alpha;
                    l *= alpha;
                }
                for (size_t d = 0; d < hd; ++d) o[d] += p * (elem ? bf16_to_f32(vr[d]) : f16_to_f32(vr[d]));
                l += p;
                m = m_new;
            }
            if (l > 0.0f) {
                const float inv = 1.0f / l;
                for (size_t d = 0; d < hd; ++d) o[d] *= inv;
            }
        }
    }
    return 0;
}

/* ---- next: MoE dispatch / gather / combine around the expert FFNs ---------
 * crates/backend-cpu/src/kernels/moe.rs:839-848 groups the routed assignments
 * per expert while walking tokens in order and each token's selected experts
 * in rank order (groups[expert].push((token, weight))), so inside an expert
 * the assignments a = token * k + slot appear in ascending a; moe.rs:954-957
 * copies each group's x rows; moe.rs:1024-1033 adds every group's outputs
 * into y expert by expert (value += weight * contribution, no FMA), so a
 * token's contributions arrive in ascending expert id order.  The CUDA
 * plugin's count / prefix / scatter / weighted-reduce kernels
 * (oxide_kernels.rs:2289-2327, 2507-2532) compute the same grouping with an
 * atomic (unordered) scatter and a rank-order reduce from zero. */
int oracle_moe_dispatch(const uint32_t *ids, size_t tokens, size_t k, size_t n_experts, uint32_t *counts,
                        uint32_t *offsets, uint32_t *order, uint32_t *inv) {
    const size_t n = tokens * k;
    for (size_t e = 0; e < n_experts; ++e) counts[e] = 0;
    for (size_t a = 0; a < n; ++a) {
        if (ids[a] >= n_experts) return -2;
        counts[ids[a]]++;
    }
    uint32_t run = 0;
    for (size_t e = 0; e < n_experts; ++e) {
        offsets[e] = run;
        run += counts[e];
    }
    offsets[n_experts] = run;
    uint32_t *cursor = calloc(n_experts, sizeof(uint32_t));
    for (size_t a = 0; a < n; ++a) {
        const uint32_t e = ids[a], pos = offsets[e] + cursor[e]++;
        order[pos] = (uint32_t)a;
        inv[a] = pos;
    }
    free(cursor);
    return 0;
}

/* grouped[i] = x[order[i] / k] (moe.rs:954-957), f32 rows of width h. */
void oracle_moe_gather(const float *x, size_t tokens, size_t k, size_t h, const uint32_t *order, float *grouped) {
    for (size_t i = 0; i < tokens * k; ++i) memcpy(grouped + i * h, x + (size_t)(order[i] / k) * h, h * sizeof(float));
}

/* y[t] = y0[t] + sum over t's assignments in ascending (expert id, slot) of
 * weight * expert_out[inv[a]] (moe.rs:1024-1033). */
void oracle_moe_combine(const float *y0, const float *expert_out, const uint32_t *ids, const float *weights,
                        const uint32_t *inv, size_t tokens, size_t k, size_t h, float *y) {
    for (size_t t = 0; t < tokens; ++t) {
        float *yr = y + t * h;
        memcpy(yr, y0 + t * h, h * sizeof(float));
        /* next slot by (expert id, slot): a selection sort over the k slots */
        uint64_t last = 0;
        for (size_t done = 0; done < k; ++done) {
            size_t best = k;
            uint64_t best_key = 0;
            for (size_t s = 0; s < k; ++s) {
                const uint64_t key = (uint64_t)ids[t * k + s] * k + s;
                if ((done == 0 || key > last) && (best == k || key < best_key)) best = s, best_key = key;
            }
            const float w = weights[t * k + best];
            const float *src = expert_out + (size_t)inv[t * k + best] * h;
            for (size_t d = 0; d < h; ++d) yr[d] += w * src[d];
            last = best_key;
        }
    }
}
