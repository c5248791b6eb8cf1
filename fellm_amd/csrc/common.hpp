// Shared device helpers for the gfx950 kernels: activation dtypes, wavefront
// reductions, bit-exact glibc expf, launch bookkeeping.
#pragma once

#include <type_traits>

// Build knob: BF16HW stores through the hardware conversion (1) or integer
// rounding (0); both round to nearest even.
#ifndef FELLM_BF16_HW
#define FELLM_BF16_HW 1
#endif

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include "fellm_abi.h"
#include "fellm_rocm.h"

// Build knob: the 16-bit SwiGLU interval test rounds both ends with one
// packed hardware conversion (1) or through the output type's store (0).
#ifndef FELLM_SILU_PK
#define FELLM_SILU_PK 1
#endif

// Bit distance bound of silu_fast; kept equal to the measured maximum.
// Build knob: the packed interval test evaluates every element without a
// branch on the fast domain (1; the domain and NaN tests join the final
// compare) or returns early outside it (0).
#ifndef FELLM_SILU_BRANCHLESS
#define FELLM_SILU_BRANCHLESS 1
#endif

// Build knob: silu_fast's exp(-g) from the hardware exp2 of the whole
// argument with a first-order correction (1) or after a reduction by ln 2 (0).
#ifndef FELLM_SILU_EXP_DIRECT
#define FELLM_SILU_EXP_DIRECT 1
#endif

// Build knob (with FELLM_SILU_EXP_DIRECT): g / d in silu_fast as g times the
// hardware reciprocal (0), with one Newton step on the reciprocal (1), and
// one residual correction of the quotient (2).
#ifndef FELLM_SILU_DIV_STEPS
#define FELLM_SILU_DIV_STEPS 0
#endif

#ifndef FELLM_SILU_FAST_DIST
#define FELLM_SILU_FAST_DIST 5
#endif

namespace fellm {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// Activation element types.  Arithmetic is always f32; storage is f32, f16
// (IEEE binary16) or bf16.  Narrowing rounds to nearest-even once.
// ---------------------------------------------------------------------------
struct F32 {
    using T = float;
    static constexpr uint32_t code = FELLM_DTYPE_F32;
    __device__ __forceinline__ static float load(T v) { return v; }
    __device__ __forceinline__ static T store(float v) { return v; }
};

struct F16 {
    using T = _Float16;
    static constexpr uint32_t code = FELLM_DTYPE_F16;
    __device__ __forceinline__ static float load(T v) { return (float)v; }
    // v_cvt_f16_f32 under the default MODE register rounds to nearest-even.
    // The empty asm pins the f32 value: without it the compiler folds
    // fptrunc(f32 * fpext(f16)) into one mixed-precision FMA that rounds the
    // exact product straight to f16, skipping the f32 rounding the CPU does.
    __device__ __forceinline__ static T store(float v) {
        __asm__("" : "+v"(v));
        return (_Float16)v;
    }
};

struct BF16 {
    using T = uint16_t;
    static constexpr uint32_t code = FELLM_DTYPE_BF16;
    // Widening is exact: bits << 16 (dequant.rs:36-42).
    __device__ __forceinline__ static float load(T v) { return __uint_as_float((uint32_t)v << 16); }
    // Round to nearest-even on the top 16 bits; NaN stays a quiet NaN.
    __device__ __forceinline__ static T store(float v) {
        uint32_t u = __float_as_uint(v);
        if ((u & 0x7fffffffu) > 0x7f800000u) return (T)((u >> 16) | 0x0040u);
        u += 0x7fffu + ((u >> 16) & 1u);
        return (T)(u >> 16);
    }
};

// The same bf16 storage and rounding with non-NaN values converted by
// gfx950's hardware (v_cvt_pk_bf16_f32, round to nearest even; equal to
// BF16::store for every f32 input, checked exhaustively on the device).  NaN
// keeps the bit path.  Used where it measured faster: SwiGLU's output, which
// rounds each element twice on its fast path (c4 10.9 -> 10.5 us, c5 routed
// 95.7 -> 94.0 us).  Elsewhere the extra select raised register use (the
// fused decode step spilled, add + RMSNorm measured 5% slower), so other
// kernels keep BF16.
struct BF16HW : BF16 {
    __device__ __forceinline__ static T store(float v) {
        if constexpr (FELLM_BF16_HW) {
            const uint32_t u = __float_as_uint(v);
            const T hw = __builtin_bit_cast(T, (__bf16)v);
            return (u & 0x7fffffffu) > 0x7f800000u ? (T)((u >> 16) | 0x0040u) : hw;
        } else {
            return BF16::store(v);
        }
    }
};

// Output type of kernels that take the hardware bf16 rounding.
template <typename A> struct HwStore { using type = A; };
template <> struct HwStore<BF16> { using type = BF16HW; };

// bf16 by truncation: the CPU backend's Cast f32 -> bf16 keeps the top 16
// bits (backend.rs:1648-1656).  Store-only policy.
struct BF16Trunc {
    using T = uint16_t;
    static constexpr uint32_t code = FELLM_DTYPE_BF16;
    __device__ __forceinline__ static float load(T v) { return __uint_as_float((uint32_t)v << 16); }
    __device__ __forceinline__ static T store(float v) { return (T)(__float_as_uint(v) >> 16); }
};

// Compute units of the current device (the first call's device; every
// device this library runs on is the same part), for persistent grids.
inline int cu_count() {
    static int n = [] {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
            v = 256;
        return v;
    }();
    return n;
}

// Grid of a persistent kernel whose rows are assigned statically (workgroup b
// takes rows b, b + grid, ...): every workgroup must be resident from the
// start, or the late ones would run their rows after the others finish.  At
// most `cap` workgroups per compute unit, fewer when the kernel's registers
// or LDS (`lds` bytes, the largest the caller uses) allow fewer.  Cached per
// kernel: call it from one instantiation per kernel.
template <typename K>
inline uint32_t resident_grid(K kernel, int block, size_t lds, int cap) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, block, lds) != hipSuccess || n <= 0) n = 1;
    return (uint32_t)cu_count() * (uint32_t)(n < cap ? n : cap);
}

// Host-side dispatch helper: call f.template operator()<Type>() for a dtype code.
template <typename Fn>
inline int dispatch_act(uint32_t dtype, Fn &&f) {
    switch (dtype) {
        case FELLM_DTYPE_F32: return f.template operator()<F32>();
        case FELLM_DTYPE_F16: return f.template operator()<F16>();
        case FELLM_DTYPE_BF16: return f.template operator()<BF16>();
        default: return FELLM_ERR_DTYPE;
    }
}

inline size_t act_bytes(uint32_t dtype) {
    return dtype == FELLM_DTYPE_F32 ? 4 : (dtype == FELLM_DTYPE_F16 || dtype == FELLM_DTYPE_BF16) ? 2 : 0;
}

// ---------------------------------------------------------------------------
// Vector load/store of N elements (N * sizeof(T) must be 4, 8, 16 or 32 bytes).
// ---------------------------------------------------------------------------
template <typename T, int N>
struct alignas(sizeof(T) * N) Pack {
    T v[N];
};

template <typename A, int N>
__device__ __forceinline__ void load_f32(const typename A::T *p, float (&out)[N]) {
    Pack<typename A::T, N> pk = *reinterpret_cast<const Pack<typename A::T, N> *>(p);
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = A::load(pk.v[i]);
}

template <typename A, int N>
__device__ __forceinline__ void store_f32(typename A::T *p, const float (&in)[N]) {
    Pack<typename A::T, N> pk;
#pragma unroll
    for (int i = 0; i < N; ++i) pk.v[i] = A::store(in[i]);
    *reinterpret_cast<Pack<typename A::T, N> *>(p) = pk;
}

// Streaming variants: data touched exactly once bypasses cache retention.
template <typename A, int N>
__device__ __forceinline__ void load_f32_nt(const typename A::T *p, float (&out)[N]) {
    using P = Pack<typename A::T, N>;
    if constexpr (sizeof(P) % 4 != 0) {
        load_f32<A, N>(p, out);
    } else {
        constexpr int W = sizeof(P) / 4;
        uint32_t w[W];
        const uint32_t *src = reinterpret_cast<const uint32_t *>(p);
#pragma unroll
        for (int i = 0; i < W; ++i) w[i] = __builtin_nontemporal_load(src + i);
        P pk;
        memcpy(&pk, w, sizeof(P));
#pragma unroll
        for (int i = 0; i < N; ++i) out[i] = A::load(pk.v[i]);
    }
}

// Raw N-element packs with non-temporal access (N * sizeof(T) a multiple of 4).
template <typename T, int N>
__device__ __forceinline__ Pack<T, N> load_pack_nt(const T *p) {
    using P = Pack<T, N>;
    constexpr int W = sizeof(P) / 4;
    uint32_t w[W];
    const uint32_t *src = reinterpret_cast<const uint32_t *>(p);
#pragma unroll
    for (int i = 0; i < W; ++i) w[i] = __builtin_nontemporal_load(src + i);
    P pk;
    memcpy(&pk, w, sizeof(P));
    return pk;
}

// Raw N-element packs with the default cache policy.
template <typename T, int N>
__device__ __forceinline__ Pack<T, N> load_pack(const T *p) {
    return *reinterpret_cast<const Pack<T, N> *>(p);
}

template <typename T, int N>
__device__ __forceinline__ void store_pack_nt(T *p, const Pack<T, N> &pk) {
    constexpr int W = sizeof(Pack<T, N>) / 4;
    uint32_t w[W];
    memcpy(w, &pk, sizeof(w));
    uint32_t *dst = reinterpret_cast<uint32_t *>(p);
#pragma unroll
    for (int i = 0; i < W; ++i) __builtin_nontemporal_store(w[i], dst + i);
}

template <typename A, int N>
__device__ __forceinline__ void store_f32_nt(typename A::T *p, const float (&in)[N]) {
    using P = Pack<typename A::T, N>;
    if constexpr (sizeof(P) % 4 != 0) {
        store_f32<A, N>(p, in);
    } else {
        constexpr int W = sizeof(P) / 4;
        P pk;
#pragma unroll
        for (int i = 0; i < N; ++i) pk.v[i] = A::store(in[i]);
        uint32_t w[W];
        memcpy(w, &pk, sizeof(P));
        uint32_t *dst = reinterpret_cast<uint32_t *>(p);
#pragma unroll
        for (int i = 0; i < W; ++i) __builtin_nontemporal_store(w[i], dst + i);
    }
}

// ---------------------------------------------------------------------------
// Reductions.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
    return v;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
        uint64_t o = __shfl_xor(v, off, kWave);
        v = o > v ? o : v;
    }
    return v;
}

// ---- DPP row permutes: intra-row data movement at VALU latency -------------
// dpp_ctrl encodings (GCN/CDNA DPP): quad_perm [1,0,3,2] = 0xB1 (lane ^ 1),
// quad_perm [2,3,0,1] = 0x4E (lane ^ 2), row_half_mirror = 0x141 (i <-> 7-i in
// each half-row of 8), row_mirror = 0x140 (i <-> 15-i in each row of 16),
// row_shr:1 = 0x111 (lane i reads lane i-1 of its row).
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __uint_as_float(dpp_u32<CTRL>(__float_as_uint(v)));
}
template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
    return ((uint64_t)dpp_u32<CTRL>((uint32_t)(v >> 32)) << 32) | dpp_u32<CTRL>((uint32_t)v);
}

// Max over aligned groups of G lanes (G = 1, 2, 4, 8 or 16); every lane of the
// group gets the result.  Mirrors pair up halves, then quad xor 2 and xor 1.
template <int G>
__device__ __forceinline__ float group_max_f32(float v) {
    static_assert(G == 1 || G == 2 || G == 4 || G == 8 || G == 16, "group size");
    if constexpr (G >= 16) v = fmaxf(v, dpp_f32<0x140>(v));
    if constexpr (G >= 8) v = fmaxf(v, dpp_f32<0x141>(v));
    if constexpr (G >= 4) v = fmaxf(v, dpp_f32<0x4E>(v));
    if constexpr (G >= 2) v = fmaxf(v, dpp_f32<0xB1>(v));
    return v;
}
template <int G>
__device__ __forceinline__ uint64_t group_max_u64(uint64_t v) {
    static_assert(G == 1 || G == 2 || G == 4 || G == 8 || G == 16, "group size");
    if constexpr (G >= 16) { const uint64_t o = dpp_u64<0x140>(v); v = o > v ? o : v; }
    if constexpr (G >= 8) { const uint64_t o = dpp_u64<0x141>(v); v = o > v ? o : v; }
    if constexpr (G >= 4) { const uint64_t o = dpp_u64<0x4E>(v); v = o > v ? o : v; }
    if constexpr (G >= 2) { const uint64_t o = dpp_u64<0xB1>(v); v = o > v ? o : v; }
    return v;
}

template <int G>
__device__ __forceinline__ uint32_t dpp_max_group(uint32_t v) {
    static_assert(G == 1 || G == 2 || G == 4 || G == 8 || G == 16, "group size");
    if constexpr (G >= 16) { const uint32_t o = dpp_u32<0x140>(v); v = o > v ? o : v; }
    if constexpr (G >= 8) { const uint32_t o = dpp_u32<0x141>(v); v = o > v ? o : v; }
    if constexpr (G >= 4) { const uint32_t o = dpp_u32<0x4E>(v); v = o > v ? o : v; }
    if constexpr (G >= 2) { const uint32_t o = dpp_u32<0xB1>(v); v = o > v ? o : v; }
    return v;
}

// Block-wide f32 sum; every thread gets the result.  `scratch` holds one
// float per wave.  Contains __syncthreads, so all threads must call it.
template <int BLOCK>
__device__ __forceinline__ float block_sum(float v, float *scratch) {
    constexpr int NW = BLOCK / kWave;
    v = wave_sum(v);
    if constexpr (NW == 1) {
        return v;
    } else {
        const int lane = threadIdx.x % kWave, wid = threadIdx.x / kWave;
        if (lane == 0) scratch[wid] = v;
        __syncthreads();
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < NW; ++i) t += scratch[i];
        __syncthreads();
        return t;
    }
}

// ---------------------------------------------------------------------------
// expf, bit-exact with glibc >= 2.27 on x86_64 (the libm that Rust's f32::exp
// calls on linux-gnu).  Algorithm: Szabolcs Nagy's expf from ARM
// optimized-routines (MIT), as shipped in glibc: x*32/ln2 = k + r,
// exp(x) = 2^(k/32) * p(r), p cubic, all in double, one final rounding.
// The x86_64 build contracts r = x*InvLn2N - kd and the Horner steps into FMA;
// this restatement does the same.  Table: tab[i] = bits(2^(i/32)) - (i << 47).
// Checked on the GPU against the host's glibc expf for all 2^32 inputs.
// ---------------------------------------------------------------------------
struct ExpfTable {
    uint64_t tab[32];
};

__host__ __device__ constexpr ExpfTable make_expf_table() {
    // 2^(i/32) rounded to double; verified against exp2l at build-test time.
    return ExpfTable{{0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full,
                      0x3fef9301d0125b51ull, 0x3fef72b83c7d517bull, 0x3fef54873168b9aaull,
                      0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, 0x3fef06fe0a31b715ull,
                      0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
                      0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull,
                      0x3feea47eb03a5585ull, 0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull,
                      0x3feea11473eb0187ull, 0x3feea589994cce13ull, 0x3feeace5422aa0dbull,
                      0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
                      0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull,
                      0x3fef3720dcef9069ull, 0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full,
                      0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull}};
}

__device__ __forceinline__ float expf_glibc(float x, const uint64_t *tab) {
    const uint32_t ux = __float_as_uint(x);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {  // |x| >= 88 or NaN/Inf
        if (ux == 0xff800000u) return 0.0f;          // -inf
        if (abstop >= 0x7f8u) return x + x;           // +inf or NaN
        if (x > 0x1.62e42ep6f) return __uint_as_float(0x7f800000u);  // overflow
        if (x < -0x1.9fe368p6f) return 0.0f;          // underflow
    }
    const double InvLn2N = 0x1.71547652b82fep+0 * 32.0;
    const double C0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double C1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double C2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x;
    const double z = InvLn2N * xd;
    // glibc rounds z to the nearest integer with the add/subtract-0x1.8p52
    // trick; |z| < 2^13 here, so rint gives the identical kd in one op.
    const double kd = __builtin_rint(z);
    const int32_t ki = (int32_t)kd;
    const double r = __fma_rn(InvLn2N, xd, -kd);
    uint64_t t = tab[ki & 31];
    t += (uint64_t)(int64_t)ki << 47;
    const double s = __longlong_as_double((long long)t);
    const double zz = __fma_rn(C0, r, C1);
    const double r2 = __dmul_rn(r, r);
    double y = __fma_rn(C2, r, 1.0);
    y = __fma_rn(zz, r2, y);
    y = __dmul_rn(y, s);
    return (float)y;
}

// expf_glibc without branches, for x <= 0 or NaN (softmax's exp(l - max)):
// the main path runs on x raised to glibc's underflow bound, and the cases
// glibc treats apart (x below that bound, -inf: 0; NaN: x + x) are selected
// afterwards.  On this domain glibc's own special cases are exactly these,
// and every other input takes the same main path, so the results are
// identical (checked on every non-positive and NaN input).
__device__ __forceinline__ float expf_glibc_nonpos(float x, const uint64_t *tab) {
    const float lo = -0x1.9fe368p6f;
    const float xc = x < lo ? lo : (x != x ? 0.0f : x);
    const double InvLn2N = 0x1.71547652b82fep+0 * 32.0;
    const double C0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double C1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double C2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)xc;
    const double z = InvLn2N * xd;
    const double kd = __builtin_rint(z);
    const int32_t ki = (int32_t)kd;
    const double r = __fma_rn(InvLn2N, xd, -kd);
    uint64_t t = tab[ki & 31];
    t += (uint64_t)(int64_t)ki << 47;
    const double sc = __longlong_as_double((long long)t);
    const double zz = __fma_rn(C0, r, C1);
    const double r2 = __dmul_rn(r, r);
    double y = __fma_rn(C2, r, 1.0);
    y = __fma_rn(zz, r2, y);
    y = __dmul_rn(y, sc);
    const float res = (float)y;
    return x < lo ? 0.0f : (x != x ? x + x : res);
}

// ---------------------------------------------------------------------------
// sinf / cosf, bit-exact with glibc >= 2.28 on x86_64 (Rust's f32::sin_cos on
// linux-gnu calls these; kernels/rope.rs:46-58 rotates with them).  Algorithm:
// Szabolcs Nagy's sinf/cosf from ARM optimized-routines (MIT), as glibc ships
// it.  All arithmetic in double, one final rounding:
//  * |x| < pi/4: odd polynomial (sin) or even polynomial (cos) in x directly;
//  * |x| < 120: n = nearest integer to x * 2/pi (taken from the top bits of
//    x * 2^24 * 2/pi), r = x - n * pi/2 with one FMA;
//  * larger: Payne-Hanek reduction with 96 bits of 4/pi picked by exponent
//    (kInvPio4 below), r = (fraction in 2^62 units) * pi/2^62;
//  * quadrant n selects sin or cos polynomial, its sign and whether the cos
//    coefficients are negated.
// glibc's x86_64 FMA variant (chosen at load time on FMA hosts) contracts the
// Horner steps and r = x - n*pi/2 into FMAs; this restatement does the same.
// kInvPio4[i] = floor((4/pi) * 2^(8i+7)) mod 2^32, i.e. 32-bit windows of the
// binary expansion of 4/pi stepping 8 bits (recomputed from an integer pi in
// the CPU test suite).  The polynomial coefficients are the published ones of
// that source.  Checked against the host's glibc on all 2^32 inputs.
// ---------------------------------------------------------------------------
__device__ __constant__ inline constexpr uint32_t kInvPio4[24] = {
    0xa2u,       0xa2f9u,     0xa2f983u,   0xa2f9836eu, 0xf9836e4eu, 0x836e4e44u, 0x6e4e4415u, 0x4e441529u,
    0x441529fcu, 0x1529fc27u, 0x29fc2757u, 0xfc2757d1u, 0x2757d1f5u, 0x57d1f534u, 0xd1f534ddu, 0xf534ddc0u,
    0x34ddc0dbu, 0xddc0db62u, 0xc0db6295u, 0xdb629599u, 0x6295993cu, 0x95993c43u, 0x993c4390u, 0x3c439041u};

// One of the two polynomials of the optimized-routines sinf/cosf on the
// reduced argument x (x2 = x*x).  odd: sin polynomial; else cos polynomial,
// whose coefficients are negated when neg_cos (quadrants 2 and 3).
__device__ __forceinline__ float sincosf_poly(double x, double x2, bool odd, bool neg_cos) {
    if (odd) {
        const double S1 = -0x1.555545995a603p-3, S2 = 0x1.1107605230bc4p-7, S3 = -0x1.994eb3774cf24p-13;
        const double x3 = __dmul_rn(x, x2);
        const double s1 = __fma_rn(x2, S3, S2);
        const double x7 = __dmul_rn(x3, x2);
        const double s = __fma_rn(x3, S1, x);
        return (float)__fma_rn(x7, s1, s);
    }
    const double g = neg_cos ? -1.0 : 1.0;  // exact sign flip of every coefficient
    const double C0 = g * 0x1p0, C1 = g * -0x1.ffffffd0c621cp-2, C2 = g * 0x1.55553e1068f19p-5,
                 C3 = g * -0x1.6c087e89a359dp-10, C4 = g * 0x1.99343027bf8c3p-16;
    const double x4 = __dmul_rn(x2, x2);
    const double c2 = __fma_rn(x2, C4, C3);
    const double c1 = __fma_rn(x2, C1, C0);
    const double x6 = __dmul_rn(x4, x2);
    const double c = __fma_rn(x4, C2, c1);
    return (float)__fma_rn(x6, c2, c);
}

__device__ __forceinline__ void sincosf_glibc(float y, float *sp, float *cp) {
    const uint32_t xi = __float_as_uint(y);
    const uint32_t top = (xi >> 20) & 0x7ffu;
    double x = (double)y;
    if (top < 0x3f4u) {      // |y| < pi/4 (abstop12 of 0x1.921FB6p-1f)
        if (top < 0x398u) {  // |y| < 2^-12
            *sp = y;
            *cp = 1.0f;
            return;
        }
        const double x2 = __dmul_rn(x, x);
        *sp = sincosf_poly(x, x2, true, false);
        *cp = sincosf_poly(x, x2, false, false);
        return;
    }
    if (top >= 0x7f8u) {  // inf or NaN
        *sp = *cp = y - y;
        return;
    }
    int n, q;  // n: polynomial parity; q: quadrant of the signs and coefficient set
    if (top < 0x42fu) {  // |y| < 120
        const double r = __dmul_rn(x, 0x1.45F306DC9C883p+23);
        n = ((int32_t)r + 0x800000) >> 24;
        x = __fma_rn(-(double)n, 0x1.921FB54442D18p0, x);
        q = n & 3;
    } else {
        const uint32_t *arr = &kInvPio4[(xi >> 26) & 15];
        const int shift = (xi >> 23) & 7;
        const uint32_t m = ((xi & 0xffffffu) | 0x800000u) << shift;
        uint64_t r0 = (uint64_t)(uint32_t)(m * arr[0]);
        const uint64_t r1 = (uint64_t)m * arr[4];
        const uint64_t r2 = (uint64_t)m * arr[8];
        r0 = (r2 >> 32) | (r0 << 32);
        r0 += r1;
        const uint64_t nn = (r0 + (1ull << 61)) >> 62;
        r0 -= nn << 62;
        x = __dmul_rn((double)(int64_t)r0, 0x1.921FB54442D18p-62);
        n = (int)nn;
        q = (n + (int)(xi >> 31)) & 3;  // the reduction took |y|: its sign joins the quadrant
    }
    const double s = (q == 1 || q == 2) ? -1.0 : 1.0;
    const double xs = __dmul_rn(x, s), x2 = __dmul_rn(x, x);
    const bool neg = (q & 2) != 0;
    // Quadrant parity swaps the roles of the two polynomials.
    *sp = sincosf_poly(xs, x2, (n & 1) == 0, neg);
    *cp = sincosf_poly(xs, x2, (n & 1) != 0, neg);
}

// ---------------------------------------------------------------------------
// logf, bit-exact with glibc >= 2.28 on x86_64 (Rust's f32::ln on linux-gnu;
// the router's sqrt-softplus gating, kernels/moe.rs:68-77, takes it).
// Algorithm: Szabolcs Nagy's logf from ARM optimized-routines (MIT), as glibc
// ships it: x = 2^k z with z in [0x1.66p-1, 0x1.66p0) (the bits minus 0x3f330000
// pick k and one of 16 subintervals), log(x) = k ln2 + log(c) + log1p(z/c - 1)
// with a cubic for log1p, all in double, one final rounding.  The 16 (1/c,
// log c) pairs and the cubic's coefficients are the published ones; glibc's
// x86_64 FMA variant contracts r = z/c - 1, k ln2 + log c and the Horner
// steps into FMAs, as below.  Checked against the host's glibc on all 2^32
// inputs.
// ---------------------------------------------------------------------------
__device__ __constant__ inline constexpr double kLogfTab[16][2] = {
    {0x1.661ec79f8f3bep+0, -0x1.57bf7808caadep-2}, {0x1.571ed4aaf883dp+0, -0x1.2bef0a7c06ddbp-2},
    {0x1.49539f0f010bp+0, -0x1.01eae7f513a67p-2},  {0x1.3c995b0b80385p+0, -0x1.b31d8a68224e9p-3},
    {0x1.30d190c8864a5p+0, -0x1.6574f0ac07758p-3}, {0x1.25e227b0b8eap+0, -0x1.1aa2bc79c81p-3},
    {0x1.1bb4a4a1a343fp+0, -0x1.a4e76ce8c0e5ep-4}, {0x1.12358f08ae5bap+0, -0x1.1973c5a611cccp-4},
    {0x1.0953f419900a7p+0, -0x1.252f438e10c1ep-5}, {0x1p+0, 0x0p+0},
    {0x1.e608cfd9a47acp-1, 0x1.aa5aa5df25984p-5},  {0x1.ca4b31f026aap-1, 0x1.c5e53aa362eb4p-4},
    {0x1.b2036576afce6p-1, 0x1.526e57720db08p-3},  {0x1.9c2d163a1aa2dp-1, 0x1.bc2860d22477p-3},
    {0x1.886e6037841edp-1, 0x1.1058bc8a07ee1p-2},  {0x1.767dcf5534862p-1, 0x1.4043057b6ee09p-2}};

__device__ __forceinline__ float logf_glibc(float x) {
    uint32_t ix = __float_as_uint(x);
    if (ix == 0x3f800000u) return 0.0f;
    if (ix - 0x00800000u >= 0x7f800000u - 0x00800000u) {
        if (ix * 2 == 0) return -__builtin_inff();             // log(+-0) = -inf
        if (ix == 0x7f800000u) return x;                       // log(inf) = inf
        if ((ix & 0x80000000u) || ix * 2 >= 0xff000000u) return __builtin_nanf("");  // x < 0 or NaN
        ix = __float_as_uint(x * 0x1p23f) - (23u << 23);       // subnormal: normalise
    }
    const uint32_t tmp = ix - 0x3f330000u;
    const uint32_t i = (tmp >> (23 - 4)) % 16;
    const int32_t k = (int32_t)tmp >> 23;
    const uint32_t iz = ix - (tmp & 0xff800000u);
    const double invc = kLogfTab[i][0], logc = kLogfTab[i][1];
    const double z = (double)__uint_as_float(iz);
    const double A0 = -0x1.00ea348b88334p-2, A1 = 0x1.5575b0be00b6ap-2, A2 = -0x1.ffffef20a4123p-2;
    const double Ln2 = 0x1.62e42fefa39efp-1;
    const double r = __fma_rn(z, invc, -1.0);
    const double y0 = __fma_rn((double)k, Ln2, logc);
    const double r2 = __dmul_rn(r, r);
    double y = __fma_rn(A1, r, A2);
    y = __fma_rn(A0, r2, y);
    y = __fma_rn(y, r2, __dadd_rn(y0, r));
    return (float)y;
}

// Correctly rounded f32 square root (IEEE sqrtf, what f32::sqrt gives).  The
// hardware square root is an approximation; the seed is moved to the
// neighbour on the other side of a rounding midpoint while one exists.  A
// midpoint m of two adjacent floats has 25 significant bits, so m*m is exact
// in double and the comparison with x decides the rounding exactly (x never
// equals m*m: a 25-bit odd significand squared has bit 50 set).  Checked
// against the host's sqrtf on every positive f32 from seeds up to 2 ulps off.
__device__ __forceinline__ float sqrtf_rn(float x) {
    if (!(x > 0.0f) || x == __builtin_inff()) return __builtin_sqrtf(x);  // +-0, negative, NaN, inf
    float s = __builtin_sqrtf(x);
    const double dx = (double)x;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const float up = __uint_as_float(__float_as_uint(s) + 1u), dn = __uint_as_float(__float_as_uint(s) - 1u);
        const double hu = __dmul_rn(__dadd_rn((double)s, (double)up), 0.5);
        const double hd = __dmul_rn(__dadd_rn((double)s, (double)dn), 0.5);
        if (dx > __dmul_rn(hu, hu))
            s = up;
        else if (dx < __dmul_rn(hd, hd))
            s = dn;
        else
            break;
    }
    return s;
}

// get_scale_min_k4 (dequant.rs:295-305): 6-bit scale and min j (0..7) of a
// Q4_K/Q5_K block from its 12 scale bytes held as 3 little-endian dwords.
__device__ __forceinline__ void k4_scale_min(uint32_t j, uint32_t s0, uint32_t s1, uint32_t s2, uint32_t &sc,
                                             uint32_t &m) {
    if (j < 4) {
        sc = (s0 >> (8 * j)) & 63u;
        m = (s1 >> (8 * j)) & 63u;
    } else {
        const uint32_t k = 8 * (j - 4);
        const uint32_t b_hi = (s2 >> k) & 0xffu;                // q[j + 4]
        sc = (b_hi & 0x0fu) | (((s0 >> k) & 0xffu) >> 6) << 4;  // q[j - 4] >> 6
        m = (b_hi >> 4) | (((s1 >> k) & 0xffu) >> 6) << 4;      // q[j] >> 6
    }
}

// silu(g) = g / (1 + exp(-g)) as swiglu.rs:5-7 computes it in f32.
// g / d for d = 1 + exp(-g) >= 1: hardware reciprocal, one Newton step on the
// reciprocal, one residual correction of the quotient (Markstein's sequence).
// Inputs outside [2^-100, 2^126) take the IEEE division.  Proven equal to the
// IEEE quotient for this use by comparing silu(g) for all 2^32 values of g.
__device__ __forceinline__ float silu_div(float g, float d) {
    const float ag = __builtin_fabsf(g);
    if (!(ag >= 0x1p-100f && ag < 0x1p+126f && d < 0x1p+126f)) return g / d;
    const float y0 = __builtin_amdgcn_rcpf(d);
    const float e0 = __builtin_fmaf(-d, y0, 1.0f);
    const float y1 = __builtin_fmaf(e0, y0, y0);
    const float q0 = g * y1;
    const float r0 = __builtin_fmaf(-d, q0, g);
    return __builtin_fmaf(r0, y1, q0);
}

__device__ __forceinline__ float silu(float g, const uint64_t *tab) {
    return silu_div(g, 1.0f + expf_glibc(-g, tab));
}

// Fast silu for outputs rounded to 16 bits.  exp(-g) comes from the hardware
// exp2 after a two-constant reduction by ln 2 (ln 2 = kLn2Hi + kLn2Lo), and
// the division is one hardware reciprocal and a multiply.  On the fast domain
// 2^-100 <= |g| < 64 its bit distance to silu() (same sign, normal results)
// is at most kSiluFastDist; fellm_rocm_silu_fast_bound measures the largest
// distance over every f32 g in the domain.
constexpr uint32_t kSiluFastDist = FELLM_SILU_FAST_DIST;

__device__ __forceinline__ bool silu_fast_domain(float g) {
    const float ag = __builtin_fabsf(g);
    return ag >= 0x1p-100f && ag < 64.0f;
}

__device__ __forceinline__ float silu_fast(float g) {
#if FELLM_SILU_EXP_DIRECT
    // -g log2(e) as an unevaluated sum xh + xl (log2 e = kL2eHi + kL2eLo,
    // the product's rounding error recovered by an FMA); the hardware exp2
    // takes xh whole and the first-order factor 1 + xl ln 2 carries xl.
    constexpr float kL2eHi = 0x1.715476p+0f, kL2eLo = 0x1.4ae0c0p-26f, kLn2 = 0x1.62e430p-1f;
    const float xh = -g * kL2eHi;
    const float xl = __builtin_fmaf(-g, kL2eLo, __builtin_fmaf(-g, kL2eHi, -xh));
    const float e0 = __builtin_amdgcn_exp2f(xh);
    const float e = __builtin_fmaf(e0, xl * kLn2, e0);
    const float d = 1.0f + e;
    const float y0 = __builtin_amdgcn_rcpf(d);
    if constexpr (FELLM_SILU_DIV_STEPS == 0) return g * y0;
    const float y1 = __builtin_fmaf(__builtin_fmaf(-d, y0, 1.0f), y0, y0);
    const float q0 = g * y1;
    if constexpr (FELLM_SILU_DIV_STEPS == 1) return q0;
    return __builtin_fmaf(__builtin_fmaf(-d, q0, g), y1, q0);
#else
    constexpr float kLog2e = 0x1.715476p+0f;
    constexpr float kLn2Hi = 0x1.62e430p-1f;   // ln 2 rounded up to 24 bits
    constexpr float kLn2Lo = -0x1.05c610p-29f;  // ln 2 - kLn2Hi
    const float t = -g;
    const float n = __builtin_rintf(t * kLog2e);
    float r = __builtin_fmaf(n, -kLn2Hi, t);
    r = __builtin_fmaf(n, -kLn2Lo, r);
    const float e = __builtin_ldexpf(__builtin_amdgcn_exp2f(r * kLog2e), (int)n);
    return g * __builtin_amdgcn_rcpf(1.0f + e);
#endif
}

// out = O::store(RN(silu(g) * u)) without evaluating the exact silu when the
// answer is already fixed: the exact f32 silu s lies within kSiluFastDist
// steps of the fast value in bit order, hence in [sa, sb]; RN(s * u) then lies
// between RN(sa * u) and RN(sb * u) (rounding and multiplication by u are
// monotone), and so does its 16-bit rounding, which therefore equals O::store
// of either end when those agree.  Returns false (out unset) otherwise, and
// outside the fast domain.
// Two f32 values rounded to nearest-even f16 by one v_cvt_pk_f16_f32 (a in
// the low half); equal to the scalar conversion of F16::store for every f32,
// NaNs included (checked exhaustively on the device).
__device__ __forceinline__ uint32_t f16_pack_bits(float a, float b) {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    __asm__("" : "+v"(a), "+v"(b));  // keep the f32 roundings (see F16::store)
    const f32x2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
}
__device__ __forceinline__ uint32_t bf16_pack_bits(float a, float b) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    const f32x2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// N f32 values (N even) rounded to the 16-bit type A as N/2 packed words,
// element 2i in the low half of word i.  f16: the packed conversion, equal
// to F16::store for every input.  bf16: the packed conversion when the lane
// holds no NaN (equal to BF16::store for every non-NaN f32), else BF16::store
// per element (a NaN keeps its top payload bits, quiet bit set): one compare
// per element instead of BF16::store's per-element NaN select.
template <typename A, int N>
__device__ __forceinline__ void round_words(const float (&v)[N], uint32_t (&w)[N / 2]) {
    static_assert(N % 2 == 0, "pairs");
    if constexpr (std::is_same_v<A, F16>) {
#pragma unroll
        for (int i = 0; i < N; i += 2) w[i / 2] = f16_pack_bits(v[i], v[i + 1]);
    } else {
        static_assert(std::is_base_of_v<BF16, A>, "16-bit types");
        bool nan = false;
#pragma unroll
        for (int i = 0; i < N; i += 2) {
            nan |= (v[i] != v[i]) | (v[i + 1] != v[i + 1]);
            w[i / 2] = bf16_pack_bits(v[i], v[i + 1]);
        }
        if (nan) {
#pragma unroll
            for (int i = 0; i < N; i += 2)
                w[i / 2] = (uint32_t)BF16::store(v[i]) | (uint32_t)BF16::store(v[i + 1]) << 16;
        }
    }
}
template <int N>
__device__ __forceinline__ void bf16_round_words(const float (&v)[N], uint32_t (&w)[N / 2]) {
    round_words<BF16, N>(v, w);
}

// W packed words stored at dst, as 16-byte (or 8-byte) vectors (dst aligned
// to the vector size), or with WORD_NT non-temporal stores word by word.
// Which non-temporal form is faster depends on the kernel: the prefill RoPE
// walk measured 55.0 against 55.9 us with word stores, the
// one-launch decode step 15.8 against 16.2 us with vector stores.
template <int W, bool WORD_NT = false>
__device__ __forceinline__ void store_words(uint32_t *dst, const uint32_t (&w)[W], bool nt) {
    typedef uint32_t v4 __attribute__((ext_vector_type(4)));
    typedef uint32_t v2 __attribute__((ext_vector_type(2)));
    if (WORD_NT && nt) {
#pragma unroll
        for (int i = 0; i < W; ++i) __builtin_nontemporal_store(w[i], dst + i);
    } else if constexpr (W % 4 == 0) {
#pragma unroll
        for (int i = 0; i < W; i += 4) {
            const v4 x = {w[i], w[i + 1], w[i + 2], w[i + 3]};
            v4 *d = reinterpret_cast<v4 *>(dst + i);
            if (nt)
                __builtin_nontemporal_store(x, d);
            else
                *d = x;
        }
    } else if constexpr (W % 2 == 0) {
#pragma unroll
        for (int i = 0; i < W; i += 2) {
            const v2 x = {w[i], w[i + 1]};
            v2 *d = reinterpret_cast<v2 *>(dst + i);
            if (nt)
                __builtin_nontemporal_store(x, d);
            else
                *d = x;
        }
    } else {
#pragma unroll
        for (int i = 0; i < W; ++i) {
            if (nt)
                __builtin_nontemporal_store(w[i], dst + i);
            else
                dst[i] = w[i];
        }
    }
}

// 16-bit outputs (F16, BF16, BF16HW): with u not NaN neither end product is NaN (s
// is finite and nonzero on the fast domain), so both ends are rounded by one
// packed conversion (v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32), which equals
// the output type's rounding for every non-NaN f32; a NaN u takes the exact
// path.
template <typename O>
__device__ __forceinline__ bool silu_mul_fast(float g, float u, typename O::T &out) {
    static_assert(sizeof(typename O::T) == 2, "the interval test needs a 16-bit output");
    constexpr bool kBf = std::is_base_of_v<BF16, O>, kF16 = std::is_same_v<O, F16>;
    if constexpr ((kBf || kF16) && FELLM_SILU_PK && FELLM_SILU_BRANCHLESS) {
        // Straight-line code: outside the domain the fast value is computed
        // and discarded.  With the reduction by ln 2, med3 keeps the
        // exponent's integer conversion in range for any g; inside the domain
        // it changes nothing.
        // f16: a NaN u gives both ends u's NaN, quieted, which the packed
        // conversion rounds as F16::store does (equal for every input), and
        // the exact path's product is that same NaN: no NaN test needed.
        const bool ok = silu_fast_domain(g) && (kF16 || u == u);
        const float gc = FELLM_SILU_EXP_DIRECT ? g : __builtin_amdgcn_fmed3f(g, -64.0f, 64.0f);
        const uint32_t b = __float_as_uint(silu_fast(gc));
        float lo = __uint_as_float(b - kSiluFastDist) * u, hi = __uint_as_float(b + kSiluFastDist) * u;
        __asm__("" : "+v"(lo), "+v"(hi));
        const uint32_t r = kBf ? bf16_pack_bits(lo, hi) : f16_pack_bits(lo, hi);
        out = __builtin_bit_cast(typename O::T, (uint16_t)(r & 0xffffu));
        return ok && (r & 0xffffu) == (r >> 16);
    } else if constexpr ((kBf || kF16) && FELLM_SILU_PK) {
        if (!silu_fast_domain(g) || u != u) return false;
        const uint32_t b = __float_as_uint(silu_fast(g));
        float lo = __uint_as_float(b - kSiluFastDist) * u, hi = __uint_as_float(b + kSiluFastDist) * u;
        // Pin the f32 products (see F16::store): a mixed-precision FMA would
        // round the exact product straight to 16 bits.
        __asm__("" : "+v"(lo), "+v"(hi));
        const uint32_t r = kBf ? bf16_pack_bits(lo, hi) : f16_pack_bits(lo, hi);
        out = __builtin_bit_cast(typename O::T, (uint16_t)(r & 0xffffu));
        return (r & 0xffffu) == (r >> 16);
    } else {
        if (!silu_fast_domain(g)) return false;
        const uint32_t b = __float_as_uint(silu_fast(g));
        const typename O::T lo = O::store(__uint_as_float(b - kSiluFastDist) * u);
        const typename O::T hi = O::store(__uint_as_float(b + kSiluFastDist) * u);
        out = lo;
        return __builtin_bit_cast(uint16_t, lo) == __builtin_bit_cast(uint16_t, hi);
    }
}

// Copies the 32-entry table into LDS once per block; returns the LDS pointer.
// Contains __syncthreads.
__device__ __forceinline__ const uint64_t *stage_expf_table(uint64_t *lds) {
    constexpr ExpfTable T = make_expf_table();
    if (threadIdx.x < 32) lds[threadIdx.x] = T.tab[threadIdx.x];
    __syncthreads();
    return lds;
}

// ---------------------------------------------------------------------------
// Host helpers.
// ---------------------------------------------------------------------------
// Kernel timing for measurement.  fellm_rocm_timing_arm(start, stop) arms the
// calling thread: until fellm_rocm_timing_disarm(), the first kernel this
// library launches records `start` at its beginning and every kernel records
// `stop` at its end (hipExtLaunchKernel attaches the events to the kernel
// itself, so no marker packet runs between kernels).  The elapsed time of
// the pair is then the device time of the op's kernels, as a profiler's
// kernel trace reports it.  Unarmed launches are plain hipLaunchKernelGGL.
struct LaunchTiming {
    hipEvent_t start = nullptr, stop = nullptr;
    bool armed = false, started = false;
};
inline thread_local LaunchTiming g_launch_timing;

#define FELLM_LAUNCH(kernel, grid, block, lds, stream, ...)                                                   \
    do {                                                                                                     \
        ::fellm::LaunchTiming &lt_ = ::fellm::g_launch_timing;                                               \
        if (lt_.armed) {                                                                                     \
            hipExtLaunchKernelGGL(kernel, grid, block, lds, stream, lt_.started ? nullptr : lt_.start, lt_.stop, \
                                  0, __VA_ARGS__);                                                           \
            lt_.started = true;                                                                              \
        } else {                                                                                             \
            hipLaunchKernelGGL(kernel, grid, block, lds, stream, __VA_ARGS__);                               \
        }                                                                                                    \
    } while (0)

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

inline int launch_status() {
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? FELLM_OK : FELLM_ERR_LAUNCH;
}

inline bool aligned_to(const void *p, size_t a) {
    return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

}  // namespace fellm
