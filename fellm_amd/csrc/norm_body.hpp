// Device body of the residual add + RMSNorm row kernel (norm.hip), shared with
// the fused decode-step launch (rope.hip).
//
// Reference semantics: Add (crates/backend-cpu/src/kernels/simd_f32.rs:175-197)
// then RmsNorm (crates/backend-cpu/src/kernels/norm.rs:6-53, launcher
// crates/backend-cpu/src/backend.rs:1104-1133): per row of `group` elements,
// sumsq = sum(h^2), scale = 1 / sqrt(sumsq / group + eps), y = (h * scale) * w.
#pragma once

#include <type_traits>

#include "common.hpp"

#ifndef FELLM_NORM_W_EARLY
#define FELLM_NORM_W_EARLY 1
#endif

namespace fellm {

// x and residual are read once with non-temporal loads, and h and y are
// written with non-temporal stores.  For the many-row (prefill) layout
// regular stores make this kernel alone faster (26.7 vs 28.4 us at
// 4096 x 4096 f16) but leave 67 MB of dirty lines that the next kernel pays
// to write back; judged on a whole chain the non-temporal stores win
// (embedding -> add+RMSNorm -> RoPE -> SwiGLU at T 4096: 123.0 -> 116.4 us).
template <typename A, int N>
__device__ __forceinline__ void norm_load(const typename A::T *p, float (&v)[N]) {
    load_f32_nt<A, N>(p, v);
}
// Build knob: 16-bit rows rounded by the packed hardware conversions
// (round_words) (1), or element by element (0).
#ifndef FELLM_NORM_BF16_PK
#define FELLM_NORM_BF16_PK 1
#endif
// Build knob: non-temporal stores of the packed rows word by word (1) or as
// 16-byte vectors (0).
#ifndef FELLM_NORM_WORD_NT
#define FELLM_NORM_WORD_NT 0
#endif
template <typename A>
constexpr bool kNormPk = FELLM_NORM_BF16_PK && (std::is_base_of_v<BF16, A> || std::is_same_v<A, F16>);

template <typename A, int N, bool NT>
__device__ __forceinline__ void norm_store(typename A::T *p, const float (&v)[N]) {
    if constexpr (kNormPk<A> && N % 2 == 0) {
        uint32_t w[N / 2];
        round_words<A, N>(v, w);
        store_words<N / 2, FELLM_NORM_WORD_NT != 0>(reinterpret_cast<uint32_t *>(p), w, NT);
    } else {
        if constexpr (NT) store_f32_nt<A, N>(p, v); else store_f32<A, N>(p, v);
    }
}
// h = x + r rounded to the activation type, in place, for VEC values; with
// STORE the rounded values are also stored (non-temporally) at p.
template <typename A, int N, bool STORE>
__device__ __forceinline__ void norm_add_round(float (&v)[N], const float (&r)[N], typename A::T *p) {
    if constexpr (kNormPk<A> && N % 2 == 0) {
        float s[N];
#pragma unroll
        for (int i = 0; i < N; ++i) s[i] = v[i] + r[i];
        uint32_t w[N / 2];
        round_words<A, N>(s, w);
#pragma unroll
        for (int i = 0; i < N; i += 2) {
            v[i] = A::load(__builtin_bit_cast(typename A::T, (uint16_t)(w[i / 2] & 0xffffu)));
            v[i + 1] = A::load(__builtin_bit_cast(typename A::T, (uint16_t)(w[i / 2] >> 16)));
        }
        if constexpr (STORE) store_words<N / 2, FELLM_NORM_WORD_NT != 0>(reinterpret_cast<uint32_t *>(p), w, true);
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) v[i] = A::load(A::store(v[i] + r[i]));
        if constexpr (STORE) norm_store<A, N, true>(p, v);
    }
}
namespace {


// Row `row` of add + RMSNorm by one BLOCK-thread workgroup (every thread of
// the workgroup calls it; contains a barrier).  red: BLOCK / 64 floats of LDS.
template <typename A, typename O, int BLOCK, int VEC, int NCHUNK, bool ADD, bool STORE_H>
__device__ __forceinline__ void add_rmsnorm_row(
    // h may alias x or r (in-place residual update): no __restrict__ on them.
    const typename A::T *x, const typename A::T *r, typename A::T *h, const float *__restrict__ w,
    typename O::T *y, uint32_t group, float eps, size_t row, float *red) {
    const typename A::T *xr = x + row * group;
    float v[NCHUNK][VEC];
    float ss = 0.0f;
    // Every chunk's x and r are requested before the first h store: h may
    // alias x or r, so the compiler cannot move a later chunk's loads above
    // an earlier chunk's store by itself, which would expose one memory
    // latency per chunk.
    float rv[ADD ? NCHUNK : 1][VEC];
#pragma unroll
    for (int c = 0; c < NCHUNK; ++c) {
        const uint32_t base = (uint32_t)(c * BLOCK + threadIdx.x) * VEC;
        if (base < group) {
            norm_load<A, VEC>(xr + base, v[c]);
            if constexpr (ADD) norm_load<A, VEC>(r + row * group + base, rv[c]);
        }
    }
#pragma unroll
    for (int c = 0; c < NCHUNK; ++c) {
        const uint32_t base = (uint32_t)(c * BLOCK + threadIdx.x) * VEC;
        if (base < group) {
            if constexpr (ADD) {
                // h is stored in the activation dtype and normalised as stored.
                norm_add_round<A, VEC, STORE_H>(v[c], rv[c], STORE_H ? h + row * group + base : nullptr);
            }
#pragma unroll
            for (int i = 0; i < VEC; ++i) ss += v[c][i] * v[c][i];
        }
    }
    // The weights do not depend on the reduction: with FELLM_NORM_W_EARLY they
    // are requested before the barrier, so their (cache) latency overlaps it.
    float wv[NCHUNK][VEC];
    if constexpr (FELLM_NORM_W_EARLY) {
#pragma unroll
        for (int c = 0; c < NCHUNK; ++c) {
            const uint32_t base = (uint32_t)(c * BLOCK + threadIdx.x) * VEC;
            if (base < group) load_f32<F32, VEC>(w + base, wv[c]);
        }
    }
    ss = block_sum<BLOCK>(ss, red);
    const float scale = 1.0f / sqrtf(ss / (float)group + eps);
#pragma unroll
    for (int c = 0; c < NCHUNK; ++c) {
        const uint32_t base = (uint32_t)(c * BLOCK + threadIdx.x) * VEC;
        if (base < group) {
            float o[VEC];
            if constexpr (!FELLM_NORM_W_EARLY) load_f32<F32, VEC>(w + base, wv[c]);
#pragma unroll
            for (int i = 0; i < VEC; ++i) o[i] = (v[c][i] * scale) * wv[c][i];
            norm_store<O, VEC, true>(y + row * group + base, o);
        }
    }
}

}  // namespace
}  // namespace fellm
