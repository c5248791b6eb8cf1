// Device body of the residual add + RMSNorm row kernel (norm.hip), shared with
// the fused decode-step launch (rope.hip).
//
// Reference semantics: Add (crates/backend-cpu/src/kernels/simd_f32.rs:175-197)
// then RmsNorm (crates/backend-cpu/src/kernels/norm.rs:6-53, launcher
// crates/backend-cpu/src/backend.rs:1104-1133): per row of `group` elements,
// sumsq = sum(h^2), scale = 1 / sqrt(sumsq / group + eps), y = (h * scale) * w.
#pragma once

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
template <typename A, int N, bool NT>
__device__ __forceinline__ void norm_store(typename A::T *p, const float (&v)[N]) {
    if constexpr (NT) store_f32_nt<A, N>(p, v); else store_f32<A, N>(p, v);
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
#pragma unroll
                for (int i = 0; i < VEC; ++i) {
                    // h is stored in the activation dtype and normalised as stored.
                    v[c][i] = A::load(A::store(v[c][i] + rv[c][i]));
                }
                if constexpr (STORE_H) norm_store<A, VEC, true>(h + row * group + base, v[c]);
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
