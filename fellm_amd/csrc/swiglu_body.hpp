// Device body of the SwiGLU kernel (elementwise.hip), shared with the fused
// decode-step launch (rope.hip).
//
// SiluGate reference: crates/backend-cpu/src/kernels/swiglu.rs:5-16
//   out[i] = (g / (1 + exp(-g))) * u       (f32, libm expf)
#pragma once

#include <type_traits>

#include "common.hpp"

namespace fellm {
namespace {

constexpr int kEwBlock = 256;

// Build knob: 16-bit outputs take the interval fast path of silu_mul_fast (1).
#ifndef FELLM_SWIGLU_FAST
#define FELLM_SWIGLU_FAST 1
#endif

// Non-temporal store of VEC already-rounded output elements.
template <typename O, int VEC>
__device__ __forceinline__ void store_raw_nt(typename O::T *p, const typename O::T (&v)[VEC]) {
    using P = Pack<typename O::T, VEC>;
    constexpr int W = sizeof(P) / 4;
    P pk;
#pragma unroll
    for (int i = 0; i < VEC; ++i) pk.v[i] = v[i];
    uint32_t w[W];
    memcpy(w, &pk, sizeof(P));
    uint32_t *dst = reinterpret_cast<uint32_t *>(p);
#pragma unroll
    for (int i = 0; i < W; ++i) __builtin_nontemporal_store(w[i], dst + i);
}

// SwiGLU over n elements by a grid of nblk kEwBlock-thread workgroups, this
// workgroup being number bid (every thread calls it; contains a barrier).
// tab_lds: 32 u64 of LDS for the expf table.
template <typename I, typename O, int VEC, int UNROLL>
__device__ __forceinline__ void silu_gate_blocks(const typename I::T *__restrict__ g,
                                                 const typename I::T *__restrict__ u, typename O::T *__restrict__ out,
                                                 uint64_t n, uint32_t bid, uint32_t nblk, uint64_t *tab_lds) {
    const uint64_t *tab = stage_expf_table(tab_lds);
    const uint64_t nvec = n / VEC;
    const uint64_t stride = (uint64_t)nblk * kEwBlock * UNROLL;
    for (uint64_t base = (uint64_t)bid * kEwBlock * UNROLL + threadIdx.x; base < nvec; base += stride) {
        float gv[UNROLL][VEC], uv[UNROLL][VEC];
#pragma unroll
        for (int j = 0; j < UNROLL; ++j) {
            const uint64_t i = base + (uint64_t)j * kEwBlock;
            if (i < nvec) {
                load_f32_nt<I, VEC>(g + i * VEC, gv[j]);
                load_f32_nt<I, VEC>(u + i * VEC, uv[j]);
            }
        }
#pragma unroll
        for (int j = 0; j < UNROLL; ++j) {
            const uint64_t i = base + (uint64_t)j * kEwBlock;
            if (i < nvec) {
                if constexpr (FELLM_SWIGLU_FAST && sizeof(typename O::T) == 2 && VEC % 2 == 0) {
                    // The exact silu runs only for the elements (and only in
                    // the wavefronts) whose rounding the interval leaves open.
                    // bf16: one branch per vector for the exact fallback
                    // (configs[4] routed 94.6 -> 92.8 us); f16 keeps one per
                    // element (configs[1] 56.3 against 57.3 us the other way).
                    typename O::T o[VEC];
                    if constexpr (std::is_same_v<O, F16>) {
#pragma unroll
                        for (int k = 0; k < VEC; ++k)
                            if (__builtin_expect(!silu_mul_fast<O>(gv[j][k], uv[j][k], o[k]), 0))
                                o[k] = O::store(silu(gv[j][k], tab) * uv[j][k]);
                    } else {
                        bool fast[VEC];
                        bool all = true;
#pragma unroll
                        for (int k = 0; k < VEC; ++k) {
                            fast[k] = silu_mul_fast<O>(gv[j][k], uv[j][k], o[k]);
                            all = all && fast[k];
                        }
                        if (__builtin_expect(!all, 0)) {
#pragma unroll
                            for (int k = 0; k < VEC; ++k)
                                if (!fast[k]) o[k] = O::store(silu(gv[j][k], tab) * uv[j][k]);
                        }
                    }
                    store_raw_nt<O, VEC>(out + i * VEC, o);
                } else {
                    float o[VEC];
#pragma unroll
                    for (int k = 0; k < VEC; ++k) o[k] = silu(gv[j][k], tab) * uv[j][k];
                    store_f32_nt<O, VEC>(out + i * VEC, o);
                }
            }
        }
    }
    // Tail (n % VEC elements), handled by the first threads of block 0.
    if (bid == 0) {
        const uint64_t t = nvec * VEC + threadIdx.x;
        if (t < n) out[t] = O::store(silu(I::load(g[t]), tab) * I::load(u[t]));
    }
}

}  // namespace
}  // namespace fellm
