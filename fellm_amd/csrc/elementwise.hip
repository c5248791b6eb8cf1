// Elementwise kernels for gfx950: SwiGLU (SiLU-gate * up), Add, expf and
// sinf/cosf checks.
//
// SiluGate reference: crates/backend-cpu/src/kernels/swiglu.rs:5-16
//   out[i] = (g / (1 + exp(-g))) * u       (f32, libm expf)
// Add reference: crates/backend-cpu/src/kernels/simd_f32.rs:175-197.
//
// Pure streaming kernels: each thread moves 2 x VEC elements per iteration
// (both 16-byte loads of g and u for the two units issued before any math)
// with non-temporal loads/stores; the grid covers the tensor in one pass.
// exp is the glibc-exact double-precision restatement (common.hpp) and the
// division uses silu_div below, so the f32 result equals the CPU reference
// bit for bit.  With ~30 ALU ops per element the kernel sits close to the
// ALU/HBM balance point, which is why the division is not left to the
// default 13-instruction IEEE sequence.  For 16-bit outputs most elements
// skip that exact evaluation altogether: a fast f32 silu whose distance to
// the exact one is bounded over every input decides the rounded output
// whenever the interval it implies holds a single 16-bit value
// (silu_mul_fast, common.hpp); the rest take the exact path.
#include "swiglu_body.hpp"

namespace fellm {
namespace {

// Build knob: 8-element vectors per thread in the SwiGLU launch.  Measured
// interleaved on one box: configs[1] 55.6-56.7 us at 1 and 2, 60.0-60.5 at 4;
// configs[4] routed 95.6 (1), 92.5 (2), 97.6 (4).
#ifndef FELLM_SWIGLU_UNROLL
#define FELLM_SWIGLU_UNROLL 2
#endif

inline uint32_t ew_grid(uint64_t units) {
    uint64_t g = (units + kEwBlock - 1) / kEwBlock;
    const uint64_t cap = 256ull * 32;  // 256 CUs x 32 blocks: enough to saturate HBM
    if (g > cap) g = cap;
    return (uint32_t)(g == 0 ? 1 : g);
}

template <typename I, typename O, int VEC, int UNROLL>
__global__ __launch_bounds__(kEwBlock) void silu_gate_kernel(const typename I::T *__restrict__ g,
                                                             const typename I::T *__restrict__ u,
                                                             typename O::T *__restrict__ out, uint64_t n) {
    __shared__ uint64_t tab_lds[32];
    silu_gate_blocks<I, O, VEC, UNROLL>(g, u, out, n, blockIdx.x, gridDim.x, tab_lds);
}

template <typename I, typename O, int VEC>
__global__ __launch_bounds__(kEwBlock) void add_kernel(const typename I::T *__restrict__ a,
                                                       const typename I::T *__restrict__ b,
                                                       typename O::T *__restrict__ out, uint64_t n) {
    const uint64_t nvec = n / VEC;
    const uint64_t stride = (uint64_t)gridDim.x * kEwBlock;
    for (uint64_t i = (uint64_t)blockIdx.x * kEwBlock + threadIdx.x; i < nvec; i += stride) {
        float av[VEC], bv[VEC], o[VEC];
        load_f32_nt<I, VEC>(a + i * VEC, av);
        load_f32_nt<I, VEC>(b + i * VEC, bv);
#pragma unroll
        for (int k = 0; k < VEC; ++k) o[k] = av[k] + bv[k];
        store_f32_nt<O, VEC>(out + i * VEC, o);
    }
    if (blockIdx.x == 0) {
        const uint64_t t = nvec * VEC + threadIdx.x;
        if (t < n) out[t] = O::store(I::load(a[t]) + I::load(b[t]));
    }
}

__global__ __launch_bounds__(kEwBlock) void expf_kernel(const float *__restrict__ in,
                                                        float *__restrict__ out, uint64_t n) {
    __shared__ uint64_t tab_lds[32];
    const uint64_t *tab = stage_expf_table(tab_lds);
    const uint64_t stride = (uint64_t)gridDim.x * kEwBlock;
    for (uint64_t i = (uint64_t)blockIdx.x * kEwBlock + threadIdx.x; i < n; i += stride)
        out[i] = expf_glibc(in[i], tab);
}

// Streaming probe: reads nr units of 16 bytes from a (and b), writes nw
// units to out (out[i] = a[i] ^ b[i] where both exist, else whatever was
// read or a constant), U units per thread in one pass, all loads issued
// before the stores, non-temporal or regular accesses.  No arithmetic: the
// speed of moving an op's read and write bytes, the ceiling the op is
// measured against.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int NR, int U, bool NT>
__global__ __launch_bounds__(kEwBlock) void stream_probe_kernel(const u32x4 *__restrict__ a,
                                                                const u32x4 *__restrict__ b, uint64_t nr,
                                                                u32x4 *__restrict__ out, uint64_t nw) {
    const uint64_t base = (uint64_t)blockIdx.x * kEwBlock * U + threadIdx.x;
    u32x4 v[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
        const uint64_t i = base + (uint64_t)k * kEwBlock;
        v[k] = u32x4{(uint32_t)i, 0u, 0u, 0u};
        if (i < nr) {
            v[k] = NT ? __builtin_nontemporal_load(a + i) : a[i];
            if constexpr (NR == 2) v[k] ^= NT ? __builtin_nontemporal_load(b + i) : b[i];
        }
    }
#pragma unroll
    for (int k = 0; k < U; ++k) {
        const uint64_t i = base + (uint64_t)k * kEwBlock;
        if (i < nw) {
            if (NT)
                __builtin_nontemporal_store(v[k], out + i);
            else
                out[i] = v[k];
        } else if (i < nr && v[k].x == 0x9e3779b9u && v[k].y == 0x7f4a7c15u) {
            out[0] = v[k];  // keeps reads past the write range live; practically never taken
        }
    }
}

__global__ __launch_bounds__(kEwBlock) void sincosf_kernel(const float *__restrict__ in, float *__restrict__ sin_out,
                                                           float *__restrict__ cos_out, uint64_t n) {
    const uint64_t stride = (uint64_t)gridDim.x * kEwBlock;
    for (uint64_t i = (uint64_t)blockIdx.x * kEwBlock + threadIdx.x; i < n; i += stride) {
        float sv, cv;
        sincosf_glibc(in[i], &sv, &cv);
        sin_out[i] = sv;
        cos_out[i] = cv;
    }
}

__global__ __launch_bounds__(kEwBlock) void mathf_kernel(uint32_t fn, const float *__restrict__ in,
                                                         float *__restrict__ out, uint64_t n) {
    __shared__ uint64_t tab_lds[32];
    const uint64_t *tab = stage_expf_table(tab_lds);
    const uint64_t stride = (uint64_t)gridDim.x * kEwBlock;
    for (uint64_t i = (uint64_t)blockIdx.x * kEwBlock + threadIdx.x; i < n; i += stride)
        out[i] = fn == 0   ? logf_glibc(in[i])
                 : fn == 1 ? sqrtf_rn(in[i])
                 : fn == 2 ? __uint_as_float((uint32_t)BF16HW::store(in[i]))  // bf16 bits in the low half
                 : fn == 4 ? __uint_as_float((f16_pack_bits(in[i], in[i]) & 0xffffu) |
                                             (uint32_t)__builtin_bit_cast(uint16_t, F16::store(in[i])) << 16)
                           : expf_glibc_nonpos(in[i], tab);
}

// Largest bit distance between silu_fast and silu over every f32 g of the
// fast domain, one grid-stride sweep of all 2^32 patterns.
__global__ __launch_bounds__(kEwBlock) void silu_fast_bound_kernel(uint32_t *__restrict__ max_dist) {
    __shared__ uint64_t tab_lds[32];
    const uint64_t *tab = stage_expf_table(tab_lds);
    uint32_t m = 0;
    const uint64_t stride = (uint64_t)gridDim.x * kEwBlock;
    for (uint64_t i = (uint64_t)blockIdx.x * kEwBlock + threadIdx.x; i < (1ull << 32); i += stride) {
        const float g = __uint_as_float((uint32_t)i);
        if (!silu_fast_domain(g)) continue;
        const uint32_t a = __float_as_uint(silu_fast(g)), b = __float_as_uint(silu(g, tab));
        // Opposite signs give a distance of at least 2^31, far above any bound.
        const uint32_t d = a > b ? a - b : b - a;
        m = d > m ? d : m;
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
        const uint32_t o = __shfl_xor(m, off, kWave);
        m = o > m ? o : m;
    }
    if (threadIdx.x % kWave == 0) atomicMax(max_dist, m);
}

// VEC = 8 elements: 16 B for 16-bit types, 32 B for f32.
template <typename I, typename O>
int launch_silu(const void *g, const void *u, void *out, uint64_t n, hipStream_t s) {
    constexpr int VEC = 8, UNROLL = FELLM_SWIGLU_UNROLL;
    using TI = typename I::T;
    using TO = typename O::T;
    if (!aligned_to(g, sizeof(TI) * VEC) || !aligned_to(u, sizeof(TI) * VEC) ||
        !aligned_to(out, sizeof(TO) * VEC)) {
        FELLM_LAUNCH((silu_gate_kernel<I, O, 1, 1>), dim3(ew_grid(n)), dim3(kEwBlock), 0, s,
                           (const TI *)g, (const TI *)u, (TO *)out, n);
        return launch_status();
    }
    // One pass over the tensor: ceil(units / (block * UNROLL)) blocks.
    const uint64_t units = n / VEC;
    uint64_t blocks = (units + kEwBlock * UNROLL - 1) / (kEwBlock * UNROLL);
    if (blocks == 0) blocks = 1;
    if (blocks > 0x7fffffffull) blocks = 0x7fffffffull;
    FELLM_LAUNCH((silu_gate_kernel<I, O, VEC, UNROLL>), dim3((uint32_t)blocks), dim3(kEwBlock), 0, s,
                       (const TI *)g, (const TI *)u, (TO *)out, n);
    return launch_status();
}

template <typename I, typename O>
int launch_add(const void *a, const void *b, void *out, uint64_t n, hipStream_t s) {
    constexpr int VEC = 8;
    using TI = typename I::T;
    using TO = typename O::T;
    if (!aligned_to(a, sizeof(TI) * VEC) || !aligned_to(b, sizeof(TI) * VEC) ||
        !aligned_to(out, sizeof(TO) * VEC)) {
        FELLM_LAUNCH((add_kernel<I, O, 1>), dim3(ew_grid(n)), dim3(kEwBlock), 0, s,
                           (const TI *)a, (const TI *)b, (TO *)out, n);
        return launch_status();
    }
    FELLM_LAUNCH((add_kernel<I, O, VEC>), dim3(ew_grid(n / VEC)), dim3(kEwBlock), 0, s,
                       (const TI *)a, (const TI *)b, (TO *)out, n);
    return launch_status();
}

}  // namespace
}  // namespace fellm

extern "C" int fellm_rocm_silu_gate(const void *gate, const void *up, uint32_t in_dtype, void *out,
                                    uint32_t out_dtype, uint64_t n_elems, void *stream) {
    using namespace fellm;
    if (n_elems == 0) return FELLM_OK;
    if (!gate || !up || !out) return FELLM_ERR_ARITY;
    hipStream_t s = as_stream(stream);
    return dispatch_act(in_dtype, [&]<typename I>() -> int {
        if (out_dtype == in_dtype) return launch_silu<I, typename HwStore<I>::type>(gate, up, out, n_elems, s);
        if (out_dtype == FELLM_DTYPE_F32) return launch_silu<I, F32>(gate, up, out, n_elems, s);
        return FELLM_ERR_DTYPE;
    });
}

extern "C" int fellm_rocm_add(const void *a, const void *b, uint32_t in_dtype, void *out,
                              uint32_t out_dtype, uint64_t n_elems, void *stream) {
    using namespace fellm;
    if (n_elems == 0) return FELLM_OK;
    if (!a || !b || !out) return FELLM_ERR_ARITY;
    hipStream_t s = as_stream(stream);
    return dispatch_act(in_dtype, [&]<typename I>() -> int {
        if (out_dtype == in_dtype) return launch_add<I, I>(a, b, out, n_elems, s);
        if (out_dtype == FELLM_DTYPE_F32) return launch_add<I, F32>(a, b, out, n_elems, s);
        return FELLM_ERR_DTYPE;
    });
}

extern "C" int fellm_rocm_stream_probe(const void *a, const void *b, uint64_t read_bytes, void *out,
                                       uint64_t write_bytes, uint32_t variant, void *stream) {
    using namespace fellm;
    if (read_bytes == 0 && write_bytes == 0) return FELLM_OK;
    if ((read_bytes && !a) || !out || read_bytes % 16 || write_bytes % 16 || !aligned_to(a, 16) ||
        !aligned_to(out, 16) || (b && !aligned_to(b, 16)))
        return FELLM_ERR_SHAPE;
    const uint64_t nr = read_bytes / 16, nw = write_bytes / 16, n = nr > nw ? nr : nw;
    hipStream_t s = as_stream(stream);
    const int u = variant & 3 ? 1 << (variant & 3) >> 1 : 1;  // variant bits 0-1: U = 1, 1, 2, 4
    const bool nt = (variant & 4) != 0;
    auto go = [&]<int U>() -> int {
        const uint64_t blocks = (n + (uint64_t)kEwBlock * U - 1) / ((uint64_t)kEwBlock * U);
        if (blocks > 0x7fffffffull) return FELLM_ERR_SHAPE;
        const dim3 grid((uint32_t)blocks);
        const u32x4 *pa = static_cast<const u32x4 *>(a), *pb = static_cast<const u32x4 *>(b);
        u32x4 *po = static_cast<u32x4 *>(out);
        if (b) {
            if (nt) FELLM_LAUNCH((stream_probe_kernel<2, U, true>), grid, dim3(kEwBlock), 0, s, pa, pb, nr, po, nw);
            else FELLM_LAUNCH((stream_probe_kernel<2, U, false>), grid, dim3(kEwBlock), 0, s, pa, pb, nr, po, nw);
        } else {
            if (nt) FELLM_LAUNCH((stream_probe_kernel<1, U, true>), grid, dim3(kEwBlock), 0, s, pa, pb, nr, po, nw);
            else FELLM_LAUNCH((stream_probe_kernel<1, U, false>), grid, dim3(kEwBlock), 0, s, pa, pb, nr, po, nw);
        }
        return launch_status();
    };
    if (u == 4) return go.template operator()<4>();
    if (u == 2) return go.template operator()<2>();
    return go.template operator()<1>();
}

extern "C" int fellm_rocm_timing_arm(void *start_event, void *stop_event) {
    if (!start_event || !stop_event) return FELLM_ERR_ARITY;
    fellm::g_launch_timing = fellm::LaunchTiming{static_cast<hipEvent_t>(start_event),
                                                 static_cast<hipEvent_t>(stop_event), true, false};
    return FELLM_OK;
}

extern "C" void fellm_rocm_timing_disarm(void) { fellm::g_launch_timing = fellm::LaunchTiming{}; }

extern "C" int fellm_rocm_mathf(uint32_t fn, const float *in, float *out, uint64_t n, void *stream) {
    using namespace fellm;
    if (fn > 4) return FELLM_ERR_SHAPE;
    if (n == 0) return FELLM_OK;
    if (!in || !out) return FELLM_ERR_ARITY;
    FELLM_LAUNCH(mathf_kernel, dim3(ew_grid(n)), dim3(kEwBlock), 0, as_stream(stream), fn, in, out, n);
    return launch_status();
}

extern "C" int fellm_rocm_sincosf(const float *in, float *sin_out, float *cos_out, uint64_t n, void *stream) {
    using namespace fellm;
    if (n == 0) return FELLM_OK;
    if (!in || !sin_out || !cos_out) return FELLM_ERR_ARITY;
    FELLM_LAUNCH(sincosf_kernel, dim3(ew_grid(n)), dim3(kEwBlock), 0, as_stream(stream), in, sin_out, cos_out,
                       n);
    return launch_status();
}

extern "C" int fellm_rocm_expf(const float *in, float *out, uint64_t n, void *stream) {
    using namespace fellm;
    if (!in || !out) return FELLM_ERR_ARITY;
    if (n == 0) return FELLM_OK;
    FELLM_LAUNCH(expf_kernel, dim3(ew_grid(n)), dim3(kEwBlock), 0, as_stream(stream), in, out, n);
    return launch_status();
}

extern "C" int fellm_rocm_silu_fast_bound(uint32_t *max_dist, void *stream) {
    using namespace fellm;
    if (!max_dist) return FELLM_ERR_ARITY;
    FELLM_LAUNCH(silu_fast_bound_kernel, dim3(256 * 16), dim3(kEwBlock), 0, as_stream(stream), max_dist);
    return launch_status();
}

extern "C" uint32_t fellm_rocm_silu_fast_dist(void) { return fellm::kSiluFastDist; }
