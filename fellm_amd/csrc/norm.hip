// Residual add + RMSNorm for gfx950.
//
// Reference semantics: Add (crates/backend-cpu/src/kernels/simd_f32.rs:175-197)
// then RmsNorm (crates/backend-cpu/src/kernels/norm.rs:6-53, launcher
// crates/backend-cpu/src/backend.rs:1104-1133): per row of `group` elements,
// sumsq = sum(h^2), scale = 1 / sqrt(sumsq / group + eps), y = (h * scale) * w.
//
// Layout: one workgroup per row.  Each thread owns NCHUNK chunks of VEC
// consecutive elements (16-byte accesses for 16-bit types), keeps them in
// registers between the reduction and the scaling pass, so x and residual are
// read exactly once and h and y written exactly once: 4 row-passes of HBM
// traffic with the residual fused (the unfused graph needs 6).
// The sum of squares is one wavefront shuffle reduction plus one LDS exchange.
#include <algorithm>

#include "norm_body.hpp"

// Build knob: the one-wavefront-per-row layout reads the weights from one
// LDS copy per workgroup (1) or from the caches per wavefront (0).  Per row
// the f32 weights are twice the bytes of a 16-bit row, and two thirds of the
// kernel's load instructions.  Measured at configs[4] (16384 x 2048 bf16,
// interleaved on one box): 25.0-25.3 against 25.9-26.5 us.
#ifndef FELLM_NORM_WAVE_WLDS
#define FELLM_NORM_WAVE_WLDS 1
#endif

// Build knob: with many rows, rows of at most FELLM_NORM_WAVE_BYTES bytes
// take one wavefront per row instead of one workgroup per row (0: never).
// Measured on MI355X inside the op chains: 16384 x 2048 bf16 RMSNorm
// 26.2-26.3 us (wavefront per row) against 27.3-27.5 us; 4096 x 4096 f16
// add+RMSNorm (8 KB rows) 28.4 us against 25.2 us, with the RoPE launched
// after it slowed from 15.6 to 19.5 us.  So rows up to 4 KB only.
// Build knob: many-row add + RMSNorm with h, rows of 2049..4096 16-bit
// elements, as a persistent pipelined grid of FELLM_NORM_PIPE workgroups per
// CU (0: one workgroup per row).  Measured inside the op chain at 4096 x 4096
// f16: 3 per CU 23.6-24.0 us, 2 per CU 24.1-24.5, 4 per CU 24.4, one
// workgroup per row 24.1-25.0.
#ifndef FELLM_NORM_PIPE
#define FELLM_NORM_PIPE 3
#endif
// Build knob: threads per workgroup of the wavefront-per-row kernel (one row
// per wavefront; the workgroup's rows share one LDS copy of the weights).
// Measured at configs[4] (16384 x 2048 bf16, interleaved on one box): 256
// 25.1-25.2 us, 512 25.1-25.2, 1024 26.8-27.0, 128 27.2-27.6.
// Build knob: rows per wavefront in the wavefront-per-row layout (each
// wavefront requests all of its rows before reducing the first).
#ifndef FELLM_NORM_WAVE_ROWS
#define FELLM_NORM_WAVE_ROWS 1
#endif
// Build knob: the wavefront-per-row layout reads x and r non-temporally (1)
// or with the default cache policy (0).
#ifndef FELLM_NORM_WAVE_XNT
#define FELLM_NORM_WAVE_XNT 1
#endif
#ifndef FELLM_NORM_WAVE_BLOCK
#define FELLM_NORM_WAVE_BLOCK 256
#endif
#ifndef FELLM_NORM_WAVE_BYTES
#define FELLM_NORM_WAVE_BYTES 4096
#endif
// Build knob: threads per row for rows of 2049..4096 (16-bit) elements at
// >= 1024 rows (256: two 8-element chunks per thread; 512: one).  Measured
// inside the op chain at 4096 x 4096 f16: 24.4-24.5 us (512) against
// 25.2-25.9 us (256).
#ifndef FELLM_NORM_PREFILL_BLOCK
#define FELLM_NORM_PREFILL_BLOCK 512
#endif

namespace fellm {

namespace {

template <typename A, typename O, int BLOCK, int VEC, int NCHUNK, bool ADD, bool STORE_H>
__global__ __launch_bounds__(BLOCK) void add_rmsnorm_kernel(const typename A::T *x, const typename A::T *r,
                                                            typename A::T *h, const float *__restrict__ w,
                                                            typename O::T *y, uint32_t group, float eps) {
    __shared__ float red[BLOCK / kWave];
    add_rmsnorm_row<A, O, BLOCK, VEC, NCHUNK, ADD, STORE_H>(x, r, h, w, y, group, eps, blockIdx.x, red);
}

// Persistent, software-pipelined add + RMSNorm for many rows: a grid of
// about `waves_per_cu` workgroups per CU loops over rows bid, bid + grid, ...
// and requests row i+1's x and r before it reduces and stores row i, so the
// loads of the next row overlap the barrier and the stores of this one.  The
// weights are read once per workgroup.  Same arithmetic as add_rmsnorm_row.
template <typename A, typename O, int BLOCK, int VEC, int NCHUNK>
__global__ __launch_bounds__(BLOCK) void add_rmsnorm_pipe_kernel(const typename A::T *x, const typename A::T *r,
                                                                 typename A::T *h, const float *__restrict__ w,
                                                                 typename O::T *y, uint32_t group, uint32_t rows,
                                                                 float eps) {
    __shared__ float red[2][BLOCK / kWave];
    float wv[NCHUNK][VEC];
#pragma unroll
    for (int c = 0; c < NCHUNK; ++c) {
        const uint32_t base = (uint32_t)(c * BLOCK + threadIdx.x) * VEC;
        if (base < group) load_f32<F32, VEC>(w + base, wv[c]);
    }
    float xv[NCHUNK][VEC], rv[NCHUNK][VEC];
    auto load_row = [&](uint32_t row, float (&xo)[NCHUNK][VEC], float (&ro)[NCHUNK][VEC]) {
#pragma unroll
        for (int c = 0; c < NCHUNK; ++c) {
            const uint32_t base = (uint32_t)(c * BLOCK + threadIdx.x) * VEC;
            if (base < group) {
                norm_load<A, VEC>(x + (size_t)row * group + base, xo[c]);
                norm_load<A, VEC>(r + (size_t)row * group + base, ro[c]);
            }
        }
    };
    uint32_t row = blockIdx.x;
    if (row < rows) load_row(row, xv, rv);
    int parity = 0;
    for (; row < rows; row += gridDim.x) {
        float hv[NCHUNK][VEC];
#pragma unroll
        for (int c = 0; c < NCHUNK; ++c) {
#pragma unroll
            for (int i = 0; i < VEC; ++i) hv[c][i] = xv[c][i];
            norm_add_round<A, VEC, false>(hv[c], rv[c], nullptr);
        }
        const uint32_t next = row + gridDim.x;
        if (next < rows) load_row(next, xv, rv);  // in flight during this row's reduction and stores
        float ss = 0.0f;
#pragma unroll
        for (int c = 0; c < NCHUNK; ++c) {
            const uint32_t base = (uint32_t)(c * BLOCK + threadIdx.x) * VEC;
            if (base < group) {
                norm_store<A, VEC, true>(h + (size_t)row * group + base, hv[c]);
#pragma unroll
                for (int i = 0; i < VEC; ++i) ss += hv[c][i] * hv[c][i];
            }
        }
        // Alternate the LDS slots so one barrier per row suffices.
        ss = wave_sum(ss);
        if (threadIdx.x % kWave == 0) red[parity][threadIdx.x / kWave] = ss;
        __syncthreads();
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < BLOCK / kWave; ++i) t += red[parity][i];
        parity ^= 1;
        const float scale = 1.0f / sqrtf(t / (float)group + eps);
#pragma unroll
        for (int c = 0; c < NCHUNK; ++c) {
            const uint32_t base = (uint32_t)(c * BLOCK + threadIdx.x) * VEC;
            if (base < group) {
                float o[VEC];
#pragma unroll
                for (int i = 0; i < VEC; ++i) o[i] = (hv[c][i] * scale) * wv[c][i];
                norm_store<O, VEC, true>(y + (size_t)row * group + base, o);
            }
        }
    }
}

// One wavefront per row, four rows per workgroup, for rows of at most 8 KB
// (NCH 16-byte chunks per lane, chunk c of the row at lanes' c * 1 KB).  Every
// lane requests all of its x and r chunks before any arithmetic; the sum of
// squares is one wavefront reduction (no LDS, no barrier), so a row's stores
// follow its loads by one reduction and nothing waits on other rows.  x and r
// stay in registers in storage form, h is rounded in place, and y is formed
// from it with the weights read per chunk.
template <typename A, typename O, int NCH, bool ADD, bool STORE_H>
__global__ __launch_bounds__(FELLM_NORM_WAVE_BLOCK) void add_rmsnorm_wave_kernel(
    const typename A::T *x, const typename A::T *r, typename A::T *h, const float *__restrict__ w,
    typename O::T *y, uint32_t group, uint32_t rows, float eps) {
    using T = typename A::T;
    constexpr int VEC = 16 / sizeof(T);
    using P = Pack<T, VEC>;
    constexpr int RW = FELLM_NORM_WAVE_ROWS;
    const uint32_t lane = threadIdx.x % kWave;
    const uint32_t row0 = (blockIdx.x * (FELLM_NORM_WAVE_BLOCK / kWave) + threadIdx.x / kWave) * RW;
    const bool live = row0 < rows;
    const uint32_t nvec = group / VEC;
    // The rows' x and r are requested first: their latency overlaps the
    // weight staging and its barrier.
    P xv[RW][NCH], rv[RW][ADD ? NCH : 1];
#pragma unroll
    for (int q = 0; q < RW; ++q) {
        const size_t off = (size_t)(row0 + q) * group;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const uint32_t i = c * kWave + lane;
            if (row0 + q < rows && i < nvec) {
                xv[q][c] = FELLM_NORM_WAVE_XNT ? load_pack_nt<T, VEC>(x + off + (size_t)i * VEC)
                                               : load_pack<T, VEC>(x + off + (size_t)i * VEC);
                if constexpr (ADD)
                    rv[q][c] = FELLM_NORM_WAVE_XNT ? load_pack_nt<T, VEC>(r + off + (size_t)i * VEC)
                                                   : load_pack<T, VEC>(r + off + (size_t)i * VEC);
            }
        }
    }
    if constexpr (FELLM_NORM_WAVE_WLDS) {
        // The workgroup's rows share one copy of the weights in LDS (group
        // floats, at most 8 KB), instead of each wavefront reading them from
        // the caches.
        extern __shared__ float4 w_lds4[];
        for (uint32_t i = threadIdx.x; i < group / 4; i += FELLM_NORM_WAVE_BLOCK)
            w_lds4[i] = reinterpret_cast<const float4 *>(w)[i];
        __syncthreads();
        w = reinterpret_cast<const float *>(w_lds4);
    }
    if (!live) return;  // whole wavefronts only: no block-level barrier follows
#pragma unroll
    for (int q = 0; q < RW; ++q) {
        const size_t off = (size_t)(row0 + q) * group;
        const bool qlive = row0 + q < rows;
        float ss = 0.0f;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const uint32_t i = c * kWave + lane;
            if (qlive && i < nvec) {
#pragma unroll
                for (int k = 0; k < VEC; ++k) {
                    float hv = A::load(xv[q][c].v[k]);
                    if constexpr (ADD) {
                        // h is stored in the activation dtype and normalised as stored.
                        xv[q][c].v[k] = A::store(hv + A::load(rv[q][c].v[k]));
                        hv = A::load(xv[q][c].v[k]);
                    }
                    ss += hv * hv;
                }
                if constexpr (STORE_H) store_pack_nt<T, VEC>(h + off + (size_t)i * VEC, xv[q][c]);
            }
        }
        ss = wave_sum(ss);
        const float scale = 1.0f / sqrtf(ss / (float)group + eps);
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const uint32_t i = c * kWave + lane;
            if (qlive && i < nvec) {
                float wv[VEC], o[VEC];
                load_f32<F32, VEC>(w + (size_t)i * VEC, wv);
#pragma unroll
                for (int k = 0; k < VEC; ++k) o[k] = (A::load(xv[q][c].v[k]) * scale) * wv[k];
                norm_store<O, VEC, true>(y + off + (size_t)i * VEC, o);
            }
        }
    }
}

template <typename A, typename O, int NCH>
int launch_wave(const void *x, const void *r, void *h, const float *w, void *y, uint32_t group, uint64_t rows,
                float eps, hipStream_t s) {
    using TA = typename A::T;
    using TO = typename O::T;
    constexpr uint32_t RPB = FELLM_NORM_WAVE_BLOCK / kWave * FELLM_NORM_WAVE_ROWS;  // rows per workgroup
    const dim3 grid((uint32_t)((rows + RPB - 1) / RPB)), block(FELLM_NORM_WAVE_BLOCK);
    const size_t wl = FELLM_NORM_WAVE_WLDS ? (size_t)group * sizeof(float) : 0;
    if (r == nullptr) {
        FELLM_LAUNCH((add_rmsnorm_wave_kernel<A, O, NCH, false, false>), grid, block, wl, s, (const TA *)x, nullptr,
                     nullptr, w, (TO *)y, group, (uint32_t)rows, eps);
    } else if (h == nullptr) {
        FELLM_LAUNCH((add_rmsnorm_wave_kernel<A, O, NCH, true, false>), grid, block, wl, s, (const TA *)x,
                     (const TA *)r, nullptr, w, (TO *)y, group, (uint32_t)rows, eps);
    } else {
        FELLM_LAUNCH((add_rmsnorm_wave_kernel<A, O, NCH, true, true>), grid, block, wl, s, (const TA *)x,
                     (const TA *)r, (TA *)h, w, (TO *)y, group, (uint32_t)rows, eps);
    }
    return launch_status();
}

// Generic fallback for rows that do not fit the register-resident layout
// (group % VEC != 0 or group > BLOCK * VEC * 8): two passes, the second
// re-reading h (or x) from cache.
template <typename A, typename O, bool ADD>
__global__ __launch_bounds__(256) void add_rmsnorm_generic(
    const typename A::T *x, const typename A::T *r, typename A::T *h, const float *__restrict__ w,
    typename O::T *y, uint32_t group, float eps) {
    __shared__ float red[256 / kWave];
    const size_t off = (size_t)blockIdx.x * group;
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < group; i += 256) {
        float hv = A::load(x[off + i]);
        if constexpr (ADD) {
            hv = A::load(A::store(hv + A::load(r[off + i])));
            if (h) h[off + i] = A::store(hv);
        }
        ss += hv * hv;
    }
    ss = block_sum<256>(ss, red);
    const float scale = 1.0f / sqrtf(ss / (float)group + eps);
    for (uint32_t i = threadIdx.x; i < group; i += 256) {
        float hv;
        if (ADD && h) {
            hv = A::load(h[off + i]);  // x or r may have been overwritten by h
        } else {
            hv = A::load(x[off + i]);
            if constexpr (ADD) hv = A::load(A::store(hv + A::load(r[off + i])));
        }
        y[off + i] = O::store((hv * scale) * w[i]);
    }
}

template <typename A, typename O, int BLOCK, int VEC, int NCHUNK>
int launch_fast(const void *x, const void *r, void *h, const float *w, void *y, uint32_t group,
                uint64_t rows, float eps, hipStream_t s) {
    using TA = typename A::T;
    using TO = typename O::T;
    dim3 grid((uint32_t)rows), block(BLOCK);
    if (r == nullptr) {
        FELLM_LAUNCH((add_rmsnorm_kernel<A, O, BLOCK, VEC, NCHUNK, false, false>), grid, block, 0, s,
                           (const TA *)x, nullptr, nullptr, w, (TO *)y, group, eps);
    } else if (h == nullptr) {
        FELLM_LAUNCH((add_rmsnorm_kernel<A, O, BLOCK, VEC, NCHUNK, true, false>), grid, block, 0, s,
                           (const TA *)x, (const TA *)r, nullptr, w, (TO *)y, group, eps);
    } else {
        FELLM_LAUNCH((add_rmsnorm_kernel<A, O, BLOCK, VEC, NCHUNK, true, true>), grid, block, 0, s,
                           (const TA *)x, (const TA *)r, (TA *)h, w, (TO *)y, group, eps);
    }
    return launch_status();
}

template <typename A, typename O>
int launch_typed(const void *x, const void *r, void *h, const float *w, void *y, uint32_t group,
                 uint64_t rows, float eps, hipStream_t s) {
    constexpr int VEC = 8;
    const bool vec_ok = group % VEC == 0 && aligned_to(x, 16) && aligned_to(y, 16) &&
                        aligned_to(w, 32) && (!r || aligned_to(r, 16)) && (!h || aligned_to(h, 16));
    if (vec_ok) {
        // Few rows (decode): wide blocks keep more bytes in flight per CU.
        if (rows < 1024 && group <= 1024 * VEC * 2) {
            if (group <= 1024 * VEC) return launch_fast<A, O, 1024, VEC, 1>(x, r, h, w, y, group, rows, eps, s);
            return launch_fast<A, O, 1024, VEC, 2>(x, r, h, w, y, group, rows, eps, s);
        }
        // Many rows of at most 8 KB: one wavefront per row.
        constexpr uint32_t WV = 16 / sizeof(typename A::T);  // elements per 16-byte chunk
        if (group % WV == 0 && group * sizeof(typename A::T) <= FELLM_NORM_WAVE_BYTES) {
            const uint32_t nch = (group / WV + kWave - 1) / kWave;
            if (nch <= 1) return launch_wave<A, O, 1>(x, r, h, w, y, group, rows, eps, s);
            if (nch <= 2) return launch_wave<A, O, 2>(x, r, h, w, y, group, rows, eps, s);
            if (nch <= 4) return launch_wave<A, O, 4>(x, r, h, w, y, group, rows, eps, s);
            return launch_wave<A, O, 8>(x, r, h, w, y, group, rows, eps, s);
        }
        if (FELLM_NORM_PIPE && r && h && group > 256 * VEC && group <= 512 * VEC) {
            using TA = typename A::T;
            using TO = typename O::T;
            const uint32_t grid = (uint32_t)std::min<uint64_t>(rows, (uint64_t)cu_count() * FELLM_NORM_PIPE);
            FELLM_LAUNCH((add_rmsnorm_pipe_kernel<A, O, 512, VEC, 1>), dim3(grid), dim3(512), 0, s, (const TA *)x,
                         (const TA *)r, (TA *)h, w, (TO *)y, group, (uint32_t)rows, eps);
            return launch_status();
        }
        if (FELLM_NORM_PREFILL_BLOCK == 512 && group > 256 * VEC && group <= 512 * VEC)
            return launch_fast<A, O, 512, VEC, 1>(x, r, h, w, y, group, rows, eps, s);
        if (group <= 256 * VEC) return launch_fast<A, O, 256, VEC, 1>(x, r, h, w, y, group, rows, eps, s);
        if (group <= 256 * VEC * 2) return launch_fast<A, O, 256, VEC, 2>(x, r, h, w, y, group, rows, eps, s);
        if (group <= 256 * VEC * 4) return launch_fast<A, O, 256, VEC, 4>(x, r, h, w, y, group, rows, eps, s);
        if (group <= 256 * VEC * 8) return launch_fast<A, O, 256, VEC, 8>(x, r, h, w, y, group, rows, eps, s);
    }
    using TA = typename A::T;
    using TO = typename O::T;
    if (r == nullptr)
        FELLM_LAUNCH((add_rmsnorm_generic<A, O, false>), dim3((uint32_t)rows), dim3(256), 0, s,
                           (const TA *)x, nullptr, nullptr, w, (TO *)y, group, eps);
    else
        FELLM_LAUNCH((add_rmsnorm_generic<A, O, true>), dim3((uint32_t)rows), dim3(256), 0, s,
                           (const TA *)x, (const TA *)r, (TA *)h, w, (TO *)y, group, eps);
    return launch_status();
}

}  // namespace
}  // namespace fellm

extern "C" int fellm_rocm_add_rmsnorm(const void *x, const void *residual, void *h_out,
                                      uint32_t act_dtype, const float *weight, uint32_t group,
                                      void *y, uint32_t y_dtype, uint64_t n_elems, float eps,
                                      void *stream) {
    using namespace fellm;
    if (group == 0 || n_elems % group != 0) return FELLM_ERR_SHAPE;
    if (n_elems == 0) return FELLM_OK;  // no rows: nothing to do, as on the CPU (backend.rs:1125-1128)
    if (!x || !weight || !y) return FELLM_ERR_ARITY;
    if (!residual && h_out) return FELLM_ERR_ARITY;
    const uint64_t rows = n_elems / group;
    if (rows > 0x7fffffffull) return FELLM_ERR_SHAPE;
    hipStream_t s = as_stream(stream);
    return dispatch_act(act_dtype, [&]<typename A>() -> int {
        if (y_dtype == act_dtype) return launch_typed<A, A>(x, residual, h_out, weight, y, group, rows, eps, s);
        if (y_dtype == FELLM_DTYPE_F32) return launch_typed<A, F32>(x, residual, h_out, weight, y, group, rows, eps, s);
        return FELLM_ERR_DTYPE;
    });
}
