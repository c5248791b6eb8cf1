// K-quant GEMV (one activation vector) and the fused gate/up GEMV with the
// SwiGLU epilogue.
//
// Reference: crates/backend-cpu/src/backend.rs:944-1002 (launch_gate_up_swiglu)
//   -> kernels/matmul.rs:404-531 (matvec_quant_multi: x quantized once to
//      Q8_K, every gate row then every up row dotted against it) and
//      swiglu.rs:5-16 (out = silu(gate) * up);
//   matmul.rs:534-600 (matvec_quant) for the plain GEMV;
//   Q8_K activations: matmul.rs:213-270 (quantize_row_q8_k_avx2: amax,
//      iscale = 127/amax, round-to-nearest-even, saturate, bsums, d = amax/127);
//   block dots: Q4_K vec_dot_q4k.rs:296-333, Q5_K vec_dot_q5k.rs:189-218,
//      Q6_K matmul.rs:1597-1644 (fused_q6_k_block).
//
// Layout and schedule.  Weights are the GGUF row-major block streams
// (row r = cols/256 blocks of 144 / 176 / 210 bytes), read exactly once with
// non-temporal loads; they are the only HBM traffic that scales with the
// problem.  Each workgroup quantizes x to Q8_K in LDS (cols bytes of qs,
// cols/16 int16 bsums, cols/256 f32 scales) while its first weight loads are
// in flight.  A wavefront then walks units of at most 32 blocks per matrix
// (a group of 32/cols*256 whole rows, or one 32-block pass of a long row):
// the unit's bytes arrive by coalesced 16-byte loads (lane l, chunk 64i + l)
// into registers one unit ahead, are written to the wavefront's LDS stage,
// and are reduced from there by lane pairs, two lanes per block (lane half h
// covers elements 128h .. 128h+127).  After a row's last unit, lanes
// 0 .. 2*rows-1 fold the rows' gate and up sums in parallel and the even
// lanes apply silu(gate) * up.
//
// Arithmetic.  Integer parts are exact: 4-byte dot products (v_dot4) give the
// per-group sums, combined with the 6-bit scales/mins exactly as the CPU's
// i32 arithmetic does, reduced over the lane pair of a block.  The f32 part
// follows the CPU's portable path operation by operation:
//   Q4_K/Q5_K block: ((-dmin)*xd)*f(sumi_min) + (d*xd)*f(sumi);
//   Q6_K block: 16 terms (d*sc)*f(dot) accumulated in (half, group, k)
//     order, times xd;
//   row: serial f32 sum over blocks from 0.0.
// The CPU's SIMD paths for Q4_K/Q5_K (AVX2/VNNI/AVX-512) share the integer
// parts and reorder only that f32 combine.
#include <mutex>
#include <tuple>
#include <vector>

#include "common.hpp"

// Build knob: workgroups in the grid-stride launch (each quantizes x once).
// 512 = two resident workgroups per CU for the LDS-heavy fused formats.
#ifndef FELLM_GEMV_MAX_GRID
#define FELLM_GEMV_MAX_GRID 512
#endif

// Build knob: the widest grid for launches with many units per wavefront.
#ifndef FELLM_GEMV_WIDE_GRID
#define FELLM_GEMV_WIDE_GRID 768
#endif

// Build knob: weight units in flight per wavefront (1 or 2 register sets).
#ifndef FELLM_GEMV_DEPTH
#define FELLM_GEMV_DEPTH 1
#endif


namespace fellm {
namespace {

constexpr int kGemvBlock = 256;
constexpr int kGemvWaves = kGemvBlock / kWave;
// Build knob: wavefronts per workgroup for rows of more than 32 blocks (the
// multi-pass layout), whose workgroups each quantize all of a long x: 8
// halves that work against 4.  Measured interleaved on one box: Llama-3-8B
// down projection (4096 x 14336 Q4_K) 12.9 against 15.5 us; the 8B gate/up
// shape (one pass per row) measured 16.1 against 14.4 us with 8, so it
// keeps 4.
// Build knob: wavefronts per workgroup for rows of at most 32 blocks.  8
// measured slower at the 8B gate/up shape: 16.2 us with 384 workgroups, 18.8
// with 512, against 14.5 us for 4.
#ifndef FELLM_GEMV_ONE_WAVES
#define FELLM_GEMV_ONE_WAVES 4
#endif
#ifndef FELLM_GEMV_MULTI_WAVES
#define FELLM_GEMV_MULTI_WAVES 8
#endif
constexpr uint32_t kGemvMaxCols = 49152;
// Dynamic LDS a workgroup may take: the CU's 160 KB less the kernel's static
// LDS (the exp table) with room to spare.
constexpr uint32_t kGemvLdsLimit = 160 * 1024 - 1024;
#ifndef FELLM_GEMV_MAX_GRID_PRE
#define FELLM_GEMV_MAX_GRID_PRE 1024
#endif
constexpr uint32_t kGemvMaxGridPre = FELLM_GEMV_MAX_GRID_PRE;

// Q8_K copy of x in (dynamic) LDS: qs[cols], bsums[cols/16], d[cols/256],
// then the per-wavefront row-fold buffers [waves][rows][matrices][nb rounded up to 4].
struct XLds {
    int8_t *qs;
    int16_t *bs;
    float *d;
    float *fold;
};
__host__ __device__ constexpr uint32_t gemv_fold_off(uint32_t nb) { return (nb * 292 + 15) / 16 * 16; }
// fold_per_wave: floats of row-fold buffer per wavefront.
__host__ __device__ constexpr uint32_t gemv_lds_bytes(uint32_t nb, uint32_t fold_per_wave,
                                                     uint32_t waves = kGemvWaves) {
    return gemv_fold_off(nb) + waves * fold_per_wave * 4;
}
__device__ __forceinline__ XLds carve_lds(uint8_t *base, uint32_t nb) {
    return {reinterpret_cast<int8_t *>(base), reinterpret_cast<int16_t *>(base + nb * 256),
            reinterpret_cast<float *>(base + nb * 288), reinterpret_cast<float *>(base + gemv_fold_off(nb))};
}

// quantize_row_q8_k_avx2 (matmul.rs:213-270) for the 256-element blocks of x:
// wavefront `first` takes blocks first, first + stride, ...; lane l holds
// elements 4l..4l+3.  xl may point into LDS or global memory.  The x loads of
// kXBatch blocks go out together before any of them is reduced, and the
// batch's amax reductions (DPP inside each 16-lane row, then the four rows'
// values read as scalars) run side by side: the prologue is a short chain,
// not one LDS shuffle round trip per reduction step and block.
// fmaxf ignores a NaN operand, so the reduction order does not change amax.
__device__ __forceinline__ float block_absmax(const float4 v) {
    float a = fmaxf(fmaxf(__builtin_fabsf(v.x), __builtin_fabsf(v.y)), fmaxf(__builtin_fabsf(v.z), __builtin_fabsf(v.w)));
    a = group_max_f32<16>(a);
    const int ai = __float_as_int(a);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(ai, 0)), r1 = __int_as_float(__builtin_amdgcn_readlane(ai, 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(ai, 32)), r3 = __int_as_float(__builtin_amdgcn_readlane(ai, 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

__device__ __forceinline__ void quantize_block(const float4 v, const float a, uint32_t b, const XLds &xl,
                                               uint32_t lane) {
    int32_t q[4] = {0, 0, 0, 0};
    if (a != 0.0f) {
        const float iscale = 127.0f / a;
        const float e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            // x86 cvtps_epi32 gives INT32_MIN for NaN and |p| >= 2^31 (iscale is
            // inf when amax < ~3.7e-37); the saturating packs make it -128.
            const float p = e[k] * iscale;
            const float r = __builtin_rintf(p);
            q[k] = !(__builtin_fabsf(p) < 0x1p31f) ? -128 : r < -128.0f ? -128 : r > 127.0f ? 127 : (int32_t)r;
        }
    }
    const uint32_t packed = (uint32_t)(q[0] & 0xff) | (uint32_t)(q[1] & 0xff) << 8 | (uint32_t)(q[2] & 0xff) << 16 |
                            (uint32_t)(q[3] & 0xff) << 24;
    *reinterpret_cast<uint32_t *>(&xl.qs[b * 256 + lane * 4]) = packed;
    int32_t s = q[0] + q[1] + q[2] + q[3];
    s += (int32_t)dpp_u32<0xB1>((uint32_t)s);  // quad xor 1
    s += (int32_t)dpp_u32<0x4E>((uint32_t)s);  // quad xor 2
    if ((lane & 3) == 0) xl.bs[b * 16 + lane / 4] = (int16_t)s;
    if (lane == 0) xl.d[b] = a / 127.0f;
}

constexpr int kXBatch = 8;

__device__ __forceinline__ void load_x_batch(const float *__restrict__ x, uint32_t nb, uint32_t b0, uint32_t stride,
                                             float4 (&v)[kXBatch]) {
    const uint32_t lane = threadIdx.x % kWave;
#pragma unroll
    for (int j = 0; j < kXBatch; ++j) {
        const uint32_t b = b0 + j * stride;
        v[j] = b < nb ? *reinterpret_cast<const float4 *>(x + (size_t)b * 256 + lane * 4)
                      : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
}

__device__ __forceinline__ void quantize_batch(const float4 (&v)[kXBatch], uint32_t nb, uint32_t b0, uint32_t stride,
                                               const XLds &xl) {
    const uint32_t lane = threadIdx.x % kWave;
    float a[kXBatch];
#pragma unroll
    for (int j = 0; j < kXBatch; ++j) a[j] = block_absmax(v[j]);
#pragma unroll
    for (int j = 0; j < kXBatch; ++j) {
        const uint32_t b = b0 + j * stride;
        if (b < nb) quantize_block(v[j], a[j], b, xl, lane);
    }
}

__device__ void quantize_x(const float *__restrict__ x, uint32_t nb, const XLds &xl, uint32_t first,
                           uint32_t stride) {
    for (uint32_t b0 = first; b0 < nb; b0 += stride * kXBatch) {
        float4 v[kXBatch];
        load_x_batch(x, nb, b0, stride, v);
        quantize_batch(v, nb, b0, stride, xl);
    }
}

// The Q8_K activation blob: the same layout in global memory as in LDS
// (qs[nb * 256] int8, bsums[nb * 16] int16, d[nb] f32; nb * 292 bytes).
__host__ __device__ constexpr uint32_t q8k_blob_bytes(uint32_t nb) { return nb * 292; }

// x into the workgroup's LDS: quantized here (PREQ = false), or copied from a
// blob that fellm_rocm_quantize_q8k wrote once for the whole launch.  In two
// halves: x_issue requests the thread's first batch of x (or of the blob)
// into registers, x_finish quantizes (copies) it and the rest.  The kernel
// issues x before its first weight loads, so that x does not queue behind
// the weight stream (x is on every wavefront's critical path).
constexpr int kBlobBatch = 4;
template <bool PREQ>
struct XFirst {
    float4 v[kXBatch];
};
template <>
struct XFirst<true> {
    uint32_t v[kBlobBatch];
};

template <bool PREQ>
__device__ __forceinline__ void x_issue(const void *__restrict__ xsrc, uint32_t nb, XFirst<PREQ> &f) {
    if constexpr (PREQ) {
        const uint32_t words = q8k_blob_bytes(nb) / 4;
        const uint32_t *src = static_cast<const uint32_t *>(xsrc);
#pragma unroll
        for (int j = 0; j < kBlobBatch; ++j) {
            const uint32_t i = threadIdx.x + j * blockDim.x;
            f.v[j] = i < words ? src[i] : 0u;
        }
    } else {
        load_x_batch(static_cast<const float *>(xsrc), nb, threadIdx.x / kWave, blockDim.x / kWave, f.v);
    }
}

template <bool PREQ>
__device__ __forceinline__ void x_finish(const void *__restrict__ xsrc, uint32_t nb, const XLds &xl, uint8_t *smem,
                                         const XFirst<PREQ> &f) {
    if constexpr (PREQ) {
        const uint32_t words = q8k_blob_bytes(nb) / 4;
        const uint32_t *src = static_cast<const uint32_t *>(xsrc);
        uint32_t *dst = reinterpret_cast<uint32_t *>(smem);
#pragma unroll
        for (int j = 0; j < kBlobBatch; ++j) {
            const uint32_t i = threadIdx.x + j * blockDim.x;
            if (i < words) dst[i] = f.v[j];
        }
        for (uint32_t i0 = threadIdx.x + blockDim.x * kBlobBatch; i0 < words; i0 += blockDim.x * kBlobBatch) {
            uint32_t v[kBlobBatch];
#pragma unroll
            for (int j = 0; j < kBlobBatch; ++j) {
                const uint32_t i = i0 + j * blockDim.x;
                v[j] = i < words ? src[i] : 0u;
            }
#pragma unroll
            for (int j = 0; j < kBlobBatch; ++j) {
                const uint32_t i = i0 + j * blockDim.x;
                if (i < words) dst[i] = v[j];
            }
        }
    } else {
        const float *x = static_cast<const float *>(xsrc);
        const uint32_t first = threadIdx.x / kWave;
        const uint32_t nw = blockDim.x / kWave;
        quantize_batch(f.v, nb, first, nw, xl);
        quantize_x(x, nb, xl, first + nw * kXBatch, nw);
    }
}

template <bool PREQ>
__device__ __forceinline__ void fill_x(const void *__restrict__ xsrc, uint32_t nb, const XLds &xl, uint8_t *smem) {
    XFirst<PREQ> f;
    x_issue<PREQ>(xsrc, nb, f);
    x_finish<PREQ>(xsrc, nb, xl, smem, f);
}

__device__ __forceinline__ uint4 lds_u4(const void *p) { return *reinterpret_cast<const uint4 *>(p); }

// Weight streams are read through a buffer resource whose range is the
// launch's rows: a load past the end returns zeros without touching memory,
// so the next row group is requested unconditionally (no branch around the
// loads, hence exact wait counts) and the last request costs nothing.
// Cache policy 2 = non-temporal (read once).
using Rsrc = __amdgpu_buffer_rsrc_t;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ Rsrc weight_rsrc(const uint8_t *w, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(w), 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 bld16(Rsrc r, uint32_t off) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 bld8(Rsrc r, uint32_t off) {
    const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 2);
    return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t bld2(Rsrc r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 2);
}

__device__ __forceinline__ float f16_bits(uint32_t b) { return (float)__builtin_bit_cast(_Float16, (uint16_t)b); }

__device__ __forceinline__ uint32_t bld4(Rsrc r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 2);
}

// Partner lane of a pair (lane ^ 1): DPP quad_perm [1,0,3,2].
__device__ __forceinline__ uint32_t pair_swap(uint32_t v) { return dpp_u32<0xB1>(v); }

__device__ __forceinline__ uint32_t mask_shr(uint32_t v, uint32_t s, uint32_t m) { return (v >> s) & m; }

// ---- lane layout ----------------------------------------------------------------
// Two lanes per 256-element block: lane half h (= lane & 1) covers elements
// 128h .. 128h+127.  The 32 lane pairs of a wavefront take 32 block slots:
// with nb <= 32 blocks per row, slot s is block s % nb of row s / nb of the
// wavefront's current row group (32 / nb rows at once); with nb > 32 a row is
// walked in passes of 32 blocks.  Bytes both lanes of a block need (the
// Q4_K/Q5_K header, the Q5_K high bits) are loaded half by each lane and
// exchanged with one DPP swap: lanes reading the same address in one load
// slow the memory pipeline measurably.

// Lane's Q8_K slice of x for its half block.
struct XHalf {
    uint4 q[8];      // x quants of elements 128h .. 128h+127
    int32_t s2[4];   // Q4_K/Q5_K: bsums of the 4 32-element groups
    int32_t s1[8];   // Q6_K: bsums of the 8 16-element groups
    float d;
};

__device__ __forceinline__ void load_x(const XLds &xl, uint32_t b, uint32_t h, XHalf &x) {
    const int8_t *q = xl.qs + b * 256 + 128 * h;
#pragma unroll
    for (int i = 0; i < 8; ++i) x.q[i] = lds_u4(q + 16 * i);
    const int16_t *bs = xl.bs + b * 16 + 8 * h;
#pragma unroll
    for (int g = 0; g < 8; ++g) x.s1[g] = bs[g];
#pragma unroll
    for (int j = 0; j < 4; ++j) x.s2[j] = x.s1[2 * j] + x.s1[2 * j + 1];
    x.d = xl.d[b];
}

// The 4 (scale, min) pairs of groups j = 4h .. 4h+3 from the 12 scale bytes
// (get_scale_min_k4, dequant.rs:295-305) as packed bytes, four at a time:
// h = 0: sc = q[j] & 63, m = q[j+4] & 63;
// h = 1: sc = (q[j+4] & 15) | (q[j-4] >> 6) << 4, m = (q[j+4] >> 4) | (q[j] >> 6) << 4.
__device__ __forceinline__ void k4_scales_half(uint32_t s0, uint32_t s1, uint32_t s2, uint32_t h, uint32_t &sc,
                                               uint32_t &m) {
    const uint32_t sc_hi = (s2 & 0x0f0f0f0fu) | ((s0 >> 2) & 0x30303030u);
    const uint32_t m_hi = ((s2 >> 4) & 0x0f0f0f0fu) | ((s1 >> 2) & 0x30303030u);
    sc = h ? sc_hi : (s0 & 0x3f3f3f3fu);
    m = h ? m_hi : (s1 & 0x3f3f3f3fu);
}

// ---- weight formats ---------------------------------------------------------------
// Raw per-lane block bytes, read from the wavefront's LDS stage (where the
// row group was streamed with coalesced 16-byte loads).  Lane half h.
struct Q4K {
    static constexpr uint32_t kBytes = 144;
    struct Raw {
        uint4 hdr;   // d, dmin, 12 scale bytes
        uint4 q[4];  // qs bytes 64h .. 64h+63
    };
    __device__ static Raw read(const uint8_t *blk, uint32_t h) {
        Raw r;
        r.hdr = lds_u4(blk);
#pragma unroll
        for (int i = 0; i < 4; ++i) r.q[i] = lds_u4(blk + 16 + 64 * h + 16 * i);
        return r;
    }
};

struct Q5K {
    static constexpr uint32_t kBytes = 176;
    struct Raw {
        uint4 hdr;
        uint4 qh[2];  // the 32 high-bit bytes
        uint4 q[4];   // qs bytes 64h .. 64h+63
    };
    __device__ static Raw read(const uint8_t *blk, uint32_t h) {
        Raw r;
        r.hdr = lds_u4(blk);
        r.qh[0] = lds_u4(blk + 16);
        r.qh[1] = lds_u4(blk + 32);
#pragma unroll
        for (int i = 0; i < 4; ++i) r.q[i] = lds_u4(blk + 48 + 64 * h + 16 * i);
        return r;
    }
};

// 210-byte Q6_K blocks sit at 2-byte aligned LDS offsets; gfx950 serves the
// unaligned 16- and 8-byte LDS reads directly.
__device__ __forceinline__ uint4 lds_u4_any(const uint8_t *p) {
    uint4 v;
    __builtin_memcpy(&v, p, 16);
    return v;
}

struct Q6K {
    static constexpr uint32_t kBytes = 210;
    struct Raw {
        uint4 ql[4];  // ql bytes 64h .. 64h+63
        uint4 qh[2];  // qh bytes 32h .. 32h+31
        uint2 sc;     // int8 scales 8h .. 8h+7
        uint32_t d;
    };
    __device__ static Raw read(const uint8_t *blk, uint32_t h) {
        Raw r;
#pragma unroll
        for (int i = 0; i < 4; ++i) r.ql[i] = lds_u4_any(blk + 64 * h + 16 * i);
        r.qh[0] = lds_u4_any(blk + 128 + 32 * h);
        r.qh[1] = lds_u4_any(blk + 144 + 32 * h);
        __builtin_memcpy(&r.sc, blk + 192 + 8 * h, 8);
        uint16_t dd;
        __builtin_memcpy(&dd, blk + 208, 2);
        r.d = dd;
        return r;
    }
};

__device__ __forceinline__ uint32_t u4_at(const uint4 &v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }

// Q4_K / Q5_K block value.  Lane h: chunks c = 2h, 2h+1 (qs bytes 32c .. 32c+31,
// low nibbles -> group 2c, high -> 2c+1), groups j = 4h .. 4h+3.  The exact
// integers of both halves are summed over the lane pair; both lanes then form
// ((-dmin)*xd)*f(sumi_min) + (d*xd)*f(sumi) (vec_dot_q4k.rs:296-333).
template <typename W>
__device__ __forceinline__ float k45_value(const typename W::Raw &r, uint32_t h, const XHalf &x) {
    uint32_t scp, mp;
    k4_scales_half(r.hdr.y, r.hdr.z, r.hdr.w, h, scp, mp);
    uint32_t qh[8];
    if constexpr (W::kBytes == 176) {
        qh[0] = r.qh[0].x;
        qh[1] = r.qh[0].y;
        qh[2] = r.qh[0].z;
        qh[3] = r.qh[0].w;
        qh[4] = r.qh[1].x;
        qh[5] = r.qh[1].y;
        qh[6] = r.qh[1].z;
        qh[7] = r.qh[1].w;
    }
    int32_t si = 0, sm = 0;
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
        int32_t dlo = 0, dhi = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t q = u4_at(r.q[2 * cc + i / 4], i % 4);
            uint32_t lo = q & 0x0f0f0f0fu, hi = (q >> 4) & 0x0f0f0f0fu;
            if constexpr (W::kBytes == 176) {
                // bit 2c (low) / 2c+1 (high) of qh byte l adds 16 (unpack_q5_k_aux8)
                const uint32_t c2 = 2 * (2 * h + cc);
                lo |= ((qh[i] >> c2) & 0x01010101u) << 4;
                hi |= ((qh[i] >> (c2 + 1)) & 0x01010101u) << 4;
            }
            dlo = __builtin_amdgcn_sdot4((int)lo, (int)u4_at(x.q[4 * cc + i / 4], i % 4), dlo, false);
            dhi = __builtin_amdgcn_sdot4((int)hi, (int)u4_at(x.q[4 * cc + 2 + i / 4], i % 4), dhi, false);
        }
        const int32_t sc_lo = (scp >> (16 * cc)) & 0xff, sc_hi = (scp >> (16 * cc + 8)) & 0xff;
        const int32_t m_lo = (mp >> (16 * cc)) & 0xff, m_hi = (mp >> (16 * cc + 8)) & 0xff;
        si += sc_lo * dlo + sc_hi * dhi;
        sm += m_lo * x.s2[2 * cc] + m_hi * x.s2[2 * cc + 1];
    }
    si += (int32_t)pair_swap((uint32_t)si);
    sm += (int32_t)pair_swap((uint32_t)sm);
    const float d = f16_bits(r.hdr.x & 0xffffu), dmin = f16_bits(r.hdr.x >> 16);
    const float t_min = (-dmin * x.d) * (float)sm;
    const float t_sc = (d * x.d) * (float)si;
    return t_min + t_sc;
}

// Q6_K block value (matmul.rs:1597-1644).  Lane h covers half h: for group
// parity is and k = 0..3 the run 128h + 16is + 32k.  The lane forms its 8
// terms (d*sc[8h+is+2k]) * dot in (is, k) order; lane 0's partial sum is
// handed to lane 1, which adds its 8 terms: the CPU's (h, is, k) order.  The
// block value acc * xd is valid in lane h = 1.
__device__ __forceinline__ float q6k_value(const Q6K::Raw &r, uint32_t h, const XHalf &x) {
    const float d = f16_bits(r.d);
    float t[8];
#pragma unroll
    for (int is = 0; is < 2; ++is) {
        int32_t dots[4] = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 4; ++i) {  // dword i of the 16-byte run l = 16is + 4i ..
            const uint32_t A = u4_at(r.ql[is], i), B = u4_at(r.ql[2 + is], i), H = u4_at(r.qh[is], i);
            const uint32_t w1 = (A & 0x0f0f0f0fu) | ((H << 4) & 0x30303030u);
            const uint32_t w2 = (B & 0x0f0f0f0fu) | ((H << 2) & 0x30303030u);
            const uint32_t w3 = ((A >> 4) & 0x0f0f0f0fu) | (H & 0x30303030u);
            const uint32_t w4 = ((B >> 4) & 0x0f0f0f0fu) | ((H >> 2) & 0x30303030u);
            dots[0] = __builtin_amdgcn_sdot4((int)w1, (int)u4_at(x.q[is], i), dots[0], false);
            dots[1] = __builtin_amdgcn_sdot4((int)w2, (int)u4_at(x.q[2 + is], i), dots[1], false);
            dots[2] = __builtin_amdgcn_sdot4((int)w3, (int)u4_at(x.q[4 + is], i), dots[2], false);
            dots[3] = __builtin_amdgcn_sdot4((int)w4, (int)u4_at(x.q[6 + is], i), dots[3], false);
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            // q - 32 in every weight: dot(q - 32, x) = dot(q, x) - 32 * bsum of the run
            const int32_t dk = dots[k] - 32 * x.s1[is + 2 * k];
            const uint32_t sb = is + 2 * k;  // scale byte within the half's 8
            const int32_t sc = (int8_t)((sb < 4 ? r.sc.x : r.sc.y) >> (8 * (sb & 3)));
            t[4 * is + k] = (d * (float)sc) * (float)dk;
        }
    }
    float a = 0.0f;
    if (h == 0) {
#pragma unroll
        for (int i = 0; i < 8; ++i) a += t[i];
    }
    const float from0 = __uint_as_float(dpp_u32<0x111>(__float_as_uint(a)));  // row_shr:1
    if (h == 1) {
        a = from0;
#pragma unroll
        for (int i = 0; i < 8; ++i) a += t[i];
    }
    return a * x.d;
}

template <typename W>
__device__ __forceinline__ float block_value(const typename W::Raw &r, uint32_t h, const XHalf &x) {
    if constexpr (W::kBytes == 210)
        return q6k_value(r, h, x);
    else
        return k45_value<W>(r, h, x);
}

__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

// Serial f32 sum of a row's n block values in LDS, in block order, onto acc
// (16-byte reads; f is 16-byte aligned).
__device__ __forceinline__ float fold_serial(const float *f, uint32_t n, float acc) {
    const float4 *f4 = reinterpret_cast<const float4 *>(f);
    uint32_t i = 0;
    for (; i + 4 <= n; i += 4) {
        const float4 t = f4[i / 4];
        acc += t.x;
        acc += t.y;
        acc += t.z;
        acc += t.w;
    }
    for (; i < n; ++i) acc += f[i];
    return acc;
}

// ---- staging: coalesced 16-byte loads of a contiguous byte range ---------------
// A wavefront's unit of work is a contiguous byte range of each matrix (a
// group of whole rows, or one 32-block pass of a row) of at most 32 blocks.
// It is fetched as aligned 16-byte chunks, lane l taking chunk 64i + l, so
// one load instruction covers 1 KB of consecutive bytes (the pattern that
// reaches the copy-kernel bandwidth; per-block lane patterns measured
// 25-45% slower), and written to the wavefront's LDS stage.  The lanes then
// read their block's bytes from the stage.  Chunks past the unit read outside
// the buffer range: zeros, no traffic.
// 1 KB chunks per lane per unit: 32 blocks + up to 15 alignment bytes
// (Q4_K 5, Q5_K 6, Q6_K 7).
template <typename W>
constexpr uint32_t kChunks = (32 * W::kBytes + 15 + 1023) / 1024;

template <typename W>
struct Staged {
    u32x4 v[kChunks<W>];
};
template <typename W>
__device__ __forceinline__ void stage_issue(Rsrc w, uint32_t begin, uint32_t end, uint32_t lane, Staged<W> &s) {
    const uint32_t a0 = begin & ~15u;
#pragma unroll
    for (uint32_t i = 0; i < kChunks<W>; ++i) {
        const uint32_t off = a0 + 1024 * i + 16 * lane;
        s.v[i] = __builtin_amdgcn_raw_buffer_load_b128(w, off < end ? off : 0x80000000u, 0, 2);
    }
}
template <typename W>
__device__ __forceinline__ void stage_store(uint8_t *st, uint32_t lane, const Staged<W> &s) {
#pragma unroll
    for (uint32_t i = 0; i < kChunks<W>; ++i) *reinterpret_cast<u32x4 *>(st + 1024 * i + 16 * lane) = s.v[i];
}
// LDS stage bytes per wavefront.
template <typename GW, typename UW, bool FUSED>
constexpr uint32_t kStagePerWave = 1024 * (kChunks<GW> + (FUSED ? kChunks<UW> : 0));

// GW: gate (or the only) format; UW: up format (unused unless FUSED).
// MULTI = false (nb <= 32): a unit is a group of rp = 32/nb consecutive rows;
//   lane pair slot s works on block s % nb of row s / nb; the lane's x slice
//   stays in registers for the whole launch.
// MULTI = true (nb > 32): a unit is pass p (blocks 32p ..) of one row; x
//   slices are read from LDS per unit.
// Each step: next unit's loads issued -> block values of the staged unit ->
// fold buffer; after a row's last unit, lanes 0 .. mats*rows-1 each fold one
// (row, matrix) serially over its block values from 0.0 and the even lanes
// apply silu(gate) * up; then the next unit is written to the stage.
template <typename GW, typename UW, bool FUSED, bool MULTI, bool PREQ, int NW = kGemvWaves>
__global__ __launch_bounds__(NW * kWave) void kquant_gemv_kernel(const uint8_t *__restrict__ gw,
                                                                  const uint8_t *__restrict__ uw,
                                                                  const void *__restrict__ x, float *__restrict__ out,
                                                                  uint32_t rows, uint32_t nb, uint32_t rp) {
    constexpr uint32_t kMats = FUSED ? 2 : 1;
    extern __shared__ __align__(16) uint8_t gemv_smem[];
    __shared__ uint64_t tab_lds[32];
    const XLds xl = carve_lds(gemv_smem, nb);
    const uint32_t wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const uint32_t h = lane & 1, slot = lane >> 1;
    const uint32_t nbp = (nb + 3) & ~3u;
    const uint32_t fold_floats = MULTI ? kMats * nbp : kMats * rp * nbp;
    uint8_t *stage = reinterpret_cast<uint8_t *>(xl.fold + NW * fold_floats) + wave * kStagePerWave<GW, UW, FUSED>;
    uint8_t *ustage = stage + 1024 * kChunks<GW>;
    float *fold = xl.fold + wave * fold_floats;
    const uint32_t grb = nb * GW::kBytes, urb = nb * UW::kBytes;
    const uint32_t g_end = rows * grb, u_end = rows * urb;
    const Rsrc wg = weight_rsrc(gw, g_end);
    const Rsrc wu = weight_rsrc(FUSED ? uw : gw, FUSED ? u_end : g_end);
    const uint32_t passes = MULTI ? (nb + 31) / 32 : 1;
    const uint32_t wstride = gridDim.x * NW;
    const uint32_t wid = blockIdx.x * NW + wave;

    // unit n of this wavefront: (first row, pass) and its byte range per matrix
    auto unit_row = [&](uint32_t n) { return MULTI ? wid + (n / passes) * wstride : (wid + n * wstride) * rp; };
    auto unit_pass = [&](uint32_t n) { return MULTI ? n % passes : 0u; };
    auto range = [&](uint32_t n, uint32_t rb, uint32_t kb, uint32_t lim, uint32_t &b0, uint32_t &b1) {
        const uint32_t r = unit_row(n), p = unit_pass(n);
        if (r >= rows) {
            b0 = b1 = 0;
            return;
        }
        if constexpr (MULTI) {
            b0 = r * rb + 32 * p * kb;
            const uint32_t nblk = nb - 32 * p < 32 ? nb - 32 * p : 32;
            b1 = b0 + nblk * kb;
        } else {
            b0 = r * rb;
            b1 = b0 + rp * rb;
            if (b1 > lim) b1 = lim;
        }
    };

    // Everything the prologue waits for (x, the exp table) is requested
    // before the first unit's weights: loads complete in order, so a wait
    // for a later load would wait for the whole weight burst too.
    XFirst<PREQ> xf;
    x_issue<PREQ>(x, nb, xf);
    uint64_t tab_v = 0;
    {
        constexpr ExpfTable T = make_expf_table();
        if (threadIdx.x < 32) tab_v = T.tab[threadIdx.x];
    }
    Staged<GW> sg;
    Staged<UW> su;
    uint32_t gb0, gb1, ub0 = 0, ub1 = 0;
    range(0, grb, GW::kBytes, g_end, gb0, gb1);
    stage_issue(wg, gb0, gb1, lane, sg);
    if constexpr (FUSED) {
        range(0, urb, UW::kBytes, u_end, ub0, ub1);
        stage_issue(wu, ub0, ub1, lane, su);
    }
#if FELLM_GEMV_DEPTH == 2
    Staged<GW> sg2;
    Staged<UW> su2;
    uint32_t gb0b, gb1b, ub0b = 0, ub1b = 0;
    range(1, grb, GW::kBytes, g_end, gb0b, gb1b);
    stage_issue(wg, gb0b, gb1b, lane, sg2);
    if constexpr (FUSED) {
        range(1, urb, UW::kBytes, u_end, ub0b, ub1b);
        stage_issue(wu, ub0b, ub1b, lane, su2);
    }
#endif
    if (threadIdx.x < 32) tab_lds[threadIdx.x] = tab_v;
    x_finish<PREQ>(x, nb, xl, gemv_smem, xf);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");

    const uint32_t ro = MULTI ? 0 : slot / nb, bfix = MULTI ? 0 : slot - (slot / nb) * nb;
    const bool slot_on = MULTI || ro < rp;
    XHalf xh;
    if constexpr (!MULTI) load_x(xl, bfix, h, xh);
    stage_store(stage, lane, sg);
    if constexpr (FUSED) stage_store(ustage, lane, su);

    // Block values of the staged unit n (byte ranges starting at cg0 / cu0),
    // and after a row's last unit the row folds and the stores.
    auto work = [&](uint32_t n, uint32_t cg0, uint32_t cu0) {
        const uint32_t row0 = unit_row(n), p = unit_pass(n);
        wave_lds_sync();
        const uint32_t b = MULTI ? 32 * p + slot : bfix;  // block index within its row
        const bool on = MULTI ? b < nb : slot_on;
        if constexpr (MULTI) load_x(xl, on ? b : 0, h, xh);
        {
            const uint8_t *blk = stage + (cg0 & 15u) + (MULTI ? slot * GW::kBytes : ro * grb + bfix * GW::kBytes);
            const float v = block_value<GW>(GW::read(blk, h), h, xh);
            if (on && h == (GW::kBytes == 210 ? 1u : 0u)) fold[(MULTI ? 0 : ro * kMats) * nbp + b] = v;
        }
        if constexpr (FUSED) {
            const uint8_t *blk = ustage + (cu0 & 15u) + (MULTI ? slot * UW::kBytes : ro * urb + bfix * UW::kBytes);
            const float v = block_value<UW>(UW::read(blk, h), h, xh);
            if (on && h == (UW::kBytes == 210 ? 1u : 0u)) fold[(MULTI ? 1 : ro * kMats + 1) * nbp + b] = v;
        }
        wave_lds_sync();
        if (!MULTI || p == passes - 1) {
            const uint32_t nf = MULTI ? kMats : kMats * rp;
            float acc = 0.0f;
            if (lane < nf) acc = fold_serial(fold + lane * nbp, nb, 0.0f);
            const uint32_t nrow = MULTI ? 1 : rp;
            if constexpr (FUSED) {
                const float up = dpp_f32<0x101>(acc);  // row_shl:1, lane i reads lane i+1
                const uint32_t r = row0 + lane / 2;
                if (lane < 2 * nrow && (lane & 1) == 0 && r < rows) out[r] = silu(acc, tab_lds) * up;
            } else {
                if (lane < nrow && row0 + lane < rows) out[row0 + lane] = acc;
            }
            wave_lds_sync();
        }
    };

#if FELLM_GEMV_DEPTH == 2
    // Two units in flight: register sets A (sg, su) and B (sg2, su2) take
    // alternate units; the LDS stage holds the unit being reduced.
    for (uint32_t n = 0;; n += 2) {
        if (unit_row(n) >= rows) break;
        uint32_t cg0 = gb0, cu0 = ub0;
        range(n + 2, grb, GW::kBytes, g_end, gb0, gb1);
        stage_issue(wg, gb0, gb1, lane, sg);
        if constexpr (FUSED) {
            range(n + 2, urb, UW::kBytes, u_end, ub0, ub1);
            stage_issue(wu, ub0, ub1, lane, su);
        }
        work(n, cg0, cu0);
        stage_store(stage, lane, sg2);
        if constexpr (FUSED) stage_store(ustage, lane, su2);
        if (unit_row(n + 1) >= rows) break;
        cg0 = gb0b;
        cu0 = ub0b;
        range(n + 3, grb, GW::kBytes, g_end, gb0b, gb1b);
        stage_issue(wg, gb0b, gb1b, lane, sg2);
        if constexpr (FUSED) {
            range(n + 3, urb, UW::kBytes, u_end, ub0b, ub1b);
            stage_issue(wu, ub0b, ub1b, lane, su2);
        }
        work(n + 1, cg0, cu0);
        stage_store(stage, lane, sg);
        if constexpr (FUSED) stage_store(ustage, lane, su);
    }
#else
    for (uint32_t n = 0;; ++n) {
        if (unit_row(n) >= rows) break;
        const uint32_t cg0 = gb0, cu0 = ub0;  // staged unit's byte ranges start here
        range(n + 1, grb, GW::kBytes, g_end, gb0, gb1);
        stage_issue(wg, gb0, gb1, lane, sg);
        if constexpr (FUSED) {
            range(n + 1, urb, UW::kBytes, u_end, ub0, ub1);
            stage_issue(wu, ub0, ub1, lane, su);
        }
        work(n, cg0, cu0);
        stage_store(stage, lane, sg);
        if constexpr (FUSED) stage_store(ustage, lane, su);
    }
#endif
}

// Rows whose bytes do not end on a 16-byte boundary (Q6_K rows of nb % 8 != 0
// blocks) are finished by this direct kernel so that no staged chunk reaches
// past the matrix: one wavefront per row, blocks read straight from memory.
template <typename GW, typename UW, bool FUSED, bool PREQ>
__global__ __launch_bounds__(kGemvBlock) void kquant_gemv_direct(const uint8_t *__restrict__ gw,
                                                                  const uint8_t *__restrict__ uw,
                                                                  const void *__restrict__ x, float *__restrict__ out,
                                                                  uint32_t rows, uint32_t nb) {
    constexpr uint32_t kMats = FUSED ? 2 : 1;
    extern __shared__ __align__(16) uint8_t gemv_smem[];
    __shared__ uint64_t tab_lds[32];
    const XLds xl = carve_lds(gemv_smem, nb);
    const uint32_t wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const uint32_t h = lane & 1, slot = lane >> 1;
    const uint32_t nbp = (nb + 3) & ~3u;
    stage_expf_table(tab_lds);
    fill_x<PREQ>(x, nb, xl, gemv_smem);
    __syncthreads();
    float *fold = xl.fold + wave * kMats * nbp;
    for (uint32_t row = blockIdx.x * kGemvWaves + wave; row < rows; row += gridDim.x * kGemvWaves) {
        for (uint32_t b0 = 0; b0 < nb; b0 += 32) {
            const uint32_t b = b0 + slot, bb = b < nb ? b : nb - 1;
            XHalf xh;
            load_x(xl, bb, h, xh);
            const float vg = block_value<GW>(GW::read(gw + ((size_t)row * nb + bb) * GW::kBytes, h), h, xh);
            if (b < nb && h == (GW::kBytes == 210 ? 1u : 0u)) fold[b] = vg;
            if constexpr (FUSED) {
                const float vu = block_value<UW>(UW::read(uw + ((size_t)row * nb + bb) * UW::kBytes, h), h, xh);
                if (b < nb && h == (UW::kBytes == 210 ? 1u : 0u)) fold[nbp + b] = vu;
            }
        }
        wave_lds_sync();
        float acc = 0.0f;
        if (lane < kMats) acc = fold_serial(fold + lane * nbp, nb, 0.0f);
        if constexpr (FUSED) {
            const float up = dpp_f32<0x101>(acc);
            if (lane == 0) out[row] = silu(acc, tab_lds) * up;
        } else {
            if (lane == 0) out[row] = acc;
        }
        wave_lds_sync();
    }
}

// Standalone Q8_K quantization of x into a blob (one wavefront per block).
__global__ __launch_bounds__(kGemvBlock) void quantize_q8k_kernel(const float *__restrict__ x, uint32_t nb,
                                                                   uint8_t *__restrict__ blob) {
    const XLds xl = carve_lds(blob, nb);
    quantize_x(x, nb, xl, blockIdx.x * kGemvWaves + threadIdx.x / kWave, gridDim.x * kGemvWaves);
}

// Workgroups for `units` row groups (or rows of passes).  Each workgroup
// quantizes x once, so a launch keeps to FELLM_GEMV_MAX_GRID (512) unless
// its wavefronts would each get more than two units; then it widens to at
// most FELLM_GEMV_WIDE_GRID (768), and never past the workgroups that can be
// resident at once (the LDS stage sets that).  With x already quantized the
// prologue is a copy, so more workgroups pay off at every size.
template <bool PREQ, typename K>
uint32_t gemv_grid(K kernel, uint32_t lds, uint32_t units, uint32_t nw = kGemvWaves) {
    const uint32_t need = (units + nw - 1) / nw;
    // the caps count wavefronts in kGemvWaves-wavefront workgroups
    uint32_t grid = (PREQ ? kGemvMaxGridPre : FELLM_GEMV_MAX_GRID) * kGemvWaves / nw;
    if (!PREQ && units / (2 * nw) > grid) {
        // resident workgroups for this kernel and LDS size, looked up once each
        static std::mutex mu;
        static std::vector<std::tuple<const void *, uint32_t, uint32_t>> seen;
        uint32_t cap = 0;
        {
            std::lock_guard<std::mutex> lock(mu);
            for (const auto &[k, l, c] : seen)
                if (k == reinterpret_cast<const void *>(kernel) && l == lds) cap = c;
            if (cap == 0) {
                cap = resident_grid(kernel, (int)nw * kWave, lds, 8);
                seen.emplace_back(reinterpret_cast<const void *>(kernel), lds, cap);
            }
        }
        uint32_t wide = units / (2 * nw);
        if (wide > FELLM_GEMV_WIDE_GRID * kGemvWaves / nw) wide = FELLM_GEMV_WIDE_GRID * kGemvWaves / nw;
        if (wide > cap) wide = cap;
        if (wide > grid) grid = wide;
    }
    return need < grid ? need : grid;
}

template <typename GW, typename UW, bool FUSED, bool PREQ = false>
int launch_gemv(const void *gw, const void *uw, const void *x, float *out, uint32_t rows, uint32_t cols,
                hipStream_t s) {
    const uint32_t nb = cols / 256;
    const uint32_t mats = FUSED ? 2 : 1;
    const uint32_t nbp = (nb + 3) & ~3u;
    const uint8_t *g8 = static_cast<const uint8_t *>(gw), *u8 = static_cast<const uint8_t *>(uw);
    // Staged rows: every matrix's staged bytes end on a 16-byte boundary.
    uint32_t m = 1;
    while ((uint64_t)m * nb * GW::kBytes % 16 || (FUSED && (uint64_t)m * nb * UW::kBytes % 16)) ++m;
    const uint32_t rows_main = rows / m * m;
    // Buffer ranges are 32-bit: stage at most 2^31 - 1 bytes of a matrix per launch.
    const uint64_t rb = (uint64_t)nb * (GW::kBytes > UW::kBytes ? GW::kBytes : UW::kBytes);
    const uint32_t chunk = (uint32_t)(((1ull << 31) - 1) / rb) / m * m;
    for (uint32_t r0 = 0; r0 < rows_main; r0 += chunk) {
        const uint32_t n = rows_main - r0 < chunk ? rows_main - r0 : chunk;
        const uint8_t *g = g8 + (uint64_t)r0 * nb * GW::kBytes;
        const uint8_t *u = FUSED ? u8 + (uint64_t)r0 * nb * UW::kBytes : nullptr;
        if (nb <= 32) {
            const uint32_t rp = 32 / nb;
            constexpr int NWO = FELLM_GEMV_ONE_WAVES;
            const uint32_t lds = gemv_lds_bytes(nb, mats * rp * nbp, NWO) + NWO * kStagePerWave<GW, UW, FUSED>;
            const uint32_t units = (n + rp - 1) / rp;
            const uint32_t grid = gemv_grid<PREQ>(kquant_gemv_kernel<GW, UW, FUSED, false, PREQ, NWO>, lds, units, NWO);
            FELLM_LAUNCH((kquant_gemv_kernel<GW, UW, FUSED, false, PREQ, NWO>), dim3(grid), dim3(NWO * kWave), lds, s, g, u, x,
                               out + r0, n, nb, rp);
        } else {
            auto go_multi = [&]<int NW>() {
                const uint32_t lds = gemv_lds_bytes(nb, mats * nbp, NW) + NW * kStagePerWave<GW, UW, FUSED>;
                const uint32_t grid = gemv_grid<PREQ>(kquant_gemv_kernel<GW, UW, FUSED, true, PREQ, NW>, lds, n, NW);
                FELLM_LAUNCH((kquant_gemv_kernel<GW, UW, FUSED, true, PREQ, NW>), dim3(grid), dim3(NW * kWave), lds, s, g,
                             u, x, out + r0, n, nb, 1u);
            };
            // FELLM_GEMV_MULTI_WAVES wavefronts while their stages and x fit the
            // workgroup's LDS (fused Q5_K / Q6_K rows of ~40k columns do not).
            constexpr int NWM = FELLM_GEMV_MULTI_WAVES;
            if (gemv_lds_bytes(nb, mats * nbp, NWM) + NWM * kStagePerWave<GW, UW, FUSED> <= kGemvLdsLimit)
                go_multi.template operator()<NWM>();
            else
                go_multi.template operator()<kGemvWaves>();
        }
        const int rc = launch_status();
        if (rc != FELLM_OK) return rc;
    }
    if (rows_main < rows) {
        const uint32_t n = rows - rows_main;
        const uint8_t *g = g8 + (uint64_t)rows_main * nb * GW::kBytes;
        const uint8_t *u = FUSED ? u8 + (uint64_t)rows_main * nb * UW::kBytes : nullptr;
        FELLM_LAUNCH((kquant_gemv_direct<GW, UW, FUSED, PREQ>), dim3((n + kGemvWaves - 1) / kGemvWaves),
                           dim3(kGemvBlock), gemv_lds_bytes(nb, mats * nbp), s, g, u, x, out + rows_main, n, nb);
        const int rc = launch_status();
        if (rc != FELLM_OK) return rc;
    }
    return FELLM_OK;
}

bool kquant_ok(uint32_t dt) { return dt == FELLM_DTYPE_Q4K || dt == FELLM_DTYPE_Q5K || dt == FELLM_DTYPE_Q6K; }

// Q4_K and Q5_K blocks (144 and 176 bytes) are read with aligned 16-byte loads.
bool weight_aligned(const void *w, uint32_t dt) { return dt == FELLM_DTYPE_Q6K || aligned_to(w, 16); }

int check_gemv(const void *w, uint32_t dt, const void *x, const float *out, uint32_t cols) {
    if (!w || !x || !out) return FELLM_ERR_ARITY;
    if (!kquant_ok(dt)) return FELLM_ERR_DTYPE;
    if (cols == 0 || cols % 256 != 0 || cols > kGemvMaxCols) return FELLM_ERR_SHAPE;
    if (!aligned_to(x, 16) || !weight_aligned(w, dt)) return FELLM_ERR_SHAPE;
    return FELLM_OK;
}

}  // namespace
}  // namespace fellm

extern "C" int fellm_rocm_gate_up_swiglu(const void *gate_w, uint32_t gate_dtype, const void *up_w, uint32_t up_dtype,
                                         uint32_t rows, uint32_t cols, const float *x, float *out, void *stream) {
    using namespace fellm;
    if (rows == 0 && kquant_ok(gate_dtype) && kquant_ok(up_dtype) && cols % 256 == 0) return FELLM_OK;
    int rc = check_gemv(gate_w, gate_dtype, x, out, cols);
    if (rc == FELLM_OK) rc = check_gemv(up_w, up_dtype, x, out, cols);
    if (rc != FELLM_OK) return rc;
    hipStream_t s = as_stream(stream);
#define FELLM_GU(GT, GD, UT, UD) \
    if (gate_dtype == GD && up_dtype == UD) return launch_gemv<GT, UT, true>(gate_w, up_w, x, out, rows, cols, s);
#define FELLM_GU_ROW(GT, GD)                 \
    FELLM_GU(GT, GD, Q4K, FELLM_DTYPE_Q4K)   \
    FELLM_GU(GT, GD, Q5K, FELLM_DTYPE_Q5K)   \
    FELLM_GU(GT, GD, Q6K, FELLM_DTYPE_Q6K)
    FELLM_GU_ROW(Q4K, FELLM_DTYPE_Q4K)
    FELLM_GU_ROW(Q5K, FELLM_DTYPE_Q5K)
    FELLM_GU_ROW(Q6K, FELLM_DTYPE_Q6K)
#undef FELLM_GU_ROW
#undef FELLM_GU
    return FELLM_ERR_DTYPE;
}

extern "C" int fellm_rocm_matvec_kquant(const void *w, uint32_t w_dtype, uint32_t rows, uint32_t cols, const float *x,
                                        float *y, void *stream) {
    using namespace fellm;
    if (rows == 0 && kquant_ok(w_dtype) && cols % 256 == 0) return FELLM_OK;
    const int rc = check_gemv(w, w_dtype, x, y, cols);
    if (rc != FELLM_OK) return rc;
    hipStream_t s = as_stream(stream);
    if (w_dtype == FELLM_DTYPE_Q4K) return launch_gemv<Q4K, Q4K, false>(w, nullptr, x, y, rows, cols, s);
    if (w_dtype == FELLM_DTYPE_Q5K) return launch_gemv<Q5K, Q5K, false>(w, nullptr, x, y, rows, cols, s);
    return launch_gemv<Q6K, Q6K, false>(w, nullptr, x, y, rows, cols, s);
}

extern "C" uint64_t fellm_rocm_q8k_bytes(uint32_t cols) {
    using namespace fellm;
    return cols % 256 ? 0 : q8k_blob_bytes(cols / 256);
}

extern "C" int fellm_rocm_quantize_q8k(const float *x, uint32_t cols, void *xq, void *stream) {
    using namespace fellm;
    if (!x || !xq) return FELLM_ERR_ARITY;
    if (cols == 0 || cols % 256 != 0 || cols > kGemvMaxCols) return FELLM_ERR_SHAPE;
    if (!aligned_to(x, 16) || !aligned_to(xq, 16)) return FELLM_ERR_SHAPE;
    const uint32_t nb = cols / 256;
    FELLM_LAUNCH(quantize_q8k_kernel, dim3((nb + kGemvWaves - 1) / kGemvWaves), dim3(kGemvBlock), 0,
                       as_stream(stream), x, nb, static_cast<uint8_t *>(xq));
    return launch_status();
}

extern "C" int fellm_rocm_gate_up_swiglu_q8k(const void *gate_w, uint32_t gate_dtype, const void *up_w,
                                             uint32_t up_dtype, uint32_t rows, uint32_t cols, const void *xq,
                                             float *out, void *stream) {
    using namespace fellm;
    if (rows == 0 && kquant_ok(gate_dtype) && kquant_ok(up_dtype) && cols % 256 == 0) return FELLM_OK;
    int rc = check_gemv(gate_w, gate_dtype, xq, out, cols);
    if (rc == FELLM_OK) rc = check_gemv(up_w, up_dtype, xq, out, cols);
    if (rc != FELLM_OK) return rc;
    hipStream_t s = as_stream(stream);
#define FELLM_GU(GT, GD, UT, UD) \
    if (gate_dtype == GD && up_dtype == UD) return launch_gemv<GT, UT, true, true>(gate_w, up_w, xq, out, rows, cols, s);
#define FELLM_GU_ROW(GT, GD)                 \
    FELLM_GU(GT, GD, Q4K, FELLM_DTYPE_Q4K)   \
    FELLM_GU(GT, GD, Q5K, FELLM_DTYPE_Q5K)   \
    FELLM_GU(GT, GD, Q6K, FELLM_DTYPE_Q6K)
    FELLM_GU_ROW(Q4K, FELLM_DTYPE_Q4K)
    FELLM_GU_ROW(Q5K, FELLM_DTYPE_Q5K)
    FELLM_GU_ROW(Q6K, FELLM_DTYPE_Q6K)
#undef FELLM_GU_ROW
#undef FELLM_GU
    return FELLM_ERR_DTYPE;
}

extern "C" int fellm_rocm_matvec_kquant_q8k(const void *w, uint32_t w_dtype, uint32_t rows, uint32_t cols,
                                            const void *xq, float *y, void *stream) {
    using namespace fellm;
    if (rows == 0 && kquant_ok(w_dtype) && cols % 256 == 0) return FELLM_OK;
    const int rc = check_gemv(w, w_dtype, xq, y, cols);
    if (rc != FELLM_OK) return rc;
    hipStream_t s = as_stream(stream);
    if (w_dtype == FELLM_DTYPE_Q4K) return launch_gemv<Q4K, Q4K, false, true>(w, nullptr, xq, y, rows, cols, s);
    if (w_dtype == FELLM_DTYPE_Q5K) return launch_gemv<Q5K, Q5K, false, true>(w, nullptr, xq, y, rows, cols, s);
    return launch_gemv<Q6K, Q6K, false, true>(w, nullptr, xq, y, rows, cols, s);
}
