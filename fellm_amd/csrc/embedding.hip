// Token-embedding gather with dequant-on-gather, optionally fused with RMSNorm.
//
// Reference: crates/backend-cpu/src/backend.rs:1026-1046 (launch_embedding)
//   -> kernels/embedding.rs:10-23 (embedding_row) -> dequant.rs:19-55
//   F32 copy, F16 widen (half::f16::to_f32), BF16 bits << 16,
//   Q4_K dequant.rs:251-305, Q6_K dequant.rs:315-370, Q5_K dequant.rs:59-107,
//   Q8_0 dequant.rs:172-192 (the last two only through the LDS gather).
//
// One workgroup gathers one token row.  A row is cut into "parts", each a
// fixed set of output elements one thread produces:
//   dense : 8 consecutive elements (one 16-byte load for 16-bit tables);
//   Q4_K  : 16 elements = one 8-byte slice of a 32-byte qs chunk, whose low
//           nibbles are 8 consecutive outputs and high nibbles the 8 outputs
//           32 further on; the 16-byte block header (d, dmin, 12 scale bytes,
//           16-byte aligned because a block is 144 = 9*16 bytes) is loaded
//           straight from global memory and shared via L1 by the 16 parts of
//           the block;
//   Q6_K  : 16 elements = 4 runs of 4, read with unaligned dword loads
//           (210-byte blocks are only 2-byte aligned).  Gathers by id take
//           kquant_gather_lds_kernel instead: the raw row is copied into LDS
//           with coalesced 16-byte loads and decoded there in 8-output parts.
// The arithmetic order is the reference's, with FMA contraction disabled at
// compile time:  Q4_K  y = (d*sc)*q - (dmin*m);   Q6_K  y = (d*sc)*(q-32).
// With NORM the decoded row stays in registers for the sum of squares and
// is written once as h (gathered row) and once as y (normalised row).
#include "common.hpp"

// Build knob: threads per workgroup (one token row per workgroup).
// Build knob: non-temporal loads of dense table rows (1).  Alone the gather
// runs the same either way; after a kernel that leaves dirty lines they
// measured 19.9 -> 16.5 us at 4096 rows x 4096 f16 inside the op chain.
#ifndef FELLM_EMB_NT_LOAD
#define FELLM_EMB_NT_LOAD 1
#endif
// Build knob: non-temporal stores for the fused gather + RMSNorm (1) or regular (0).
// Regular stores make the fused kernel alone faster, but leave h and y dirty
// in the caches for the next kernel to write back.  Measured at configs[2]
// with the four ops run in turn (interleaved on one box): non-temporal
// stores took the fused Q4_K / Q6_K gathers + RMSNorm from 22.7-22.8 /
// 24.9-25.0 to 21.2-21.4 / 24.2 us and the plain Q4_K / Q6_K gathers that
// follow them from 15.2-15.4 / 16.5-16.8 to 11.1-11.3 / 14.8-15.0 us.
#ifndef FELLM_EMB_NORM_NT
#define FELLM_EMB_NORM_NT 1
#endif
#ifndef FELLM_EMB_BLOCK
#define FELLM_EMB_BLOCK 256
#endif
// Build knob: Q4_K / Q6_K scale factors staged in LDS once per row (1) or
// decoded from the block header by every part (0); 2 also takes Q4_K in
// parts of 8 consecutive outputs, every part of a thread decoded before its
// stores.  Measured at configs[2] (Q4_K / Q6_K gather, interleaved on one
// box): staged 15.2-15.4 / 19.0-19.3 us; 8-output Q4_K parts 14.8-15.0 us
// (decoding all parts first; 16.0 us part by part); 8-output Q6_K parts
// 22.2-22.8 us, so Q6_K keeps its 16-output parts.
#ifndef FELLM_EMB_STAGE
#define FELLM_EMB_STAGE 2
#endif
// Build knob: plain gathers decode and store part by part (1) or decode all
// parts into registers first (0).
#ifndef FELLM_EMB_LOOP
#define FELLM_EMB_LOOP 1
#endif
// Build knob: workgroup size of the plain Q4_K gather (parts of 8 outputs,
// all of a thread's parts decoded before its stores).  Measured at
// configs[2] (8192 Zipf rows of 3584, interleaved on one box): 128 threads
// 13.3-13.4 us against 15.0-15.1 us for 256, 13.5-13.9 us for 64 and
// 17.4-17.6 us for 512.  The fused gather + RMSNorm measured slower with 128
// threads (23.2-23.5 against 21.8-22.0 us) and keeps FELLM_EMB_BLOCK.  Q6_K
// stays on the part-by-part loop: on this all-parts layout it measured
// 19.0-19.3 us with 256 threads (level with the loop's 19.4), 21.0-21.1 with
// 128 and 22.1-22.7 with 64.
// Build knob: plain gathers through the looping staged layout (Q6_K)
// assemble each row in LDS and write it with 16-byte stores (1), or store
// each part's four 4-element runs directly (0).  A Q6_K part's outputs are
// four 8-byte runs, so the direct stores issue 2.3x the store instructions
// of Q4_K's 16-byte parts for the same bytes (SQ_INSTS_VMEM_WR).  Measured
// at configs[2], interleaved on one box: 18.1-18.2 against 19.2-19.4 us.
// The Q4_K layouts already store 16 bytes per part.
#ifndef FELLM_EMB_LDS_OUT
#define FELLM_EMB_LDS_OUT 1
#endif
#ifndef FELLM_EMB_Q4K_BLOCK
#define FELLM_EMB_Q4K_BLOCK 128
#endif
// Build knob: workgroups per compute unit of the persistent, pipelined plain
// gather (0: one workgroup per row).  Measured at configs[1] (4096 f16 rows of
// 4096, interleaved on one box): one workgroup per row 13.2-13.4 us; 2 per CU
// 16.6-16.7 us; 4 per CU 13.4-13.5 us; 8 per CU (the occupancy limit of
// 256-thread workgroups) 12.3-12.4 us.  With other workgroup sizes
// (FELLM_EMB_BLOCK): 512 threads at 4 or 2 per CU 13.0-13.2 us, 128 threads
// at 16 per CU 13.0-13.2 us, against 12.4 us.  A one-shot grid with every
// part of a row loaded before its stores: 64 threads per row 13.1, 128 12.7,
// 256 13.8, 512 13.1 us.
#ifndef FELLM_EMB_PIPE
#define FELLM_EMB_PIPE 8
#endif
// Build knob: dense gathers in one-shot workgroups of this many threads per
// row, every part of a thread loaded before its stores (0: the persistent
// pipelined kernel when there are enough rows).
#ifndef FELLM_EMB_DENSE_BLOCK
#define FELLM_EMB_DENSE_BLOCK 0
#endif
// Build knobs of the K-quant gathers that copy each raw row (segment) into
// LDS with coalesced 16-byte loads and decode it from there
// (kquant_gather_lds_kernel): its workgroup size, which gathers take it
// (plain Q6_K, fused Q6_K + RMSNorm, plain Q4_K, fused Q4_K + RMSNorm; the
// others keep the staged layouts above), and the 256-element blocks a
// workgroup takes (FELLM_EMB_Q6K_BPW; 0: the whole row).  Measured at
// configs[2] (8192 Zipf rows of 3584, interleaved on one box), plain Q6_K,
// whole rows: 64 threads 16.2-16.3 us, 128 17.6-17.7, 256 19.3-19.4 (the
// staged layout 17.8-17.9); storing each part as soon as the next is decoded
// 16.6 (64) and 17.6-17.8 (128); one wavefront per row walking rows with the
// next row's chunks in flight 16.6-16.9 at 8 workgroups per CU, 17.2 at 4,
// 19.7 at 2; 7, 4, 2 or 1 blocks per workgroup 19.7, 21.6-21.8, 23.3-23.4,
// 34.8-35.0.  In isolation (the same call repeated, table rows warm in the
// caches) the staged layout is faster (14.8-15.0 against 17.0-17.3 us); with
// a 768 MB fill between calls the LDS layout is (21.6 against 22.8 us).  The
// fused Q6_K gather + RMSNorm, rows of up to 4096 elements: 29.5 -> 25.1 us.
// Q4_K's 16-byte-aligned blocks gain nothing from the copy: the LDS layout
// measured 13.1-13.2 against 11.4 us (plain) and 25.2-25.4 against
// 21.2-21.4 us (fused), so Q4_K keeps its staged 8-output parts.
#ifndef FELLM_EMB_KQ_LDS_BLOCK
#define FELLM_EMB_KQ_LDS_BLOCK 64
#endif
#ifndef FELLM_EMB_Q6K_LDS
#define FELLM_EMB_Q6K_LDS 1
#endif
#ifndef FELLM_EMB_Q6K_LDS_NORM
#define FELLM_EMB_Q6K_LDS_NORM 1
#endif
#ifndef FELLM_EMB_Q4K_LDS
#define FELLM_EMB_Q4K_LDS 0
#endif
#ifndef FELLM_EMB_Q4K_LDS_NORM
#define FELLM_EMB_Q4K_LDS_NORM 0
#endif
#ifndef FELLM_EMB_Q6K_BPW
#define FELLM_EMB_Q6K_BPW 0
#endif


namespace fellm {
namespace {

__device__ __forceinline__ float half_bits_to_f32(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}

// ---- decoders --------------------------------------------------------------
template <typename A, int VEC>
struct DenseDec {
    static constexpr bool STAGED = false;
    static constexpr bool DENSE = true;  // gathers may take the persistent kernel
    static constexpr int OUT = VEC, RUNS = 1, RUNLEN = VEC;
    __host__ __device__ static uint64_t row_bytes(uint32_t dim) { return (uint64_t)dim * sizeof(typename A::T); }
    __host__ __device__ static uint32_t parts(uint32_t dim) { return dim / VEC; }
    __device__ static uint32_t run_off(uint32_t p, int) { return p * VEC; }
    __device__ static void decode(const uint8_t *row, uint32_t p, float (&v)[OUT]) {
        if constexpr (FELLM_EMB_NT_LOAD)
            load_f32_nt<A, VEC>(reinterpret_cast<const typename A::T *>(row) + (size_t)p * VEC, v);
        else
            load_f32<A, VEC>(reinterpret_cast<const typename A::T *>(row) + (size_t)p * VEC, v);
    }
};

struct Q4KDec {
    static constexpr bool STAGED = false;
    static constexpr int OUT = 16, RUNS = 2, RUNLEN = 8;
    __host__ __device__ static uint64_t row_bytes(uint32_t dim) { return (uint64_t)(dim / 256) * 144; }
    __host__ __device__ static uint32_t parts(uint32_t dim) { return (dim / 256) * 16; }
    __device__ static uint32_t run_off(uint32_t p, int r) {
        const uint32_t q = p % 16;
        return (p / 16) * 256 + 64 * (q / 4) + 8 * (q % 4) + 32 * r;
    }
    __device__ static void decode(const uint8_t *row, uint32_t p, float (&v)[OUT]) {
        const uint8_t *blk = row + (size_t)(p / 16) * 144;
        const uint32_t q = p % 16, c = q / 4, j = q % 4;
        const uint4 hdr = *reinterpret_cast<const uint4 *>(blk);
        const float d = half_bits_to_f32(hdr.x & 0xffffu);
        const float dmin = half_bits_to_f32(hdr.x >> 16);
        uint32_t sc0, m0, sc1, m1;
        k4_scale_min(2 * c, hdr.y, hdr.z, hdr.w, sc0, m0);
        k4_scale_min(2 * c + 1, hdr.y, hdr.z, hdr.w, sc1, m1);
        const float d1 = d * (float)sc0, m1f = dmin * (float)m0;
        const float d2 = d * (float)sc1, m2f = dmin * (float)m1;
        const uint2 qs = *reinterpret_cast<const uint2 *>(blk + 16 + 32 * c + 8 * j);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t b = ((k < 4 ? qs.x : qs.y) >> (8 * (k % 4))) & 0xffu;
            v[k] = d1 * (float)(b & 0x0fu) - m1f;
            v[8 + k] = d2 * (float)(b >> 4) - m2f;
        }
    }
};

struct Q6KDec {
    static constexpr bool STAGED = false;
    static constexpr int OUT = 16, RUNS = 4, RUNLEN = 4;
    __host__ __device__ static uint64_t row_bytes(uint32_t dim) { return (uint64_t)(dim / 256) * 210; }
    __host__ __device__ static uint32_t parts(uint32_t dim) { return (dim / 256) * 16; }
    __device__ static uint32_t run_off(uint32_t p, int r) {
        const uint32_t q = p % 16;
        return (p / 16) * 256 + 128 * (q / 8) + 4 * (q % 8) + 32 * r;
    }
    // Block layout (dequant.rs:315-370): ql[128], qh[64], int8 scales[16],
    // f16 d at 208.  210-byte blocks are only 2-byte aligned; gfx950 serves
    // unaligned dword loads directly, so each part reads its 4+4+4 quant
    // bytes and the 8 scale bytes of its half as unaligned dwords.
    __device__ static uint32_t ld32(const uint8_t *p) {
        uint32_t v;
        __builtin_memcpy(&v, p, 4);
        return v;
    }
    __device__ static void decode(const uint8_t *row, uint32_t p, float (&v)[OUT]) {
        const uint8_t *blk = row + (size_t)(p / 16) * 210;
        const uint32_t q = p % 16, hh = q / 8, l0 = 4 * (q % 8), is = l0 / 16;
        const uint32_t qa = ld32(blk + 64 * hh + l0);       // ql[l0 .. l0+3]
        const uint32_t qb = ld32(blk + 64 * hh + 32 + l0);  // ql[l0+32 .. l0+35]
        const uint32_t qhw = ld32(blk + 128 + 32 * hh + l0);
        const uint32_t s0 = ld32(blk + 192 + 8 * hh), s1 = ld32(blk + 196 + 8 * hh);
        uint16_t dbits;
        __builtin_memcpy(&dbits, blk + 208, 2);
        const float d = half_bits_to_f32(dbits);
        // scales[is + 2k] for k = 0..3 (is is 0 or 1): bytes is, is+2 of s0 and of s1.
        const int32_t sc0 = (int8_t)(s0 >> (8 * is)), sc1 = (int8_t)(s0 >> (8 * (is + 2)));
        const int32_t sc2 = (int8_t)(s1 >> (8 * is)), sc3 = (int8_t)(s1 >> (8 * (is + 2)));
        const float ds0 = d * (float)sc0, ds1 = d * (float)sc1;
        const float ds2 = d * (float)sc2, ds3 = d * (float)sc3;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int32_t a = (qa >> (8 * m)) & 0xff, b = (qb >> (8 * m)) & 0xff, h = (qhw >> (8 * m)) & 0xff;
            const int32_t q1 = ((a & 0xf) | ((h & 3) << 4)) - 32;
            const int32_t q2 = ((b & 0xf) | (((h >> 2) & 3) << 4)) - 32;
            const int32_t q3 = ((a >> 4) | (((h >> 4) & 3) << 4)) - 32;
            const int32_t q4 = ((b >> 4) | (((h >> 6) & 3) << 4)) - 32;
            v[m] = ds0 * (float)q1;
            v[4 + m] = ds1 * (float)q2;
            v[8 + m] = ds2 * (float)q3;
            v[12 + m] = ds3 * (float)q4;
        }
    }
};

// Staged decoders: the row's per-group scale factors are computed once per
// workgroup into LDS (4 float4 slots per 256-element block), so a part reads
// 16 bytes of LDS instead of the block header from global memory and skips
// the scale unpacking.  Same parts, same arithmetic, same order as Q4KDec /
// Q6KDec:  load() issues the part's quant-byte loads, stage() fills one LDS
// slot, finish() decodes once the slots are visible.
struct Q4KStaged {
    static constexpr bool STAGED = true;
    static constexpr int OUT = 16, RUNS = 2, RUNLEN = 8;
    using Raw = uint2;
    __host__ __device__ static uint64_t row_bytes(uint32_t dim) { return (uint64_t)(dim / 256) * 144; }
    __host__ __device__ static uint32_t parts(uint32_t dim) { return (dim / 256) * 16; }
    __device__ static uint32_t run_off(uint32_t p, int r) { return Q4KDec::run_off(p, r); }
    __device__ static Raw load(const uint8_t *row, uint32_t p) {
        const uint32_t q = p % 16;
        return *reinterpret_cast<const uint2 *>(row + (size_t)(p / 16) * 144 + 16 + 32 * (q / 4) + 8 * (q % 4));
    }
    // Slot 4b + c: (d * sc[2c], dmin * m[2c], d * sc[2c+1], dmin * m[2c+1]) of block b.
    __device__ static float4 stage(const uint8_t *row, uint32_t slot) {
        const uint4 hdr = *reinterpret_cast<const uint4 *>(row + (size_t)(slot / 4) * 144);
        const uint32_t c = slot % 4;
        const float d = half_bits_to_f32(hdr.x & 0xffffu);
        const float dmin = half_bits_to_f32(hdr.x >> 16);
        uint32_t sc0, m0, sc1, m1;
        k4_scale_min(2 * c, hdr.y, hdr.z, hdr.w, sc0, m0);
        k4_scale_min(2 * c + 1, hdr.y, hdr.z, hdr.w, sc1, m1);
        return make_float4(d * (float)sc0, dmin * (float)m0, d * (float)sc1, dmin * (float)m1);
    }
    __device__ static void finish(Raw qs, uint32_t p, const float4 *lds, float (&v)[OUT]) {
        const float4 f = lds[(p / 16) * 4 + (p % 16) / 4];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t b = ((k < 4 ? qs.x : qs.y) >> (8 * (k % 4))) & 0xffu;
            v[k] = f.x * (float)(b & 0x0fu) - f.y;
            v[8 + k] = f.z * (float)(b >> 4) - f.w;
        }
    }
};

struct Q6KStaged {
    static constexpr bool STAGED = true;
    static constexpr int OUT = 16, RUNS = 4, RUNLEN = 4;
    using Raw = uint3;
    __host__ __device__ static uint64_t row_bytes(uint32_t dim) { return (uint64_t)(dim / 256) * 210; }
    __host__ __device__ static uint32_t parts(uint32_t dim) { return (dim / 256) * 16; }
    __device__ static uint32_t run_off(uint32_t p, int r) { return Q6KDec::run_off(p, r); }
    __device__ static Raw load(const uint8_t *row, uint32_t p) {
        const uint8_t *blk = row + (size_t)(p / 16) * 210;
        const uint32_t q = p % 16, hh = q / 8, l0 = 4 * (q % 8);
        return make_uint3(Q6KDec::ld32(blk + 64 * hh + l0), Q6KDec::ld32(blk + 64 * hh + 32 + l0),
                          Q6KDec::ld32(blk + 128 + 32 * hh + l0));
    }
    // Slot 4b + 2hh + is: d * sc[8hh + is + 2k] for k = 0..3 of block b.
    __device__ static float4 stage(const uint8_t *row, uint32_t slot) {
        const uint8_t *blk = row + (size_t)(slot / 4) * 210;
        const uint32_t hh = (slot % 4) / 2, is = slot % 2;
        const uint32_t s0 = Q6KDec::ld32(blk + 192 + 8 * hh), s1 = Q6KDec::ld32(blk + 196 + 8 * hh);
        uint16_t dbits;
        __builtin_memcpy(&dbits, blk + 208, 2);
        const float d = half_bits_to_f32(dbits);
        return make_float4(d * (float)(int8_t)(s0 >> (8 * is)), d * (float)(int8_t)(s0 >> (8 * (is + 2))),
                           d * (float)(int8_t)(s1 >> (8 * is)), d * (float)(int8_t)(s1 >> (8 * (is + 2))));
    }
    __device__ static void finish(Raw raw, uint32_t p, const float4 *lds, float (&v)[OUT]) {
        const uint32_t q = p % 16, hh = q / 8, is = (4 * (q % 8)) / 16;
        const float4 f = lds[(p / 16) * 4 + 2 * hh + is];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int32_t a = (raw.x >> (8 * m)) & 0xff, b = (raw.y >> (8 * m)) & 0xff, h = (raw.z >> (8 * m)) & 0xff;
            const int32_t q1 = ((a & 0xf) | ((h & 3) << 4)) - 32;
            const int32_t q2 = ((b & 0xf) | (((h >> 2) & 3) << 4)) - 32;
            const int32_t q3 = ((a >> 4) | (((h >> 4) & 3) << 4)) - 32;
            const int32_t q4 = ((b >> 4) | (((h >> 6) & 3) << 4)) - 32;
            v[m] = f.x * (float)q1;
            v[4 + m] = f.y * (float)q2;
            v[8 + m] = f.z * (float)q3;
            v[12 + m] = f.w * (float)q4;
        }
    }
};

// Staged decoders with parts of 8 consecutive outputs (one 16-byte store
// of a 16-bit output per part, so a wavefront writes 1 KB of a row
// contiguously); same scale slots and arithmetic as Q4KStaged / Q6KStaged.
// Q4_K: outputs o = 8p' .. 8p'+7 of block p / 32 (p' = p % 32): chunk
// c = o / 64, offset j = o % 64, low nibbles of qs[32c + j ..] when j < 32,
// else high nibbles of qs[32c + j - 32 ..] (dequant.rs:268-289).
struct Q4KStaged8 {
    static constexpr bool STAGED = true;
    static constexpr bool ALL_PARTS_IN_REGS = true;  // plain gathers decode every part before storing
    static constexpr int OUT = 8, RUNS = 1, RUNLEN = 8;
    using Raw = uint2;
    __host__ __device__ static uint64_t row_bytes(uint32_t dim) { return (uint64_t)(dim / 256) * 144; }
    __host__ __device__ static uint32_t parts(uint32_t dim) { return dim / 8; }
    __device__ static uint32_t run_off(uint32_t p, int) { return p * 8; }
    __device__ static Raw load(const uint8_t *row, uint32_t p) {
        const uint32_t o = 8 * (p % 32);
        return *reinterpret_cast<const uint2 *>(row + (size_t)(p / 32) * 144 + 16 + 32 * (o / 64) + (o % 32));
    }
    __device__ static float4 stage(const uint8_t *row, uint32_t slot) { return Q4KStaged::stage(row, slot); }
    __device__ static void finish(Raw qs, uint32_t p, const float4 *lds, float (&v)[OUT]) {
        const uint32_t o = 8 * (p % 32);
        const float4 f = lds[(p / 32) * 4 + o / 64];
        const bool hi = (o % 64) >= 32;
        const float dq = hi ? f.z : f.x, mq = hi ? f.w : f.y;
        const uint32_t sh = hi ? 4 : 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t b = ((k < 4 ? qs.x : qs.y) >> (8 * (k % 4) + sh)) & 0x0fu;
            v[k] = dq * (float)b - mq;
        }
    }
};

// Plain gathers stream their output with non-temporal stores; the fused
// gather + RMSNorm stores after its reduction barrier and measured faster
// with regular stores.
template <typename D, typename O, bool NT>
__device__ __forceinline__ void store_part(typename O::T *row, uint32_t p, const float (&v)[D::OUT]) {
#pragma unroll
    for (int r = 0; r < D::RUNS; ++r) {
        float t[D::RUNLEN];
#pragma unroll
        for (int k = 0; k < D::RUNLEN; ++k) t[k] = v[r * D::RUNLEN + k];
        if constexpr (NT)
            store_f32_nt<O, D::RUNLEN>(row + D::run_off(p, r), t);
        else
            store_f32<O, D::RUNLEN>(row + D::run_off(p, r), t);
    }
}

// Stores of the fused gather + RMSNorm (FELLM_EMB_NORM_NT policy).
template <typename O, int N>
__device__ __forceinline__ void norm_out_store(typename O::T *p, const float (&v)[N]) {
    if constexpr (FELLM_EMB_NORM_NT) store_f32_nt<O, N>(p, v); else store_f32<O, N>(p, v);
}

constexpr int kEmbBlock = FELLM_EMB_BLOCK;

// One workgroup per token row.  Each thread decodes its (up to MAXC) parts
// into registers before storing anything, so all of its loads are in flight
// together.  MAXC == 0 selects a looping variant for rows longer than
// 8 * kEmbBlock parts (no fused norm).
template <typename D, typename O, int MAXC, bool NORM, int BLOCK = kEmbBlock, bool LDS_OUT = false>
__global__ __launch_bounds__(BLOCK) void embedding_kernel(
    const uint8_t *__restrict__ table, uint64_t vocab, uint32_t dim, const uint32_t *__restrict__ ids,
    typename O::T *__restrict__ h, typename O::T *__restrict__ y, const float *__restrict__ w, float eps,
    uint32_t *__restrict__ err) {
    __shared__ float red[BLOCK / kWave];
    const uint32_t row = blockIdx.x;
    const uint32_t id = ids ? ids[row] : row;  // no ids: row r of the table (Cast's dequantization)
    const bool bad = id >= vocab;
    if (bad && threadIdx.x == 0 && err) atomicOr(err, 1u);
    const uint64_t rb = D::row_bytes(dim);
    const uint8_t *src = table + (bad ? 0 : (uint64_t)id * rb);
    const uint32_t parts = D::parts(dim);
    const size_t obase = (size_t)row * dim;
    extern __shared__ float4 stage_lds[];  // staged decoders: 4 scale slots per 256-element block
    if constexpr (MAXC == 0 && D::STAGED) {
        // The first part's quant bytes are requested before the scale slots
        // are built, so their latency overlaps the staging and the barrier.
        typename D::Raw raw0{};
        if (threadIdx.x < parts) raw0 = D::load(src, threadIdx.x);
        for (uint32_t t = threadIdx.x; t < dim / 64; t += BLOCK) stage_lds[t] = D::stage(src, t);
        __syncthreads();
        using TO = typename O::T;
        // LDS_OUT: the decoded row is assembled in LDS (after the scale
        // slots) in natural order and then written with 16-byte
        // non-temporal stores, instead of each part storing its short runs.
        TO *out_lds = reinterpret_cast<TO *>(stage_lds + dim / 64);
        for (uint32_t p = threadIdx.x; p < parts; p += BLOCK) {
            float v[D::OUT];
            D::finish(p == threadIdx.x ? raw0 : D::load(src, p), p, stage_lds, v);
            if (bad) {
#pragma unroll
                for (int k = 0; k < D::OUT; ++k) v[k] = 0.0f;
            }
            if constexpr (LDS_OUT) {
#pragma unroll
                for (int r = 0; r < D::RUNS; ++r) {
                    Pack<TO, D::RUNLEN> pk;
#pragma unroll
                    for (int k = 0; k < D::RUNLEN; ++k) pk.v[k] = O::store(v[r * D::RUNLEN + k]);
                    *reinterpret_cast<Pack<TO, D::RUNLEN> *>(out_lds + D::run_off(p, r)) = pk;
                }
            } else {
                store_part<D, O, true>(h + obase, p, v);
            }
        }
        if constexpr (LDS_OUT) {
            constexpr int W = 16 / sizeof(TO);
            __syncthreads();
            for (uint32_t i = threadIdx.x; i < dim / W; i += BLOCK)
                store_pack_nt<TO, W>(h + obase + (size_t)i * W, *reinterpret_cast<const Pack<TO, W> *>(out_lds + i * W));
        }
        return;
    } else if constexpr (MAXC == 0) {
        for (uint32_t p = threadIdx.x; p < parts; p += BLOCK) {
            float v[D::OUT];
            D::decode(src, p, v);
            if (bad) {
#pragma unroll
                for (int k = 0; k < D::OUT; ++k) v[k] = 0.0f;
            }
            store_part<D, O, true>(h + obase, p, v);
        }
        return;
    } else {
        float v[MAXC][D::OUT];
        float ss = 0.0f;
        if constexpr (D::STAGED) {
            typename D::Raw raw[MAXC];
#pragma unroll
            for (int c = 0; c < MAXC; ++c) {
                const uint32_t p = c * BLOCK + threadIdx.x;
                if (p < parts) raw[c] = D::load(src, p);
            }
            for (uint32_t t = threadIdx.x; t < dim / 64; t += BLOCK) stage_lds[t] = D::stage(src, t);
            __syncthreads();
#pragma unroll
            for (int c = 0; c < MAXC; ++c) {
                const uint32_t p = c * BLOCK + threadIdx.x;
                if (p < parts) D::finish(raw[c], p, stage_lds, v[c]);
            }
        }
#pragma unroll
        for (int c = 0; c < MAXC; ++c) {
            const uint32_t p = c * BLOCK + threadIdx.x;
            if (p < parts) {
                if constexpr (!D::STAGED) D::decode(src, p, v[c]);
#pragma unroll
                for (int k = 0; k < D::OUT; ++k) {
                    if (bad) v[c][k] = 0.0f;
                    if constexpr (NORM) ss += v[c][k] * v[c][k];
                }
            }
        }
        if constexpr (!NORM) {
#pragma unroll
            for (int c = 0; c < MAXC; ++c) {
                const uint32_t p = c * BLOCK + threadIdx.x;
                if (p < parts) store_part<D, O, true>(h + obase, p, v[c]);
            }
        } else {
            ss = block_sum<BLOCK>(ss, red);
            const float scale = 1.0f / sqrtf(ss / (float)dim + eps);
#pragma unroll
            for (int c = 0; c < MAXC; ++c) {
                const uint32_t p = c * BLOCK + threadIdx.x;
                if (p < parts) {
                    if (h) store_part<D, O, FELLM_EMB_NORM_NT>(h + obase, p, v[c]);
                    float o[D::OUT];
#pragma unroll
                    for (int r = 0; r < D::RUNS; ++r) {
                        const uint32_t off = D::run_off(p, r);
#pragma unroll
                        for (int k = 0; k < D::RUNLEN; ++k)
                            o[r * D::RUNLEN + k] = (v[c][r * D::RUNLEN + k] * scale) * w[off + k];
                    }
                    store_part<D, O, FELLM_EMB_NORM_NT>(y + obase, p, o);
                }
            }
        }
    }
}

// One row's parts of this thread, for embedding_pipe_kernel below (an
// out-of-range id reads row 0; the caller zeroes what it stores).
template <typename D, int C>
__device__ __forceinline__ void emb_pipe_load(const uint8_t *table, uint64_t vocab, uint64_t rb, uint32_t parts,
                                              uint32_t id, float (&v)[C][D::OUT]) {
    const uint8_t *src = table + (id < vocab ? (uint64_t)id * rb : 0);
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const uint32_t p = c * kEmbBlock + threadIdx.x;
        if (p < parts) D::decode(src, p, v[c]);
    }
}

template <typename D, typename O, int C>
__device__ __forceinline__ void emb_pipe_store(typename O::T *hrow, uint32_t parts, bool bad, float (&v)[C][D::OUT]) {
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const uint32_t p = c * kEmbBlock + threadIdx.x;
        if (p < parts) {
            if (bad) {
#pragma unroll
                for (int k = 0; k < D::OUT; ++k) v[c][k] = 0.0f;
            }
            store_part<D, O, true>(hrow, p, v[c]);
        }
    }
}

// Plain (unquantized) gather, persistent: workgroup b copies rows b, b + G,
// b + 2G, ... (G = the grid).  The id of the row after next is requested a
// row ahead, and the next row's data are loaded before the current row is
// stored, so neither the id's latency nor the data's is paid per row.  A
// thread moves C parts of VEC elements per row; two register sets alternate.
template <typename D, typename O, int C>
__global__ __launch_bounds__(kEmbBlock) void embedding_pipe_kernel(
    const uint8_t *__restrict__ table, uint64_t vocab, uint32_t dim, const uint32_t *__restrict__ ids,
    uint32_t n_ids, typename O::T *__restrict__ h, uint32_t *__restrict__ err) {
    static_assert(D::DENSE, "plain tables only");
    const uint64_t rb = D::row_bytes(dim);
    const uint32_t parts = D::parts(dim);
    const uint32_t G = gridDim.x;
    uint32_t row = blockIdx.x;
    if (row >= n_ids) return;
    uint32_t id_a = ids[row];
    uint32_t id_b = row + G < n_ids ? ids[row + G] : 0u;
    float va[C][D::OUT], vb[C][D::OUT];
    emb_pipe_load<D, C>(table, vocab, rb, parts, id_a, va);
    uint32_t bad_rows = 0;
    for (;;) {
        // va holds row (id_a); id_b is row + G's id.
        uint32_t next = row + G;
        if (next < n_ids) emb_pipe_load<D, C>(table, vocab, rb, parts, id_b, vb);
        uint32_t id_c = next + G < n_ids ? ids[next + G] : 0u;
        bad_rows |= id_a >= vocab;
        emb_pipe_store<D, O, C>(h + (size_t)row * dim, parts, id_a >= vocab, va);
        if (next >= n_ids) break;
        row = next;
        // vb holds row (id_b); id_c is row + G's id.
        next = row + G;
        if (next < n_ids) emb_pipe_load<D, C>(table, vocab, rb, parts, id_c, va);
        id_a = next + G < n_ids ? ids[next + G] : 0u;
        bad_rows |= id_b >= vocab;
        emb_pipe_store<D, O, C>(h + (size_t)row * dim, parts, id_b >= vocab, vb);
        if (next >= n_ids) break;
        row = next;
        const uint32_t t = id_a;  // va now holds row (id_c); id_a is row + G's id
        id_a = id_c;
        id_b = t;
    }
    if (bad_rows && threadIdx.x == 0 && err) atomicOr(err, 1u);
}

// K-quant gathers through LDS.  A Q6_K row is dim/256 blocks of 210 bytes,
// so blocks are only 2-byte aligned and a per-part layout reads each block
// with short unaligned loads at 210-byte strides (Q4_K: 144-byte blocks, one
// 8-byte qs load per part at 144-byte strides).  Here the workgroup first
// copies the whole raw row into LDS with 16-byte loads of consecutive
// addresses (the row's span rounded out to 16-byte boundaries, which never
// leaves the pages the row lies on), then each thread decodes parts of 8
// consecutive outputs from LDS and writes them with one 16-byte store of a
// 16-bit output (a wavefront writes 1 KB of the row contiguously).
// Q6_K output o = 8p' of block b, at n = o % 256 = 128 hh + 32 k + l:
//   q  = ((ql[64 hh + 32 (k & 1) + l] >> 4 (k >> 1)) & 15)
//        | ((qh[32 hh + l] >> 2k) & 3) << 4,
//   y  = (d * sc[8 hh + l / 16 + 2k]) * (q - 32)      (dequant.rs:315-370).
// NL 16-byte loads and NP parts per thread, all loads issued before the LDS
// writes and all parts decoded before the stores.
__device__ __forceinline__ uint64_t lds_u64_at(const uint32_t *w, uint32_t off) {
    const uint32_t i = off / 4, sh = off % 4;
    const uint32_t w0 = w[i], w1 = w[i + 1], w2 = w[i + 2];
    return (uint64_t)__builtin_amdgcn_alignbyte(w1, w0, sh) |
           ((uint64_t)__builtin_amdgcn_alignbyte(w2, w1, sh) << 32);
}

//
// NORM (whole rows, bpw = dim / 256): the gather fused with RMSNorm.  The
// decoded row stays in registers for the sum of squares; h (when non-null)
// and y = (v * scale) * w are stored once each.
// Formats of the LDS gather: kBytes per 256-element block, and decode8,
// the 8 consecutive outputs n .. n+7 (n a multiple of 8) of the block whose
// bytes start at byte `blk` of the LDS row copy `w`.
struct Q6KLds {
    static constexpr uint32_t kBytes = 210, kElems = 256;
    __device__ static void decode8(const uint32_t *w, uint32_t blk, uint32_t n, float (&v)[8]) {
        const uint32_t hh = n / 128, k = (n / 32) % 4, l = n % 32;
        const uint64_t ql = lds_u64_at(w, blk + 64 * hh + 32 * (k & 1) + l);
        const uint64_t qh = lds_u64_at(w, blk + 128 + 32 * hh + l);
        const uint32_t so = blk + 192 + 8 * hh + l / 16 + 2 * k;
        const int32_t sc = (int8_t)(w[so / 4] >> (8 * (so % 4)));
        const uint32_t dof = blk + 208;  // even, so the f16 never straddles a dword
        const float d = half_bits_to_f32(w[dof / 4] >> (8 * (dof % 4)));
        const float ds = d * (float)sc;
        const uint32_t qs = 4 * (k >> 1), hs = 2 * k;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int32_t q = (int32_t)((((uint32_t)(ql >> (8 * e)) >> qs) & 15u) |
                                        ((((uint32_t)(qh >> (8 * e)) >> hs) & 3u) << 4)) -
                              32;
            v[e] = ds * (float)q;
        }
    }
};

// Q4_K (dequant.rs:251-305): output n of a block is chunk c = n / 64, offset
// j = n % 64: the low nibbles of qs[32c + j] for j < 32, else the high
// nibbles of qs[32c + j - 32], scaled by group 2c (+1 for the high nibbles):
// y = (d * sc) * q - (dmin * m).  Blocks are 144 = 9 * 16 bytes and the table
// is 16-byte aligned, so every word read here is aligned.
struct Q4KLds {
    static constexpr uint32_t kBytes = 144, kElems = 256;
    __device__ static void decode8(const uint32_t *w, uint32_t blk, uint32_t n, float (&v)[8]) {
        const uint32_t c = n / 64, j = n % 64, hi = j >= 32;
        const uint32_t *hw = w + blk / 4;
        const uint32_t h0 = hw[0];
        const float d = half_bits_to_f32(h0 & 0xffffu), dmin = half_bits_to_f32(h0 >> 16);
        uint32_t sc, m;
        k4_scale_min(2 * c + hi, hw[1], hw[2], hw[3], sc, m);
        const float dq = d * (float)sc, mq = dmin * (float)m;
        const uint32_t qo = (blk + 16 + 32 * c + j % 32) / 4;
        const uint32_t q0 = w[qo], q1 = w[qo + 1], sh = 4 * hi;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t b = ((e < 4 ? q0 : q1) >> (8 * (e % 4) + sh)) & 15u;
            v[e] = dq * (float)b - mq;
        }
    }
};

// Q5_K (dequant.rs:59-107): 176-byte blocks of d, dmin, 12 scale bytes,
// qh[32] at 16 and qs[128] at 48.  Output n is chunk c = n / 64, offset
// j = n % 64, l = j % 32: the low (j < 32) or high nibble of qs[32c + l]
// plus 16 when bit 2c (low) or 2c + 1 (high) of qh[l] is set, scaled by
// group 2c (+1 for the high nibbles): y = (d * sc) * q - (dmin * m).
// 176 = 11 * 16, so with a 4-byte-aligned table every word read is aligned.
struct Q5KLds {
    static constexpr uint32_t kBytes = 176, kElems = 256;
    __device__ static void decode8(const uint32_t *w, uint32_t blk, uint32_t n, float (&v)[8]) {
        const uint32_t c = n / 64, j = n % 64, hi = j >= 32, l = j % 32;
        const uint32_t *hw = w + blk / 4;
        const uint32_t h0 = hw[0];
        const float d = half_bits_to_f32(h0 & 0xffffu), dmin = half_bits_to_f32(h0 >> 16);
        uint32_t sc, m;
        k4_scale_min(2 * c + hi, hw[1], hw[2], hw[3], sc, m);
        const float dq = d * (float)sc, mq = dmin * (float)m;
        const uint32_t qo = (blk + 48 + 32 * c + l) / 4, ho = (blk + 16 + l) / 4;
        const uint32_t q0 = w[qo], q1 = w[qo + 1], g0 = w[ho], g1 = w[ho + 1];
        const uint32_t sh = 4 * hi, hb = 2 * c + hi;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t lo = ((e < 4 ? q0 : q1) >> (8 * (e % 4) + sh)) & 15u;
            const uint32_t up = (((e < 4 ? g0 : g1) >> (8 * (e % 4) + hb)) & 1u) << 4;
            v[e] = dq * (float)(lo + up) - mq;
        }
    }
};

// Q8_0 (dequant.rs:172-192): 34-byte blocks of 32 elements, f16 d then 32
// int8 values, y = d * (float)q.  Blocks are only 2-byte aligned: d sits at
// an even offset (never straddling a dword) and the 8 values of a part are
// assembled from unaligned LDS words.
struct Q8_0Lds {
    static constexpr uint32_t kBytes = 34, kElems = 32;
    __device__ static void decode8(const uint32_t *w, uint32_t blk, uint32_t n, float (&v)[8]) {
        const float d = half_bits_to_f32(w[blk / 4] >> (8 * (blk % 4)));
        const uint64_t q = lds_u64_at(w, blk + 2 + n);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = d * (float)(int8_t)(q >> (8 * e));
    }
};

template <typename F, typename O, int BLOCK, int NL, int NP, bool NORM>
__global__ __launch_bounds__(BLOCK) void kquant_gather_lds_kernel(const uint8_t *__restrict__ table, uint64_t vocab,
                                                                  uint32_t dim, const uint32_t *__restrict__ ids,
                                                                  uint32_t bpw, typename O::T *__restrict__ h,
                                                                  typename O::T *__restrict__ y,
                                                                  const float *__restrict__ w_norm, float eps,
                                                                  uint32_t *__restrict__ err) {
    extern __shared__ uint4 raw_lds[];
    __shared__ float red[BLOCK / kWave];
    // Workgroup = (row, segment of bpw blocks).  Without ids (a Cast) row r
    // of the table is gathered.
    constexpr uint32_t PPB = F::kElems / 8;  // parts per block
    const uint32_t nb = dim / F::kElems, nseg = (nb + bpw - 1) / bpw;
    const uint32_t row = blockIdx.x / nseg, b0 = (blockIdx.x % nseg) * bpw;
    const uint32_t nblk = nb - b0 < bpw ? nb - b0 : bpw;
    const uint32_t id = ids ? ids[row] : row;
    const bool bad = id >= vocab;
    if (bad && threadIdx.x == 0 && b0 == 0 && err) atomicOr(err, 1u);
    const uint8_t *segp = table + (bad ? 0 : (uint64_t)id * nb * F::kBytes) + F::kBytes * b0;
    const uint32_t lead = (uint32_t)(reinterpret_cast<uintptr_t>(segp) & 15);
    const uint4 *src = reinterpret_cast<const uint4 *>(segp - lead);
    const uint32_t n16 = (lead + F::kBytes * nblk + 15) / 16;
    // Threads past the span re-read its last chunk (a cache hit), so every
    // load is unconditional and the chunks stay in registers.
    uint4 c[NL];
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        const uint32_t j = i * BLOCK + threadIdx.x;
        c[i] = src[j < n16 ? j : n16 - 1];
    }
#pragma unroll
    for (int i = 0; i < NL; ++i) raw_lds[i * BLOCK + threadIdx.x] = c[i];  // LDS holds NL * BLOCK chunks
    __syncthreads();
    const uint32_t *w = reinterpret_cast<const uint32_t *>(raw_lds);
    const uint32_t parts = nblk * PPB;
    typename O::T *out = h + (size_t)row * dim + F::kElems * (size_t)b0;
    float v[NP][8];
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        const uint32_t p = i * BLOCK + threadIdx.x;
        if (p < parts) {
            F::decode8(w, lead + F::kBytes * (p / PPB), 8 * (p % PPB), v[i]);
            if (bad) {
#pragma unroll
                for (int e = 0; e < 8; ++e) v[i][e] = 0.0f;
            }
        }
    }
    if constexpr (!NORM) {
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const uint32_t p = i * BLOCK + threadIdx.x;
            if (p < parts) store_f32_nt<O, 8>(out + 8 * (size_t)p, v[i]);
        }
    } else {
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const uint32_t p = i * BLOCK + threadIdx.x;
            if (p < parts) {
#pragma unroll
                for (int e = 0; e < 8; ++e) ss += v[i][e] * v[i][e];
            }
        }
        ss = block_sum<BLOCK>(ss, red);
        const float scale = 1.0f / sqrtf(ss / (float)dim + eps);
        typename O::T *yrow = y + (size_t)row * dim;
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const uint32_t p = i * BLOCK + threadIdx.x;
            if (p < parts) {
                if (h) norm_out_store<O, 8>(out + 8 * (size_t)p, v[i]);
                float wv[8], o[8];
                load_f32<F32, 8>(w_norm + 8 * p, wv);
#pragma unroll
                for (int e = 0; e < 8; ++e) o[e] = (v[i][e] * scale) * wv[e];
                norm_out_store<O, 8>(yrow + 8 * (size_t)p, o);
            }
        }
    }
}

// Build knob: the fused gather + RMSNorm has an instantiation for 7 parts a
// thread (1), so rows of 3584 elements hold 56 decoded values in registers
// instead of 64 (Q6_K f16: 74 VGPRs, 6 waves per SIMD, against 82 and 5):
// configs[2] Q6_K gather + RMSNorm 24.16-24.24 against 24.48-24.72 us.
#ifndef FELLM_EMB_NORM_NP7
#define FELLM_EMB_NORM_NP7 1
#endif
// Build knob: the plain Q5_K / Q6_K gathers take the 7-part instantiation
// too (1).  configs[2], interleaved on one box: Q6_K 13.2 against 13.4-13.56
// us, Q5_K 12.4 against 12.8-12.9; Q8_0 slower with it (12.48 against
// 12.08), so it keeps 8.
#ifndef FELLM_EMB_PLAIN_NP7
#define FELLM_EMB_PLAIN_NP7 1
#endif

// Launches kquant_gather_lds_kernel with B threads per workgroup when a
// thread's share fits the unrolled counts (whole rows of up to 16384
// elements at 64 threads); -1 otherwise.  Without the norm, `split` cuts
// rows that do not fit into segments of blocks, one workgroup each.
template <typename F, typename O, int B>
int launch_kquant_lds_b(const void *table, uint64_t vocab, uint32_t dim, const uint32_t *ids, uint32_t n_ids,
                        void *h, void *y, const float *w, float eps, uint32_t *err, hipStream_t s, bool split) {
    if constexpr (B == 0) {
        return -1;
    } else {
        if (w && !aligned_to(w, 32)) return -1;  // 8-float weight vectors
        constexpr uint32_t PPB = F::kElems / 8;
        const uint32_t nb = dim / F::kElems;
        uint32_t bpw = !w && FELLM_EMB_Q6K_BPW && FELLM_EMB_Q6K_BPW < nb ? FELLM_EMB_Q6K_BPW : nb;
        // Chunks a segment of bpw blocks spans (its start rounded down and its
        // end rounded up to 16 bytes) and parts a thread decodes.
        auto n16_of = [](uint32_t nblk) { return (F::kBytes * nblk + 15 + 15) / 16; };
        if (split && !w && (n16_of(bpw) * 16 + 16 > 16u * B * 16 || (PPB * bpw + B - 1) / B > 32)) {
            const uint32_t by_lds = (8u * B * 16 - 16 - 30) / F::kBytes, by_parts = 16u * B / PPB;
            bpw = by_lds < by_parts ? by_lds : by_parts;
        }
        const uint64_t grid = (uint64_t)n_ids * ((nb + bpw - 1) / bpw);
        if (grid > 0x7fffffffull) return -1;
        const uint32_t n16 = n16_of(bpw);
        const uint32_t nl = (n16 + B - 1) / B, np = (PPB * bpw + B - 1) / B;
        // The fused norm keeps the row in registers: at most 8 parts a thread.
        if (w && np > 8) return -1;
        const uint8_t *tb = static_cast<const uint8_t *>(table);
        using TO = typename O::T;
        // Every thread writes its NL chunks; the segment's span (n16 chunks)
        // plus the dword lds_u64_at may read past it fit below NL * B chunks.
#define FELLM_Q6L(NL, NP)                                                                                      \
    if (nl <= NL && np <= NP && (size_t)NL * B * 16 >= (size_t)n16 * 16 + 16) {                                \
        if (w)                                                                                                 \
            FELLM_LAUNCH((kquant_gather_lds_kernel<F, O, B, NL, NP, true>), dim3((uint32_t)grid), dim3(B),             \
                         (size_t)NL * B * 16, s, tb, vocab, dim, ids, bpw, (TO *)h, (TO *)y, w, eps, err);     \
        else                                                                                                   \
            FELLM_LAUNCH((kquant_gather_lds_kernel<F, O, B, NL, NP, false>), dim3((uint32_t)grid), dim3(B),            \
                         (size_t)NL * B * 16, s, tb, vocab, dim, ids, bpw, (TO *)h, nullptr, nullptr, 0.0f, err); \
        return launch_status();                                                                                \
    }
        FELLM_Q6L(1, 1)
        FELLM_Q6L(1, 2)
        FELLM_Q6L(2, 4)
        // 7 parts a thread: rows of 3584 (Qwen2-7B) at 64 threads
        if ((w || (FELLM_EMB_PLAIN_NP7 && F::kElems == 256)) && FELLM_EMB_NORM_NP7) FELLM_Q6L(4, 7)
        FELLM_Q6L(4, 8)
        if (!w) {
            FELLM_Q6L(8, 16)
            FELLM_Q6L(16, 32)
        } else {
            FELLM_Q6L(8, 8)  // Q8_0 rows carry 34/32 bytes per element
        }
#undef FELLM_Q6L
        return -1;
    }
}

// The LDS gather at FELLM_EMB_KQ_LDS_BLOCK threads.  Q4_K and Q6_K keep
// their staged layouts for what it does not fit; Q5_K and Q8_0 (`full`) have
// only this kernel, so a fused norm over longer rows takes 256-thread
// workgroups and longer plain rows are split into segments.
template <typename F, typename O>
int launch_kquant_lds(const void *table, uint64_t vocab, uint32_t dim, const uint32_t *ids, uint32_t n_ids, void *h,
                      void *y, const float *w, float eps, uint32_t *err, hipStream_t s, bool full = false) {
    const int st = launch_kquant_lds_b<F, O, FELLM_EMB_KQ_LDS_BLOCK>(table, vocab, dim, ids, n_ids, h, y, w, eps, err,
                                                                     s, full);
    if (st >= 0 || !full || !w) return st;
    return launch_kquant_lds_b<F, O, 256>(table, vocab, dim, ids, n_ids, h, y, w, eps, err, s, false);
}

template <typename D, typename O>
int launch_emb(const void *table, uint64_t vocab, uint32_t dim, const uint32_t *ids, uint32_t n_ids,
               void *h, void *y, const float *w, float eps, uint32_t *err, hipStream_t s) {
    using TO = typename O::T;
    const dim3 grid(n_ids), block(kEmbBlock);
    const uint8_t *tb = static_cast<const uint8_t *>(table);
    const uint32_t chunks = (D::parts(dim) + kEmbBlock - 1) / kEmbBlock;
    const uint32_t lds = D::STAGED ? dim / 64 * sizeof(float4) : 0;
    if (lds > 65536) return FELLM_ERR_SHAPE;  // dim > 262144
#define FELLM_EMB(C, NORM)                                                                          \
    if (chunks <= C) {                                                                              \
        FELLM_LAUNCH((embedding_kernel<D, O, C, NORM>), grid, block, lds, s, tb, vocab, dim, ids, \
                           (TO *)h, (TO *)y, w, eps, err);                                          \
        return launch_status();                                                                     \
    }
    if (!w) {
        if constexpr (requires { D::DENSE; } && FELLM_EMB_PIPE > 0) {
            // Many rows (at least two per workgroup, so the pipeline has rows
            // to overlap): persistent workgroups, all resident.
            if (ids && chunks <= 4) {
#define FELLM_EMB_P(C)                                                                                         \
    if (chunks <= C) {                                                                                         \
        static const uint32_t pgrid = resident_grid(embedding_pipe_kernel<D, O, C>, kEmbBlock, 0, FELLM_EMB_PIPE); \
        if (n_ids >= 2 * pgrid) {                                                                              \
            FELLM_LAUNCH((embedding_pipe_kernel<D, O, C>), dim3(pgrid), block, 0, s, tb, vocab, dim, ids, n_ids, \
                         (TO *)h, err);                                                                        \
            return launch_status();                                                                            \
        }                                                                                                      \
    } else
                FELLM_EMB_P(1)
                FELLM_EMB_P(2)
                FELLM_EMB_P(4) {}
#undef FELLM_EMB_P
            }
        }
        if constexpr (requires { D::DENSE; } && FELLM_EMB_DENSE_BLOCK > 0) {
            // One workgroup per row, every part of a thread loaded before its stores.
            constexpr int B = FELLM_EMB_DENSE_BLOCK;
            const uint32_t ch = (D::parts(dim) + B - 1) / B;
#define FELLM_EMB_B(C)                                                                                         \
    if (ch <= C) {                                                                                             \
        FELLM_LAUNCH((embedding_kernel<D, O, C, false, B>), grid, dim3(B), lds, s, tb, vocab, dim, ids, (TO *)h, \
                     nullptr, nullptr, 0.0f, err);                                                             \
        return launch_status();                                                                                \
    }
            FELLM_EMB_B(1)
            FELLM_EMB_B(2)
            FELLM_EMB_B(4)
            FELLM_EMB_B(8)
#undef FELLM_EMB_B
        }
        constexpr bool regs = requires { D::ALL_PARTS_IN_REGS; };
        if constexpr (regs && FELLM_EMB_Q4K_BLOCK != kEmbBlock) {
            constexpr int B = FELLM_EMB_Q4K_BLOCK;
            const uint32_t ch = (D::parts(dim) + B - 1) / B;
#define FELLM_EMB_B(C)                                                                                         \
    if (ch <= C) {                                                                                             \
        FELLM_LAUNCH((embedding_kernel<D, O, C, false, B>), grid, dim3(B), lds, s, tb, vocab, dim, ids, (TO *)h, \
                     nullptr, nullptr, 0.0f, err);                                                             \
        return launch_status();                                                                                \
    }
            FELLM_EMB_B(1)
            FELLM_EMB_B(2)
            FELLM_EMB_B(4)
            FELLM_EMB_B(8)
#undef FELLM_EMB_B
        }
        if constexpr (D::STAGED && !regs && FELLM_EMB_LDS_OUT) {
            const uint32_t out_bytes = dim * (uint32_t)sizeof(TO);
            if (FELLM_EMB_LOOP && out_bytes % 16 == 0 && aligned_to(h, 16) && lds + out_bytes <= 65536) {
                FELLM_LAUNCH((embedding_kernel<D, O, 0, false, kEmbBlock, true>), grid, block, lds + out_bytes, s, tb,
                             vocab, dim, ids, (TO *)h, nullptr, nullptr, 0.0f, err);
                return launch_status();
            }
        }
        if (FELLM_EMB_LOOP && !regs) {
            FELLM_LAUNCH((embedding_kernel<D, O, 0, false>), grid, block, lds, s, tb, vocab, dim, ids, (TO *)h,
                               nullptr, nullptr, 0.0f, err);
            return launch_status();
        }
        FELLM_EMB(1, false)
        FELLM_EMB(2, false)
        FELLM_EMB(4, false)
        FELLM_EMB(8, false)
        FELLM_LAUNCH((embedding_kernel<D, O, 0, false>), grid, block, lds, s, tb, vocab, dim, ids, (TO *)h,
                           nullptr, nullptr, 0.0f, err);
        return launch_status();
    }
    FELLM_EMB(1, true)
    FELLM_EMB(2, true)
    FELLM_EMB(4, true)
    FELLM_EMB(8, true)
#undef FELLM_EMB
    return FELLM_ERR_SHAPE;
}

template <typename O>
int dispatch_table(const void *table, uint32_t table_dtype, uint64_t vocab, uint32_t dim,
                   const uint32_t *ids, uint32_t n_ids, void *h, void *y, const float *w, float eps,
                   uint32_t *err, hipStream_t s) {
    switch (table_dtype) {
        case FELLM_DTYPE_Q4K:
            if (dim % 256 || !aligned_to(table, 16)) return FELLM_ERR_SHAPE;
            if (ids && dim * sizeof(typename O::T) % 16 == 0 && (w ? FELLM_EMB_Q4K_LDS_NORM : FELLM_EMB_Q4K_LDS)) {
                const int st = launch_kquant_lds<Q4KLds, O>(table, vocab, dim, ids, n_ids, h, y, w, eps, err, s);
                if (st >= 0) return st;
            }
            if (FELLM_EMB_STAGE == 2) return launch_emb<Q4KStaged8, O>(table, vocab, dim, ids, n_ids, h, y, w, eps, err, s);
            if (FELLM_EMB_STAGE) return launch_emb<Q4KStaged, O>(table, vocab, dim, ids, n_ids, h, y, w, eps, err, s);
            return launch_emb<Q4KDec, O>(table, vocab, dim, ids, n_ids, h, y, w, eps, err, s);
        case FELLM_DTYPE_Q6K:
            if (dim % 256 || !aligned_to(table, 2)) return FELLM_ERR_SHAPE;
            if (ids && dim * sizeof(typename O::T) % 16 == 0 && (w ? FELLM_EMB_Q6K_LDS_NORM : FELLM_EMB_Q6K_LDS)) {
                const int st = launch_kquant_lds<Q6KLds, O>(table, vocab, dim, ids, n_ids, h, y, w, eps, err, s);
                if (st >= 0) return st;
            }
            if (FELLM_EMB_STAGE) return launch_emb<Q6KStaged, O>(table, vocab, dim, ids, n_ids, h, y, w, eps, err, s);
            return launch_emb<Q6KDec, O>(table, vocab, dim, ids, n_ids, h, y, w, eps, err, s);
        case FELLM_DTYPE_Q5K: {
            if (dim % 256 || !aligned_to(table, 4) || dim * sizeof(typename O::T) % 16) return FELLM_ERR_SHAPE;
            const int st = launch_kquant_lds<Q5KLds, O>(table, vocab, dim, ids, n_ids, h, y, w, eps, err, s, true);
            return st >= 0 ? st : FELLM_ERR_SHAPE;
        }
        case FELLM_DTYPE_Q8_0: {
            if (dim % 32 || !aligned_to(table, 2) || dim * sizeof(typename O::T) % 16) return FELLM_ERR_SHAPE;
            const int st = launch_kquant_lds<Q8_0Lds, O>(table, vocab, dim, ids, n_ids, h, y, w, eps, err, s, true);
            return st >= 0 ? st : FELLM_ERR_SHAPE;
        }
        default:
            break;
    }
    return dispatch_act(table_dtype, [&]<typename A>() -> int {
        constexpr int VEC = 8;
        const bool vec = dim % VEC == 0 && aligned_to(table, sizeof(typename A::T) * VEC);
        if (vec) return launch_emb<DenseDec<A, VEC>, O>(table, vocab, dim, ids, n_ids, h, y, w, eps, err, s);
        return launch_emb<DenseDec<A, 1>, O>(table, vocab, dim, ids, n_ids, h, y, w, eps, err, s);
    });
}

int embedding_common(const void *table, uint32_t table_dtype, uint64_t vocab, uint32_t dim,
                     const uint32_t *ids, uint32_t n_ids, void *h, void *y, uint32_t out_dtype,
                     const float *w, float eps, uint32_t *err, void *stream) {
    if (dim == 0 || vocab == 0) return FELLM_ERR_SHAPE;
    if (n_ids == 0) return FELLM_OK;
    if (!table || !ids) return FELLM_ERR_ARITY;
    // Output runs are up to 8 elements: 16-byte alignment covers every case.
    if ((h && !aligned_to(h, 16)) || (y && !aligned_to(y, 16))) return FELLM_ERR_SHAPE;
    hipStream_t s = as_stream(stream);
    return dispatch_act(out_dtype, [&]<typename O>() -> int {
        return dispatch_table<O>(table, table_dtype, vocab, dim, ids, n_ids, h, y, w, eps, err, s);
    });
}

}  // namespace
}  // namespace fellm

extern "C" int fellm_rocm_embedding(const void *table, uint32_t table_dtype, uint64_t vocab,
                                    uint32_t dim, const uint32_t *ids, uint32_t n_ids, void *out,
                                    uint32_t out_dtype, uint32_t *err_flag, void *stream) {
    if (!out && n_ids) return FELLM_ERR_ARITY;
    return fellm::embedding_common(table, table_dtype, vocab, dim, ids, n_ids, out, nullptr, out_dtype,
                                   nullptr, 0.0f, err_flag, stream);
}

extern "C" int fellm_rocm_embedding_rmsnorm(const void *table, uint32_t table_dtype, uint64_t vocab,
                                            uint32_t dim, const uint32_t *ids, uint32_t n_ids,
                                            const float *norm_weight, float eps, void *h_out, void *y,
                                            uint32_t out_dtype, uint32_t *err_flag, void *stream) {
    if ((!norm_weight || !y) && n_ids) return FELLM_ERR_ARITY;
    return fellm::embedding_common(table, table_dtype, vocab, dim, ids, n_ids, h_out, y, out_dtype,
                                   norm_weight, eps, err_flag, stream);
}

namespace fellm {
namespace {

// Rows of `dim` elements covering n: the widest of 4096 .. `unit` that divides n.
uint32_t cast_dim(uint64_t n, uint32_t unit) {
    for (uint32_t d = 4096; d >= unit; d /= 2)
        if (n % d == 0 && n / d <= 0x7fffffffull) return d;
    return 0;
}

}  // namespace
}  // namespace fellm

extern "C" int fellm_rocm_cast(const void *src, uint32_t src_dtype, void *dst, uint32_t dst_dtype, uint64_t n_elems,
                               void *stream) {
    using namespace fellm;
    if (n_elems == 0) return FELLM_OK;
    if (!src || !dst) return FELLM_ERR_ARITY;
    hipStream_t s = as_stream(stream);
    const bool out_vec = aligned_to(dst, 16);
    // Dense pairs of the CPU backend's Cast (backend.rs:1616-1656): f32 copy,
    // f16 / bf16 widening, f32 -> f16 round-to-nearest-even, f32 -> bf16 truncation.
    auto dense = [&]<typename A, typename O>() -> int {
        constexpr int VEC = 8;
        const bool vec = out_vec && n_elems % VEC == 0 && aligned_to(src, sizeof(typename A::T) * VEC);
        const uint32_t dim = cast_dim(n_elems, vec ? VEC : 1);
        if (!dim) return FELLM_ERR_SHAPE;
        const uint64_t rows = n_elems / dim;
        if (vec)
            return launch_emb<DenseDec<A, VEC>, O>(src, rows, dim, nullptr, (uint32_t)rows, dst, nullptr, nullptr,
                                                   0.0f, nullptr, s);
        return launch_emb<DenseDec<A, 1>, O>(src, rows, dim, nullptr, (uint32_t)rows, dst, nullptr, nullptr, 0.0f,
                                             nullptr, s);
    };
    if (dst_dtype == FELLM_DTYPE_F32) {
        switch (src_dtype) {
            case FELLM_DTYPE_F32: return dense.template operator()<F32, F32>();
            case FELLM_DTYPE_F16: return dense.template operator()<F16, F32>();
            case FELLM_DTYPE_BF16: return dense.template operator()<BF16, F32>();
            case FELLM_DTYPE_Q4K:
            case FELLM_DTYPE_Q6K: {
                // Quantized -> f32 via the row dequantization (backend.rs:1657-1661,
                // dequant.rs:19-55): the block stream as rows of `dim` elements.
                if (n_elems % 256 || !out_vec) return FELLM_ERR_SHAPE;
                const uint32_t dim = cast_dim(n_elems, 256);
                if (!dim) return FELLM_ERR_SHAPE;
                const uint64_t rows = n_elems / dim;
                if (src_dtype == FELLM_DTYPE_Q4K) {
                    if (!aligned_to(src, 16)) return FELLM_ERR_SHAPE;
                    return launch_emb<Q4KDec, F32>(src, rows, dim, nullptr, (uint32_t)rows, dst, nullptr, nullptr, 0.0f,
                                                   nullptr, s);
                }
                if (!aligned_to(src, 2)) return FELLM_ERR_SHAPE;
                return launch_emb<Q6KDec, F32>(src, rows, dim, nullptr, (uint32_t)rows, dst, nullptr, nullptr, 0.0f,
                                               nullptr, s);
            }
            case FELLM_DTYPE_Q5K:
            case FELLM_DTYPE_Q8_0: {
                // Through the LDS gather with row r = table row r (no ids).
                const bool q5 = src_dtype == FELLM_DTYPE_Q5K;
                if (n_elems % (q5 ? 256 : 32) || !out_vec || !aligned_to(src, q5 ? 4 : 2)) return FELLM_ERR_SHAPE;
                const uint32_t dim = cast_dim(n_elems, q5 ? 256 : 32);
                if (!dim) return FELLM_ERR_SHAPE;
                const uint64_t rows = n_elems / dim;
                const int st = q5 ? launch_kquant_lds<Q5KLds, F32>(src, rows, dim, nullptr, (uint32_t)rows, dst, nullptr,
                                                                   nullptr, 0.0f, nullptr, s, true)
                                  : launch_kquant_lds<Q8_0Lds, F32>(src, rows, dim, nullptr, (uint32_t)rows, dst,
                                                                    nullptr, nullptr, 0.0f, nullptr, s, true);
                return st >= 0 ? st : FELLM_ERR_SHAPE;
            }
            default: return FELLM_ERR_DTYPE;
        }
    }
    if (src_dtype == FELLM_DTYPE_F32 && dst_dtype == FELLM_DTYPE_F16) return dense.template operator()<F32, F16>();
    if (src_dtype == FELLM_DTYPE_F32 && dst_dtype == FELLM_DTYPE_BF16)
        return dense.template operator()<F32, BF16Trunc>();
    return FELLM_ERR_DTYPE;
}
