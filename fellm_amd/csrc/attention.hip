// Paged decode attention over the KV cache the fused RoPE + KV append writes.
//
// Reference: crates/fellm-plugin-abi/src/attention_provider.rs:391-459
//   (reference_attention_paged_f32: per query head, online softmax over the
//   keys 0 .. seq-1, score = (q . k) * scale, keys older than the window
//   skipped when causal; out = sum p v / sum p), driven per batch row as
//   crates/backend-cpu/src/backend.rs:1286-1323 does (seq = row_lengths[row],
//   causal, window = attention_window) and as the CUDA plugin's
//   attention_paged_batch_heads launch (plugins/cuda_kernels/src/launchers.rs
//   :3394-3446) is fed; K/V rows as crates/fellm-plugin-abi/src/paged_ctx.rs
//   :138-174 address them.
//
// Work split.  One wavefront per (batch row b, KV head g, key split s); the
// G = n_heads / n_kv query heads that share KV head g are processed together,
// so every K/V byte is read once.  Keys go in cache blocks of 16 tokens:
//  * Q.K^T on the matrix cores: v_mfma_f32_16x16x16f16 with A = the block's K
//    rows (16 tokens x 16 dims per step) and B = q^T (16 dims x 16 head slots).
//    q is split into f16 high and low parts (two MFMAs per step), so the
//    products with the f16 cache are exact and the f32 accumulation carries
//    q to ~2^-22 relative; a bf16 cache uses bf16 MFMAs with a three-way split.
//    The contraction order over dims is a permutation shared by A and B: lane
//    group i = lane / 16 holds dims 32(s/2) + 8i + 4(s%2) .. +3 of step s.
//  * Online softmax in f32 per head (block max across the 64 lanes, exp,
//    rescale by exp(m_old - m_new)), probabilities exchanged through LDS.
//  * P.V on the vector ALUs: lane (token group tg = lane / 16, dim slice
//    ds = lane % 16) accumulates HD/16 dims of all G heads over tokens
//    4i + tg, in f32; the four token groups are summed at the end.
// Splits (several wavefronts per (b, g) when b * n_kv is small) write
// unnormalised partial sums with their running max and denominator; a second
// kernel combines them.  Tokens outside [lo, seq) are masked with -inf and
// their V rows read as zero, so stale cache bytes never reach the output.
#include "common.hpp"

#include "fellm_rocm.h"

namespace fellm {
namespace {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
using Rsrc = __amdgpu_buffer_rsrc_t;

constexpr uint32_t kBlockTokens = 16;  // tokens per cache block handled by one MFMA tile
// A split's partial record per head slot: HD sums, m, l and two unused
// floats, so that every record starts on a 16-byte boundary.
constexpr uint32_t kRecTail = 4;

struct PagedGeom {
    const uint8_t *arena;
    uint64_t arena_len;
    const uint32_t *table;
    uint64_t n_table;
    uint32_t n_logical, n_layers, layer, block_size;
    uint64_t block_bytes;
    uint32_t stride;  // elements per token row (n_kv * head_dim)
};

// Cache element policies: MFMA operand split of q and widening of V.
struct CacheF16 {
    static constexpr int kParts = 2;
    using Op = half4_t;
    __device__ static Op part(const float (&v)[4], int p, float (&rem)[4]) {
        Op o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const _Float16 h = (_Float16)rem[e];
            o[e] = h;
            rem[e] = rem[e] - (float)h;
        }
        (void)v;
        (void)p;
        return o;
    }
    __device__ static Op from_bits(uint32_t lo, uint32_t hi) {
        Op o;
        o[0] = __builtin_bit_cast(_Float16, (uint16_t)(lo & 0xffffu));
        o[1] = __builtin_bit_cast(_Float16, (uint16_t)(lo >> 16));
        o[2] = __builtin_bit_cast(_Float16, (uint16_t)(hi & 0xffffu));
        o[3] = __builtin_bit_cast(_Float16, (uint16_t)(hi >> 16));
        return o;
    }
    __device__ static f32x4 mfma(Op a, Op b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0); }
    __device__ static float widen(uint32_t bits16) { return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16); }
};

struct CacheBF16 {
    static constexpr int kParts = 3;
    using Op = short4_t;
    __device__ static Op part(const float (&v)[4], int p, float (&rem)[4]) {
        Op o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            // round to nearest even bf16, keep the remainder for the next part
            const uint32_t u = __float_as_uint(rem[e]);
            const uint32_t r = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
            o[e] = (short)(r >> 16);
            rem[e] = rem[e] - __uint_as_float(r);
        }
        (void)v;
        (void)p;
        return o;
    }
    __device__ static Op from_bits(uint32_t lo, uint32_t hi) {
        Op o;
        o[0] = (short)(lo & 0xffffu);
        o[1] = (short)(lo >> 16);
        o[2] = (short)(hi & 0xffffu);
        o[3] = (short)(hi >> 16);
        return o;
    }
    __device__ static f32x4 mfma(Op a, Op b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
    }
    __device__ static float widen(uint32_t bits16) { return __uint_as_float(bits16 << 16); }
};

// Keys of split s for a row of length seq: blocks [b0, b1) of the range
// [lo, seq) (lo > 0 only for a causal window), in chunks of bps blocks.
__device__ __forceinline__ void split_range(uint32_t seq, uint32_t lo, uint32_t s, uint32_t bps, uint32_t &b0,
                                            uint32_t &b1) {
    const uint32_t first = lo / kBlockTokens, last = (seq + kBlockTokens - 1) / kBlockTokens;
    b0 = first + s * bps;
    b1 = b0 + bps < last ? b0 + bps : last;
    if (b0 > last) b0 = last;
}

// Q: query activation policy, O: output policy, C: cache policy, HD: head
// dim (64, 128 or 256), GM: maximum query heads per KV head (8 or 16).
template <typename Q, typename O, typename C, int HD, int GM, int DEPTH>
__global__ __launch_bounds__(kWave) void paged_decode_kernel(const typename Q::T *__restrict__ q,
                                                             typename O::T *__restrict__ out,
                                                             float *__restrict__ part, const uint32_t *__restrict__ lens,
                                                             const uint32_t *__restrict__ table, PagedGeom geo,
                                                             uint32_t n_heads, uint32_t n_kv, float scale,
                                                             uint32_t causal, uint32_t window, uint32_t splits,
                                                             uint32_t bps) {
    constexpr int NS = HD / 16;  // MFMA k-steps
    constexpr int NKL = HD / 32; // 16-byte K loads per lane per block
    constexpr int DP = HD / 16;  // dims per lane in P.V
    __shared__ __align__(16) float lds_p[kBlockTokens * 16];
    __shared__ __align__(16) float lds_h[16];

    const uint32_t lane = threadIdx.x;
    const uint32_t col = lane % 16, grp = lane / 16;  // MFMA column (head slot) / lane group
    const uint32_t s = blockIdx.x % splits;
    const uint32_t bg = blockIdx.x / splits;
    const uint32_t g = bg % n_kv, b = bg / n_kv;
    const uint32_t G = n_heads / n_kv;
    const size_t row_bytes = (size_t)geo.stride * 2;
    const size_t table_base = ((size_t)b * geo.n_layers + geo.layer) * geo.n_logical;
    // One cache block's K and V slices for this lane, fetched through a
    // buffer resource spanning the block: an absent or out-of-range block has
    // range 0 and reads as zeros without memory traffic, so the next block is
    // requested unconditionally while the current one is reduced.
    struct BlockRegs {
        uint4 kr[NKL];         // K: token col, dims 32c + 8 grp .. +7 of load c
        uint32_t vr[4][DP / 2]; // V: token 4i + grp, dims col*DP .. +DP-1
        bool ok;
    };
    auto fetch = [&](uint32_t blk, uint32_t lim, BlockRegs &R) {
        const size_t ti = table_base + blk;
        const uint64_t phys =
            (blk < lim && blk < geo.n_logical && ti < geo.n_table) ? (uint64_t)table[ti] : ~0ull;
        const bool ok = phys != ~0ull && (phys + 1) * geo.block_bytes <= geo.arena_len;
        const uint8_t *base = geo.arena + (ok ? phys * geo.block_bytes : 0);
        const Rsrc rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(base), 0,
                                                          ok ? (int)geo.block_bytes : 0, 0x00020000);
        const uint32_t koff = g * HD * 2 + col * (uint32_t)row_bytes + 16 * grp;
#pragma unroll
        for (int c = 0; c < NKL; ++c) {
            const u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(rs, koff + 64 * c, 0, 2);
            R.kr[c] = make_uint4(t.x, t.y, t.z, t.w);
        }
        const uint32_t voff = geo.block_size * (uint32_t)row_bytes + g * HD * 2 + col * DP * 2;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t o = voff + (4 * i + grp) * (uint32_t)row_bytes;
            if constexpr (DP == 4) {  // 8 bytes per lane
                const u32x2 t = __builtin_amdgcn_raw_buffer_load_b64(rs, o, 0, 2);
                R.vr[i][0] = t.x;
                R.vr[i][1] = t.y;
            } else {  // 16 or 32 bytes per lane
#pragma unroll
                for (int w = 0; w < DP / 2; w += 4) {
                    const u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(rs, o + 4 * w, 0, 2);
                    R.vr[i][w] = t.x;
                    R.vr[i][w + 1] = t.y;
                    R.vr[i][w + 2] = t.z;
                    R.vr[i][w + 3] = t.w;
                }
            }
        }
        R.ok = ok;
    };
    // Without a sliding window the split's first block is s * bps whatever
    // the sequence length, so it is requested before the length arrives
    // (tokens past the length are masked in process); with a window the
    // first block depends on the length and is fetched once it is known.
    const bool spec = !(causal && window);
    // DEPTH blocks are in flight ahead of the one being reduced.
    BlockRegs ra, rb, rc;
    if constexpr (DEPTH == 2) fetch(s * bps + 1, spec ? s * bps + bps : 0u, rb);
    fetch(s * bps, spec ? s * bps + bps : 0u, ra);
    const uint32_t seq = lens[b];
    const uint32_t lo = (causal && window && seq > window) ? seq - window : 0;
    uint32_t blk0, blk1;
    split_range(seq, lo, s, bps, blk0, blk1);

    // q^T as the B operand: head slot col (= query head g*G + col), dims of step st.
    typename C::Op qb[NS][C::kParts];
    {
        // Steps 2j and 2j+1 use dims 32j + 8 grp .. +7: one vector load each.
        const bool hv = col < G;
        const typename Q::T *qh = q + ((size_t)b * n_heads + (size_t)g * G + (hv ? col : 0)) * HD;
        float qv[NS / 2][8];
#pragma unroll
        for (int j = 0; j < NS / 2; ++j) {
            load_f32<Q, 8>(qh + 32 * j + 8 * grp, qv[j]);
            if (!hv)
#pragma unroll
                for (int e = 0; e < 8; ++e) qv[j][e] = 0.0f;
        }
#pragma unroll
        for (int st = 0; st < NS; ++st) {
            float v[4], rem[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) rem[e] = v[e] = qv[st / 2][4 * (st % 2) + e];
#pragma unroll
            for (int p = 0; p < C::kParts; ++p) qb[st][p] = C::part(v, p, rem);
        }
    }

    float acc[GM][DP];
#pragma unroll
    for (int h = 0; h < GM; ++h)
#pragma unroll
        for (int d = 0; d < DP; ++d) acc[h][d] = 0.0f;
    float m = -__builtin_inff(), l = 0.0f;  // running max / denominator of head slot col

    auto process = [&](uint32_t blk, const BlockRegs &R) {
        const bool blk_ok = R.ok;
        const uint4(&kr)[NKL] = R.kr;
        const uint32_t(&vr)[4][DP / 2] = R.vr;
        const uint32_t t0 = blk * kBlockTokens;
        // S^T[token 4 grp + e][head slot col]
        f32x4 sacc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int st = 0; st < NS; ++st) {
            const uint4 &k4 = kr[st / 2];
            const typename C::Op a = (st % 2) ? C::from_bits(k4.z, k4.w) : C::from_bits(k4.x, k4.y);
#pragma unroll
            for (int p = 0; p < C::kParts; ++p) sacc = C::mfma(a, qb[st][p], sacc);
        }
        float sc[4];
        float bmax = -__builtin_inff();
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t t = t0 + 4 * grp + e;
            const bool valid = blk_ok && t >= lo && t < seq;
            sc[e] = valid ? sacc[e] * scale : -__builtin_inff();
            bmax = fmaxf(bmax, sc[e]);
        }
        bmax = fmaxf(bmax, __shfl_xor(bmax, 16, kWave));
        bmax = fmaxf(bmax, __shfl_xor(bmax, 32, kWave));
        const float m_new = fmaxf(m, bmax);
        const float alpha = (m > -__builtin_inff()) ? __expf(m - m_new) : 0.0f;
        float psum = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float p = sc[e] > -__builtin_inff() ? __expf(sc[e] - m_new) : 0.0f;
            lds_p[(4 * grp + e) * 16 + col] = p;
            psum += p;
        }
        psum += __shfl_xor(psum, 16, kWave);
        psum += __shfl_xor(psum, 32, kWave);
        // a head with no valid key yet keeps m = -inf, l = 0, alpha = 0
        if (m_new > -__builtin_inff()) {
            l = l * alpha + psum;
            m = m_new;
        }
        if (grp == 0) lds_h[col] = m_new > -__builtin_inff() ? alpha : 1.0f;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");

        float al[GM];
#pragma unroll
        for (int h = 0; h < GM; h += 4) {
            const float4 t = *reinterpret_cast<const float4 *>(&lds_h[h]);
            al[h] = t.x;
            al[h + 1] = t.y;
            al[h + 2] = t.z;
            al[h + 3] = t.w;
        }
#pragma unroll
        for (int h = 0; h < GM; ++h)
#pragma unroll
            for (int d = 0; d < DP; ++d) acc[h][d] *= al[h];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t t = 4 * i + grp;
            const bool tv = blk_ok && t0 + t >= lo && t0 + t < seq;
            float v[DP];
#pragma unroll
            for (int w = 0; w < DP / 2; ++w) {
                v[2 * w] = tv ? C::widen(vr[i][w] & 0xffffu) : 0.0f;
                v[2 * w + 1] = tv ? C::widen(vr[i][w] >> 16) : 0.0f;
            }
            float p[GM];
#pragma unroll
            for (int h = 0; h < GM; h += 4) {
                const float4 t4 = *reinterpret_cast<const float4 *>(&lds_p[t * 16 + h]);
                p[h] = t4.x;
                p[h + 1] = t4.y;
                p[h + 2] = t4.z;
                p[h + 3] = t4.w;
            }
#pragma unroll
            for (int h = 0; h < GM; ++h)
#pragma unroll
                for (int d = 0; d < DP; ++d) acc[h][d] = __builtin_fmaf(p[h], v[d], acc[h][d]);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
        };
    if constexpr (DEPTH == 2) {
        if (!spec) {
            fetch(blk0, blk1, ra);
            fetch(blk0 + 1, blk1, rb);
        }
        for (uint32_t blk = blk0; blk < blk1; blk += 3) {
            fetch(blk + 2, blk1, rc);
            process(blk, ra);
            if (blk + 1 >= blk1) break;
            fetch(blk + 3, blk1, ra);
            process(blk + 1, rb);
            if (blk + 2 >= blk1) break;
            fetch(blk + 4, blk1, rb);
            process(blk + 2, rc);
        }
    } else {
        if (!spec) fetch(blk0, blk1, ra);
        for (uint32_t blk = blk0; blk < blk1; blk += 2) {
            fetch(blk + 1, blk1, rb);
            process(blk, ra);
            if (blk + 1 >= blk1) break;
            fetch(blk + 2, blk1, ra);
            process(blk + 1, rb);
        }
    }

    // Sum the four token groups; lanes 0..15 then hold dims col*DP .. of every head.
#pragma unroll
    for (int h = 0; h < GM; ++h)
#pragma unroll
        for (int d = 0; d < DP; ++d) {
            acc[h][d] += __shfl_xor(acc[h][d], 16, kWave);
            acc[h][d] += __shfl_xor(acc[h][d], 32, kWave);
        }
    if (grp == 0) lds_h[col] = l;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
    // The epilogue loops over head slots are unrolled (with a guard rather
    // than a break: a loop with a second exit is not fully unrolled at GM 16,
    // and acc then lives in scratch), except where acc (GM x HD / 16 floats
    // per lane) cannot stay in registers anyway: at 16 x 256 unrolling only
    // multiplies the compile time.
    constexpr int kEpiUnroll = GM * DP > 128 ? 1 : GM;
    if (splits == 1) {
        if (grp == 0) {
#pragma unroll kEpiUnroll
            for (int h = 0; h < GM; ++h) {
                if ((uint32_t)h < G) {
                    const float lh = lds_h[h];
                    const float inv = lh > 0.0f ? 1.0f / lh : 0.0f;
                    typename O::T *o = out + ((size_t)b * n_heads + (size_t)g * G + h) * HD + col * DP;
                    float r[DP];
#pragma unroll
                    for (int d = 0; d < DP; ++d) r[d] = lh > 0.0f ? acc[h][d] * inv : 0.0f;
                    store_f32<O, DP>(o, r);
                }
            }
        }
    } else {
        // partial record per (b, g, s, head slot): HD sums, then m, l
        float *rec = part + ((size_t)bg * splits + s) * GM * (HD + kRecTail);
        if (grp == 0) {
#pragma unroll kEpiUnroll
            for (int h = 0; h < GM; ++h) {
                if ((uint32_t)h < G) {
#pragma unroll
                    for (int d = 0; d < DP; ++d) rec[h * (HD + kRecTail) + col * DP + d] = acc[h][d];
                }
            }
            if (col < G) {
                rec[col * (HD + kRecTail) + HD] = m;
                rec[col * (HD + kRecTail) + HD + 1] = l;
            }
        }
    }
}

// Combine the splits of one (b, query head): M = max m_s, w_s = exp(m_s - M),
// out = sum w_s acc_s / sum w_s l_s.  1024 threads: thread (p, d) owns
// dimension d of splits p, p + kParts, ...  Every load (the partial sums and
// each split's m, l) is issued up front, so the kernel pays one memory
// latency; the maxima, weights and denominators then go through LDS.
constexpr int kCombineThreads = 1024;
constexpr uint32_t kMaxSplits = 256;

template <typename O, int HD, int GM>
__global__ __launch_bounds__(kCombineThreads) void paged_decode_combine(const float *__restrict__ part,
                                                                        typename O::T *__restrict__ out,
                                                                        uint32_t n_heads, uint32_t n_kv,
                                                                        uint32_t splits) {
    constexpr int kParts = kCombineThreads / HD;
    constexpr int kPer = kMaxSplits / kParts;  // splits per thread at most
    constexpr int kWaves = kCombineThreads / kWave;
    __shared__ float w_lds[kMaxSplits];
    __shared__ float red[kWaves];
    __shared__ float acc_lds[kParts][HD];
    const uint32_t bh = blockIdx.x, h = bh % n_heads, b = bh / n_heads;
    const uint32_t G = n_heads / n_kv, g = h / G, slot = h % G;
    constexpr uint32_t kRec = GM * (HD + kRecTail);
    const float *base = part + ((size_t)(b * n_kv + g) * splits) * kRec + slot * (HD + kRecTail);
    const uint32_t t = threadIdx.x, d = t % HD, p = t / HD;
    float av[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const uint32_t sp = p + (uint32_t)i * kParts;
        av[i] = sp < splits ? base[(size_t)sp * kRec + d] : 0.0f;
    }
    const float ms = t < splits ? base[(size_t)t * kRec + HD] : -__builtin_inff();
    const float ls = t < splits ? base[(size_t)t * kRec + HD + 1] : 0.0f;
    float M = wave_max(ms);
    if (t % kWave == 0) red[t / kWave] = M;
    __syncthreads();
    M = red[0];
#pragma unroll
    for (int i = 1; i < kWaves; ++i) M = fmaxf(M, red[i]);
    const float w = (t < splits && ms > -__builtin_inff()) ? __expf(ms - M) : 0.0f;
    if (t < kMaxSplits) w_lds[t] = w;
    float L = wave_sum(w * ls);
    __syncthreads();
    if (t % kWave == 0) red[t / kWave] = L;
    __syncthreads();
    L = 0.0f;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) L += red[i];
    float o = 0.0f;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const uint32_t sp = p + (uint32_t)i * kParts;
        if (sp < splits) o += w_lds[sp] * av[i];
    }
    acc_lds[p][d] = o;
    __syncthreads();
    if (t < (uint32_t)HD) {
        float r = 0.0f;
#pragma unroll
        for (int q = 0; q < kParts; ++q) r += acc_lds[q][t];
        out[((size_t)b * n_heads + h) * HD + t] = O::store(L > 0.0f ? r * (1.0f / L) : 0.0f);
    }
}

// The same combine by one wavefront per (b, query head), for the launches
// where the 1024-thread form's barriers and width cost more than its work:
// lanes take the splits for m and l (wavefront reductions, no barrier); for
// the sums HD/4 lanes cover a record's dims with 16-byte loads and the
// 64 / (HD/4) lane groups take interleaved splits, every load issued before
// the sums.  M, the weights and L as in paged_decode_combine.
template <typename O, int HD, int GM>
__global__ __launch_bounds__(kWave) void paged_decode_combine_wave(const float *__restrict__ part,
                                                                   typename O::T *__restrict__ out,
                                                                   uint32_t n_heads, uint32_t n_kv,
                                                                   uint32_t splits) {
    constexpr uint32_t kRec = HD + kRecTail;
    constexpr uint32_t LPR = HD / 4, SG = kWave / LPR;  // lanes per record, split groups
    constexpr uint32_t kPerLane = kMaxSplits / kWave;
    __shared__ float w_lds[kMaxSplits];
    const uint32_t bh = blockIdx.x, h = bh % n_heads, b = bh / n_heads;
    const uint32_t G = n_heads / n_kv, g = h / G, slot = h % G;
    const float *base = part + ((size_t)(b * n_kv + g) * splits * GM + slot) * kRec;  // split s: + s * GM * kRec
    const uint32_t lane = threadIdx.x, dq = lane % LPR, sg = lane / LPR;
    // the first batch of record sums first: its latency overlaps the m / l
    // reductions
    constexpr uint32_t kBatch = 16;
    float4 v[kBatch];
    auto load_batch = [&](uint32_t s0) {
#pragma unroll
        for (uint32_t j = 0; j < kBatch; ++j) {
            const uint32_t sp = s0 + sg + j * SG;
            v[j] = sp < splits ? *reinterpret_cast<const float4 *>(base + (size_t)sp * GM * kRec + 4 * dq)
                               : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    };
    load_batch(0);
    float ms[kPerLane], ls[kPerLane];
    float M = -__builtin_inff();
#pragma unroll
    for (uint32_t i = 0; i < kPerLane; ++i) {
        const uint32_t sp = lane + i * kWave;
        ms[i] = sp < splits ? base[(size_t)sp * GM * kRec + HD] : -__builtin_inff();
        ls[i] = sp < splits ? base[(size_t)sp * GM * kRec + HD + 1] : 0.0f;
        M = fmaxf(M, ms[i]);
    }
    M = wave_max(M);
    float Lp = 0.0f;
#pragma unroll
    for (uint32_t i = 0; i < kPerLane; ++i) {
        const uint32_t sp = lane + i * kWave;
        const float w = (sp < splits && ms[i] > -__builtin_inff()) ? __expf(ms[i] - M) : 0.0f;
        w_lds[sp] = w;
        Lp += w * ls[i];
    }
    const float L = wave_sum(Lp);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
    float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (uint32_t s0 = 0;;) {
#pragma unroll
        for (uint32_t j = 0; j < kBatch; ++j) {
            const uint32_t sp = s0 + sg + j * SG;
            const float w = sp < splits ? w_lds[sp] : 0.0f;
            o.x += w * v[j].x;
            o.y += w * v[j].y;
            o.z += w * v[j].z;
            o.w += w * v[j].w;
        }
        s0 += kBatch * SG;
        if (s0 >= splits) break;
        load_batch(s0);
    }
#pragma unroll
    for (uint32_t off = LPR; off < kWave; off *= 2) {
        o.x += __shfl_xor(o.x, off, kWave);
        o.y += __shfl_xor(o.y, off, kWave);
        o.z += __shfl_xor(o.z, off, kWave);
        o.w += __shfl_xor(o.w, off, kWave);
    }
    if (sg == 0) {
        const float inv = 1.0f / L;
        const float r[4] = {L > 0.0f ? o.x * inv : 0.0f, L > 0.0f ? o.y * inv : 0.0f, L > 0.0f ? o.z * inv : 0.0f,
                            L > 0.0f ? o.w * inv : 0.0f};
        store_f32<O, 4>(out + ((size_t)b * n_heads + h) * HD + 4 * dq, r);
    }
}

// Split count: about kTargetWaves wavefronts when batch * n_kv is small, at
// least kMinSplitBlocks blocks per split, at most kMaxSplits.
// Measured (one Llama-3-8B sequence, 8 KV heads): 2048 keys took 32 us with
// 16-block splits and 17.5 us with 2-block ones; 32768 keys did best at
// 128 splits (1024 wavefronts) rather than 256.
constexpr uint32_t kMinSplitBlocks = 2;
// Build knobs: the one-wavefront combine for launches of at most
// COMBINE_WAVE_MAX splits (1), or the 1024-thread combine always (0).
// Measured interleaved on one box: one 2048-key sequence (64 splits) 11.96
// against 12.16 us; one 32768-key sequence (128 splits) 35.9 against 34.0 us
// with the wavefront form, hence the limit.
#ifndef FELLM_ATT_COMBINE_WAVE
#define FELLM_ATT_COMBINE_WAVE 1
#endif
#ifndef FELLM_ATT_COMBINE_WAVE_MAX
#define FELLM_ATT_COMBINE_WAVE_MAX 64
#endif
// Build knob: wavefronts the split policy aims for.  With two blocks in
// flight from 8-block walks, one 32768-key sequence measured 34.0-34.2 us at
// 1024, 41.3-41.4 at 2048 and 52.3 at 512 (interleaved on one box).
#ifndef FELLM_ATT_TARGET_WAVES
#define FELLM_ATT_TARGET_WAVES 1024
#endif
constexpr uint32_t kTargetWaves = FELLM_ATT_TARGET_WAVES;
// Build knob: blocks per wavefront from which DEPTH 2 is used.  Measured
// (interleaved on one box): one Llama-3-8B sequence of 32768 keys (splits of
// 16 blocks) 37.8-37.9 us from 64, 33.9 us from 4, 8 or 16; 2048 keys (splits
// of 2 blocks) and 256 sequences x 4096 keys level.
#ifndef FELLM_ATT_DEEP_WALK
#define FELLM_ATT_DEEP_WALK 8
#endif
constexpr uint32_t kDeepWalk = FELLM_ATT_DEEP_WALK;
uint32_t choose_splits(uint32_t batch, uint32_t n_kv, uint32_t max_seq) {
    const uint32_t pairs = batch * n_kv;
    const uint32_t blocks = (max_seq + kBlockTokens - 1) / kBlockTokens;
    uint32_t s = pairs >= kTargetWaves ? 1 : (kTargetWaves + pairs - 1) / pairs;
    const uint32_t cap = blocks / kMinSplitBlocks > 0 ? blocks / kMinSplitBlocks : 1;
    if (s > cap) s = cap;
    if (s > kMaxSplits) s = kMaxSplits;
    return s ? s : 1;
}

template <typename Q, typename O, typename C, int HD, int GM>
int launch_decode(const void *q, void *out, uint32_t batch, uint32_t n_heads, uint32_t n_kv, const uint32_t *lens,
                  uint32_t max_seq, float scale, uint32_t causal, uint32_t window, const PagedGeom &geo,
                  float *ws, uint64_t ws_bytes, hipStream_t st) {
    uint32_t splits = choose_splits(batch, n_kv, max_seq);
    const uint64_t need = (uint64_t)batch * n_kv * splits * GM * (HD + kRecTail) * 4;
    if (splits > 1 && (!ws || ws_bytes < need)) splits = 1;
    const uint32_t blocks = (max_seq + kBlockTokens - 1) / kBlockTokens;
    const uint32_t bps = (blocks + splits - 1) / splits;
    // Two blocks in flight pay off on walks of 8 blocks and more (256
    // sequences x 4096 keys: 754 -> 720 us); splits of a few blocks do better
    // with one.
    if (bps >= kDeepWalk)
        FELLM_LAUNCH((paged_decode_kernel<Q, O, C, HD, GM, 2>), dim3(batch * n_kv * splits), dim3(kWave), 0,
                           st, static_cast<const typename Q::T *>(q), static_cast<typename O::T *>(out), ws, lens,
                           geo.table, geo, n_heads, n_kv, scale, causal, window, splits, bps);
    else
        FELLM_LAUNCH((paged_decode_kernel<Q, O, C, HD, GM, 1>), dim3(batch * n_kv * splits), dim3(kWave), 0,
                           st, static_cast<const typename Q::T *>(q), static_cast<typename O::T *>(out), ws, lens,
                           geo.table, geo, n_heads, n_kv, scale, causal, window, splits, bps > 0 ? bps : 1);
    int rc = launch_status();
    if (rc != FELLM_OK || splits == 1) return rc;
    if (FELLM_ATT_COMBINE_WAVE && splits <= FELLM_ATT_COMBINE_WAVE_MAX && aligned_to(ws, 16))
        FELLM_LAUNCH((paged_decode_combine_wave<O, HD, GM>), dim3(batch * n_heads), dim3(kWave), 0, st, ws,
                     static_cast<typename O::T *>(out), n_heads, n_kv, splits);
    else
        FELLM_LAUNCH((paged_decode_combine<O, HD, GM>), dim3(batch * n_heads), dim3(kCombineThreads), 0, st, ws,
                     static_cast<typename O::T *>(out), n_heads, n_kv, splits);
    return launch_status();
}

template <typename Q, typename O, typename C>
int dispatch_hd(uint32_t hd, uint32_t G, const void *q, void *out, uint32_t batch, uint32_t n_heads, uint32_t n_kv,
                const uint32_t *lens, uint32_t max_seq, float scale, uint32_t causal, uint32_t window,
                const PagedGeom &geo, float *ws, uint64_t ws_bytes, hipStream_t st) {
#define FELLM_ATT(HDV, GMV)                                                                                    \
    if (hd == HDV && G <= GMV)                                                                                 \
        return launch_decode<Q, O, C, HDV, GMV>(q, out, batch, n_heads, n_kv, lens, max_seq, scale, causal, window, \
                                                 geo, ws, ws_bytes, st);
    FELLM_ATT(64, 8)
    FELLM_ATT(64, 16)
    FELLM_ATT(128, 8)
    FELLM_ATT(128, 16)
    FELLM_ATT(256, 8)
    FELLM_ATT(256, 16)
#undef FELLM_ATT
    return FELLM_ERR_SHAPE;
}

// ---------------------------------------------------------------------------
// Attention over f32 K/V rows held contiguously ([t, n_kv * head_dim]), the
// non-paged arms of the reference's Attention launch:
//  * decode (backend.rs:1371-1397; CUDA attention_heads, launchers.rs:
//    3719-3760): one query row against keys [max(0, seq - window), seq) of
//    one K/V pair;
//  * canvas (backend.rs:1412-1535; CUDA attention_canvas_heads,
//    launchers.rs:3270-3333): every query row against the prefix keys
//    [prefix_start, past) of one pair and then all `rows` canvas keys of a
//    second pair, with no causal mask.
// One workgroup (four wavefronts) per (query row, KV head): the G query heads
// of the KV head share every K/V byte.  Keys go in tiles of 64, tile i to
// wavefront i % 4.  Scores: lane = key, the full q . k over the head
// dimension from 16-byte K loads against q held in LDS.  Online softmax per
// head (tile max and sum across the wavefront).  P.V: lane = dimension slot
// (dims lane, lane + 64, ...), probabilities read back from LDS.  The four
// wavefronts' (max, sum, accumulators) are merged in LDS at the end.
constexpr int kF32kvWaves = 4;

template <int VD, int GM>
__global__ __launch_bounds__(kF32kvWaves * kWave) void attention_f32kv_kernel(
    const float *__restrict__ q, float *__restrict__ out, uint32_t n_heads, uint32_t n_kv, uint32_t hd,
    const float *__restrict__ k1, const float *__restrict__ v1, uint32_t b1, uint32_t e1,
    const float *__restrict__ k2, const float *__restrict__ v2, uint32_t n2, float scale, uint32_t rows,
    uint32_t row_mode, uint32_t window, uint32_t head_major) {
    extern __shared__ float f32kv_lds[];
    __shared__ uint64_t exp_tab[32];
    const uint32_t G = n_heads / n_kv;
    const uint32_t row = blockIdx.x / n_kv, g = blockIdx.x % n_kv;
    const uint32_t lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const size_t kv_w = (size_t)n_kv * hd;  // elements per K/V row
    float *q_lds = f32kv_lds;                        // [G][hd]
    float *p_lds = f32kv_lds + GM * hd;              // [waves][GM][64]
    // q (and out) rows: [row][head][d], or head-major [head][row][d].
    const size_t hstride = head_major ? (size_t)rows * hd : hd;
    const size_t qbase = head_major ? ((size_t)g * G * rows + row) * hd : ((size_t)row * n_heads + (size_t)g * G) * hd;
    for (uint32_t i = threadIdx.x; i < G * hd; i += kF32kvWaves * kWave)
        q_lds[i] = q[qbase + (size_t)(i / hd) * hstride + i % hd];
    if (threadIdx.x < 32) exp_tab[threadIdx.x] = make_expf_table().tab[threadIdx.x];
    // This row's keys of the first pair: [b1, e1) as given (row_mode 0);
    // causal with the query rows ending at key e1 - 1 (row_mode 1: keys up to
    // e1 - rows + row, the last `window` of them when window > 0); or within
    // `window` of the row index (row_mode 2, all keys when window == 0).
    if (row_mode == 1) {
        const uint32_t last = e1 - rows + row;
        e1 = last + 1;
        b1 = window && e1 > window ? e1 - window : 0;
    } else if (row_mode == 2) {
        b1 = window && row + 1 > window ? row + 1 - window : 0;
        if (window && row + window < e1) e1 = row + window;
    }
    __syncthreads();

    const uint32_t n1 = e1 > b1 ? e1 - b1 : 0, n = n1 + n2;
    float m[GM], l[GM], acc[GM][VD];
#pragma unroll
    for (int h = 0; h < GM; ++h) {
        m[h] = -__builtin_inff();
        l[h] = 0.0f;
#pragma unroll
        for (int c = 0; c < VD; ++c) acc[h][c] = 0.0f;
    }
    float *pw = p_lds + (size_t)wave * GM * kWave;
    for (uint32_t t0 = wave * kWave; t0 < n; t0 += kF32kvWaves * kWave) {
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");  // previous tile's p reads before new writes
        __builtin_amdgcn_wave_barrier();
        // scores: lane = key t0 + lane
        const uint32_t j = t0 + lane;
        const bool valid = j < n;
        const float *kr = nullptr;
        if (valid) kr = j < n1 ? k1 + (size_t)(b1 + j) * kv_w + (size_t)g * hd : k2 + (size_t)(j - n1) * kv_w + (size_t)g * hd;
        float sc[GM];
#pragma unroll
        for (int h = 0; h < GM; ++h) sc[h] = 0.0f;
        if (valid) {
            for (uint32_t d = 0; d < hd; d += 4) {
                const float4 kv4 = *reinterpret_cast<const float4 *>(kr + d);
#pragma unroll
                for (int h = 0; h < GM; ++h) {
                    if (h < (int)G) {
                        const float4 q4 = *reinterpret_cast<const float4 *>(q_lds + h * hd + d);
                        sc[h] += q4.x * kv4.x + q4.y * kv4.y + q4.z * kv4.z + q4.w * kv4.w;
                    }
                }
            }
        }
        float alpha[GM];
#pragma unroll
        for (int h = 0; h < GM; ++h) {
            if (h >= (int)G) continue;
            const float s = valid ? sc[h] * scale : -__builtin_inff();
            const float m_new = fmaxf(m[h], wave_max(s));
            alpha[h] = m[h] > -__builtin_inff() ? expf_glibc(m[h] - m_new, exp_tab) : 0.0f;
            const float p = valid ? expf_glibc(s - m_new, exp_tab) : 0.0f;
            l[h] = l[h] * alpha[h] + wave_sum(p);
            m[h] = m_new;
            pw[h * kWave + lane] = p;
        }
        // P.V: lane = dimension slot, reading the p values other lanes of
        // this wavefront just wrote (waves run different tile counts, so no
        // workgroup barrier here: a wavefront-scope fence orders the LDS
        // writes before the reads).
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int h = 0; h < GM; ++h)
            if (h < (int)G)
#pragma unroll
                for (int c = 0; c < VD; ++c) acc[h][c] *= alpha[h];
        const uint32_t kn = n - t0 < (uint32_t)kWave ? n - t0 : (uint32_t)kWave;
        for (uint32_t jj = 0; jj < kn; ++jj) {
            const uint32_t jt = t0 + jj;
            const float *vr = jt < n1 ? v1 + (size_t)(b1 + jt) * kv_w + (size_t)g * hd
                                      : v2 + (size_t)(jt - n1) * kv_w + (size_t)g * hd;
            float vv[VD];
#pragma unroll
            for (int c = 0; c < VD; ++c) {
                const uint32_t d = lane + c * kWave;
                vv[c] = d < hd ? vr[d] : 0.0f;
            }
#pragma unroll
            for (int h = 0; h < GM; ++h) {
                if (h < (int)G) {
                    const float p = pw[h * kWave + jj];
#pragma unroll
                    for (int c = 0; c < VD; ++c) acc[h][c] += p * vv[c];
                }
            }
        }
    }
    // Merge the wavefronts into wavefront 0, one at a time through LDS.
    float *st = f32kv_lds;  // [GM][2 + hd]: m, l, acc
    for (uint32_t w = 1; w < (uint32_t)kF32kvWaves; ++w) {
        __syncthreads();
        if (wave == w) {
#pragma unroll
            for (int h = 0; h < GM; ++h) {
                if (h >= (int)G) continue;
                float *sh = st + h * (2 + hd);
                if (lane == 0) {
                    sh[0] = m[h];
                    sh[1] = l[h];
                }
#pragma unroll
                for (int c = 0; c < VD; ++c) {
                    const uint32_t d = lane + c * kWave;
                    if (d < hd) sh[2 + d] = acc[h][c];
                }
            }
        }
        __syncthreads();
        if (wave == 0) {
#pragma unroll
            for (int h = 0; h < GM; ++h) {
                if (h >= (int)G) continue;
                const float *sh = st + h * (2 + hd);
                const float mo = sh[0], lo = sh[1];
                const float mn = fmaxf(m[h], mo);
                if (mn == -__builtin_inff()) continue;
                const float a = m[h] > -__builtin_inff() ? expf_glibc(m[h] - mn, exp_tab) : 0.0f;
                const float b = mo > -__builtin_inff() ? expf_glibc(mo - mn, exp_tab) : 0.0f;
                l[h] = l[h] * a + lo * b;
                m[h] = mn;
#pragma unroll
                for (int c = 0; c < VD; ++c) {
                    const uint32_t d = lane + c * kWave;
                    acc[h][c] = acc[h][c] * a + (d < hd ? sh[2 + d] : 0.0f) * b;
                }
            }
        }
    }
    if (wave == 0) {
        float *orow = out + qbase;
#pragma unroll
        for (int h = 0; h < GM; ++h) {
            if (h >= (int)G) continue;
            const float inv = l[h] > 0.0f ? 1.0f / l[h] : 0.0f;
#pragma unroll
            for (int c = 0; c < VD; ++c) {
                const uint32_t d = lane + c * kWave;
                if (d < hd) orow[(size_t)h * hstride + d] = l[h] > 0.0f ? acc[h][c] * inv : 0.0f;
            }
        }
    }
}

}  // namespace
}  // namespace fellm

extern "C" uint64_t fellm_rocm_paged_attention_workspace(uint32_t batch, uint32_t n_heads, uint32_t n_kv_heads,
                                                         uint32_t head_dim, uint32_t max_seq) {
    using namespace fellm;
    if (!n_kv_heads || n_heads % n_kv_heads) return 0;
    const uint32_t splits = choose_splits(batch, n_kv_heads, max_seq);
    if (splits <= 1) return 0;
    const uint32_t gm = n_heads / n_kv_heads <= 8 ? 8 : 16;
    return (uint64_t)batch * n_kv_heads * splits * gm * (head_dim + kRecTail) * 4;
}

extern "C" int fellm_rocm_paged_attention(const void *q, uint32_t q_dtype, void *out, uint32_t out_dtype,
                                          uint32_t batch, uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                                          const uint32_t *row_lengths, uint32_t max_seq, float scale,
                                          uint32_t causal, uint32_t window, const FellmRocmPagedKv *kv,
                                          float *workspace, uint64_t workspace_bytes, void *stream) {
    using namespace fellm;
    if (!q || !out || !row_lengths || !kv || !kv->arena || !kv->block_table) return FELLM_ERR_ARITY;
    if (!n_kv_heads || n_heads % n_kv_heads || n_heads / n_kv_heads > 16) return FELLM_ERR_SHAPE;
    if (kv->stride != n_kv_heads * head_dim || kv->block_size != kBlockTokens) return FELLM_ERR_SHAPE;
    if (kv->block_bytes < 2ull * kv->block_size * kv->stride * 2 || kv->block_bytes % 16) return FELLM_ERR_SHAPE;
    if (kv->layer >= kv->n_layers) return FELLM_ERR_SHAPE;
    if (!aligned_to(kv->arena, 16) || !aligned_to(q, 16) || !aligned_to(out, 16)) return FELLM_ERR_SHAPE;
    if (batch == 0) return FELLM_OK;
    if (!(scale > 0.0f)) scale = 1.0f / sqrtf((float)head_dim);
    const PagedGeom geo{static_cast<const uint8_t *>(kv->arena), kv->arena_len, kv->block_table, kv->n_block_table,
                        kv->n_logical_blocks, kv->n_layers, kv->layer, kv->block_size, kv->block_bytes, kv->stride};
    hipStream_t st = as_stream(stream);
    const uint32_t G = n_heads / n_kv_heads;
    if (kv->kv_dtype != FELLM_DTYPE_F16 && kv->kv_dtype != FELLM_DTYPE_BF16) return FELLM_ERR_DTYPE;
    const bool bf = kv->kv_dtype == FELLM_DTYPE_BF16;
#define FELLM_ATT_QO(QD, QT, OD, OT)                                                                              \
    if (q_dtype == QD && out_dtype == OD)                                                                         \
        return bf ? dispatch_hd<QT, OT, CacheBF16>(head_dim, G, q, out, batch, n_heads, n_kv_heads, row_lengths,  \
                                                   max_seq, scale, causal, window, geo, workspace, workspace_bytes, \
                                                   st)                                                            \
                  : dispatch_hd<QT, OT, CacheF16>(head_dim, G, q, out, batch, n_heads, n_kv_heads, row_lengths,   \
                                                  max_seq, scale, causal, window, geo, workspace, workspace_bytes,  \
                                                  st);
    FELLM_ATT_QO(FELLM_DTYPE_F32, F32, FELLM_DTYPE_F32, F32)
    FELLM_ATT_QO(FELLM_DTYPE_F16, F16, FELLM_DTYPE_F16, F16)
    FELLM_ATT_QO(FELLM_DTYPE_BF16, BF16, FELLM_DTYPE_BF16, BF16)
    FELLM_ATT_QO(FELLM_DTYPE_F16, F16, FELLM_DTYPE_F32, F32)
    FELLM_ATT_QO(FELLM_DTYPE_BF16, BF16, FELLM_DTYPE_F32, F32)
#undef FELLM_ATT_QO
    return FELLM_ERR_DTYPE;
}

namespace fellm {
namespace {

int attention_f32kv_common(const float *q, float *out, uint32_t rows, uint32_t n_heads, uint32_t n_kv_heads,
                           uint32_t head_dim, const float *k1, const float *v1, uint32_t begin1, uint32_t end1,
                           const float *k2, const float *v2, uint32_t n2, float scale, uint32_t row_mode,
                           uint32_t window, uint32_t head_major, void *stream) {
    if (!q || !out) return FELLM_ERR_ARITY;
    if (end1 > begin1 && (!k1 || !v1)) return FELLM_ERR_ARITY;
    if (n2 && (!k2 || !v2)) return FELLM_ERR_ARITY;
    if (!n_kv_heads || n_heads % n_kv_heads || head_dim == 0 || head_dim % 4 || head_dim > 256) return FELLM_ERR_SHAPE;
    const uint32_t G = n_heads / n_kv_heads;
    if (G > 16 || (uint64_t)G * head_dim > 2048) return FELLM_ERR_SHAPE;
    for (const void *p : {(const void *)q, (const void *)k1, (const void *)v1, (const void *)k2, (const void *)v2})
        if (p && !aligned_to(p, 16)) return FELLM_ERR_SHAPE;
    if (rows == 0) return FELLM_OK;
    if (!(scale > 0.0f)) scale = 1.0f / sqrtf((float)head_dim);
    hipStream_t st = as_stream(stream);
    const uint32_t vd = (head_dim + kWave - 1) / kWave;
    auto go = [&]<int VD, int GM>() -> int {
        const size_t a = (size_t)GM * head_dim + (size_t)kF32kvWaves * GM * kWave;
        const size_t b = (size_t)GM * (2 + head_dim);
        const size_t lds = (a > b ? a : b) * sizeof(float);
        FELLM_LAUNCH((attention_f32kv_kernel<VD, GM>), dim3(rows * n_kv_heads), dim3(kF32kvWaves * kWave), lds, st,
                     q, out, n_heads, n_kv_heads, head_dim, k1, v1, begin1, end1, k2, v2, n2, scale, rows, row_mode,
                     window, head_major);
        return launch_status();
    };
    auto go_vd = [&]<int GM>() -> int {
        if (vd <= 1) return go.template operator()<1, GM>();
        if (vd <= 2) return go.template operator()<2, GM>();
        return go.template operator()<4, GM>();
    };
    if (G <= 1) return go_vd.template operator()<1>();
    if (G <= 2) return go_vd.template operator()<2>();
    if (G <= 4) return go_vd.template operator()<4>();
    if (G <= 8) return go_vd.template operator()<8>();
    return go_vd.template operator()<16>();
}

}  // namespace
}  // namespace fellm

extern "C" int fellm_rocm_attention_f32kv(const float *q, float *out, uint32_t rows, uint32_t n_heads,
                                          uint32_t n_kv_heads, uint32_t head_dim, const float *k1, const float *v1,
                                          uint32_t begin1, uint32_t end1, const float *k2, const float *v2, uint32_t n2,
                                          float scale, void *stream) {
    return fellm::attention_f32kv_common(q, out, rows, n_heads, n_kv_heads, head_dim, k1, v1, begin1, end1, k2, v2,
                                         n2, scale, 0, 0, 0, stream);
}

extern "C" int fellm_rocm_attention_f32kv_rows(const float *q, float *out, uint32_t query_len, uint32_t n_heads,
                                               uint32_t n_kv_heads, uint32_t head_dim, const float *k,
                                               const float *v, uint32_t kv_len, float scale, uint32_t causal,
                                               uint32_t window, void *stream) {
    if (query_len == 0) return FELLM_OK;
    if (causal && kv_len < query_len) return FELLM_ERR_SHAPE;  // the query rows end at the last key
    if (kv_len == 0) return FELLM_ERR_SHAPE;
    return fellm::attention_f32kv_common(q, out, query_len, n_heads, n_kv_heads, head_dim, k, v, 0, kv_len, nullptr,
                                         nullptr, 0, scale, causal ? 1 : 2, window, 1, stream);
}
