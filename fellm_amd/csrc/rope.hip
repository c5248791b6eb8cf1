// Rotary position embedding, paged KV append, and the two fused.
//
// RoPE reference: crates/backend-cpu/src/backend.rs:1135-1172 (launch_rope)
//   -> kernels/rope.rs:28-62 (rope_inplace_with_freqs_ex):
//   theta = (pos as f32) * inv_freq[i]; (s, c) = sin_cos(theta)
//   a' = a*c - b*s;  b' = a*s + b*c        (no FMA contraction)
//   pairing 0: (2i, 2i+1); 1: (i, i + rope_dim/2); 2: adjacent over the last
//   rope_dim dims of the head.  Dims outside the rotated span pass through.
// KvWrite reference: backend.rs:1734-1775 and the paged addressing of
//   crates/fellm-plugin-abi/src/paged_ctx.rs:341-360 (row_mut_for),
//   block bytes from crates/backend-cuda/src/vram_pool.rs:31-35.
//
// One workgroup handles one token row.  The rope_dim/2 (sin, cos) pairs for
// that row's position are computed once into LDS (a bit-exact restatement of
// glibc's sinf/cosf, the libm behind Rust's f32::sin_cos) and shared
// by every head of q and k, instead of once per (head, pair) as on the CPU.
// The row is then cut into items of PV pairs (PV = 4: one 16-byte access per
// item for 16-bit activations) spread over the block.  In KV mode the rotated
// K row and the V row are also rounded once to the cache dtype and written
// into their paged slots, so K never makes an extra HBM round trip.
#include <algorithm>
#include <initializer_list>
#include <type_traits>

#include "common.hpp"
#include "norm_body.hpp"
#include "swiglu_body.hpp"

// Build knob: non-temporal activation loads (bit 0) and stores (bit 1).
#ifndef FELLM_ROPE_NT
#define FELLM_ROPE_NT 2
#endif
// Build knob: MODE 0 slot walk with per-thread constants hoisted (1) or the
// generic walk shared with MODE 1 (0).  Measured interleaved on one box:
// configs[1] q+k 15.0-15.4 against 15.5-16.3 us, f32 and split-half
// pairings 4-8% faster.
#ifndef FELLM_ROPE_FAST
#define FELLM_ROPE_FAST 1
#endif
// Build knobs: the hoisted walk serves row groups of up to FAST_MAX_R rows,
// and prefill RoPE launches ask for FELLM_ROPE_WAVES waves per SIMD.  With
// row groups the hoisted walk needs 67 VGPRs for bf16 (7 waves): alone it
// measured 61.4-62.8 us at configs[4]; with 8 waves requested it spills
// 20 bytes per lane for bf16 and measured 57.0-57.1 against 58.7-59.3 us for
// the generic walk (interleaved on one box), configs[1] level.
#ifndef FELLM_ROPE_FAST_MAX_R
#define FELLM_ROPE_FAST_MAX_R 4
#endif
#ifndef FELLM_ROPE_WAVES
#define FELLM_ROPE_WAVES 8
#endif
// Build knob: (row, head) slots each thread loads before rotating/storing.
// Build knob: 16-bit items kept packed in registers between load and
// rotation in the fast slot walk (1) or widened to f32 at the load (0).
#ifndef FELLM_ROPE_RAW
#define FELLM_ROPE_RAW 1
#endif
// Build knob: 16-bit outputs of the prefill walk through the packed
// hardware conversions (round_words: a bf16 lane holding a NaN rounds
// element by element) (1), or element by element (0).  Measured interleaved
// on one box with word-wise non-temporal stores: configs[1] 14.4-14.5
// against 14.7-14.8 us, configs[4] 54.4-54.7 against 55.0 us.
#ifndef FELLM_ROPE_BF16_HW
#define FELLM_ROPE_BF16_HW 1
#endif
// The same for the RoPE + K/V append launches (q outputs and cache slots).
#ifndef FELLM_ROPE_BF16_HW_KV
#define FELLM_ROPE_BF16_HW_KV 1
#endif
// Build knob: row-group launches (R > 1: 8192 rows and more) read their
// packed 16-bit items non-temporally (1).  Measured interleaved on one box:
// configs[4] 53.6 against 54.8-54.9 us; one-row launches stay regular
// (configs[1] 17.1-17.3 against 14.1-14.3 us with non-temporal loads: its
// 42 MB of inputs are read from the last-level cache).
#ifndef FELLM_ROPE_RAW_NT
#define FELLM_ROPE_RAW_NT 1
#endif
#ifndef FELLM_ROPE_UNROLL
#define FELLM_ROPE_UNROLL 3
#endif
// Build knob: workgroups per row of the standalone RoPE + K/V append launch
// (0: rope_head_split).  Measured at configs[3], interleaved on one box: the
// rule's 4 6.24-6.28 us, 1 8.08-8.16, 2 6.64-6.72, 8 7.16.
#ifndef FELLM_KV_HSPLIT
#define FELLM_KV_HSPLIT 0
#endif

namespace fellm {
namespace {

constexpr int kRopeBlock = 256;
// Build knobs: workgroup size of the prefill RoPE launch with one row per
// workgroup (BLOCK1) and with row groups (BLOCKN).  Measured interleaved on
// one box: configs[1] (one row) 128 threads 14.6-14.7 us, level with 256
// (14.4-15.5), 512 18.9-19.4; configs[4] (four rows) 256 59.1-59.6 us, 128
// 64.1-64.4, 512 61.9-62.4.
#ifndef FELLM_ROPE_BLOCK1
#define FELLM_ROPE_BLOCK1 256
#endif
#ifndef FELLM_ROPE_BLOCKN
#define FELLM_ROPE_BLOCKN 256
#endif
constexpr uint32_t kMaxHalf = 512;  // rope_dim <= 1024

struct KvDev {
    uint8_t *arena;
    uint64_t arena_len;
    const uint32_t *table;
    uint64_t n_table;
    uint32_t n_logical, n_layers, layer, block_size;
    uint64_t block_bytes;
    uint32_t stride;
};

// Byte offset of (batch row, position)'s K row, or UINT64_MAX if the slot lies
// outside the table or the arena.  V rows sit block_size rows further on.
__device__ __forceinline__ uint64_t kv_slot_offset(const KvDev &kv, uint32_t row, uint32_t pos) {
    const uint32_t logical = pos / kv.block_size;
    const uint32_t slot = pos % kv.block_size;
    if (logical >= kv.n_logical) return ~0ull;
    const uint64_t idx = ((uint64_t)row * kv.n_layers + kv.layer) * kv.n_logical + logical;
    if (idx >= kv.n_table) return ~0ull;
    const uint64_t phys = kv.table[idx];
    const uint64_t row_bytes = (uint64_t)kv.stride * 2;
    const uint64_t base = phys * kv.block_bytes + (uint64_t)slot * row_bytes;
    if (base + (uint64_t)kv.block_size * row_bytes + row_bytes > kv.arena_len) return ~0ull;
    return base;
}

// 16-bit stores through the packed hardware conversions (round_words: f16
// always, bf16 for lanes without a NaN, which otherwise round element by
// element).  HW = false (or an f32 type): the type's own rounding.
template <typename A, int N, bool NT, bool HW, bool WORD_NT = false>
__device__ __forceinline__ void store16(typename A::T *p, const float (&v)[N]) {
    if constexpr (HW && (std::is_same_v<A, BF16> || std::is_same_v<A, F16>) && N % 2 == 0) {
        uint32_t w[N / 2];
        round_words<A, N>(v, w);
        store_words<N / 2, WORD_NT>(reinterpret_cast<uint32_t *>(p), w, NT);
    } else {
        if constexpr (NT) store_f32_nt<A, N>(p, v); else store_f32<A, N>(p, v);
    }
}

template <typename C, int N, bool HW = false>
__device__ __forceinline__ void store_cache(uint8_t *arena, uint64_t byte_off, uint32_t elem,
                                            const float (&v)[N]) {
    store16<C, N, false, HW>(reinterpret_cast<typename C::T *>(arena + byte_off) + elem, v);
}

template <typename A, int N>
__device__ __forceinline__ void act_load(const typename A::T *p, float (&v)[N]) {
    if constexpr (FELLM_ROPE_NT & 1) load_f32_nt<A, N>(p, v); else load_f32<A, N>(p, v);
}

// The prefill walk (MODE 0) stores word by word, the append path (MODE 1)
// as vectors (see store_words).
template <typename A, int N, bool HW = (FELLM_ROPE_BF16_HW != 0), bool WORD_NT = true>
__device__ __forceinline__ void act_store(typename A::T *p, const float (&v)[N]) {
    store16<A, N, (FELLM_ROPE_NT & 2) != 0, HW, WORD_NT>(p, v);
}

// Element offset, within its head, of item `it`'s first run and of its
// second run (PV elements each).  Items [0, n_rot) are rotated; the rest are
// the pass-through span.  Adjacent pairings keep both runs contiguous.
__device__ __forceinline__ void item_offsets(uint32_t it, uint32_t n_rot, uint32_t head_dim, uint32_t rope_dim,
                                             uint32_t pairing, int PV, uint32_t &lo, uint32_t &hi) {
    if (it >= n_rot) {
        lo = (pairing == 2 ? 0 : rope_dim) + (it - n_rot) * 2 * PV;
        hi = lo + PV;
    } else if (pairing == 1) {
        lo = it * PV;
        hi = lo + rope_dim / 2;
    } else {
        lo = (pairing == 2 ? head_dim - rope_dim : 0) + 2 * it * PV;
        hi = lo + PV;
    }
}

// Loads the 2*PV elements of item `it` of head `hd` (q heads, then k heads,
// then v heads) of `row`: e[0..PV) is the first run, e[PV..2PV) the second.
template <typename A, int PV>
__device__ __forceinline__ void rope_load(const typename A::T *x1, const typename A::T *x2,
                                          const typename A::T *x3, uint32_t nh1, uint32_t nh2, size_t w1, size_t w2,
                                          uint32_t row, uint32_t hd, uint32_t it, uint32_t head_dim, uint32_t rope_dim,
                                          uint32_t pairing, uint32_t n_rot, float (&e)[2 * PV]) {
    if constexpr (sizeof(typename A::T) * 2 * PV > 16) {
        // Items wider than one 16-byte access (f32) take two loads whatever
        // the layout: the branches pick the two addresses and the loads
        // follow unconditionally, so e is written at fixed indices only
        // (writes of e merged across branches would move it to scratch).
        const typename A::T *p0, *p1;
        if (hd < nh1 + nh2) {
            const bool first = hd < nh1;
            const typename A::T *src = first ? x1 : x2;
            const size_t base = first ? (size_t)row * w1 + (size_t)hd * head_dim
                                      : (size_t)row * w2 + (size_t)(hd - nh1) * head_dim;
            uint32_t lo, hi;
            item_offsets(it, n_rot, head_dim, rope_dim, pairing, PV, lo, hi);
            p0 = src + base + lo;
            p1 = src + base + hi;
        } else {  // V head: plain 2*PV-element run
            p0 = x3 + (size_t)row * w2 + (size_t)(hd - nh1 - nh2) * head_dim + it * 2 * PV;
            p1 = p0 + PV;
        }
        float a[PV], b[PV];
        act_load<A, PV>(p0, a);
        act_load<A, PV>(p1, b);
#pragma unroll
        for (int k = 0; k < PV; ++k) {
            e[k] = a[k];
            e[PV + k] = b[k];
        }
        return;
    }
    const typename A::T *src;
    size_t base;
    if (hd < nh1) {
        src = x1;
        base = (size_t)row * w1 + (size_t)hd * head_dim;
    } else if (hd < nh1 + nh2) {
        src = x2;
        base = (size_t)row * w2 + (size_t)(hd - nh1) * head_dim;
    } else {  // V head: plain 2*PV-element run
        act_load<A, 2 * PV>(x3 + (size_t)row * w2 + (size_t)(hd - nh1 - nh2) * head_dim + it * 2 * PV, e);
        return;
    }
    uint32_t lo, hi;
    item_offsets(it, n_rot, head_dim, rope_dim, pairing, PV, lo, hi);
    if (hi == lo + PV) {
        act_load<A, 2 * PV>(src + base + lo, e);
    } else {
        float a[PV], b[PV];
        act_load<A, PV>(src + base + lo, a);
        act_load<A, PV>(src + base + hi, b);
#pragma unroll
        for (int k = 0; k < PV; ++k) {
            e[k] = a[k];
            e[PV + k] = b[k];
        }
    }
}

// Rotates a loaded item and stores it (and the K/V cache copies in MODE 1).
template <typename A, typename C, int PV, int MODE>
__device__ __forceinline__ void rope_finish(const typename A::T *x1, typename A::T *out1, const typename A::T *x2,
                                            typename A::T *out2, uint32_t nh1, uint32_t nh2, size_t w1, size_t w2,
                                            uint32_t row, uint32_t hd, uint32_t it, uint32_t head_dim,
                                            uint32_t rope_dim, uint32_t pairing, uint32_t n_rot, const float2 *cs,
                                            float (&e)[2 * PV], uint64_t kbase, const KvDev &kv, uint64_t v_off) {
    if (hd >= nh1 + nh2) {  // V head (MODE 1 only)
        if constexpr (MODE == 1) {
            const uint32_t el = (hd - nh1 - nh2) * head_dim + it * 2 * PV;
            if (kbase != ~0ull)
                store_f32<C, 2 * PV>(reinterpret_cast<typename C::T *>(kv.arena + kbase + v_off) + el, e);
        }
        return;
    }
    const bool second = hd >= nh1;
    const uint32_t h = second ? hd - nh1 : hd;
    const typename A::T *src = second ? x2 : x1;
    typename A::T *dst = second ? out2 : out1;
    const size_t base = (size_t)row * (second ? w2 : w1) + (size_t)h * head_dim;
    uint32_t lo, hi;
    item_offsets(it, n_rot, head_dim, rope_dim, pairing, PV, lo, hi);
    if (it < n_rot) {
        const uint32_t i0 = it * PV;
        if (pairing == 1) {
#pragma unroll
            for (int k = 0; k < PV; ++k) {
                const float2 sc = cs[i0 + k];  // (sin, cos)
                const float a = e[k], b = e[PV + k];
                e[k] = a * sc.y - b * sc.x;
                e[PV + k] = a * sc.x + b * sc.y;
            }
        } else {
#pragma unroll
            for (int k = 0; k < PV; ++k) {
                const float2 sc = cs[i0 + k];
                const float a = e[2 * k], b = e[2 * k + 1];
                e[2 * k] = a * sc.y - b * sc.x;
                e[2 * k + 1] = a * sc.x + b * sc.y;
            }
        }
    }
    const bool write = dst && (dst != src || it < n_rot);
    const bool cache = MODE == 1 && second && kbase != ~0ull;
    constexpr bool HW = MODE == 1 ? FELLM_ROPE_BF16_HW_KV != 0 : FELLM_ROPE_BF16_HW != 0;
    if (hi == lo + PV) {
        if (write) act_store<A, 2 * PV, HW, MODE != 1>(dst + base + lo, e);
        if constexpr (MODE == 1)
            if (cache) store_cache<C, 2 * PV, HW>(kv.arena, kbase, h * head_dim + lo, e);
    } else {
        float a[PV], b[PV];
#pragma unroll
        for (int k = 0; k < PV; ++k) {
            a[k] = e[k];
            b[k] = e[PV + k];
        }
        if (write) {
            act_store<A, PV, HW, MODE != 1>(dst + base + lo, a);
            act_store<A, PV, HW, MODE != 1>(dst + base + hi, b);
        }
        if constexpr (MODE == 1) {
            if (cache) {
                store_cache<C, PV, HW>(kv.arena, kbase, h * head_dim + lo, a);
                store_cache<C, PV, HW>(kv.arena, kbase, h * head_dim + hi, b);
            }
        }
    }
}

// MODE 0 with a fixed item position per thread: the slot walk with every
// per-thread constant hoisted out of it.  KIND is the thread's item kind
// (uniform over its slots): 0 pass-through (unrotated span), 1 adjacent
// pairs (e[2k], e[2k+1]) in one contiguous run, 2 split-half pairs
// (e[k], e[PV+k]) in two runs `hi - lo` apart.  With one row per workgroup
// the thread's PV (sin, cos) pairs are read from LDS once; with row groups
// they are read per slot from the slot's row.
constexpr int kRopePass = 0, kRopeAdjacent = 1, kRopeSplit = 2;

template <typename A, int PV, int R, int KIND, int BLOCK>
__device__ __forceinline__ void rope_fast_slots(const typename A::T *x1, typename A::T *out1, uint32_t nh1,
                                                const typename A::T *x2, typename A::T *out2, size_t w1, size_t w2,
                                                uint32_t row0, uint32_t total_slots, uint32_t h0, uint32_t heads,
                                                uint32_t head_dim, uint32_t lo, uint32_t hi, uint32_t i0,
                                                uint32_t step, float2 (*cs_all)[kMaxHalf / R]) {
    using T = typename A::T;
    constexpr int U = FELLM_ROPE_UNROLL;
    float2 sc1[KIND == kRopePass || R > 1 ? 1 : PV];
    if constexpr (KIND != kRopePass && R == 1) {
#pragma unroll
        for (int k = 0; k < PV; ++k) sc1[k] = cs_all[0][i0 + k];
    }
    uint32_t slot = threadIdx.x / (BLOCK / step);
    uint32_t rr = slot / heads, hd = slot % heads;
    // Per slot only its row and head stay live across the batch; the
    // element offset is recomputed at the store (cheaper in registers than
    // keeping a 64-bit offset per slot).
    auto slot_off = [&](uint32_t r, uint32_t h) -> size_t {
        return h < nh1 ? (size_t)(row0 + r) * w1 + (size_t)h * head_dim
                       : (size_t)(row0 + r) * w2 + (size_t)(h - nh1) * head_dim;
    };
    // 16-bit activations stay packed between the loads and the rotation
    // (2 elements per register): a batch of U items then holds half the
    // registers, which keeps the row-group walk at 8 waves per SIMD without
    // spilling (bf16 needs more temporaries than f16 for its rounding).
    constexpr bool RAW = sizeof(T) == 2 && FELLM_ROPE_RAW;
    constexpr int RW = RAW ? (int)sizeof(T) * PV / 4 : 1;  // 32-bit words per run
    for (; slot < total_slots; slot += step * U) {
        float e[RAW ? 1 : U][2 * PV];
        uint32_t raw[RAW ? U : 1][2 * RW];
        uint32_t srr[U], sh[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t h = h0 + hd;
            srr[u] = rr;
            sh[u] = h;
            if constexpr (RAW) {
                if (slot + u * step < total_slots) {
                    const T *src = (h < nh1 ? x1 : x2) + slot_off(rr, h);
                    const uint32_t *pa = reinterpret_cast<const uint32_t *>(src + lo);
                    const uint32_t *pb = reinterpret_cast<const uint32_t *>(src + (KIND == kRopeSplit ? hi : lo + PV));
                    if constexpr (RW == 2 && KIND != kRopeSplit) {  // one 16-byte run
                        typedef uint32_t u4v __attribute__((ext_vector_type(4)));
                        u4v av;
                        if constexpr (FELLM_ROPE_RAW_NT && R > 1)
                            av = __builtin_nontemporal_load(reinterpret_cast<const u4v *>(pa));
                        else
                            av = *reinterpret_cast<const u4v *>(pa);
                        const uint4 a = make_uint4(av.x, av.y, av.z, av.w);
                        raw[u][0] = a.x;
                        raw[u][1] = a.y;
                        raw[u][2] = a.z;
                        raw[u][3] = a.w;
                    } else if constexpr (RW == 2) {
                        const uint2 a = *reinterpret_cast<const uint2 *>(pa), b = *reinterpret_cast<const uint2 *>(pb);
                        raw[u][0] = a.x;
                        raw[u][1] = a.y;
                        raw[u][2] = b.x;
                        raw[u][3] = b.y;
                    } else {
#pragma unroll
                        for (int w = 0; w < RW; ++w) {
                            raw[u][w] = pa[w];
                            raw[u][RW + w] = pb[w];
                        }
                    }
                }
                hd += step;
                while (hd >= heads) {
                    hd -= heads;
                    ++rr;
                }
                continue;
            }
            if (slot + u * step < total_slots) {
                const T *src = (h < nh1 ? x1 : x2) + slot_off(rr, h);
                if constexpr (KIND == kRopeSplit) {
                    float a[PV], b[PV];
                    act_load<A, PV>(src + lo, a);
                    act_load<A, PV>(src + hi, b);
#pragma unroll
                    for (int k = 0; k < PV; ++k) {
                        e[u][k] = a[k];
                        e[u][PV + k] = b[k];
                    }
                } else if constexpr (sizeof(T) * 2 * PV > 16) {
                    float a[PV], b[PV];
                    act_load<A, PV>(src + lo, a);
                    act_load<A, PV>(src + lo + PV, b);
#pragma unroll
                    for (int k = 0; k < PV; ++k) {
                        e[u][k] = a[k];
                        e[u][PV + k] = b[k];
                    }
                } else {
                    act_load<A, 2 * PV>(src + lo, e[u]);
                }
            }
            hd += step;
            while (hd >= heads) {
                hd -= heads;
                ++rr;
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (slot + u * step >= total_slots) continue;
            const bool first = sh[u] < nh1;
            const size_t off = slot_off(srr[u], sh[u]);
            const T *src = (first ? x1 : x2) + off;
            T *dst = (first ? out1 : out2);
            if (!dst) continue;
            dst += off;
            float (&ev)[2 * PV] = e[RAW ? 0 : u];
            if constexpr (RAW) {
#pragma unroll
                for (int i = 0; i < 2 * PV; ++i)
                    ev[i] = A::load(__builtin_bit_cast(T, (uint16_t)(raw[u][i / 2] >> (16 * (i % 2)))));
            }
            if constexpr (KIND == kRopePass) {
                if (dst == src) continue;  // in place: the span is already there
            } else {
#pragma unroll
                for (int k = 0; k < PV; ++k) {
                    const float2 sc = R == 1 ? sc1[k] : cs_all[srr[u]][i0 + k];  // (sin, cos)
                    const int ia = KIND == kRopeSplit ? k : 2 * k, ib = KIND == kRopeSplit ? PV + k : 2 * k + 1;
                    const float a = ev[ia], b = ev[ib];
                    ev[ia] = a * sc.y - b * sc.x;
                    ev[ib] = a * sc.x + b * sc.y;
                }
            }
            if constexpr (KIND == kRopeSplit) {
                float a[PV], b[PV];
#pragma unroll
                for (int k = 0; k < PV; ++k) {
                    a[k] = ev[k];
                    b[k] = ev[PV + k];
                }
                act_store<A, PV>(dst + lo, a);
                act_store<A, PV>(dst + hi, b);
            } else {
                act_store<A, 2 * PV>(dst + lo, ev);
            }
        }
    }
}

// MODE 0: rotate x1 -> out1 and x2 -> out2.
// MODE 1: additionally write rotated x2 (K) and x3 (V) into the paged cache
//         (cache element type C).
// Each workgroup handles R consecutive rows: all threads first fill the
// R x rope_dim/2 (sin, cos) table (one barrier), then stream every item of
// the R rows.
// The work of workgroup `bid` of a RoPE launch (every thread calls it;
// contains a barrier).  cs_all / kbase_all: the LDS tables below.
template <typename A, typename C, int PV, int MODE, int R, int BLOCK = kRopeBlock>
__device__ __forceinline__ void rope_block(
    // x1/out1 and x2/out2 may alias (in-place rotation): no __restrict__.
    const typename A::T *x1, typename A::T *out1, uint32_t nh1,
    const typename A::T *x2, typename A::T *out2, uint32_t nh2,
    const typename A::T *__restrict__ x3, uint32_t rows, uint32_t head_dim, uint32_t rope_dim, uint32_t pairing,
    const float *__restrict__ inv_freqs, const uint32_t *__restrict__ rope_pos, uint32_t pos0,
    const uint32_t *__restrict__ kv_pos, const KvDev &kv, uint32_t *__restrict__ err, uint32_t hsplit, uint32_t bid,
    float2 (*cs_all)[kMaxHalf / R], uint64_t *kbase_all) {
    // hsplit workgroups share a row group, each taking a contiguous range of
    // its (q, k, v) heads.
    const uint32_t part = bid % hsplit;
    const uint32_t row0 = bid / hsplit * R;
    const uint32_t half = rope_dim / 2;
    for (uint32_t t = threadIdx.x; t < R * half; t += BLOCK) {
        const uint32_t rr = t / half, i = t % half;
        const uint32_t row = row0 + rr;
        if (row >= rows) continue;
        uint32_t pos;
        if constexpr (MODE == 1)
            pos = rope_pos ? rope_pos[row] : kv_pos[row];
        else
            pos = rope_pos ? rope_pos[row] : pos0 + row;
        const float theta = (float)pos * inv_freqs[i];
        float sf, cf;
        sincosf_glibc(theta, &sf, &cf);
        cs_all[rr][i] = make_float2(sf, cf);
    }
    if constexpr (MODE == 1) {
        if (threadIdx.x < R) {
            const uint32_t row = row0 + threadIdx.x;
            uint64_t kb = ~0ull;
            if (row < rows) {
                kb = kv_slot_offset(kv, row, kv_pos[row]);
                if (kb == ~0ull && err) atomicOr(err, 1u);
            }
            kbase_all[threadIdx.x] = kb;
        }
    }
    __syncthreads();

    const uint32_t n_rot = half / PV;                // rotated items of PV pairs
    const uint32_t items_head = head_dim / (2 * PV);  // all items of a head
    const uint32_t nh_x2 = x2 ? nh2 : 0;
    const uint32_t nh_v = (MODE == 1) ? nh2 : 0;
    const uint32_t all_heads = nh1 + nh_x2 + nh_v;   // q heads, k heads, v heads
    const uint32_t h0 = part * all_heads / hsplit;
    const uint32_t heads = (part + 1) * all_heads / hsplit - h0;  // this workgroup's heads
    const size_t w1 = (size_t)nh1 * head_dim, w2 = (size_t)nh2 * head_dim;
    const uint64_t v_off = (uint64_t)kv.block_size * kv.stride * 2;
    const uint32_t nrows = rows - row0 < (uint32_t)R ? rows - row0 : (uint32_t)R;

    // When items_head divides the block (head_dim a power of two), each thread
    // keeps one item position `it` and walks (row, head) slots with a fixed
    // step, U slots per batch: all U loads are issued before any rotation or
    // store, so each thread keeps U 16-byte requests in flight.  Other shapes
    // enumerate items one by one with divisions.
    const bool fixed_item = items_head <= BLOCK && BLOCK % items_head == 0;
    const uint32_t total_slots = nrows * heads;
    if constexpr (MODE == 0 && FELLM_ROPE_FAST && R <= FELLM_ROPE_FAST_MAX_R) {
        if (fixed_item) {
            const uint32_t it = threadIdx.x % items_head;
            uint32_t lo, hi;
            item_offsets(it, n_rot, head_dim, rope_dim, pairing, PV, lo, hi);
            const uint32_t step = BLOCK / items_head;
            if (it >= n_rot)
                rope_fast_slots<A, PV, R, kRopePass, BLOCK>(x1, out1, nh1, x2, out2, w1, w2, row0, total_slots, h0, heads,
                                                     head_dim, lo, hi, 0, step, cs_all);
            else if (hi == lo + PV)
                rope_fast_slots<A, PV, R, kRopeAdjacent, BLOCK>(x1, out1, nh1, x2, out2, w1, w2, row0, total_slots, h0,
                                                         heads, head_dim, lo, hi, it * PV, step, cs_all);
            else
                rope_fast_slots<A, PV, R, kRopeSplit, BLOCK>(x1, out1, nh1, x2, out2, w1, w2, row0, total_slots, h0, heads,
                                                      head_dim, lo, hi, it * PV, step, cs_all);
            return;
        }
    }
    if (fixed_item) {
        const uint32_t it = threadIdx.x % items_head;
        const uint32_t step = BLOCK / items_head;
        uint32_t slot = threadIdx.x / items_head;
        uint32_t rr = slot / heads, hd = slot % heads;
        for (; slot < total_slots; slot += step * FELLM_ROPE_UNROLL) {
            uint32_t srr[FELLM_ROPE_UNROLL], shd[FELLM_ROPE_UNROLL];
            float e[FELLM_ROPE_UNROLL][2 * PV];
#pragma unroll
            for (int uu = 0; uu < FELLM_ROPE_UNROLL; ++uu) {
                srr[uu] = rr;
                shd[uu] = hd;
                if (slot + uu * step < total_slots)
                    rope_load<A, PV>(x1, x2, x3, nh1, nh_x2, w1, w2, row0 + rr, h0 + hd, it, head_dim, rope_dim,
                                     pairing, n_rot, e[uu]);
                hd += step;
                while (hd >= heads) {
                    hd -= heads;
                    ++rr;
                }
            }
#pragma unroll
            for (int uu = 0; uu < FELLM_ROPE_UNROLL; ++uu) {
                if (slot + uu * step < total_slots)
                    rope_finish<A, C, PV, MODE>(x1, out1, x2, out2, nh1, nh_x2, w1, w2, row0 + srr[uu], h0 + shd[uu], it,
                                                head_dim, rope_dim, pairing, n_rot, cs_all[srr[uu]], e[uu],
                                                kbase_all[srr[uu]], kv, v_off);
            }
        }
    } else {
        for (uint32_t t = threadIdx.x; t < total_slots * items_head; t += BLOCK) {
            const uint32_t it = t % items_head, slot = t / items_head;
            const uint32_t rr = slot / heads, hd = h0 + slot % heads;
            float e[2 * PV];
            rope_load<A, PV>(x1, x2, x3, nh1, nh_x2, w1, w2, row0 + rr, hd, it, head_dim, rope_dim, pairing, n_rot, e);
            rope_finish<A, C, PV, MODE>(x1, out1, x2, out2, nh1, nh_x2, w1, w2, row0 + rr, hd, it, head_dim, rope_dim,
                                        pairing, n_rot, cs_all[rr], e, kbase_all[rr], kv, v_off);
        }
    }
}

template <typename A, typename C, int PV, int MODE, int R, int BLOCK = kRopeBlock>
__global__ __launch_bounds__(BLOCK)
__attribute__((amdgpu_waves_per_eu(MODE == 0 && BLOCK == 256 ? FELLM_ROPE_WAVES : 1))) void rope_kernel(
    const typename A::T *x1, typename A::T *out1, uint32_t nh1, const typename A::T *x2, typename A::T *out2,
    uint32_t nh2, const typename A::T *__restrict__ x3, uint32_t rows, uint32_t head_dim, uint32_t rope_dim,
    uint32_t pairing, const float *__restrict__ inv_freqs, const uint32_t *__restrict__ rope_pos, uint32_t pos0,
    const uint32_t *__restrict__ kv_pos, KvDev kv, uint32_t *__restrict__ err, uint32_t hsplit) {
    __shared__ float2 cs_all[R][kMaxHalf / R];
    __shared__ uint64_t kbase_all[R];
    rope_block<A, C, PV, MODE, R, BLOCK>(x1, out1, nh1, x2, out2, nh2, x3, rows, head_dim, rope_dim, pairing,
                                         inv_freqs, rope_pos, pos0, kv_pos, kv, err, hsplit, blockIdx.x, cs_all,
                                         kbase_all);
}

// Rows per workgroup.  Measured on MI355X (q+k, 32/8 heads, hd 128): at
// 4096 rows one row per workgroup streams fastest (18.7 us against 21.4 us
// for four: more workgroups keep more loads in flight); at 16384 rows four
// rows per workgroup win (63.3 us against 69.1 us for one) by sharing the
// launch and sin/cos set-up.  With the row-group walk's non-temporal loads,
// two rows per workgroup measured 53.0 against 53.6 us for four at 16384
// rows (configs[4], interleaved on one box), so the cap is two.  R *
// rope_dim/2 (sin, cos) pairs must fit the LDS table.
#ifndef FELLM_ROPE_MAX_R
#define FELLM_ROPE_MAX_R 2
#endif
inline int rope_rows_per_block(uint32_t rows, uint32_t rope_dim) {
    const uint32_t half = rope_dim / 2;
    if (FELLM_ROPE_MAX_R >= 4 && rows >= 16384 && half <= kMaxHalf / 4) return 4;
    if (FELLM_ROPE_MAX_R >= 2 && rows >= 8192 && half <= kMaxHalf / 2) return 2;
    return 1;
}

// Workgroups per row group.  With few rows, one workgroup per row leaves most
// CUs idle while each thread walks many (row, head) slots one memory latency
// at a time; the row's heads are then split so that about 1024 workgroups
// run, each keeping at least 8 heads.
inline uint32_t rope_head_split(uint32_t row_groups, uint32_t heads) {
    if (row_groups >= 1024) return 1;
    const uint32_t want = (1024 + row_groups - 1) / row_groups;
    const uint32_t cap = heads / 8 > 0 ? heads / 8 : 1;
    return want < cap ? want : cap;
}

// Standalone KvWrite: one workgroup per batch row, items of VEC elements.
template <typename A, typename C, int VEC>
__global__ __launch_bounds__(kRopeBlock) void kv_write_kernel(const typename A::T *__restrict__ rows,
                                                              const uint32_t *__restrict__ kv_pos,
                                                              KvDev kv, uint32_t is_v,
                                                              uint32_t *__restrict__ err) {
    const uint32_t row = blockIdx.x;
    const uint64_t base = kv_slot_offset(kv, row, kv_pos[row]);
    if (base == ~0ull) {
        if (threadIdx.x == 0 && err) atomicOr(err, 1u);
        return;
    }
    const uint64_t off = base + (is_v ? (uint64_t)kv.block_size * kv.stride * 2 : 0);
    typename C::T *dst = reinterpret_cast<typename C::T *>(kv.arena + off);
    const typename A::T *src = rows + (size_t)row * kv.stride;
    for (uint32_t e = threadIdx.x * VEC; e < kv.stride; e += kRopeBlock * VEC) {
        float v[VEC];
        load_f32<A, VEC>(src + e, v);
        store_f32<C, VEC>(dst + e, v);
    }
}

bool make_kv(const FellmRocmPagedKv *p, KvDev &kv) {
    if (!p || !p->arena || !p->block_table || p->block_size == 0 || p->stride == 0 || p->n_layers == 0 ||
        p->n_logical_blocks == 0 || p->layer >= p->n_layers)
        return false;
    // A block holds block_size K rows then block_size V rows of 2-byte elements.
    if (p->block_bytes < (uint64_t)2 * p->block_size * p->stride * 2 || p->block_bytes % 4) return false;
    kv = KvDev{(uint8_t *)p->arena, p->arena_len, p->block_table, p->n_block_table, p->n_logical_blocks,
               p->n_layers, p->layer, p->block_size, p->block_bytes, p->stride};
    return true;
}

template <typename Fn>
int dispatch_cache(uint32_t kv_dtype, Fn &&f) {
    if (kv_dtype == FELLM_DTYPE_F16) return f.template operator()<F16>();
    if (kv_dtype == FELLM_DTYPE_BF16) return f.template operator()<BF16>();
    return FELLM_ERR_DTYPE;
}

// PV = 4 needs every item boundary on a 4-pair (8-element) grid and
// 8-element-aligned rows; otherwise single pairs.
bool rope_vec_ok(uint32_t head_dim, uint32_t rope_dim, uint32_t pairing, size_t esize,
                 std::initializer_list<const void *> ptrs) {
    if (head_dim % 8 || rope_dim % 8) return false;
    (void)pairing;
    for (const void *p : ptrs)
        if (p && !aligned_to(p, esize * 8)) return false;
    return true;
}

int check_rope_shape(uint32_t head_dim, uint32_t rope_dim, uint32_t pairing) {
    if (head_dim == 0 || head_dim % 2) return FELLM_ERR_SHAPE;
    if (rope_dim % 2 || rope_dim > head_dim || rope_dim / 2 > kMaxHalf) return FELLM_ERR_SHAPE;
    if (pairing > 2) return FELLM_ERR_SHAPE;
    return FELLM_OK;
}

}  // namespace
}  // namespace fellm

extern "C" int fellm_rocm_rope(const void *x1, void *out1, uint32_t n_heads1, const void *x2, void *out2,
                               uint32_t n_heads2, uint32_t act_dtype, uint32_t rows, uint32_t head_dim,
                               uint32_t rope_dim, uint32_t pairing, const float *inv_freqs,
                               const uint32_t *positions, uint32_t position0, void *stream) {
    using namespace fellm;
    if (int rc = check_rope_shape(head_dim, rope_dim, pairing)) return rc;
    if (rows == 0) return FELLM_OK;
    if (!x1 || !out1 || (rope_dim && !inv_freqs) || n_heads1 == 0) return FELLM_ERR_ARITY;
    if (x2 && (!out2 || n_heads2 == 0)) return FELLM_ERR_ARITY;
    hipStream_t s = as_stream(stream);
    return dispatch_act(act_dtype, [&]<typename A>() -> int {
        using T = typename A::T;
        const bool vec = rope_vec_ok(head_dim, rope_dim, pairing, sizeof(T), {x1, out1, x2, out2});
        const int R = rope_rows_per_block(rows, rope_dim);
        auto go = [&]<int PV, int RR>() {
            const uint32_t groups = (rows + RR - 1) / RR;
            const uint32_t hs = rope_head_split(groups, n_heads1 + (x2 ? n_heads2 : 0));
            constexpr int B = RR == 1 ? FELLM_ROPE_BLOCK1 : FELLM_ROPE_BLOCKN;
            FELLM_LAUNCH((rope_kernel<A, F16, PV, 0, RR, B>), dim3(groups * hs), dim3(B), 0, s,
                               (const T *)x1, (T *)out1, n_heads1, (const T *)x2, (T *)out2, x2 ? n_heads2 : 0,
                               nullptr, rows, head_dim, rope_dim, pairing, inv_freqs, positions, position0, nullptr,
                               KvDev{}, nullptr, hs);
            return launch_status();
        };
        auto go_r = [&]<int PV>() {
            if (R == 4) return go.template operator()<PV, 4>();
            if (R == 2) return go.template operator()<PV, 2>();
            return go.template operator()<PV, 1>();
        };
        return vec ? go_r.template operator()<4>() : go_r.template operator()<1>();
    });
}

extern "C" int fellm_rocm_kv_write(const void *rows, uint32_t act_dtype, uint32_t batch,
                                   const uint32_t *kv_positions, const FellmRocmPagedKv *kvp, uint32_t is_v,
                                   uint32_t *err_flag, void *stream) {
    using namespace fellm;
    if (!rows || !kv_positions || !kvp) return FELLM_ERR_ARITY;
    KvDev kv;
    if (!make_kv(kvp, kv)) return FELLM_ERR_SHAPE;
    if (batch == 0) return FELLM_OK;
    hipStream_t s = as_stream(stream);
    return dispatch_act(act_dtype, [&]<typename A>() -> int {
        return dispatch_cache(kvp->kv_dtype, [&]<typename C>() -> int {
            using T = typename A::T;
            const bool vec = kv.stride % 8 == 0 && aligned_to(rows, sizeof(T) * 8) && aligned_to(kvp->arena, 16) &&
                             kv.block_bytes % 16 == 0;
            if (vec)
                FELLM_LAUNCH((kv_write_kernel<A, C, 8>), dim3(batch), dim3(kRopeBlock), 0, s, (const T *)rows,
                                   kv_positions, kv, is_v, err_flag);
            else
                FELLM_LAUNCH((kv_write_kernel<A, C, 1>), dim3(batch), dim3(kRopeBlock), 0, s, (const T *)rows,
                                   kv_positions, kv, is_v, err_flag);
            return launch_status();
        });
    });
}

namespace fellm {
namespace {

// The reference's controlled single-row KV addressing (oxide_kernels.rs:
// 4203-4214): logical block (sequence_length - 1) / block_size (saturating),
// slot kv_write_slot.  Expressed as the position logical * block_size + slot
// that the KV kernels take; a slot outside the block gives 0xffffffff, which
// the KV kernels reject (error flag) instead of writing past the block.
__global__ void step_kv_position_kernel(const FellmDeviceStepParams *__restrict__ p, uint32_t block_size,
                                        uint32_t *__restrict__ kv_pos) {
    if (threadIdx.x != 0) return;
    const uint32_t seq = p->sequence_length, slot = p->kv_write_slot;
    const uint32_t logical = (seq ? seq - 1 : 0) / block_size;
    kv_pos[0] = slot < block_size ? logical * block_size + slot : 0xffffffffu;
}

}  // namespace
}  // namespace fellm

extern "C" int fellm_rocm_step_kv_position(const FellmDeviceStepParams *params, uint32_t block_size,
                                           uint32_t *kv_pos, void *stream) {
    using namespace fellm;
    if (!params || !kv_pos) return FELLM_ERR_ARITY;
    if (block_size == 0) return FELLM_ERR_SHAPE;
    FELLM_LAUNCH(step_kv_position_kernel, dim3(1), dim3(kWave), 0, as_stream(stream), params, block_size,
                       kv_pos);
    return launch_status();
}

extern "C" int fellm_rocm_rope_kv_write(const void *q, void *q_out, uint32_t n_q_heads, const void *k,
                                        void *k_out, const void *v, uint32_t n_kv_heads, uint32_t act_dtype,
                                        uint32_t batch, uint32_t head_dim, uint32_t rope_dim, uint32_t pairing,
                                        const float *inv_freqs, const uint32_t *rope_positions,
                                        const uint32_t *kv_positions, const FellmRocmPagedKv *kvp,
                                        uint32_t *err_flag, void *stream) {
    using namespace fellm;
    if (!q || !q_out || !k || !v || !kv_positions || !kvp || (rope_dim && !inv_freqs)) return FELLM_ERR_ARITY;
    if (n_q_heads == 0 || n_kv_heads == 0) return FELLM_ERR_SHAPE;
    if (int rc = check_rope_shape(head_dim, rope_dim, pairing)) return rc;
    KvDev kv;
    if (!make_kv(kvp, kv)) return FELLM_ERR_SHAPE;
    if (kv.stride != n_kv_heads * head_dim) return FELLM_ERR_SHAPE;
    if (batch == 0) return FELLM_OK;
    hipStream_t s = as_stream(stream);
    return dispatch_act(act_dtype, [&]<typename A>() -> int {
        return dispatch_cache(kvp->kv_dtype, [&]<typename C>() -> int {
            using T = typename A::T;
            const bool vec = rope_vec_ok(head_dim, rope_dim, pairing, sizeof(T), {q, q_out, k, k_out, v}) &&
                             aligned_to(kvp->arena, 16) && kv.block_bytes % 16 == 0;
            auto go = [&]<int PV>() {
                const uint32_t hs = FELLM_KV_HSPLIT ? FELLM_KV_HSPLIT : rope_head_split(batch, n_q_heads + 2 * n_kv_heads);
                FELLM_LAUNCH((rope_kernel<A, C, PV, 1, 1>), dim3(batch * hs), dim3(kRopeBlock), 0, s,
                                   (const T *)q, (T *)q_out, n_q_heads, (const T *)k, (T *)k_out, n_kv_heads,
                                   (const T *)v, batch, head_dim, rope_dim, pairing, inv_freqs, rope_positions, 0u,
                                   kv_positions, kv, err_flag, hs);
                return launch_status();
            };
            return vec ? go.template operator()<4>() : go.template operator()<1>();
        });
    });
}

// ---------------------------------------------------------------------------
// One decode step's three memory-bound ops in one launch.  At decode batch
// sizes each op moves 10-44 MB, a few microseconds of traffic, and as
// separate kernels each pays its own fill and drain.  Here the grid is the
// concatenation of the three launches' grids, workgroup ranges in order
// (FELLM_STEP_ORDER 1):
//   [0, rows)                   residual add + RMSNorm, one row each,
//   [rows, + nb_rope)           RoPE(q), RoPE(k) + paged K/V append,
//   [.., + nb_silu)             SwiGLU,
// each range running the same device code as its standalone kernel
// (rope_block, add_rmsnorm_row, silu_gate_blocks), so the results are the
// standalone launches' bit for bit, except y, whose sum of squares is
// reduced over 256 threads here (the few-row standalone launch uses 1024).  The ops are independent (disjoint
// outputs), as in the reference's decode graph before attention
// (crates/fellm-model/src/graph.rs:2136-2246).
// ---------------------------------------------------------------------------
// Minimum waves per SIMD requested for the fused decode step when a norm
// row takes at most 4 chunks per thread: the norm role's registers would
// otherwise set the occupancy of all three roles (82 VGPRs, 5 waves; 6 waves
// fit without spilling and measured 17.6 vs 18.5 us at 256 x H 8192 bf16).
// 8 chunks (rows above 8192 elements) keep the compiler's choice: limiting
// them spills.
#ifndef FELLM_STEP_WAVES
#define FELLM_STEP_WAVES 6
#endif
// Build knob: rows per RoPE workgroup in the one-launch decode step.
#ifndef FELLM_STEP_ROWS
#define FELLM_STEP_ROWS 1
#endif
// Build knob: workgroups per RoPE row in the one-launch decode step (0: the
// rule in fellm_rocm_decode_step).  Measured at configs[3] (256 rows, 80
// q/k/v heads), interleaved on one box: 1 per row 13.6-13.8 us, 2 14.6,
// 4 (the standalone launch's split) 15.6, 8 18.0-18.1; two or four rows per
// workgroup (one per row group) 17.1 and 24.7.
#ifndef FELLM_STEP_HSPLIT
#define FELLM_STEP_HSPLIT 0
#endif
// Build knob: role order along the grid (see decode_step_kernel).  With one
// RoPE workgroup per row: norm first 13.52 us, RoPE first 13.6-13.64.
#ifndef FELLM_STEP_ORDER
#define FELLM_STEP_ORDER 1
#endif

namespace fellm {
namespace {

template <typename A>
struct StepArgs {
    using T = typename A::T;
    // RoPE + K/V append
    const T *q;
    T *q_out;
    const T *k;
    T *k_out;
    const T *v;
    uint32_t nq, nkv, batch, head_dim, rope_dim, pairing, hsplit;
    const float *inv_freqs;
    const uint32_t *rope_pos, *kv_pos;
    KvDev kv;
    uint32_t *err;
    // add + RMSNorm
    const T *x, *r;
    T *h, *y;
    const float *w;
    uint32_t group;
    float eps;
    // SwiGLU
    const T *gate, *up;
    T *act;
    uint64_t n_silu;
    // workgroup ranges
    uint32_t nb_rope, nb_norm, nb_silu;
};

template <typename A, typename C, int NCHUNK>
__global__ __launch_bounds__(kRopeBlock)
__attribute__((amdgpu_waves_per_eu(NCHUNK <= 4 && FELLM_STEP_WAVES ? FELLM_STEP_WAVES : 1)))
void decode_step_kernel(StepArgs<A> p) {
    static_assert(kRopeBlock == 256 && kEwBlock == 256, "the three roles share one workgroup size");
    constexpr int SR = FELLM_STEP_ROWS;
    __shared__ float2 cs_all[SR][kMaxHalf / SR];
    __shared__ uint64_t kbase_all[SR];
    __shared__ float red[256 / kWave];
    __shared__ uint64_t tab_lds[32];
    // Role order along the grid (build knob FELLM_STEP_ORDER): 0 RoPE, norm,
    // SwiGLU; 1 norm, RoPE, SwiGLU; 2 SwiGLU, RoPE, norm.
    constexpr int kOrder[3][3] = {{0, 1, 2}, {1, 0, 2}, {2, 0, 1}};
    const uint32_t nb[3] = {p.nb_rope, p.nb_norm, p.nb_silu};
    uint32_t b = blockIdx.x;
    int role = kOrder[FELLM_STEP_ORDER][2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int r = kOrder[FELLM_STEP_ORDER][i];
        if (b < nb[r]) {
            role = r;
            break;
        }
        b -= nb[r];
    }
    if (role == 0) {
        rope_block<A, C, 4, 1, SR>(p.q, p.q_out, p.nq, p.k, p.k_out, p.nkv, p.v, p.batch, p.head_dim, p.rope_dim,
                                  p.pairing, p.inv_freqs, p.rope_pos, 0u, p.kv_pos, p.kv, p.err, p.hsplit, b, cs_all,
                                  kbase_all);
    } else if (role == 1) {
        add_rmsnorm_row<A, A, 256, 8, NCHUNK, true, true>(p.x, p.r, p.h, p.w, p.y, p.group, p.eps, b, red);
    } else {
        silu_gate_blocks<A, typename HwStore<A>::type, 8, 2>(p.gate, p.up, p.act, p.n_silu, b, p.nb_silu, tab_lds);
    }
}

}  // namespace
}  // namespace fellm

extern "C" int fellm_rocm_decode_step(const FellmRocmDecodeStep *d, void *stream) {
    using namespace fellm;
    if (!d) return FELLM_ERR_ARITY;
    const uint32_t dt = d->act_dtype;
    const size_t es = act_bytes(dt);
    if (!es) return FELLM_ERR_DTYPE;
    // The fused layout: 16-byte vectors everywhere, a residual and an h
    // output, rows of 2049..16384 elements (256 threads, 2-8 chunks of 8), a
    // SwiGLU length that is a whole number of 8-element vectors.
    const bool norm_fits = d->residual && d->h_out && d->group && d->group % 8 == 0 && d->group > 2048 &&
                           d->group <= 16384 && d->norm_elems % d->group == 0 && d->norm_elems / d->group <= 0x7fffffffull;
    bool fuse = norm_fits && d->swiglu_elems % 8 == 0 && d->batch > 0 && d->kv &&
                d->rope_dim / 2 <= kMaxHalf / FELLM_STEP_ROWS &&
                rope_vec_ok(d->head_dim, d->rope_dim, d->pairing, es, {d->q, d->q_out, d->k, d->k_out, d->v}) &&
                aligned_to(d->kv->arena, 16) && d->kv->block_bytes % 16 == 0;
    for (const void *p : {d->x, d->residual, (const void *)d->h_out, (const void *)d->y, d->gate, d->up,
                          (const void *)d->act_out})
        fuse = fuse && p && aligned_to(p, 16);
    fuse = fuse && aligned_to(d->norm_weight, 32);
    KvDev kv{};
    if (fuse) {
        if (!d->q || !d->q_out || !d->k || !d->v || !d->kv_positions || (d->rope_dim && !d->inv_freqs))
            return FELLM_ERR_ARITY;
        if (d->n_q_heads == 0 || d->n_kv_heads == 0) return FELLM_ERR_SHAPE;
        if (int rc = check_rope_shape(d->head_dim, d->rope_dim, d->pairing)) return rc;
        if (!make_kv(d->kv, kv) || kv.stride != d->n_kv_heads * d->head_dim) return FELLM_ERR_SHAPE;
        if (!d->norm_weight || !d->y) return FELLM_ERR_ARITY;
        if (d->swiglu_elems && (!d->gate || !d->up || !d->act_out)) return FELLM_ERR_ARITY;
        if (d->kv->kv_dtype != FELLM_DTYPE_F16 && d->kv->kv_dtype != FELLM_DTYPE_BF16) return FELLM_ERR_DTYPE;
    }
    hipStream_t s = as_stream(stream);
    if (!fuse) {  // the same three ops, launched separately
        if (d->batch) {
            if (int rc = fellm_rocm_rope_kv_write(d->q, d->q_out, d->n_q_heads, d->k, d->k_out, d->v, d->n_kv_heads, dt,
                                                  d->batch, d->head_dim, d->rope_dim, d->pairing, d->inv_freqs,
                                                  d->rope_positions, d->kv_positions, d->kv, d->err_flag, stream))
                return rc;
        }
        if (d->norm_elems) {
            if (int rc = fellm_rocm_add_rmsnorm(d->x, d->residual, d->h_out, dt, d->norm_weight, d->group, d->y, dt,
                                                d->norm_elems, d->eps, stream))
                return rc;
        }
        if (d->swiglu_elems) return fellm_rocm_silu_gate(d->gate, d->up, dt, d->act_out, dt, d->swiglu_elems, stream);
        return FELLM_OK;
    }
    const uint32_t nchunk = (d->group / 8 + 255) / 256;  // 2..8
    return dispatch_act(dt, [&]<typename A>() -> int {
        return dispatch_cache(d->kv->kv_dtype, [&]<typename C>() -> int {
            using T = typename A::T;
            StepArgs<A> p{};
            p.q = (const T *)d->q;
            p.q_out = (T *)d->q_out;
            p.k = (const T *)d->k;
            p.k_out = (T *)d->k_out;
            p.v = (const T *)d->v;
            p.nq = d->n_q_heads;
            p.nkv = d->n_kv_heads;
            p.batch = d->batch;
            p.head_dim = d->head_dim;
            p.rope_dim = d->rope_dim;
            p.pairing = d->pairing;
            // RoPE workgroups wait mostly on latency (sin/cos table, slot
            // lookups); split a row's heads only until the RoPE range covers
            // the CUs once, so that it does not hold the slots the streaming
            // roles need.
            const uint32_t cover = (cu_count() + d->batch - 1) / d->batch;
            const uint32_t auto_split = rope_head_split(d->batch, d->n_q_heads + 2 * d->n_kv_heads);
            p.hsplit = FELLM_STEP_HSPLIT ? FELLM_STEP_HSPLIT : std::max(1u, std::min(auto_split, cover));
            p.inv_freqs = d->inv_freqs;
            p.rope_pos = d->rope_positions;
            p.kv_pos = d->kv_positions;
            p.kv = kv;
            p.err = d->err_flag;
            p.x = (const T *)d->x;
            p.r = (const T *)d->residual;
            p.h = (T *)d->h_out;
            p.y = (T *)d->y;
            p.w = d->norm_weight;
            p.group = d->group;
            p.eps = d->eps;
            p.gate = (const T *)d->gate;
            p.up = (const T *)d->up;
            p.act = (T *)d->act_out;
            p.n_silu = d->swiglu_elems;
            p.nb_rope = (d->batch + FELLM_STEP_ROWS - 1) / FELLM_STEP_ROWS * p.hsplit;
            p.nb_norm = (uint32_t)(d->norm_elems / d->group);
            const uint64_t units = d->swiglu_elems / 8;
            p.nb_silu = (uint32_t)((units + kEwBlock * 2 - 1) / (kEwBlock * 2));
            const uint64_t grid = (uint64_t)p.nb_rope + p.nb_norm + p.nb_silu;
            if (grid > 0x7fffffffull) return FELLM_ERR_SHAPE;
            auto go = [&]<int NC>() -> int {
                FELLM_LAUNCH((decode_step_kernel<A, C, NC>), dim3((uint32_t)grid), dim3(kRopeBlock), 0, s, p);
                return launch_status();
            };
            if (nchunk <= 2) return go.template operator()<2>();
            if (nchunk <= 4) return go.template operator()<4>();
            return go.template operator()<8>();
        });
    });
}
