// MoE router: gate scores + top-k selection + renormalisation.
//
// Reference: crates/backend-cpu/src/kernels/moe.rs
//   gate_scores :79-111 (softmax: m = max(l); e_j = exp(l_j - m);
//       denom += e_j in expert order; s_j = e_j / denom if denom > 0;
//       sigmoid for gating 2: s_j = 1 / (1 + exp(-l_j));
//       sqrt-softplus for gating 4 (:68-77): s_j = sqrt(max(softplus(l_j), 0)))
//   select_routed_experts :142-186 (rank by s descending under f32
//       total_cmp, ties -> lower expert id)
//   finish_selected :113-140 (truncate to k; if norm_topk_prob divide by the
//       sum of the selected scores taken in rank order; times
//       routed_scaling_factor, 0 meaning 1)
//   batched variant :820-855 (same ranking and arithmetic).
//
// A group of G lanes per token (n_experts <= 512, EPL experts per lane).  exp
// is the glibc-exact restatement and the denominator is folded serially in
// expert order lane to lane, so scores, ranking and weights are bit-exact with
// the CPU.  Ranking, for non-negative scores and k <= G: unique 64-bit keys
// (score bits << 32 | ~expert, whose order is the CPU comparator's: score
// descending, ties to the lower expert id) held as doubles, ordered by f64
// max/min sorting networks within a lane and merged across the group's lanes.
// Softmax ranks the exps before the denominator is known and re-sorts the
// winners' quotients.  Otherwise 64-bit keys (total-order(score) << 32 |
// ~expert) and k group max-reductions pick the winners in rank order.
#include "common.hpp"

namespace fellm {
namespace {

// Build knob: experts per lane (8, 16 or 32).
#ifndef FELLM_ROUTER_EPL
#define FELLM_ROUTER_EPL 16
#endif

// Build knob: the sorting-network ranking on unique 64-bit keys where it
// applies (1), or the k-round selection for every wavefront (0).
#ifndef FELLM_ROUTER_FAST
#define FELLM_ROUTER_FAST 1
#endif

// Build knob: softmax with n_experts == G * EPL takes the branch-free
// specialised score kernel (1) or the general one (0).
#ifndef FELLM_ROUTER_LEAN
#define FELLM_ROUTER_LEAN 1
#endif

// Build knob: threads per workgroup.
#ifndef FELLM_ROUTER_BLOCK
#define FELLM_ROUTER_BLOCK 256
#endif

constexpr int kRouterBlock = FELLM_ROUTER_BLOCK;
constexpr int kRouterWaves = kRouterBlock / kWave;
constexpr uint32_t kMaxExperts = 512;
constexpr uint32_t kMaxTopK = kMaxExperts;

// Monotone map of f32 total order (f32::total_cmp) onto u32.
__device__ __forceinline__ uint32_t total_order_key(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float total_order_inv(uint32_t o) {
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}

// Descending sorting network on 8 keys (19 comparators, Batcher's
// odd-even merge sort) and the merge of two descending 8-lists into the
// descending top 8 of their union: c[i] = max(a[i], b[7 - i]) is bitonic and
// holds the top 8 (a half-cleaner), then a bitonic sorter orders it.  Keys
// are unique, so max/min exchanges need no tie rule.
// 64-bit keys travel as doubles whose bit patterns are the keys: with the
// high word at least 2^20 and below 0x7FF00000 they are positive normal
// finite doubles, which order exactly as their bit patterns, so one f64
// max / min does a 64-bit exchange.
template <typename K>
__device__ __forceinline__ K kmax(K a, K b) {
    if constexpr (sizeof(K) == 8) return __builtin_fmax(a, b);
    else return a > b ? a : b;
}
template <typename K>
__device__ __forceinline__ K kmin(K a, K b) {
    if constexpr (sizeof(K) == 8) return __builtin_fmin(a, b);
    else return a > b ? b : a;
}
template <typename K>
__device__ __forceinline__ void ce_desc(K &a, K &b) {
    const K hi = kmax(a, b), lo = kmin(a, b);
    a = hi;
    b = lo;
}
template <typename K>
__device__ __forceinline__ void sort8_desc(K (&a)[8]) {
    constexpr int kNet[19][2] = {{0, 2}, {1, 3}, {4, 6}, {5, 7}, {0, 4}, {1, 5}, {2, 6}, {3, 7}, {0, 1}, {2, 3},
                                 {4, 5}, {6, 7}, {2, 4}, {3, 5}, {1, 4}, {3, 6}, {1, 2}, {3, 4}, {5, 6}};
#pragma unroll
    for (int c = 0; c < 19; ++c) ce_desc(a[kNet[c][0]], a[kNet[c][1]]);
}
template <typename K>
__device__ __forceinline__ void bitonic8_desc(K (&a)[8]) {
#pragma unroll
    for (int d = 4; d >= 1; d >>= 1)
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if ((i & d) == 0) ce_desc(a[i], a[i + d]);
}
template <typename K>
__device__ __forceinline__ void merge_top8(const K (&a)[8], const K (&b)[8], K (&out)[8]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = kmax(a[i], b[7 - i]);
    bitonic8_desc(out);
}
// Merge with the partner lane that the DPP control CTRL names.
template <int CTRL, typename K>
__device__ __forceinline__ void merge_lanes(K (&l)[8]) {
    K p[8], o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        if constexpr (sizeof(K) == 8) p[i] = __longlong_as_double((long long)dpp_u64<CTRL>((uint64_t)__double_as_longlong(l[i])));
        else p[i] = dpp_u32<CTRL>(l[i]);
    }
    merge_top8(l, p, o);
#pragma unroll
    for (int i = 0; i < 8; ++i) l[i] = o[i];
}

constexpr uint32_t ilog2_u32(uint32_t v) { return v <= 1 ? 0 : 1 + ilog2_u32(v / 2); }

// Layouts the sorting-network ranking serves.
template <int EPL, int G>
constexpr bool kFastRank = (EPL == 8 || EPL == 16) && G >= 2 && G <= 16 && G * EPL <= 256 && FELLM_ROUTER_FAST;

// The descending top 8 of a token's unique keys (EPL per lane, G lanes),
// in every lane of the group, and `below`: the largest key under rank k - 1.
template <int EPL, int G, typename K>
__device__ __forceinline__ void rank_top8(const K (&a)[EPL], uint32_t k, K (&L)[8], K &below) {
    if constexpr (EPL == 8) {
#pragma unroll
        for (int j = 0; j < 8; ++j) L[j] = a[j];
        sort8_desc(L);
    } else {
        K A[8], B[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            A[j] = a[j];
            B[j] = a[8 + j];
        }
        sort8_desc(A);
        sort8_desc(B);
        merge_top8(A, B, L);
    }
    merge_lanes<0xB1>(L);                          // xor 1
    if constexpr (G >= 4) merge_lanes<0x4E>(L);    // xor 2
    if constexpr (G >= 8) merge_lanes<0x141>(L);   // mirror within 8
    if constexpr (G >= 16) merge_lanes<0x140>(L);  // mirror within 16
    K last = 0;  // rank k - 1
#pragma unroll
    for (int i = 0; i < 8; ++i)
        if ((uint32_t)i + 1 == k) last = L[i];
    below = 0;
#pragma unroll
    for (int j = 0; j < EPL; ++j) below = a[j] < last && a[j] > below ? a[j] : below;
    if constexpr (sizeof(K) == 8)
        below = __longlong_as_double((long long)group_max_u64<G>((uint64_t)__double_as_longlong(below)));
    else below = dpp_max_group<G>(below);
}

// Keys (hi, lo) as doubles for the networks: see kmax.
constexpr uint32_t kHiBias = 0x00100000u;
__device__ __forceinline__ double dkey(uint32_t hi, uint32_t lo) {
    return __longlong_as_double((long long)(((uint64_t)(hi + kHiBias) << 32) | lo));
}
__device__ __forceinline__ uint32_t dkey_hi(double v) {
    return (uint32_t)((uint64_t)__double_as_longlong(v) >> 32) - kHiBias;
}
__device__ __forceinline__ uint32_t dkey_lo(double v) { return (uint32_t)(uint64_t)__double_as_longlong(v); }

// The k-of-n_exp selection of one token held by its G lanes (scores s of
// experts e0 .. e0 + EPL - 1 in this lane), the renormalisation and the
// stores.
template <int EPL, int G, bool TRY_FAST = true>
__device__ __forceinline__ void select_and_store(const float (&s)[EPL], uint32_t lane, uint32_t sub, uint32_t token,
                                                 bool active, uint32_t n_exp, uint32_t k, uint32_t norm, float rsf,
                                                 uint32_t *__restrict__ ids, float *__restrict__ weights) {
    const uint32_t e0 = sub * EPL;
    const float scale = rsf == 0.0f ? 1.0f : rsf;
    if constexpr (TRY_FAST && kFastRank<EPL, G>) {
        // k <= G and every score non-negative and not NaN (softmax, sigmoid,
        // sqrt-softplus): exact unique keys (score bits, ~expert), whose order
        // is the reference's (score desc, expert asc), through the networks;
        // the group's top 8 in every lane.  Otherwise (a NaN, -0.0) the
        // wavefront takes the k-round selection below.
        if (k <= (uint32_t)G && n_exp <= (uint32_t)(G * EPL)) {
            double a[EPL];
            bool bad = false;
#pragma unroll
            for (int j = 0; j < EPL; ++j) {
                const uint32_t e = e0 + j, b = __float_as_uint(s[j]);
                const bool real = active && e < n_exp;
                bad |= real && b > 0x7F800000u;
                a[j] = real && b <= 0x7F800000u ? dkey(b, 0xFFFFFFFFu - e) : 0.0;
            }
            double L[8], below;
            rank_top8<EPL, G, double>(a, k, L, below);
            if (__ballot(active && bad) == 0) {
                // Rank r goes to lane r of the group; every lane sums the k
                // selected raw scores in rank order, as finish_selected does.
                float sum = 0.0f, mine = 0.0f;
                uint32_t my_e = 0;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    if ((uint32_t)i < k) {
                        const float v = __uint_as_float(dkey_hi(L[i]));
                        sum += v;
                        if ((uint32_t)i == sub) {
                            mine = v;
                            my_e = 0xFFFFFFFFu - dkey_lo(L[i]);
                        }
                    }
                }
                if (active && sub < k) {
                    float v = mine;
                    if (norm && sum > 0.0f) v = v / sum;
                    ids[(size_t)token * k + sub] = my_e;
                    weights[(size_t)token * k + sub] = v * scale;
                }
                return;
            }
        }
    }
    // k rounds: each lane scans its own candidates for the best (score desc,
    // expert asc) key, the group takes the 64-bit max, the owner marks it
    // taken.  Rank r's expert and raw score go straight to ids/weights and the
    // rank-order sum is folded on the way; a final pass rescales.
    uint64_t key[EPL];  // (total-order score << 32) | ~expert; 0 = not a candidate
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        const uint32_t e = e0 + j;
        key[j] = (active && e < n_exp) ? ((uint64_t)total_order_key(s[j]) << 32) | (uint64_t)(0xffffffffu - e) : 0ull;
    }
    // Rank r's expert and raw score stay in registers of lane r % G (ranks
    // past kHeld * G go to memory and are rescaled from there), so the final
    // rescale needs no read-back of what was just written.
    constexpr uint32_t kHeld = 4;
    uint32_t held_e[kHeld];
    float held_w[kHeld];
    float sum = 0.0f;
    for (uint32_t r = 0; r < k; ++r) {
        uint64_t best = key[0];
#pragma unroll
        for (int j = 1; j < EPL; ++j) best = key[j] > best ? key[j] : best;
        if constexpr (G <= 16) {
            best = group_max_u64<G>(best);
        } else {
#pragma unroll
            for (int off = G / 2; off > 0; off >>= 1) {
                const uint64_t o = __shfl_xor(best, off, kWave);
                best = o > best ? o : best;
            }
        }
        const uint32_t e = 0xffffffffu - (uint32_t)best;
        if (e / EPL == sub) {
#pragma unroll
            for (int j = 0; j < EPL; ++j)
                if ((uint32_t)j == e % EPL) key[j] = 0;
        }
        const float raw = total_order_inv((uint32_t)(best >> 32));
        sum += raw;  // rank order, as finish_selected sums
        if (r < kHeld * G) {
#pragma unroll
            for (uint32_t i = 0; i < kHeld; ++i)
                if (r == i * G + sub) {
                    held_e[i] = e;
                    held_w[i] = raw;
                }
        } else if (active && sub == 0) {
            ids[(size_t)token * k + r] = e;
            weights[(size_t)token * k + r] = raw;
        }
    }
    if (active) {
#pragma unroll
        for (uint32_t i = 0; i < kHeld; ++i) {
            const uint32_t r = i * G + sub;
            if (r < k) {
                float v = held_w[i];
                if (norm && sum > 0.0f) v = v / sum;
                ids[(size_t)token * k + r] = held_e[i];
                weights[(size_t)token * k + r] = v * scale;
            }
        }
    }
    // Ranks beyond the held ones: the lane that wrote them rescales them
    // (same thread, program order).
    if (active && sub == 0) {
        for (uint32_t r = kHeld * G; r < k; ++r) {
            float v = weights[(size_t)token * k + r];
            if (norm && sum > 0.0f) v = v / sum;
            weights[(size_t)token * k + r] = v * scale;
        }
    }
}

// e / d for the EPL scores of a lane: one IEEE reciprocal per token,
// y = RN(1/d), q0 = RN(e*y), r = e - d*q0 (exact), q = RN(q0 + r*y), which
// Markstein's theorem makes the correctly rounded e / d when no step
// underflows (e in [2^-100, 1], d below 2^100); tiny or non-finite operands
// take the IEEE division.  (Checked against IEEE division for 4096 values of
// d in [1, 512) and every e in [2^-100, 1].)
template <int EPL>
__device__ __forceinline__ void divide_by(float (&s)[EPL], float d) {
    const float y = 1.0f / d;
    const bool d_ok = d < 0x1p+100f;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        const float e = s[j];
        if (d_ok && e >= 0x1p-100f && e <= 1.0f) {
            const float q0 = e * y;
            const float r = __builtin_fmaf(-d, q0, e);
            s[j] = __builtin_fmaf(r, y, q0);
        } else {
            s[j] = e / d;
        }
    }
}

// General path: G = 64 / TPW lanes per token, each lane owning EPL
// consecutive experts (expert e lives in lane e / EPL of its group, slot
// e % EPL), so expert order is (lane, slot) order.
//  * max: per-lane max, then a reduction inside the group;
//  * denominator: the f32 fold in expert order runs lane to lane through the
//    group (lane q adds its EPL values to the running sum, then hands it to
//    lane q+1), i.e. exactly the CPU's left-to-right accumulation.
template <int EPL, int G>
__global__ __launch_bounds__(kRouterBlock) void router_topk_grouped(
    const float *__restrict__ logits, uint32_t tokens, uint32_t n_exp, uint32_t k, uint32_t gating,
    uint32_t norm, float rsf, uint32_t *__restrict__ ids, float *__restrict__ weights) {
    __shared__ uint64_t tab_lds[32];
    const uint64_t *tab = stage_expf_table(tab_lds);
    constexpr int TPW = kWave / G;  // tokens per wavefront
    const uint32_t lane = threadIdx.x % kWave, sub = lane % G;
    const uint32_t token = (blockIdx.x * kRouterWaves + threadIdx.x / kWave) * TPW + lane / G;
    const bool active = token < tokens;
    const float *lg = logits + (size_t)(active ? token : 0) * n_exp;
    const uint32_t e0 = sub * EPL;

    float s[EPL];
    if (EPL % 4 == 0 && n_exp % EPL == 0 && (reinterpret_cast<uintptr_t>(lg) & 15) == 0) {
        if (active && e0 < n_exp) {
#pragma unroll
            for (int j = 0; j < EPL; j += 4) {
                const float4 v = *reinterpret_cast<const float4 *>(lg + e0 + j);
                s[j] = v.x;
                s[j + 1] = v.y;
                s[j + 2] = v.z;
                s[j + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int j = 0; j < EPL; ++j) s[j] = -__builtin_inff();
        }
    } else {
#pragma unroll
        for (int j = 0; j < EPL; ++j) s[j] = (active && e0 + j < n_exp) ? lg[e0 + j] : -__builtin_inff();
    }
    if (gating == 2) {
#pragma unroll
        for (int j = 0; j < EPL; ++j) s[j] = 1.0f / (1.0f + expf_glibc(-s[j], tab));
    } else if (gating == 4) {
        // sqrt_softplus (moe.rs:68-77): softplus = v (v > 20), exp(v) (v < -20),
        // else ln(1 + exp(v)), all f32; then sqrt(max(softplus, 0)).
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            const float v = s[j];
            const float sp = v > 20.0f ? v : (v < -20.0f ? expf_glibc(v, tab) : logf_glibc(1.0f + expf_glibc(v, tab)));
            s[j] = sqrtf_rn(fmaxf(sp, 0.0f));
        }
    } else {
        float m = s[0];
#pragma unroll
        for (int j = 1; j < EPL; ++j) m = fmaxf(m, s[j]);
        if constexpr (G <= 16) {
            m = group_max_f32<G>(m);
        } else {
#pragma unroll
            for (int off = G / 2; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, kWave));
        }
#pragma unroll
        for (int j = 0; j < EPL; ++j) s[j] = expf_glibc(s[j] - m, tab);
        float d = 0.0f;
        for (uint32_t q = 0; q < (uint32_t)G; ++q) {
            if (sub == q) {
#pragma unroll
                for (int j = 0; j < EPL; ++j)
                    if (e0 + j < n_exp) d += s[j];
            }
            // lane q hands the running sum to lane q+1
            const float up = (G <= 16) ? dpp_f32<0x111>(d) : __shfl_up(d, 1, G);
            if (sub == q + 1) d = up;
        }
        d = __shfl(d, G - 1, G);  // the last lane of the group holds the full fold
        if (d > 0.0f) divide_by(s, d);
    }
    select_and_store<EPL, G>(s, lane, sub, token, active, n_exp, k, norm, rsf, ids, weights);
}

// Softmax with n_experts == G * EPL (every lane full), logits rows 16-byte
// aligned: the same arithmetic as the general path with nothing it does not
// need.  No per-expert bounds (the row is whole); exp branch-free
// (expf_glibc_nonpos: l - max <= 0 or NaN); the fold unrolled, each lane
// adding its EPL values when its turn comes (a select, no branch); the
// division's operand range checked once per wavefront.
template <int EPL, int G>
__global__ __launch_bounds__(kRouterBlock) void router_softmax_lean(
    const float *__restrict__ logits, uint32_t tokens, uint32_t k, uint32_t norm, float rsf,
    uint32_t *__restrict__ ids, float *__restrict__ weights) {
    __shared__ uint64_t tab_lds[32];
    constexpr uint32_t E = G * EPL;
    constexpr int TPW = kWave / G;
    const uint32_t lane = threadIdx.x % kWave, sub = lane % G;
    const uint32_t token = (blockIdx.x * kRouterWaves + threadIdx.x / kWave) * TPW + lane / G;
    const bool active = token < tokens;
    const float4 *lg = reinterpret_cast<const float4 *>(logits + (size_t)(active ? token : 0) * E + sub * EPL);
    float s[EPL];
#pragma unroll
    for (int j = 0; j < EPL; j += 4) {
        const float4 v = lg[j / 4];
        s[j] = v.x;
        s[j + 1] = v.y;
        s[j + 2] = v.z;
        s[j + 3] = v.w;
    }
    const uint64_t *tab = stage_expf_table(tab_lds);  // while the loads are in flight
    float m = s[0];
#pragma unroll
    for (int j = 1; j < EPL; ++j) m = fmaxf(m, s[j]);
    m = group_max_f32<G>(m);
    bool e_ok = true;  // every e >= 2^-100 (false for NaN)
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        s[j] = expf_glibc_nonpos(s[j] - m, tab);
        e_ok &= s[j] >= 0x1p-100f;
    }
    // Ranking on the exps, before and independent of the denominator, so
    // that its networks fill the gaps of the fold's dependent chain: keys
    // (e's bits << 32 | ~expert) are exact and unique, and e >= 0 orders like
    // its bits.  s = RN(e / d) is monotone in e, so the reference's order
    // (score desc, expert asc) is this order except where quotients of
    // different e tie: the k winners' scores are sorted again on
    // (score, ~expert), and a tie between rank k - 1 and the next key (which
    // could let an expert outside the k in) sends the wavefront to the
    // k-round selection on the full scores, as do NaN scores and k > G.
    double L[8], below = 0.0;
    bool bad = false;
    if constexpr (kFastRank<EPL, G>) {
        double a[EPL];
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            const uint32_t b = __float_as_uint(s[j]);
            bad |= b > 0x3F800000u;
            a[j] = dkey(bad ? 0u : b, 0xFFFFFFFFu - (sub * EPL + j));
        }
        rank_top8<EPL, G, double>(a, k, L, below);
    }
    float d = 0.0f;
#pragma unroll
    for (int q = 0; q < G; ++q) {
        float t = d;
#pragma unroll
        for (int j = 0; j < EPL; ++j) t += s[j];
        d = sub == (uint32_t)q ? t : d;
        // lane q hands the running sum to lane q + 1
        if (q + 1 < G) {
            const float up = dpp_f32<0x111>(d);
            d = sub == (uint32_t)q + 1 ? up : d;
        }
    }
    d = __shfl(d, G - 1, G);  // the last lane of the group holds the full fold
    // The quotient sequence (one IEEE reciprocal per token, Markstein's
    // correction) holds for e in [2^-100, 1] and d below 2^100; every e is at
    // most 1 (exp of a non-positive argument).
    const bool quot_ok = d > 0.0f && d < 0x1p+100f;
    if constexpr (kFastRank<EPL, G>) {
        const float y = 1.0f / d;
        auto quot = [&](float e) {
            const float q0 = e * y;
            return __builtin_fmaf(__builtin_fmaf(-d, q0, e), y, q0);
        };
        double sk[8];  // keys (score bits, ~expert) of ranks 0..k-1, 0 past k
        float e_last = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {  // branch-free: every rank's quotient, then selects
            const float e = __uint_as_float(dkey_hi(L[i]));
            const double key = dkey(__float_as_uint(quot(e)), dkey_lo(L[i]));
            e_last = (uint32_t)i + 1 == k ? e : e_last;
            sk[i] = (uint32_t)i < k ? key : 0.0;
        }
        const float e_next = below == 0.0 ? 0.0f : __uint_as_float(dkey_hi(below));
        // Every winner's e at least 2^-100 (the last one decides), so the
        // quotient sequence holds for all of them.  Below 2^-100 the next
        // key's quotient is not formed: rank k - 1 at least 2^-99 puts every
        // later quotient strictly under it (a factor of 2 survives rounding).
        const float s_last = quot(e_last);
        const bool boundary = e_next >= 0x1p-100f ? s_last > quot(e_next) : e_last >= 0x1p-99f;
        const uint64_t gmask = ((1ull << G) - 1) << (lane - sub);
        const bool ok = k <= (uint32_t)G && quot_ok && e_last >= 0x1p-100f && boundary &&
                        (__ballot(bad) & gmask) == 0;
        if (__ballot(active && !ok) == 0) {
            sort8_desc(sk);
            // Rank r goes to lane r of the group; every lane sums the k
            // scores in rank order (finish_selected).
            float sum = 0.0f, mine = 0.0f;
            uint32_t my_e = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if ((uint32_t)i < k) {
                    const float v = __uint_as_float(dkey_hi(sk[i]));
                    sum += v;
                    if ((uint32_t)i == sub) {
                        mine = v;
                        my_e = 0xFFFFFFFFu - dkey_lo(sk[i]);
                    }
                }
            }
            if (active && sub < k) {
                float v = mine;
                if (norm && sum > 0.0f) v = v / sum;
                ids[(size_t)token * k + sub] = my_e;
                weights[(size_t)token * k + sub] = v * (rsf == 0.0f ? 1.0f : rsf);
            }
            return;
        }
    }
    if (__ballot(!(quot_ok && e_ok)) == 0) {
        const float y = 1.0f / d;
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            const float q0 = s[j] * y;
            const float r = __builtin_fmaf(-d, q0, s[j]);
            s[j] = __builtin_fmaf(r, y, q0);
        }
    } else if (d > 0.0f) {
        divide_by(s, d);
    }
    select_and_store<EPL, G, false>(s, lane, sub, token, active, E, k, norm, rsf, ids, weights);
}

}  // namespace
}  // namespace fellm

extern "C" int fellm_rocm_router_topk(const float *logits, uint32_t tokens, uint32_t n_experts,
                                      uint32_t n_expert_used, uint32_t gating_func, uint32_t norm_topk_prob,
                                      float routed_scaling_factor, uint32_t *ids, float *weights,
                                      void *stream) {
    using namespace fellm;
    if (n_experts == 0 || n_experts > kMaxExperts) return FELLM_ERR_SHAPE;
    const uint32_t k = n_expert_used < n_experts ? n_expert_used : n_experts;
    if (k == 0 || k > kMaxTopK) return FELLM_ERR_SHAPE;
    if (tokens == 0) return FELLM_OK;
    if (!logits || !ids || !weights) return FELLM_ERR_ARITY;
    const dim3 block(kRouterBlock);
    hipStream_t s = as_stream(stream);
    constexpr int EPL = FELLM_ROUTER_EPL;
    // G lanes per token: a power of two <= 64 with G * EPL >= n_experts.
    const uint32_t need = (n_experts + EPL - 1) / EPL;
    uint32_t g = 1;
    while (g < need) g <<= 1;
    const uint32_t tpb = kRouterBlock / g;  // tokens per block
    const dim3 ggrid((tokens + tpb - 1) / tpb);
    if (FELLM_ROUTER_LEAN && gating_func == 1 && n_experts == g * EPL && aligned_to(logits, 16) && EPL % 4 == 0) {
#define FELLM_ROUTER_L(GG)                                                                                   \
        if (g == GG) {                                                                                       \
            FELLM_LAUNCH((router_softmax_lean<EPL, GG>), ggrid, block, 0, s, logits, tokens, k, norm_topk_prob, \
                         routed_scaling_factor, ids, weights);                                               \
            return launch_status();                                                                          \
        }
        FELLM_ROUTER_L(2)
        FELLM_ROUTER_L(4)
        FELLM_ROUTER_L(8)
        FELLM_ROUTER_L(16)
#undef FELLM_ROUTER_L
    }
#define FELLM_ROUTER_G(GG)                                                                                 \
    if (g == GG) {                                                                                         \
        FELLM_LAUNCH((router_topk_grouped<EPL, GG>), ggrid, block, 0, s, logits, tokens, n_experts, k,     \
                     gating_func, norm_topk_prob, routed_scaling_factor, ids, weights);                    \
        return launch_status();                                                                            \
    }
    FELLM_ROUTER_G(1)
    FELLM_ROUTER_G(2)
    FELLM_ROUTER_G(4)
    FELLM_ROUTER_G(8)
    FELLM_ROUTER_G(16)
    FELLM_ROUTER_G(32)
    FELLM_ROUTER_G(64)
#undef FELLM_ROUTER_G
    return FELLM_ERR_SHAPE;
}
