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
// the CPU.  Ranking uses 64-bit keys
// (total-order(score) << 32 | ~expert): k wavefront max-reductions pick the
// winners in rank order, ties resolved towards the lower expert id exactly as
// the CPU's comparator does.
#include "common.hpp"

namespace fellm {
namespace {

// Build knob: experts per lane in the grouped kernel (8, 16 or 32).
#ifndef FELLM_ROUTER_EPL
#define FELLM_ROUTER_EPL 16
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

// Grouped path: G = 64 / TPW lanes per token, each lane owning EPL
// consecutive experts (expert e lives in lane e / EPL of its group, slot
// e % EPL), so expert order is (lane, slot) order.
//  * max: per-lane max, then an xor-shuffle reduction inside the group;
//  * denominator: the f32 fold in expert order runs lane to lane through the
//    group (lane q adds its EPL values to the running sum, then hands it to
//    lane q+1), i.e. exactly the CPU's left-to-right accumulation;
//  * top-k: k rounds; each lane scans its own candidates for the best
//    (score desc, expert asc) key, the group takes the 64-bit max, the owner
//    marks it taken.  Rank r's expert and raw score go straight to ids/weights
//    and the rank-order sum is folded on the way; a final pass rescales.
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
        if (d > 0.0f) {
            // e / d for every expert with one IEEE reciprocal per token:
            // y = RN(1/d), q0 = RN(e*y), r = e - d*q0 (exact), q = RN(q0 + r*y),
            // which Markstein's theorem makes the correctly rounded e / d when no
            // step underflows; tiny or non-finite operands take the IEEE division.
            // (Checked against IEEE division for 4096 values of d in [1, 512)
            // and every e in [2^-100, 1].)
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
    }
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
    const float scale = rsf == 0.0f ? 1.0f : rsf;
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
    // Grouped path: EPL experts per lane, G lanes per token (G a power of two
    // <= 64 with G * EPL >= n_experts).
    {
        constexpr int EPL = FELLM_ROUTER_EPL;
        const uint32_t need = (n_experts + EPL - 1) / EPL;
        uint32_t g = 1;
        while (g < need) g <<= 1;
        const uint32_t tpb = kRouterBlock / g;  // tokens per block
        const dim3 ggrid((tokens + tpb - 1) / tpb);
#define FELLM_ROUTER_G(GG)                                                                                 \
        if (g == GG) {                                                                                     \
            FELLM_LAUNCH((router_topk_grouped<EPL, GG>), ggrid, block, 0, s, logits, tokens, n_experts, k, \
                               gating_func, norm_topk_prob, routed_scaling_factor, ids, weights);          \
            return launch_status();                                                                        \
        }
        FELLM_ROUTER_G(1)
        FELLM_ROUTER_G(2)
        FELLM_ROUTER_G(4)
        FELLM_ROUTER_G(8)
        FELLM_ROUTER_G(16)
        FELLM_ROUTER_G(32)
        FELLM_ROUTER_G(64)
#undef FELLM_ROUTER_G
    }
    return FELLM_ERR_SHAPE;
}
