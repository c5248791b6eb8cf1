// MoE router: gate scores + top-k selection + renormalisation.
//
// Reference: crates/backend-cpu/src/kernels/moe.rs
//   gate_scores :79-111 (softmax: m = max(l); e_j = exp(l_j - m);
//       denom += e_j in expert order; s_j = e_j / denom if denom > 0;
//       sigmoid for gating 2: s_j = 1 / (1 + exp(-l_j)))
//   select_routed_experts :142-186 (rank by s descending under f32
//       total_cmp, ties -> lower expert id)
//   finish_selected :113-140 (truncate to k; if norm_topk_prob divide by the
//       sum of the selected scores taken in rank order; times
//       routed_scaling_factor, 0 meaning 1)
//   batched variant :820-855 (same ranking and arithmetic).
//
// One wavefront per token (n_experts <= 512: EPL experts per lane).  exp is
// the glibc-exact restatement and the denominator is summed serially in
// expert order by lane 0 (through LDS), so scores, ranking and weights are
// bit-exact with the CPU.  Ranking uses 64-bit keys
// (total-order(score) << 32 | ~expert): k wavefront max-reductions pick the
// winners in rank order, ties resolved towards the lower expert id exactly as
// the CPU's comparator does.
#include "common.hpp"

namespace fellm {
namespace {

constexpr int kRouterBlock = 256;
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

template <int EPL>
__global__ __launch_bounds__(kRouterBlock) void router_topk_kernel(
    const float *__restrict__ logits, uint32_t tokens, uint32_t n_exp, uint32_t k, uint32_t gating,
    uint32_t norm, float rsf, uint32_t *__restrict__ ids, float *__restrict__ weights) {
    __shared__ uint64_t tab_lds[32];
    __shared__ float ex_lds[kRouterWaves][kMaxExperts];
    __shared__ float denom_lds[kRouterWaves];
    __shared__ uint64_t sel_lds[kRouterWaves][kMaxTopK];
    const uint64_t *tab = stage_expf_table(tab_lds);

    const uint32_t wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const uint32_t token = blockIdx.x * kRouterWaves + wave;
    const bool active = token < tokens;
    const float *lg = logits + (size_t)(active ? token : 0) * n_exp;

    float l[EPL], s[EPL];
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        const uint32_t e = lane + kWave * j;
        l[j] = (active && e < n_exp) ? lg[e] : -__builtin_inff();
    }

    if (gating == 2) {
#pragma unroll
        for (int j = 0; j < EPL; ++j) s[j] = 1.0f / (1.0f + expf_glibc(-l[j], tab));
    } else {
        // max over all experts; fmaxf skips NaN like the CPU's f32::max fold.
        float m = l[0];
#pragma unroll
        for (int j = 1; j < EPL; ++j) m = fmaxf(m, l[j]);
        m = wave_max(m);
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            const uint32_t e = lane + kWave * j;
            s[j] = expf_glibc(l[j] - m, tab);
            if (e < n_exp) ex_lds[wave][e] = s[j];
        }
        __syncthreads();
        if (lane == 0) {
            float d = 0.0f;
            for (uint32_t e = 0; e < n_exp; ++e) d += ex_lds[wave][e];  // expert order
            denom_lds[wave] = d;
        }
        __syncthreads();
        const float d = denom_lds[wave];
        if (d > 0.0f) {
#pragma unroll
            for (int j = 0; j < EPL; ++j) s[j] = s[j] / d;
        }
    }

    uint64_t key[EPL];
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        const uint32_t e = lane + kWave * j;
        key[j] = (e < n_exp) ? ((uint64_t)total_order_key(s[j]) << 32) | (uint64_t)(0xffffffffu - e) : 0ull;
    }
    for (uint32_t r = 0; r < k; ++r) {
        uint64_t best = 0;
#pragma unroll
        for (int j = 0; j < EPL; ++j) best = key[j] > best ? key[j] : best;
        const uint64_t win = wave_max_u64(best);
        const uint32_t e = 0xffffffffu - (uint32_t)win;
        if (e % kWave == lane) {
#pragma unroll
            for (int j = 0; j < EPL; ++j)
                if ((uint32_t)j == e / kWave) key[j] = 0;
        }
        if (lane == 0) sel_lds[wave][r] = win;
    }
    __syncthreads();
    if (lane == 0 && active) {
        float sum = 0.0f;
        if (norm) {
            for (uint32_t r = 0; r < k; ++r) sum += total_order_inv((uint32_t)(sel_lds[wave][r] >> 32));
        }
        const float scale = rsf == 0.0f ? 1.0f : rsf;
        for (uint32_t r = 0; r < k; ++r) {
            const uint64_t w = sel_lds[wave][r];
            float v = total_order_inv((uint32_t)(w >> 32));
            if (norm && sum > 0.0f) v = v / sum;
            v = v * scale;
            ids[(size_t)token * k + r] = 0xffffffffu - (uint32_t)w;
            weights[(size_t)token * k + r] = v;
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
    if (!logits || !ids || !weights) return FELLM_ERR_ARITY;
    if (n_experts == 0 || n_experts > kMaxExperts) return FELLM_ERR_SHAPE;
    if (gating_func == 4) return FELLM_ERR_DTYPE;  // sqrt-softplus gating not implemented
    const uint32_t k = n_expert_used < n_experts ? n_expert_used : n_experts;
    if (k == 0 || k > kMaxTopK) return FELLM_ERR_SHAPE;
    if (tokens == 0) return FELLM_OK;
    const dim3 grid((tokens + kRouterWaves - 1) / kRouterWaves), block(kRouterBlock);
    hipStream_t s = as_stream(stream);
    const uint32_t epl = (n_experts + kWave - 1) / kWave;
#define FELLM_ROUTER(E)                                                                                   \
    if (epl <= E) {                                                                                       \
        hipLaunchKernelGGL(router_topk_kernel<E>, grid, block, 0, s, logits, tokens, n_experts, k,        \
                           gating_func, norm_topk_prob, routed_scaling_factor, ids, weights);             \
        return launch_status();                                                                           \
    }
    FELLM_ROUTER(1)
    FELLM_ROUTER(2)
    FELLM_ROUTER(4)
    FELLM_ROUTER(8)
#undef FELLM_ROUTER
    return FELLM_ERR_SHAPE;
}
