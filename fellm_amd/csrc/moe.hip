// MoE dispatch around the expert FFNs: group the routed (token, slot)
// assignments per expert, gather the token rows into that grouped order, and
// add the weighted expert outputs back into the token rows.
//
// Reference behaviour:
//   grouping   crates/backend-cpu/src/kernels/moe.rs:839-848 pushes
//              (token, weight) onto groups[expert] walking tokens in order, so
//              inside one expert the assignments a = token * top_k + slot come
//              in ascending a.  plugins/cuda_kernels/src/oxide_kernels.rs:
//              2283-2327 (fill_u32 / moe_count_assignments /
//              moe_prefix_offsets / moe_scatter_assignments) computes the same
//              counts and offsets but scatters with an atomic cursor, so its
//              order inside an expert varies run to run.  Here the order is the
//              CPU backend's, deterministically: a stable counting sort.
//   gather     moe.rs:954-957 copies each group's x rows.
//   combine    moe.rs:1024-1033: y[token] += weight * out, group by group,
//              i.e. a token's contributions arrive in ascending expert id
//              (grouped rows, located through inv).  oxide_kernels.rs:2507-2532
//              (moe_weighted_reduce): value = 0; value += score * out in slot
//              order, with out indexed by assignment.  Both orders are offered;
//              neither contracts the multiply-add into an FMA, as the
//              reference's Rust does not.
//
// Layout: ids / weights are [tokens][top_k] u32 / f32 (assignment-major, as
// the router writes them); counts [E], offsets [E + 1], order [A] and inv [A]
// are u32 with A = tokens * top_k; rows are contiguous, `hidden` elements.
//
// The dispatch is integer work over A * 4 bytes of ids: it is launch- and
// latency-bound, not HBM-bound.  At most 256 blocks each take a contiguous
// chunk (>= 2048 assignments), a wavefront a quarter of it; pass 1 counts per
// block, pass 2 turns the counts into cursors and scatters stably.  Up to 2048
// assignments (decode batches) it is one launch.
#include <mutex>

#include "common.hpp"

namespace fellm {
namespace {

constexpr uint32_t kDispatchBlock = 256;                  // 4 wavefronts
constexpr uint32_t kDispatchWaves = kDispatchBlock / kWave;
constexpr uint32_t kMinChunk = 2048;                      // assignments per block, at least
constexpr uint32_t kMaxDispatchBlocks = 256;
constexpr uint32_t kMoeMaxExperts = 4096;
constexpr uint32_t kMoeMaxTopK = 64;
constexpr uint32_t kInvalid = 0xffffffffu;

__device__ __forceinline__ uint32_t lane_id() { return __lane_id(); }

// cnt[id] += 1 for every valid id in [lo, hi), `stride` threads from `t`.
// Loads go out in batches of 8 before their LDS atomics.
__device__ __forceinline__ void count_range(const uint32_t *__restrict__ ids, uint64_t lo, uint64_t hi, uint32_t t,
                                            uint32_t stride, uint32_t E, uint32_t *cnt, uint32_t *err) {
    constexpr int kBatch = 8;
    bool bad = false;
    for (uint64_t a0 = lo + t; a0 < hi; a0 += (uint64_t)stride * kBatch) {
        uint32_t v[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const uint64_t a = a0 + (uint64_t)j * stride;
            v[j] = a < hi ? ids[a] : kInvalid;
        }
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const uint64_t a = a0 + (uint64_t)j * stride;
            if (v[j] < E)
                atomicAdd(&cnt[v[j]], 1u);
            else if (a < hi)
                bad = true;
        }
    }
    if (bad && err) atomicOr(err, 1u);
}

// Stable scatter of [lo, hi) by one wavefront: cur[e] (LDS, private to the
// wavefront) holds expert e's next free grouped position.  64 assignments per
// round; an assignment's rank among the round's earlier lanes with the same
// expert comes from ballots over the id's bits (lanes agreeing on every bit
// are peers), and the round's lowest peer advances the cursor.
__device__ __forceinline__ void scatter_range(const uint32_t *__restrict__ ids, uint64_t lo, uint64_t hi, uint32_t E,
                                              uint32_t bits, uint32_t *cur, uint32_t *__restrict__ order,
                                              uint32_t *__restrict__ inv) {
    constexpr int kBatch = 8;  // rounds whose ids are loaded together
    const uint32_t lane = lane_id();
    const uint64_t lt = (1ull << lane) - 1ull;
    for (uint64_t r0 = lo; r0 < hi; r0 += (uint64_t)kWave * kBatch) {
        uint32_t idv[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const uint64_t a = r0 + (uint64_t)j * kWave + lane;
            idv[j] = a < hi ? ids[a] : kInvalid;
        }
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const uint64_t a = r0 + (uint64_t)j * kWave + lane;
            const uint32_t id = idv[j];
            const bool valid = id < E;
            if (!valid && a < hi && inv) inv[a] = kInvalid;
            uint64_t peers = __ballot(valid);
            if (peers == 0) continue;  // wave-uniform: no valid id this round
            for (uint32_t b = 0; b < bits; ++b) {
                const bool bit = (id >> b) & 1u;
                const uint64_t ones = __ballot(bit);
                peers &= bit ? ones : ~ones;
            }
            uint32_t base = 0;
            if (valid) base = cur[id];
            // Every lane has read its cursor before the leaders advance them.
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
            __builtin_amdgcn_wave_barrier();
            const uint32_t rank = __popcll(peers & lt);
            if (valid) {
                if (rank == 0) cur[id] = base + (uint32_t)__popcll(peers);
                const uint32_t pos = base + rank;
                order[pos] = (uint32_t)a;
                if (inv) inv[a] = pos;
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
            __builtin_amdgcn_wave_barrier();
        }
    }
}

// Exclusive scan of v over the wavefront; returns the prefix, *total the sum.
__device__ __forceinline__ uint32_t wave_exclusive(uint32_t v, uint32_t *total) {
    const uint32_t lane = lane_id();
    uint32_t inc = v;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const uint32_t o = __shfl_up(inc, d);
        if (lane >= (uint32_t)d) inc += o;
    }
    *total = __shfl(inc, kWave - 1);
    return inc - v;
}

// Pass 1 (only with more than one block): bc[c][e] = valid ids of expert e in
// block c's chunk [c * chunk, (c + 1) * chunk).
__global__ __launch_bounds__(kDispatchBlock) void moe_count_blocks(const uint32_t *__restrict__ ids, uint64_t n,
                                                                   uint32_t E, uint64_t chunk,
                                                                   uint32_t *__restrict__ bc, uint32_t *err) {
    extern __shared__ uint32_t cnt[];
    const uint32_t t = threadIdx.x;
    const uint64_t c = blockIdx.x;
    for (uint32_t e = t; e < E; e += kDispatchBlock) cnt[e] = 0;
    __syncthreads();
    const uint64_t lo = c * chunk, hi = min(n, lo + chunk);
    count_range(ids, lo, hi, t, kDispatchBlock, E, cnt, err);
    __syncthreads();
    for (uint32_t e = t; e < E; e += kDispatchBlock) bc[c * E + e] = cnt[e];
}

// Pass 2: block c scatters its chunk, wavefront w the w-th quarter of it.
// Every block derives what it needs from bc: the per-expert totals (their
// exclusive prefix over experts is `offsets`) and the counts of the chunks
// before its own.  Block 0 writes counts / offsets and fills the order tail
// past the valid assignments.  With one block (nblocks == 1) bc is unused and
// the whole dispatch is this one launch.
//
// LDS: wcur[kDispatchWaves][E] (per-wavefront counts, then cursors), col[E],
// bef[E].
__global__ __launch_bounds__(kDispatchBlock) void moe_scatter_blocks(const uint32_t *__restrict__ ids, uint64_t n,
                                                                     uint32_t E, uint32_t bits, uint64_t chunk,
                                                                     uint32_t nblocks,
                                                                     const uint32_t *__restrict__ bc,
                                                                     uint32_t *__restrict__ counts,
                                                                     uint32_t *__restrict__ offsets,
                                                                     uint32_t *__restrict__ order,
                                                                     uint32_t *__restrict__ inv, uint32_t *err) {
    extern __shared__ uint32_t lds[];
    uint32_t *wcur = lds;                        // [waves][E]
    uint32_t *col = lds + kDispatchWaves * E;    // [E]
    uint32_t *bef = col + E;                     // [E]
    __shared__ uint32_t wsum[kDispatchWaves];
    const uint32_t t = threadIdx.x, w = t / kWave;
    const uint32_t c = blockIdx.x;
    const uint64_t lo = (uint64_t)c * chunk, hi = min(n, lo + chunk);
    const uint64_t sub = chunk / kDispatchWaves;
    const uint64_t wlo = min(hi, lo + w * sub), whi = min(hi, wlo + sub);
    for (uint32_t i = t; i < kDispatchWaves * E; i += kDispatchBlock) wcur[i] = 0;
    __syncthreads();
    // Counts per wavefront quarter (the error flag is raised by pass 1 when
    // there is one, here otherwise).
    count_range(ids, wlo, whi, lane_id(), kWave, E, wcur + w * E, nblocks == 1 ? err : nullptr);
    __syncthreads();
    // Per expert: total over all blocks (col) and count in the blocks before
    // this one (bef), read from bc with every load of a batch in flight.
    if (nblocks == 1) {
        for (uint32_t e = t; e < E; e += kDispatchBlock) {
            uint32_t total = 0;
#pragma unroll
            for (uint32_t q = 0; q < kDispatchWaves; ++q) total += wcur[q * E + e];
            col[e] = total;
            bef[e] = 0;
        }
    } else {
        for (uint32_t e = t; e < E; e += kDispatchBlock) col[e] = bef[e] = 0;
        __syncthreads();
        constexpr int kBatch = 16;
        const uint32_t cells = nblocks * E, cut = c * E;
        for (uint32_t i0 = t; i0 < cells; i0 += kDispatchBlock * kBatch) {
            uint32_t v[kBatch];
#pragma unroll
            for (int j = 0; j < kBatch; ++j) {
                const uint32_t i = i0 + j * kDispatchBlock;
                v[j] = i < cells ? bc[i] : 0u;
            }
#pragma unroll
            for (int j = 0; j < kBatch; ++j) {
                const uint32_t i = i0 + j * kDispatchBlock;
                if (i < cells && v[j]) {
                    const uint32_t e = i % E;
                    atomicAdd(&col[e], v[j]);
                    if (i < cut) atomicAdd(&bef[e], v[j]);
                }
            }
        }
    }
    __syncthreads();
    // Per-wavefront cursors relative to the expert's first grouped position.
    for (uint32_t e = t; e < E; e += kDispatchBlock) {
        if (c == 0) counts[e] = col[e];
        uint32_t run = bef[e];
#pragma unroll
        for (uint32_t q = 0; q < kDispatchWaves; ++q) {
            const uint32_t v = wcur[q * E + e];
            wcur[q * E + e] = run;
            run += v;
        }
    }
    __syncthreads();
    // Exclusive prefix of col over experts: thread t owns a contiguous run.
    const uint32_t per = (E + kDispatchBlock - 1) / kDispatchBlock;
    const uint32_t elo = min(E, t * per), ehi = min(E, elo + per);
    uint32_t s = 0;
    for (uint32_t e = elo; e < ehi; ++e) s += col[e];
    uint32_t wtotal;
    const uint32_t wpre = wave_exclusive(s, &wtotal);
    if (lane_id() == 0) wsum[w] = wtotal;
    __syncthreads();
    uint32_t run = wpre, all = 0;
#pragma unroll
    for (uint32_t q = 0; q < kDispatchWaves; ++q) {
        const uint32_t x = wsum[q];
        run += q < w ? x : 0u;
        all += x;
    }
    for (uint32_t e = elo; e < ehi; ++e) {
        const uint32_t v = col[e];
        col[e] = run;
        if (c == 0) offsets[e] = run;
        run += v;
    }
    if (c == 0) {
        if (t == 0) offsets[E] = all;
        for (uint64_t i = all + t; i < n; i += kDispatchBlock) order[i] = kInvalid;
    }
    __syncthreads();
    for (uint32_t e = t; e < E; e += kDispatchBlock) {
#pragma unroll
        for (uint32_t q = 0; q < kDispatchWaves; ++q) wcur[q * E + e] += col[e];
    }
    __syncthreads();
    scatter_range(ids, wlo, whi, E, bits, wcur + w * E, order, inv);
}

// Block count and chunk (a multiple of kDispatchBlock, so each wavefront's
// quarter is whole rounds) for n assignments.
struct DispatchGrid {
    uint32_t nblocks;
    uint64_t chunk;
};

inline DispatchGrid dispatch_grid(uint64_t n) {
    uint64_t nb = (n + kMinChunk - 1) / kMinChunk;
    if (nb < 1) nb = 1;
    if (nb > kMaxDispatchBlocks) nb = kMaxDispatchBlocks;
    uint64_t chunk = (n + nb - 1) / nb;
    chunk = (chunk + kDispatchBlock - 1) / kDispatchBlock * kDispatchBlock;
    if (chunk == 0) chunk = kDispatchBlock;
    nb = (n + chunk - 1) / chunk;
    if (nb < 1) nb = 1;
    return {(uint32_t)nb, chunk};
}

// grouped[i] = x[order[i] / top_k]; an invalid order entry gives a zero row.
template <typename V>
__global__ __launch_bounds__(256) void moe_gather_rows(const V *__restrict__ x, const uint32_t *__restrict__ order,
                                                       uint64_t n, uint32_t top_k, uint64_t row_vecs,
                                                       V *__restrict__ grouped) {
    for (uint64_t i = blockIdx.x; i < n; i += gridDim.x) {
        const uint32_t a = order[i];
        V *dst = grouped + i * row_vecs;
        if (a < n) {
            const V *src = x + (uint64_t)(a / top_k) * row_vecs;
            for (uint64_t j = threadIdx.x; j < row_vecs; j += blockDim.x) dst[j] = src[j];
        } else {
            for (uint64_t j = threadIdx.x; j < row_vecs; j += blockDim.x) dst[j] = V{};
        }
    }
}

// Scatter form of the gather: token t's row is read once and written to
// grouped[inv[t * top_k + s]] for every slot s, so HBM sees the grouped
// writes plus one read of x.  A grouped row whose order entry is invalid (the
// tail past the valid assignments) is zeroed; rows p in [t * top_k,
// (t + 1) * top_k) are checked by token t's block.  The row is staged
// through registers in segments of kSeg 16-byte vectors per thread.
template <int kSeg>
__global__ __launch_bounds__(256) void moe_scatter_rows(const uint4 *__restrict__ x,
                                                        const uint32_t *__restrict__ order,
                                                        const uint32_t *__restrict__ inv, uint64_t tokens,
                                                        uint32_t top_k, uint64_t row_vecs,
                                                        uint4 *__restrict__ grouped) {
    __shared__ uint32_t sdst[kMoeMaxTopK];
    __shared__ uint32_t szero[kMoeMaxTopK];
    const uint32_t t = threadIdx.x;
    const uint64_t n = tokens * top_k;
    for (uint64_t tok = blockIdx.x; tok < tokens; tok += gridDim.x) {
        if (t < top_k) {
            const uint64_t a = tok * top_k + t;
            const uint32_t p = inv[a];
            sdst[t] = p < n ? p : kInvalid;
            szero[t] = order[a] < n ? kInvalid : (uint32_t)a;
        }
        __syncthreads();
        const uint4 *src = x + tok * row_vecs;
        for (uint64_t j0 = 0; j0 < row_vecs; j0 += (uint64_t)kSeg * 256) {
            uint4 v[kSeg];
#pragma unroll
            for (int u = 0; u < kSeg; ++u) {
                const uint64_t j = j0 + (uint64_t)u * 256 + t;
                if (j < row_vecs) v[u] = src[j];
            }
            for (uint32_t s = 0; s < top_k; ++s) {
                const uint32_t p = sdst[s];
                if (p == kInvalid) continue;
                uint4 *dst = grouped + (uint64_t)p * row_vecs;
#pragma unroll
                for (int u = 0; u < kSeg; ++u) {
                    const uint64_t j = j0 + (uint64_t)u * 256 + t;
                    if (j < row_vecs) dst[j] = v[u];
                }
            }
            for (uint32_t s = 0; s < top_k; ++s) {
                const uint32_t p = szero[s];
                if (p == kInvalid) continue;
                uint4 *dst = grouped + (uint64_t)p * row_vecs;
#pragma unroll
                for (int u = 0; u < kSeg; ++u) {
                    const uint64_t j = j0 + (uint64_t)u * 256 + t;
                    if (j < row_vecs) dst[j] = uint4{0, 0, 0, 0};
                }
            }
        }
        __syncthreads();
    }
}

// y[t] = y0[t] (or 0) + sum over t's slots of weight * row, one token per
// block iteration.  EXPERT_ORDER: slots in ascending (expert id, slot), rows
// expert_out[inv[a]]; otherwise slot order, rows expert_out[a].
template <bool EXPERT_ORDER, int VEC>
// Build knobs: combine workgroup size and grid cap.  512 threads (one 16-byte
// column per thread at hidden 2048) measured 3% faster than 256 in both orders.
#ifndef FELLM_MOE_COMBINE_BLOCK
#define FELLM_MOE_COMBINE_BLOCK 512
#endif
#ifndef FELLM_MOE_COMBINE_CAP
#define FELLM_MOE_COMBINE_CAP 65536
#endif
__global__ __launch_bounds__(FELLM_MOE_COMBINE_BLOCK) void moe_combine_rows(const float *y0, const float *__restrict__ expert_out,
                                                        const uint32_t *__restrict__ ids,
                                                        const float *__restrict__ weights,
                                                        const uint32_t *__restrict__ inv, uint64_t tokens,
                                                        uint32_t top_k, uint64_t hidden, uint64_t n_rows, float *y) {
#pragma clang fp contract(off)
    using Vec = Pack<float, VEC>;
    __shared__ float sw[kMoeMaxTopK];
    __shared__ uint32_t srow[kMoeMaxTopK];
    const uint32_t t = threadIdx.x;
    const uint64_t nvec = hidden / VEC;
    for (uint64_t tok = blockIdx.x; tok < tokens; tok += gridDim.x) {
        if (t < kWave) {
            const uint64_t a = tok * top_k + t;
            uint32_t rank = t, row = kInvalid;
            float w = 0.0f;
            if (t < top_k) {
                w = weights[a];
                row = (uint32_t)a;
                if (EXPERT_ORDER) row = inv[a];
            }
            if (EXPERT_ORDER) {
                const uint64_t key = t < top_k ? (uint64_t)ids[a] * kMoeMaxTopK + t : ~0ull;
                rank = 0;
                for (uint32_t j = 0; j < top_k; ++j) {
                    const uint64_t kj = __shfl(key, j);
                    rank += kj < key;
                }
            }
            if (t < top_k) {
                sw[rank] = w;
                srow[rank] = row < n_rows ? row : kInvalid;
            }
        }
        __syncthreads();
        const uint64_t ybase = tok * nvec;
        for (uint64_t j = t; j < nvec; j += blockDim.x) {
            Vec acc;
            if (y0) {
                acc = reinterpret_cast<const Vec *>(y0)[ybase + j];
            } else {
#pragma unroll
                for (int e = 0; e < VEC; ++e) acc.v[e] = 0.0f;
            }
            for (uint32_t s0 = 0; s0 < top_k; s0 += 8) {
                Vec r[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const uint32_t s = s0 + u;
                    const uint32_t row = s < top_k ? srow[s] : kInvalid;
                    if (row != kInvalid)
                        r[u] = reinterpret_cast<const Vec *>(expert_out)[(uint64_t)row * nvec + j];
                }
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const uint32_t s = s0 + u;
                    if (s < top_k && srow[s] != kInvalid) {
                        const float w = sw[s];
#pragma unroll
                        for (int e = 0; e < VEC; ++e) acc.v[e] = acc.v[e] + w * r[u].v[e];
                    }
                }
            }
            reinterpret_cast<Vec *>(y)[ybase + j] = acc;
        }
        __syncthreads();
    }
}

inline uint32_t id_bits(uint32_t E) { return E <= 1 ? 0 : 32 - __builtin_clz(E - 1); }

inline uint32_t grid_cap(uint64_t units, uint64_t cap) { return (uint32_t)(units < cap ? units : cap); }

}  // namespace
}  // namespace fellm

extern "C" uint64_t fellm_rocm_moe_dispatch_workspace(uint64_t tokens, uint32_t top_k, uint32_t n_experts) {
    using namespace fellm;
    const DispatchGrid g = dispatch_grid(tokens * top_k);
    return g.nblocks <= 1 ? 0 : (uint64_t)g.nblocks * n_experts * sizeof(uint32_t);
}

// Library-owned per-block count buffer of the allocation-free dispatch
// (fellm_rocm_moe_dispatch_noalloc): the largest grid (256 blocks) times the
// most experts (4096), 4 MiB.  Each GPU holds its own copy until the process
// ends; host code reaches it only through the address hipGetSymbolAddress
// returns for the current device, never through this name.
constexpr uint64_t kDispatchScratchWords = 256ull * 4096ull;
static __device__ __align__(256) uint32_t scratch[kDispatchScratchWords];

namespace fellm {
namespace {

// Validates the dispatch arguments and enqueues its one or two launches;
// `bc_ws` holds the per-block counts (at least nblocks * E u32) when the
// grid has more than one block.
int dispatch_launch(const uint32_t *ids, uint64_t tokens, uint32_t top_k, uint32_t n_experts, uint32_t *counts,
                    uint32_t *offsets, uint32_t *order, uint32_t *inv, uint32_t *err_flag, uint32_t *bc_ws,
                    uint64_t bc_bytes, hipStream_t st) {
    if (!counts || !offsets) return FELLM_ERR_ARITY;
    if (n_experts == 0 || n_experts > kMoeMaxExperts || top_k == 0 || top_k > kMoeMaxTopK) return FELLM_ERR_SHAPE;
    const uint64_t n = tokens * top_k;
    if (tokens > 0xffffffffull || n >= 0xffffffffull) return FELLM_ERR_SHAPE;
    if (n && (!ids || !order)) return FELLM_ERR_ARITY;
    const uint32_t E = n_experts, bits = id_bits(E);
    const DispatchGrid g = dispatch_grid(n);
    const uint32_t *bc = nullptr;
    if (g.nblocks > 1) {
        if (!bc_ws || bc_bytes < (uint64_t)g.nblocks * E * sizeof(uint32_t)) return FELLM_ERR_SHAPE;
        // Pass 1 writes every one of the nblocks * E counts before pass 2
        // reads them, so the buffer needs no clearing between calls.
        FELLM_LAUNCH(moe_count_blocks, dim3(g.nblocks), dim3(kDispatchBlock), (size_t)E * sizeof(uint32_t),
                           st, ids, n, E, g.chunk, bc_ws, err_flag);
        bc = bc_ws;
    }
    const size_t lds = (size_t)(kDispatchWaves + 2) * E * sizeof(uint32_t);
    FELLM_LAUNCH(moe_scatter_blocks, dim3(g.nblocks), dim3(kDispatchBlock), lds, st, ids, n, E, bits, g.chunk,
                       g.nblocks, bc, counts, offsets, order, inv, err_flag);
    return launch_status();
}

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint32_t *g_scratch_ptr[kMaxDevices];

// Device address of `scratch` on the current device, looked up once per device
// and kept for the life of the process.  The cache assumes the device is not
// reset and the library not unloaded in between: after hipDeviceReset the
// array's allocation is gone and a cached address would be stale, so a caller
// that resets a device must not call the allocation-free entry point again in
// that process.
static_assert(kDispatchScratchWords == (uint64_t)kMaxDispatchBlocks * kMoeMaxExperts,
              "the scratch buffer holds the per-block counts of the largest dispatch grid");

int scratch_for_current_device(uint32_t **out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return FELLM_ERR_LAUNCH;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return FELLM_ERR_ALLOC;
        g_scratch_ptr[dev] = static_cast<uint32_t *>(p);
    }
    *out = g_scratch_ptr[dev];
    return FELLM_OK;
}

}  // namespace
}  // namespace fellm

extern "C" int fellm_rocm_moe_dispatch(const uint32_t *ids, uint64_t tokens, uint32_t top_k, uint32_t n_experts,
                                       uint32_t *counts, uint32_t *offsets, uint32_t *order, uint32_t *inv,
                                       uint32_t *err_flag, void *workspace, uint64_t workspace_bytes, void *stream) {
    using namespace fellm;
    return dispatch_launch(ids, tokens, top_k, n_experts, counts, offsets, order, inv, err_flag,
                           static_cast<uint32_t *>(workspace), workspace ? workspace_bytes : 0, as_stream(stream));
}

extern "C" uint64_t fellm_rocm_moe_dispatch_noalloc_max_bytes(void) {
    return kDispatchScratchWords * sizeof(uint32_t);
}

extern "C" int fellm_rocm_moe_dispatch_noalloc(const uint32_t *ids, uint64_t tokens, uint32_t top_k,
                                               uint32_t n_experts, uint32_t *counts, uint32_t *offsets,
                                               uint32_t *order, uint32_t *inv, uint32_t *err_flag, void *stream) {
    using namespace fellm;
    if (n_experts > kMoeMaxExperts || top_k == 0 || top_k > kMoeMaxTopK) return FELLM_ERR_SHAPE;
    const uint64_t need = fellm_rocm_moe_dispatch_workspace(tokens, top_k, n_experts);
    if (need > kDispatchScratchWords * sizeof(uint32_t)) return FELLM_ERR_SHAPE;  // beyond the library's buffer
    uint32_t *ws = nullptr;
    if (need) {
        if (int rc = scratch_for_current_device(&ws)) return rc;
    }
    return dispatch_launch(ids, tokens, top_k, n_experts, counts, offsets, order, inv, err_flag, ws,
                           kDispatchScratchWords * sizeof(uint32_t), as_stream(stream));
}

extern "C" int fellm_rocm_moe_gather(const void *x, uint32_t elem_bytes, uint64_t tokens, uint32_t top_k,
                                     uint64_t hidden, const uint32_t *order, const uint32_t *inv, void *grouped,
                                     void *stream) {
    using namespace fellm;
    if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4) return FELLM_ERR_DTYPE;
    if (top_k == 0 || top_k > kMoeMaxTopK) return FELLM_ERR_SHAPE;
    const uint64_t n = tokens * top_k;
    if (tokens > 0xffffffffull || n >= 0xffffffffull) return FELLM_ERR_SHAPE;
    if (n == 0 || hidden == 0) return FELLM_OK;
    if (!x || !order || !grouped) return FELLM_ERR_ARITY;
    hipStream_t st = as_stream(stream);
    const uint64_t row_bytes = hidden * elem_bytes;
    const bool vec16 = row_bytes % 16 == 0 && aligned_to(x, 16) && aligned_to(grouped, 16);
    if (inv && vec16) {
        const uint64_t row_vecs = row_bytes / 16;
        const uint32_t grid = grid_cap(tokens, 16384);
        if (row_vecs <= 256)
            FELLM_LAUNCH(moe_scatter_rows<1>, dim3(grid), dim3(256), 0, st, static_cast<const uint4 *>(x), order,
                               inv, tokens, top_k, row_vecs, static_cast<uint4 *>(grouped));
        else
            FELLM_LAUNCH(moe_scatter_rows<4>, dim3(grid), dim3(256), 0, st, static_cast<const uint4 *>(x), order,
                               inv, tokens, top_k, row_vecs, static_cast<uint4 *>(grouped));
        return launch_status();
    }
    const uint32_t grid = grid_cap(n, 8192);
    if (vec16)
        FELLM_LAUNCH(moe_gather_rows<uint4>, dim3(grid), dim3(256), 0, st, static_cast<const uint4 *>(x),
                           order, n, top_k, row_bytes / 16, static_cast<uint4 *>(grouped));
    else if (row_bytes % 4 == 0 && aligned_to(x, 4) && aligned_to(grouped, 4))
        FELLM_LAUNCH(moe_gather_rows<uint32_t>, dim3(grid), dim3(256), 0, st,
                           static_cast<const uint32_t *>(x), order, n, top_k, row_bytes / 4,
                           static_cast<uint32_t *>(grouped));
    else
        FELLM_LAUNCH(moe_gather_rows<uint8_t>, dim3(grid), dim3(256), 0, st, static_cast<const uint8_t *>(x),
                           order, n, top_k, row_bytes, static_cast<uint8_t *>(grouped));
    return launch_status();
}

extern "C" int fellm_rocm_moe_combine(const float *y0, const float *expert_out, const uint32_t *ids,
                                      const float *weights, const uint32_t *inv, uint64_t tokens, uint32_t top_k,
                                      uint64_t hidden, float *y, void *stream) {
    using namespace fellm;
    if (top_k == 0 || top_k > kMoeMaxTopK) return FELLM_ERR_SHAPE;
    const uint64_t n = tokens * top_k;
    if (tokens > 0xffffffffull || n >= 0xffffffffull) return FELLM_ERR_SHAPE;
    if (tokens == 0 || hidden == 0) return FELLM_OK;
    if (!expert_out || !weights || !y || (inv && !ids)) return FELLM_ERR_ARITY;
    hipStream_t st = as_stream(stream);
    const uint32_t grid = grid_cap(tokens, FELLM_MOE_COMBINE_CAP);
    const bool vec = hidden % 4 == 0 && aligned_to(expert_out, 16) && aligned_to(y, 16) && (!y0 || aligned_to(y0, 16));
#define FELLM_MOE_COMBINE(ORD, V)                                                                                   \
    FELLM_LAUNCH((moe_combine_rows<ORD, V>), dim3(grid), dim3(FELLM_MOE_COMBINE_BLOCK), 0, st, y0, expert_out, ids, weights, inv, \
                       tokens, top_k, hidden, n, y)
    if (inv) {
        if (vec)
            FELLM_MOE_COMBINE(true, 4);
        else
            FELLM_MOE_COMBINE(true, 1);
    } else {
        if (vec)
            FELLM_MOE_COMBINE(false, 4);
        else
            FELLM_MOE_COMBINE(false, 1);
    }
#undef FELLM_MOE_COMBINE
    return launch_status();
}
