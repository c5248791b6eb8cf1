/*
 * fellm_rocm.h — device-pointer entry points of libfellm_rocm_kernels.so.
 *
 * These are the kernels behind the plugin launchers declared in fellm_abi.h.
 * They take DEVICE pointers that are already resident in HBM and a hipStream_t
 * (passed as void*; NULL = the null stream), enqueue work and return without
 * synchronising.  All return 0 or a negative FELLM_ERR_* code from fellm_abi.h;
 * argument validation happens on the host before anything is enqueued.
 *
 * Activation dtypes are FELLM_DTYPE_F32, FELLM_DTYPE_F16 or FELLM_DTYPE_BF16.
 * All arithmetic is f32 (the reference's op boundary is f32 everywhere:
 * crates/backend-cpu/src/backend.rs:798-816); 16-bit outputs are the f32
 * result rounded once, to nearest-even.
 *
 * Where a reference interface is replaced, the comment names it (file:line,
 * paths relative to the FeLLM repository root).
 */
#ifndef FELLM_ROCM_H
#define FELLM_ROCM_H

#include <stddef.h>
#include <stdint.h>

#include "fellm_abi.h" /* FellmDeviceStepParams, FELLM_ERR_*, FELLM_DTYPE_* */

#ifdef __cplusplus
extern "C" {
#endif

/* Library version string, e.g. "fellm-rocm 0.1.0 gfx950". */
const char *fellm_rocm_version(void);

/*
 * Residual add + RMSNorm over rows of `group` elements.
 *   replaces: Add (backend-cpu/src/backend.rs:1543-1553, kernels/simd_f32.rs:175-197)
 *             followed by RmsNorm (backend.rs:1104-1133, kernels/norm.rs:6-53).
 * x, residual, h_out: act_dtype, n_elems elements (n_elems % group == 0).
 * residual == NULL: plain RMSNorm of x (h_out must then be NULL).
 * h = x + residual is stored (rounded to act_dtype) in h_out when non-NULL and
 * the norm is taken of h as stored.  y = (h * scale) * w with
 * scale = 1 / sqrt(sum(h^2) / group + eps); y has y_dtype.
 * weight: f32 [group].
 */
int fellm_rocm_add_rmsnorm(const void *x, const void *residual, void *h_out, uint32_t act_dtype,
                           const float *weight, uint32_t group, void *y, uint32_t y_dtype,
                           uint64_t n_elems, float eps, void *stream);

/*
 * out = silu(gate) * up, silu(g) = g / (1 + exp(-g)).
 *   replaces: SiluGate (backend.rs:1174-1184, kernels/swiglu.rs:5-16).
 * exp is a bit-exact restatement of glibc's expf, so f32 output is bit-exact
 * with the CPU reference.
 */
int fellm_rocm_silu_gate(const void *gate, const void *up, uint32_t in_dtype, void *out,
                         uint32_t out_dtype, uint64_t n_elems, void *stream);

/* out = a + b elementwise (Add: backend.rs:1543-1553). */
int fellm_rocm_add(const void *a, const void *b, uint32_t in_dtype, void *out, uint32_t out_dtype,
                   uint64_t n_elems, void *stream);

/*
 * Embedding gather: out[t, :] = dequant(table[ids[t], :]).
 *   replaces: Embedding (backend.rs:1026-1046, kernels/embedding.rs:10-23,
 *             dequant.rs:19-55 F32/F16/BF16, :251-305 Q4_K, :315-370 Q6_K,
 *             :59-107 Q5_K, :172-192 Q8_0; the CUDA plugin's Q5_K and Q8_0 keys,
 *             plugins/cuda_kernels/src/lib.rs:637-661).
 * table_dtype: F32, F16, BF16, Q4K, Q5K, Q6K (dim % 256 == 0) or Q8_0 (dim % 32 == 0).
 * Q5K tables must be 4-byte aligned, Q8_0 and Q6K tables 2-byte aligned.
 * out_dtype:   F32, F16 or BF16.
 * An id >= vocab yields a zero row and sets *err_flag (device u32, may be NULL)
 * to 1; the CPU reference rejects such ids.
 * When norm_weight != NULL the gather is fused with RMSNorm over the row:
 * h_out (may be NULL) gets the gathered row and y the normalised row, with the
 * norm taken of the f32 dequantised values (out is then ignored and may be NULL).
 */
int fellm_rocm_embedding(const void *table, uint32_t table_dtype, uint64_t vocab, uint32_t dim,
                         const uint32_t *ids, uint32_t n_ids, void *out, uint32_t out_dtype,
                         uint32_t *err_flag, void *stream);
int fellm_rocm_embedding_rmsnorm(const void *table, uint32_t table_dtype, uint64_t vocab,
                                 uint32_t dim, const uint32_t *ids, uint32_t n_ids,
                                 const float *norm_weight, float eps, void *h_out, void *y,
                                 uint32_t out_dtype, uint32_t *err_flag, void *stream);

/*
 * RoPE over one or two row-major tensors sharing positions (q and k).
 *   replaces: Rope (backend.rs:1135-1172, kernels/rope.rs:28-62).
 * x1: [rows, n_heads1 * head_dim], x2: [rows, n_heads2 * head_dim] or NULL.
 * out1/out2 may alias x1/x2 (in place).  Pairing: 0 adjacent (2i, 2i+1),
 * 1 split-half (i, i + rope_dim/2), 2 adjacent over the last rope_dim dims.
 * theta = float(pos) * inv_freqs[i]; (s, c) = (sin, cos)(theta);
 * a' = a*c - b*s, b' = a*s + b*c.  pos = positions[row] when positions != NULL,
 * else position0 + row.  Dims outside the rotated span are copied.
 */
int fellm_rocm_rope(const void *x1, void *out1, uint32_t n_heads1, const void *x2, void *out2,
                    uint32_t n_heads2, uint32_t act_dtype, uint32_t rows, uint32_t head_dim,
                    uint32_t rope_dim, uint32_t pairing, const float *inv_freqs,
                    const uint32_t *positions, uint32_t position0, void *stream);

/*
 * Paged KV geometry, as FeLLM lays it out
 * (crates/fellm-plugin-abi/src/paged_ctx.rs:341-360, backend-cuda/src/vram_pool.rs:31-35):
 * block p occupies arena[p * block_bytes ...]: block_size K rows then
 * block_size V rows, each row `stride` elements of kv_dtype (F16 or BF16).
 * Row r's entry for token position t in layer L is
 *   block_table[(r * n_layers + L) * n_logical_blocks + t / block_size].
 */
typedef struct FellmRocmPagedKv {
    void *arena;               /* device */
    uint64_t arena_len;        /* bytes */
    const uint32_t *block_table; /* device */
    uint64_t n_block_table;
    uint32_t n_logical_blocks;
    uint32_t n_layers;
    uint32_t layer;
    uint32_t block_size;
    uint64_t block_bytes;
    uint32_t stride;           /* elements per K or V row (n_kv_heads * head_dim) */
    uint32_t kv_dtype;         /* FELLM_DTYPE_F16 (reference) or FELLM_DTYPE_BF16 */
} FellmRocmPagedKv;

/*
 * KvWrite: write rows[b, :] into the K (is_v = 0) or V (is_v = 1) slot of
 * batch row b at kv_positions[b].   replaces: backend.rs:1734-1775.
 * Slots outside the arena or table set *err_flag (device, may be NULL) and are skipped.
 */
int fellm_rocm_kv_write(const void *rows, uint32_t act_dtype, uint32_t batch,
                        const uint32_t *kv_positions, const FellmRocmPagedKv *kv, uint32_t is_v,
                        uint32_t *err_flag, void *stream);

/*
 * Fused RoPE(q), RoPE(k) + paged K/V append, one launch.
 *   replaces: the graph sequence q_rope -> k_rope -> k_write -> v_write
 *   (crates/fellm-model/src/graph.rs:2136-2215).
 * q_out gets rotated q; k_out (may be NULL) rotated k; rotated k and raw v are
 * rounded once to kv->kv_dtype and stored at kv_positions[b].  RoPE uses
 * rope_positions[b] (NULL: kv_positions).
 */
int fellm_rocm_rope_kv_write(const void *q, void *q_out, uint32_t n_q_heads, const void *k,
                             void *k_out, const void *v, uint32_t n_kv_heads, uint32_t act_dtype,
                             uint32_t batch, uint32_t head_dim, uint32_t rope_dim,
                             uint32_t pairing, const float *inv_freqs,
                             const uint32_t *rope_positions, const uint32_t *kv_positions,
                             const FellmRocmPagedKv *kv, uint32_t *err_flag, void *stream);

/*
 * One decode step's memory-bound ops in a single launch: RoPE(q), RoPE(k) and
 * the paged K/V append (fellm_rocm_rope_kv_write's arguments), residual add +
 * RMSNorm with y in act_dtype (fellm_rocm_add_rmsnorm's), and SwiGLU
 * (fellm_rocm_silu_gate's), all in act_dtype.
 *   replaces: the decode graph's separate launches of these ops
 *   (crates/fellm-model/src/graph.rs:2136-2246, :420-451, :1456-1510).
 * Rotated q and k, the K/V slots, h and the SwiGLU output are bit for bit
 * those of the three separate calls; y is within RMSNorm's tolerance of
 * theirs (the fused row reduces its sum of squares over 256 threads, the
 * standalone few-row launch over 1024).  The three ops must write disjoint
 * outputs.  Shapes outside the fused layout (unaligned
 * buffers, no residual or h, rows of <= 2048 or > 16384 elements) run as the
 * three separate launches; a zero batch / norm_elems / swiglu_elems skips
 * that op there.
 */
typedef struct FellmRocmDecodeStep {
    uint32_t act_dtype;
    /* RoPE + paged K/V append */
    const void *q;
    void *q_out;
    uint32_t n_q_heads;
    const void *k;
    void *k_out; /* may be NULL */
    const void *v;
    uint32_t n_kv_heads;
    uint32_t batch;
    uint32_t head_dim;
    uint32_t rope_dim;
    uint32_t pairing;
    const float *inv_freqs;
    const uint32_t *rope_positions; /* NULL: kv_positions */
    const uint32_t *kv_positions;
    const FellmRocmPagedKv *kv;
    uint32_t *err_flag;
    /* residual add + RMSNorm */
    const void *x;
    const void *residual;
    void *h_out;
    const float *norm_weight;
    uint32_t group;
    void *y;
    uint64_t norm_elems;
    float eps;
    /* SwiGLU */
    const void *gate;
    const void *up;
    void *act_out;
    uint64_t swiglu_elems;
} FellmRocmDecodeStep;

int fellm_rocm_decode_step(const FellmRocmDecodeStep *step, void *stream);

/*
 * MoE router: softmax (gating_func other than 2 and 4), sigmoid
 * (gating_func == 2) or sqrt-softplus (gating_func == 4) over each token's
 * n_experts logits, top-k by score (ties -> lower expert id),
 * optional renormalisation over the k selected, times routed_scaling_factor
 * (0 -> 1).   replaces: kernels/moe.rs:79-186 and :820-855.
 * logits f32 [tokens, n_experts] (n_experts <= 512), ids u32 [tokens, k],
 * weights f32 [tokens, k], k = min(n_expert_used, n_experts).
 * Scores use a bit-exact restatement of glibc expf and the CPU summation
 * order, so ids and weights are bit-exact with the CPU reference.
 */
int fellm_rocm_router_topk(const float *logits, uint32_t tokens, uint32_t n_experts,
                           uint32_t n_expert_used, uint32_t gating_func, uint32_t norm_topk_prob,
                           float routed_scaling_factor, uint32_t *ids, float *weights,
                           void *stream);

/*
 * Fused gate/up GEMV with the SwiGLU epilogue for one activation vector:
 * x is quantized once to Q8_K (256-element blocks: f32 scale, int8 values,
 * int16 group sums), every row of gate_w and up_w is dotted against it, and
 * out[r] = silu(gate[r]) * up[r].
 * replaces: crates/backend-cpu/src/backend.rs:944-1002 (launch_gate_up_swiglu,
 * OpKind::GateUpSwiGlu) -> kernels/matmul.rs:404-531 (matvec_quant_multi);
 * the CUDA plugin's launch_q4k_gate_up_swiglu / launch_q5k_gate_up_swiglu
 * (plugins/cuda_kernels/src/launchers.rs:1654, :1745).
 * gate_w/up_w: GGUF K-quant rows [rows, cols] of dtype 12 (Q4_K), 13 (Q5_K) or
 * 14 (Q6_K), Q4_K/Q5_K 16-byte aligned; x f32 [cols] 16-byte aligned,
 * cols % 256 == 0, cols <= 49152; out f32 [rows].
 * Integer dot products are exact; the f32 combine follows the CPU's portable
 * path (vec_dot_q4k.rs:296-333, vec_dot_q5k.rs:189-218, matmul.rs:1597-1644)
 * operation by operation.
 */
int fellm_rocm_gate_up_swiglu(const void *gate_w, uint32_t gate_dtype, const void *up_w, uint32_t up_dtype,
                              uint32_t rows, uint32_t cols, const float *x, float *out, void *stream);

/*
 * K-quant GEMV y = W x for one activation vector (same quantization and
 * arithmetic as fellm_rocm_gate_up_swiglu, no epilogue).
 * replaces: kernels/matmul.rs:534-600 (matvec_quant, Q4_K/Q5_K/Q6_K arms), the
 * rank-1 (decode) form of OpKind::MatMul [Q4K|Q5K|Q6K, F32] -> F32
 * (crates/backend-cpu/src/backend.rs:861-920, launch_matmul with rows == 1).
 */
int fellm_rocm_matvec_kquant(const void *w, uint32_t w_dtype, uint32_t rows, uint32_t cols, const float *x,
                             float *y, void *stream);

/*
 * Paged decode attention: one query token per batch row against that row's
 * paged K/V cache (the layout fellm_rocm_rope_kv_write / fellm_rocm_kv_write
 * fill).  Row b attends to keys 0 .. row_lengths[b]-1 (when causal and
 * window > 0, only the last `window` of them); query head h uses KV head
 * h / (n_heads / n_kv_heads); out = softmax(q . K^T * scale) . V with
 * scale <= 0 meaning 1/sqrt(head_dim).
 * replaces: crates/backend-cpu/src/backend.rs:1244-1368 (launch_attention, paged
 * decode arms) and the CUDA plugin's attention_paged_batch_heads /
 * attention_paged_heads paths (plugins/cuda_kernels/src/launchers.rs:3243-3560);
 * oracle crates/fellm-plugin-abi/src/attention_provider.rs:391-459.
 * q [batch, n_heads, head_dim] (F32, F16 or BF16), out same shape (the q dtype, or
 * F32); row_lengths u32 [batch] in device memory, max_seq >= every length;
 * head_dim 64, 128 or 256; n_heads / n_kv_heads <= 16; kv->block_size 16,
 * kv->stride = n_kv_heads * head_dim, kv_dtype F16 or BF16.
 * workspace: fellm_rocm_paged_attention_workspace() bytes for split-key
 * partial sums (used when batch * n_kv_heads is small; 16-byte aligned for
 * the fastest combine); with a null or short workspace every (row, KV head)
 * runs in one wavefront.
 * Products with the f16 cache are exact (q split into f16 high/low parts on
 * the matrix cores); accumulation, exp and the softmax run in f32.
 */
uint64_t fellm_rocm_paged_attention_workspace(uint32_t batch, uint32_t n_heads, uint32_t n_kv_heads,
                                              uint32_t head_dim, uint32_t max_seq);
int fellm_rocm_paged_attention(const void *q, uint32_t q_dtype, void *out, uint32_t out_dtype, uint32_t batch,
                               uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim, const uint32_t *row_lengths,
                               uint32_t max_seq, float scale, uint32_t causal, uint32_t window,
                               const FellmRocmPagedKv *kv, float *workspace, uint64_t workspace_bytes,
                               void *stream);

/*
 * Attention over f32 K/V rows stored contiguously ([t, n_kv_heads * head_dim]):
 * the non-paged arms of the Attention op.
 *   replaces: crates/backend-cpu/src/backend.rs:1371-1397 (contiguous decode:
 *   one query row, keys 0..past_len, optionally windowed) and :1412-1535
 *   (launch_canvas_attention without a paged prefix); the CUDA plugin's
 *   attention_heads / attention_canvas_heads (plugins/cuda_kernels/src/
 *   launchers.rs:3719-3760, :3270-3333; oxide_kernels.rs:3878, :4089).
 * q, out f32 [rows, n_heads, head_dim]; every query row attends, without a
 * mask, the keys t in [begin1, end1) of (k1, v1) and then t in [0, n2) of
 * (k2, v2): out = softmax(q . k * scale) . v, scale <= 0 meaning
 * 1/sqrt(head_dim); query head h uses KV head h / (n_heads / n_kv_heads).
 * No keys gives a zero row.  head_dim % 4 == 0, head_dim <= 256,
 * (n_heads / n_kv_heads) * head_dim <= 2048, 16-byte aligned buffers.
 * Accumulation and the softmax run in f32 with the device exp.
 */
int fellm_rocm_attention_f32kv(const float *q, float *out, uint32_t rows, uint32_t n_heads, uint32_t n_kv_heads,
                               uint32_t head_dim, const float *k1, const float *v1, uint32_t begin1, uint32_t end1,
                               const float *k2, const float *v2, uint32_t n2, float scale, void *stream);

/*
 * Attention of query_len rows over one contiguous f32 K/V pair of kv_len rows,
 * the CPU backend's host FA2 path for the non-paged Attention launch.
 *   replaces: backend.rs:1371-1397 -> attention_provider.rs:251-385
 *             (fa2_style_attention_f32).
 * q, out: head-major [n_heads, query_len, head_dim]; k, v: [kv_len, n_kv_heads * head_dim].
 * causal != 0: row i attends keys 0 .. kv_len - query_len + i (the last
 * `window` of them when window > 0; kv_len >= query_len).  causal == 0: keys
 * within `window` of i (|i - j| < window), every key when window == 0.
 * scale <= 0 means 1/sqrt(head_dim).  Softmax exp is the glibc-exact expf.
 */
int fellm_rocm_attention_f32kv_rows(const float *q, float *out, uint32_t query_len, uint32_t n_heads,
                                    uint32_t n_kv_heads, uint32_t head_dim, const float *k, const float *v,
                                    uint32_t kv_len, float scale, uint32_t causal, uint32_t window, void *stream);

/*
 * Cast: dst = src converted elementwise, n_elems elements.
 *   replaces: launch_cast (crates/backend-cpu/src/backend.rs:1603-1667).
 * Pairs (as the CPU backend): F32->F32, F16->F32, BF16->F32 (exact widening),
 * F32->F16 (round to nearest even), F32->BF16 (truncation: the top 16 bits),
 * Q4K/Q5K/Q6K->F32 (dequantization of the block stream, n_elems % 256 == 0,
 * dst 16-byte aligned) and Q8_0->F32 (n_elems % 32 == 0).  Other pairs return FELLM_ERR_DTYPE.
 */
int fellm_rocm_cast(const void *src, uint32_t src_dtype, void *dst, uint32_t dst_dtype, uint64_t n_elems,
                    void *stream);

/*
 * x quantized once to Q8_K for any number of K-quant GEMVs over it, as the
 * CPU backend does per matmul (matmul.rs:213-270 quantize_row_q8_k_avx2; the
 * CUDA plugin's quantize_q8_32 plays the same role for its own format).
 * The blob holds qs[cols] int8, bsums[cols / 16] int16, d[cols / 256] f32
 * (fellm_rocm_q8k_bytes(cols) = cols / 256 * 292 bytes, 16-byte aligned).
 * The _q8k GEMVs take the blob instead of x and give the same bits as
 * fellm_rocm_gate_up_swiglu / fellm_rocm_matvec_kquant on that x; their
 * workgroups copy the blob instead of quantizing x each.
 */
uint64_t fellm_rocm_q8k_bytes(uint32_t cols);
int fellm_rocm_quantize_q8k(const float *x, uint32_t cols, void *xq, void *stream);
int fellm_rocm_gate_up_swiglu_q8k(const void *gate_w, uint32_t gate_dtype, const void *up_w, uint32_t up_dtype,
                                  uint32_t rows, uint32_t cols, const void *xq, float *out, void *stream);
int fellm_rocm_matvec_kquant_q8k(const void *w, uint32_t w_dtype, uint32_t rows, uint32_t cols, const void *xq,
                                 float *y, void *stream);

/*
 * MoE dispatch: group the routed assignments a = token * top_k + slot by expert.
 *   replaces: fill_u32 + moe_count_assignments + moe_prefix_offsets +
 *             moe_scatter_assignments (plugins/cuda_kernels/src/
 *             oxide_kernels.rs:2283-2327, launched at launchers.rs:2377-2406);
 *             grouping order of crates/backend-cpu/src/kernels/moe.rs:839-848.
 * ids u32 [tokens, top_k] (device); counts u32 [n_experts]; offsets u32
 * [n_experts + 1] (exclusive prefix, offsets[n_experts] = valid assignments);
 * order u32 [A] (A = tokens * top_k): order[offsets[e] + i] is expert e's i-th
 * assignment, ascending in a (the CPU backend's order; the CUDA plugin's atomic
 * scatter leaves it unspecified); inv u32 [A] (may be NULL): inv[order[p]] = p.
 * An id >= n_experts is left out of every group (inv = 0xffffffff, the order
 * tail past offsets[n_experts] = 0xffffffff) and sets *err_flag (device u32,
 * may be NULL) to 1; the CPU reference indexes out of bounds on such ids.
 * n_experts <= 4096, top_k <= 64.  workspace: device memory of
 * fellm_rocm_moe_dispatch_workspace() bytes (0 when A <= 2048).
 */
uint64_t fellm_rocm_moe_dispatch_workspace(uint64_t tokens, uint32_t top_k, uint32_t n_experts);
int fellm_rocm_moe_dispatch(const uint32_t *ids, uint64_t tokens, uint32_t top_k, uint32_t n_experts,
                            uint32_t *counts, uint32_t *offsets, uint32_t *order, uint32_t *inv,
                            uint32_t *err_flag, void *workspace, uint64_t workspace_bytes, void *stream);

/*
 * Allocation-free MoE dispatch: fellm_rocm_moe_dispatch with the per-block
 * count buffer taken from a 4 MiB array the library keeps on each GPU
 * (fellm_rocm_moe_dispatch_noalloc_max_bytes()) instead of a workspace.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops).
 * Same arguments, results and errors as fellm_rocm_moe_dispatch; a dispatch
 * whose count buffer would exceed the array returns FELLM_ERR_SHAPE (every
 * shape the dispatch accepts fits).  It calls no allocator.  The first call
 * on a device looks the array's address up (hipGetSymbolAddress) with that
 * device current.  All calls on one GPU share the array: calls that overlap
 * on one GPU (concurrent streams or host threads) race and must be
 * serialised by the caller.  The looked-up address is kept for the process:
 * after hipDeviceReset of a device, do not call this entry point on it again.
 */
uint64_t fellm_rocm_moe_dispatch_noalloc_max_bytes(void);
int fellm_rocm_moe_dispatch_noalloc(const uint32_t *ids, uint64_t tokens, uint32_t top_k, uint32_t n_experts,
                                    uint32_t *counts, uint32_t *offsets, uint32_t *order, uint32_t *inv,
                                    uint32_t *err_flag, void *stream);

/*
 * grouped[p, :] = x[order[p] / top_k, :] for p < A (moe.rs:954-957); rows of
 * `hidden` elements of elem_bytes (1, 2 or 4) bytes, copied bit for bit.  An
 * order entry >= A (0xffffffff) gives a zero row.
 * inv (may be NULL) is the dispatch's inverse permutation; with it (and 16-byte
 * rows) each x row is read once and written to its top_k grouped positions.
 */
int fellm_rocm_moe_gather(const void *x, uint32_t elem_bytes, uint64_t tokens, uint32_t top_k, uint64_t hidden,
                          const uint32_t *order, const uint32_t *inv, void *grouped, void *stream);

/*
 * Weighted combine of the expert outputs, f32:
 *   y[t, :] = y0[t, :] (0 when y0 == NULL) + sum over t's slots of
 *             weights[t, s] * row(t, s), each step acc = acc + w * v (no FMA).
 * inv != NULL: rows are grouped, row(t, s) = expert_out[inv[t * top_k + s]],
 *   slots taken in ascending (ids[t, s], s) — crates/backend-cpu/src/kernels/
 *   moe.rs:1024-1033, which adds group by group in expert order.
 * inv == NULL: rows are per assignment, row(t, s) = expert_out[t * top_k + s],
 *   slots in order s = 0..top_k-1 — moe_weighted_reduce (oxide_kernels.rs:
 *   2507-2532, launched at launchers.rs:2228, 2533), ids unused (may be NULL).
 * y may equal y0.  A slot whose inv is 0xffffffff contributes nothing.
 */
int fellm_rocm_moe_combine(const float *y0, const float *expert_out, const uint32_t *ids, const float *weights,
                           const uint32_t *inv, uint64_t tokens, uint32_t top_k, uint64_t hidden, float *y,
                           void *stream);

/*
 * Device-resident step state (graph replay).
 *   replaces: the controlled single-row kernels of the CUDA plugin, which read
 *   DeviceStepParams (crates/fellm-plugin-abi/src/physical_plan.rs:103-128)
 *   from device memory so that a captured decode step replays with new values
 *   (oxide_kernels.rs:294-321 rope_controlled, :3578-3600 embedding rows,
 *   :4186-4223 kv_write_row, :4467 attention).
 * In the device-pointer API the block's u32 fields are themselves the device
 * arrays the kernels take: &p->token_id as ids[1], &p->position as
 * positions[1], &p->sequence_length as row_lengths[1].  The KV position of the
 * single row is written by fellm_rocm_step_kv_position:
 *   kv_pos[0] = ((sequence_length - 1) / block_size) * block_size + kv_write_slot
 * (saturating at sequence_length 0; 0xffffffff, which the KV writes reject,
 * when kv_write_slot >= block_size).
 */
int fellm_rocm_step_kv_position(const FellmDeviceStepParams *params, uint32_t block_size, uint32_t *kv_pos,
                                void *stream);

/*
 * HIP graph capture and replay on a caller stream.
 *   replaces: crates/backend-cuda/src/graph.rs (CudaGraphCapture, CudaGraphExec).
 * begin: start thread-local capture (stream must not be the null stream);
 * end: finish, instantiate and upload, returning an opaque executable;
 * abort: end an unfinished capture and drop what was recorded;
 * launch: enqueue one replay; destroy: free the executable.
 * stream_is_capturing: 1 while `stream` is capturing, 0 if not.
 * Entry points of this library enqueue kernels only (no memset, copy or
 * allocation), so any sequence of them can be captured; per-step values are
 * read from device memory at replay time.
 */
int fellm_rocm_graph_begin(void *stream);
int fellm_rocm_graph_end(void *stream, void **graph_exec);
int fellm_rocm_graph_abort(void *stream);
int fellm_rocm_graph_launch(void *graph_exec, void *stream);
void fellm_rocm_graph_destroy(void *graph_exec);
int fellm_rocm_stream_is_capturing(void *stream);

/*
 * Self-check of the device expf restatement: out[i] = expf(in[i]) on the GPU.
 * Diagnostic only (no counterpart in the reference).
 */
int fellm_rocm_expf(const float *in, float *out, uint64_t n, void *stream);

/*
 * Kernel timing (measurement only; no counterpart in the reference).
 * fellm_rocm_timing_arm(start, stop) takes two hipEvent_t handles; until
 * fellm_rocm_timing_disarm() the calling thread's launches through this
 * library record `start` at the beginning of the first kernel and `stop` at
 * the end of each kernel (hipExtLaunchKernel), so hipEventElapsedTime(start,
 * stop) is the device time of the op's kernels without marker packets in
 * between.  Not for use under graph capture.
 */
int fellm_rocm_timing_arm(void *start_event, void *stop_event);
void fellm_rocm_timing_disarm(void);

/*
 * Streaming probe (measurement only; no counterpart in the reference):
 * reads read_bytes from a (and as many from b when b != NULL) and writes
 * write_bytes to out (a ^ b where both were read), no arithmetic; sizes are
 * multiples of 16 and buffers 16-byte aligned.  It moves an op's read and
 * write bytes with nothing else: the ceiling the bench compares the op
 * against.  variant bits 0-1: 16-byte units per thread (0, 1: one; 2: two;
 * 3: four), bit 2: non-temporal loads and stores.
 */
int fellm_rocm_stream_probe(const void *a, const void *b, uint64_t read_bytes, void *out, uint64_t write_bytes,
                            uint32_t variant, void *stream);

/*
 * Self-check of the device sinf/cosf restatement that builds RoPE's per-row
 * (sin, cos) table: sin_out[i] = sinf(in[i]), cos_out[i] = cosf(in[i]).
 * Diagnostic only (no counterpart in the reference).
 */
int fellm_rocm_sincosf(const float *in, float *sin_out, float *cos_out, uint64_t n, void *stream);

/*
 * Self-check of the device logf restatement (fn 0) and correctly rounded
 * sqrtf (fn 1) used by the router's sqrt-softplus gating: out[i] =
 * logf(in[i]) or sqrtf(in[i]); fn 2: the bf16 activation store of in[i]
 * (round to nearest even), its 16 bits returned in the low half of out[i]'s
 * bit pattern; fn 3: the router's branch-free expf for in[i] <= 0 or NaN
 * (other inputs: unspecified); fn 4: in[i] rounded to f16 by the packed
 * conversion (low half of out[i]'s bits) and by the scalar conversion of the
 * f16 activation store (high half).  Diagnostic only (no counterpart in the
 * reference).
 */
int fellm_rocm_mathf(uint32_t fn, const float *in, float *out, uint64_t n, void *stream);

/*
 * Verification hook for fellm_rocm_silu_gate's 16-bit output path (no
 * counterpart in the reference).  That path skips the exact silu when an
 * interval of +-fellm_rocm_silu_fast_dist() steps around a fast f32 silu
 * already fixes the rounded output.  fellm_rocm_silu_fast_bound atomically
 * raises *max_dist (device u32, caller zeroes it) to the largest bit distance
 * between the fast and the exact silu over every f32 gate value of the fast
 * domain (2^-100 <= |g| < 64).  The path is bit-exact iff that maximum does
 * not exceed fellm_rocm_silu_fast_dist().
 */
int fellm_rocm_silu_fast_bound(uint32_t *max_dist, void *stream);
uint32_t fellm_rocm_silu_fast_dist(void);

#ifdef __cplusplus
}
#endif
#endif /* FELLM_ROCM_H */
