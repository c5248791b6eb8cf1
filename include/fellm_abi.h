/*
 * fellm_abi.h — C mirror of FeLLM's dynamic-plugin ABI (version 0.9.0).
 *
 * Every struct here is byte-for-byte the `#[repr(C)]` layout the FeLLM plugin
 * host passes across `dlopen`; the static asserts below pin each offset.
 *
 *   TensorRef / TensorMut   crates/fellm-plugin-abi/src/tensor_ref.rs:14-53
 *   OpAttrs                 crates/fellm-plugin-abi/src/op.rs:145-216
 *   OpKind raw values       crates/fellm-plugin-abi/src/op.rs:19-62, custom :69-80
 *   AbiVersion              crates/fellm-plugin-abi/src/lib.rs (ABI_VERSION 0.9.0)
 *   HostContext             crates/fellm-plugin-abi/src/c_abi.rs:29-45
 *   PluginManifestJson      crates/fellm-plugin-abi/src/c_abi.rs:80-86
 *   PluginLaunchFn          crates/fellm-plugin-abi/src/c_abi.rs:91-98
 *   PluginOpRegistration    crates/fellm-plugin-abi/src/c_abi.rs:102-113
 *   KernelRegistryVtable    crates/fellm-plugin-abi/src/c_abi.rs:115-122
 *   PagedKvSnapshot         crates/fellm-plugin-abi/src/paged_ctx.rs:14-53
 *   DeviceStepParams        crates/fellm-plugin-abi/src/physical_plan.rs:103-128
 *   DType codes             crates/fellm-core/src/dtype.rs:10-86
 *
 * Plugin entry points exported by libfellm_rocm_kernels.so (symbol names from
 * crates/fellm-plugin-abi/src/c_abi.rs:319-350).  They replace the exports of
 * plugins/cuda_kernels/src/lib.rs:96-751 for the ops this library implements.
 */
#ifndef FELLM_ABI_H
#define FELLM_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- DType (ggml codes) ------------------------------------------------- */
enum {
    FELLM_DTYPE_F32 = 0,
    FELLM_DTYPE_F16 = 1,
    FELLM_DTYPE_Q4_0 = 2,
    FELLM_DTYPE_Q5_0 = 6,
    FELLM_DTYPE_Q8_0 = 8,
    FELLM_DTYPE_Q4K = 12,
    FELLM_DTYPE_Q5K = 13,
    FELLM_DTYPE_Q6K = 14,
    FELLM_DTYPE_I32 = 26,
    FELLM_DTYPE_BF16 = 30,
    FELLM_DTYPE_U8 = 200,
    FELLM_DTYPE_U32 = 202,
};

/* ---- OpKind raw values (built-ins) -------------------------------------- */
enum {
    FELLM_OP_ADD = 0,
    FELLM_OP_MUL = 1,
    FELLM_OP_MATMUL = 2,
    FELLM_OP_RMSNORM = 3,
    FELLM_OP_ROPE = 4,
    FELLM_OP_SILU_GATE = 5,
    FELLM_OP_SOFTMAX = 6,
    FELLM_OP_ATTENTION = 7,
    FELLM_OP_EMBEDDING = 8,
    FELLM_OP_CONCAT = 9,
    FELLM_OP_RESHAPE = 10,
    FELLM_OP_CAST = 11,
    FELLM_OP_SAMPLE = 12,
    FELLM_OP_KV_WRITE = 13,
    FELLM_OP_MOE = 15,
    FELLM_OP_GATE_UP_SWIGLU = 17,
};
/* OpKind::custom(ns, name) = FNV-1a-32 over "ns:name", OR 0x8000_0000. */
#define FELLM_OP_CUSTOM_TAG 0x80000000u

#define FELLM_ABI_MAX_RANK 5
#define FELLM_PLUGIN_NAME_MAX 64
#define FELLM_PLUGIN_MAX_INPUT_DTYPES 16

typedef uint64_t FellmStreamHandle;

typedef struct FellmAbiVersion {
    uint16_t major;
    uint16_t minor;
    uint16_t patch;
} FellmAbiVersion;

typedef struct FellmTensorRef {
    uint64_t logical_id;
    uint32_t dtype;
    uint32_t rank;
    uint64_t dims[FELLM_ABI_MAX_RANK];
    uint64_t strides[FELLM_ABI_MAX_RANK];
    const uint8_t *data;
    uint64_t byte_len;
} FellmTensorRef;

typedef struct FellmTensorMut {
    uint32_t dtype;
    uint32_t rank;
    uint64_t dims[FELLM_ABI_MAX_RANK];
    uint64_t strides[FELLM_ABI_MAX_RANK];
    uint8_t *data;
    uint64_t byte_len;
} FellmTensorMut;

typedef struct FellmOpAttrs {
    float eps;
    float rope_base;
    uint32_t rope_dim;
    uint32_t rope_pairing;
    uint32_t n_heads;
    uint32_t n_kv_heads;
    uint32_t head_dim;
    uint32_t position;
    uint32_t past_len;
    float scale;
    uint32_t cast_to;
    float temperature;
    uint32_t top_k;
    float top_p;
    uint64_t seed;
    uint32_t n_experts;
    uint32_t n_expert_used;
    uint32_t expert_gating_func;
    float routed_scaling_factor;
    uint32_t norm_topk_prob;
    uint32_t shortconv_l_cache;
    uint32_t n_embd;
    uint32_t block_size;
    uint32_t kv_slot;
    uint32_t layer_ord;
    uint32_t attention_mode;
    uint32_t attention_window;
    uint32_t query_len;
    uint32_t kv_len;
    uint32_t prefix_len;
    float softcap;
    uint32_t custom_op_id;
    uint32_t gdn_inner_size;
    uint32_t gdn_state_size;
    uint32_t gdn_conv_kernel;
} FellmOpAttrs;

typedef struct FellmPagedKvSnapshot {
    uint8_t *arena;
    size_t arena_len;
    const uint32_t *block_table;
    size_t n_block_table;
    size_t n_logical_blocks;
    size_t n_layers;
    size_t tokens_stride;
    size_t block_bytes;
    size_t block_size;
    size_t elem_bytes;
    uint8_t *device_arena;
    size_t device_arena_len;
    uint32_t *device_block_table;
    size_t n_device_block_table;
    size_t device_logical_stride;
    size_t batch_size;
    const uint32_t *row_positions;
    const uint32_t *row_lengths;
    const uint32_t *row_rope_positions;
} FellmPagedKvSnapshot;

/* Returns 0 if a context is installed, 1 if none, negative on error. */
typedef int (*FellmHostSnapshotPagedFn)(FellmPagedKvSnapshot *out);

typedef struct FellmHostContext {
    FellmAbiVersion abi_version;
    uint64_t device_handle;
    FellmStreamHandle default_stream;
    void *allocator_opaque;
    char backend_id[FELLM_PLUGIN_NAME_MAX];
    FellmHostSnapshotPagedFn snapshot_paged; /* nullable (Option<fn>) */
} FellmHostContext;

typedef struct FellmPluginManifestJson {
    const uint8_t *ptr;
    size_t len;
} FellmPluginManifestJson;

typedef int (*FellmPluginLaunchFn)(const FellmOpAttrs *attrs, const FellmTensorRef *inputs,
                                   uint32_t n_inputs, FellmTensorMut *outputs,
                                   uint32_t n_outputs, FellmStreamHandle stream);

typedef struct FellmPluginOpRegistration {
    uint32_t op_kind;
    uint32_t n_input_dtypes;
    uint32_t input_dtypes[FELLM_PLUGIN_MAX_INPUT_DTYPES];
    uint32_t output_dtype;
    FellmPluginLaunchFn launch; /* nullable (Option<fn>) */
} FellmPluginOpRegistration;

typedef struct FellmKernelRegistryVtable {
    void *registry;
    int (*register_op)(void *registry, const FellmPluginOpRegistration *reg);
} FellmKernelRegistryVtable;

typedef struct __attribute__((aligned(16))) FellmDeviceStepParams {
    uint32_t token_id;
    uint32_t position;
    uint32_t sequence_length;
    uint32_t active_batch;
    uint32_t kv_write_block;
    uint32_t kv_write_slot;
    float temperature;
    float top_p;
    uint32_t top_k;
    uint32_t recent_count;
    uint64_t seed;
} FellmDeviceStepParams;

/* ---- Launch return codes (plugins/cuda_kernels/src/launchers.rs, lib.rs) -- */
enum {
    FELLM_OK = 0,
    FELLM_ERR_ARITY = -1,         /* null pointer / wrong input-output count   */
    FELLM_ERR_SHAPE = -2,         /* shape, byte_len or attribute mismatch      */
    FELLM_ERR_ALLOC = -3,         /* device allocation or H2D/D2H copy failed  */
    FELLM_ERR_LAUNCH = -4,        /* kernel launch failed                       */
    FELLM_ERR_DTYPE = -10,        /* unsupported dtype / mode                   */
    FELLM_ERR_PAGED_MISSING = -20,/* paged KV write without a host snapshot     */
    FELLM_ERR_PAGED_NO_DEVICE = -21, /* snapshot has no device arena            */
    FELLM_ERR_PAGED_RANGE = -22,  /* slot address outside the arena / table     */
    FELLM_ERR_LOCK = -30,
    FELLM_ERR_PANIC = -99,        /* exception caught at the FFI boundary       */
};

/* ---- Plugin exports ------------------------------------------------------ */
/* c_abi.rs:319-350; cuda_kernels/src/lib.rs:296-298 */
FellmAbiVersion _fellm_plugin_abi_version(void);
/* cuda_kernels/src/lib.rs:300-321 */
FellmPluginManifestJson _fellm_plugin_manifest_json(void);
/* cuda_kernels/src/lib.rs:323-335 */
int _fellm_plugin_init(const FellmHostContext *ctx);
/* cuda_kernels/src/lib.rs:337-720 */
int _fellm_plugin_register_kernels(FellmKernelRegistryVtable *registry);
/* cuda_kernels/src/lib.rs:746-751 */
void _fellm_plugin_shutdown(void);
/* cuda_kernels/src/lib.rs:722-744 (any dtype: key is (ptr, nbytes)) */
void _fellm_plugin_invalidate_f32(const float *ptr, size_t nbytes);
/* cuda_kernels/src/lib.rs:96-100 — returns the plugin's hipStream_t as u64 */
FellmStreamHandle _fellm_plugin_device_stream(void);
/* cuda_kernels/src/lib.rs:104-134 */
int _fellm_plugin_update_step_params(const FellmDeviceStepParams *params);
/* cuda_kernels/src/lib.rs:137-148 */
int _fellm_plugin_register_device_tensor(const uint8_t *host_ptr, size_t nbytes,
                                         uint64_t device_ptr);

/* ---- Layout pins --------------------------------------------------------- */
#ifdef __cplusplus
#define FELLM_STATIC_ASSERT static_assert
#else
#define FELLM_STATIC_ASSERT _Static_assert
#endif
FELLM_STATIC_ASSERT(sizeof(FellmAbiVersion) == 6, "AbiVersion");
FELLM_STATIC_ASSERT(sizeof(FellmTensorRef) == 112, "TensorRef size");
FELLM_STATIC_ASSERT(offsetof(FellmTensorRef, dtype) == 8, "TensorRef.dtype");
FELLM_STATIC_ASSERT(offsetof(FellmTensorRef, dims) == 16, "TensorRef.dims");
FELLM_STATIC_ASSERT(offsetof(FellmTensorRef, strides) == 56, "TensorRef.strides");
FELLM_STATIC_ASSERT(offsetof(FellmTensorRef, data) == 96, "TensorRef.data");
FELLM_STATIC_ASSERT(offsetof(FellmTensorRef, byte_len) == 104, "TensorRef.byte_len");
FELLM_STATIC_ASSERT(sizeof(FellmTensorMut) == 104, "TensorMut size");
FELLM_STATIC_ASSERT(offsetof(FellmTensorMut, data) == 88, "TensorMut.data");
FELLM_STATIC_ASSERT(offsetof(FellmTensorMut, byte_len) == 96, "TensorMut.byte_len");
FELLM_STATIC_ASSERT(sizeof(FellmOpAttrs) == 144, "OpAttrs size");
FELLM_STATIC_ASSERT(offsetof(FellmOpAttrs, seed) == 56, "OpAttrs.seed");
FELLM_STATIC_ASSERT(offsetof(FellmOpAttrs, block_size) == 92, "OpAttrs.block_size");
FELLM_STATIC_ASSERT(offsetof(FellmOpAttrs, kv_slot) == 96, "OpAttrs.kv_slot");
FELLM_STATIC_ASSERT(offsetof(FellmOpAttrs, layer_ord) == 100, "OpAttrs.layer_ord");
FELLM_STATIC_ASSERT(offsetof(FellmOpAttrs, custom_op_id) == 128, "OpAttrs.custom_op_id");
FELLM_STATIC_ASSERT(sizeof(FellmPagedKvSnapshot) == 152, "PagedKvSnapshot size");
FELLM_STATIC_ASSERT(offsetof(FellmPagedKvSnapshot, device_arena) == 80, "snapshot.device_arena");
FELLM_STATIC_ASSERT(offsetof(FellmPagedKvSnapshot, batch_size) == 120, "snapshot.batch_size");
FELLM_STATIC_ASSERT(offsetof(FellmPagedKvSnapshot, row_rope_positions) == 144, "snapshot.rope_pos");
FELLM_STATIC_ASSERT(sizeof(FellmHostContext) == 104, "HostContext size");
FELLM_STATIC_ASSERT(offsetof(FellmHostContext, device_handle) == 8, "HostContext.device_handle");
FELLM_STATIC_ASSERT(offsetof(FellmHostContext, backend_id) == 32, "HostContext.backend_id");
FELLM_STATIC_ASSERT(offsetof(FellmHostContext, snapshot_paged) == 96, "HostContext.snapshot");
FELLM_STATIC_ASSERT(sizeof(FellmPluginOpRegistration) == 88, "PluginOpRegistration size");
FELLM_STATIC_ASSERT(offsetof(FellmPluginOpRegistration, output_dtype) == 72, "reg.output_dtype");
FELLM_STATIC_ASSERT(offsetof(FellmPluginOpRegistration, launch) == 80, "reg.launch");
FELLM_STATIC_ASSERT(sizeof(FellmDeviceStepParams) == 48, "DeviceStepParams size");

#ifdef __cplusplus
}
#endif
#endif /* FELLM_ABI_H */
