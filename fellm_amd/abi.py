"""ctypes mirror of FeLLM's plugin ABI (include/fellm_abi.h).

Struct layouts are the ``#[repr(C)]`` types of crates/fellm-plugin-abi:
TensorRef/TensorMut (src/tensor_ref.rs:14-53), OpAttrs (src/op.rs:145-216),
PagedKvSnapshot (src/paged_ctx.rs:14-53), HostContext (src/c_abi.rs:29-45),
PluginOpRegistration (src/c_abi.rs:102-113), KernelRegistryVtable
(src/c_abi.rs:115-122), DeviceStepParams (src/physical_plan.rs:103-128).
"""
from __future__ import annotations

import ctypes as C
from enum import IntEnum

ABI_MAX_RANK = 5
PLUGIN_NAME_MAX = 64
PLUGIN_MAX_INPUT_DTYPES = 16
ABI_VERSION = (0, 9, 0)


class DType(IntEnum):
    """ggml dtype codes (crates/fellm-core/src/dtype.rs:10-86)."""

    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q5_0 = 6
    Q8_0 = 8
    Q4K = 12
    Q5K = 13
    Q6K = 14
    I32 = 26
    BF16 = 30
    U8 = 200
    U32 = 202


class OpKind(IntEnum):
    """Built-in OpKind raw values (crates/fellm-plugin-abi/src/op.rs:19-62)."""

    ADD = 0
    MUL = 1
    MATMUL = 2
    RMSNORM = 3
    ROPE = 4
    SILU_GATE = 5
    SOFTMAX = 6
    ATTENTION = 7
    EMBEDDING = 8
    CONCAT = 9
    RESHAPE = 10
    CAST = 11
    SAMPLE = 12
    KV_WRITE = 13
    MOE = 15
    GATE_UP_SWIGLU = 17


def custom_op(namespace: str, name: str) -> int:
    """OpKind::custom: FNV-1a-32 over ``ns:name``, tagged 0x8000_0000 (op.rs:69-80)."""
    h = 0x811C9DC5
    for b in namespace.encode() + b":" + name.encode():
        h ^= b
        h = (h * 0x01000193) & 0xFFFFFFFF
    return h | 0x80000000


OP_ADD_RMSNORM = custom_op("rocm", "add_rmsnorm")
OP_ROPE_KV_WRITE = custom_op("rocm", "rope_kv_write")
OP_ROUTER_TOPK = custom_op("rocm", "router_topk")
OP_EMBEDDING_RMSNORM = custom_op("rocm", "embedding_rmsnorm")


class AbiVersion(C.Structure):
    _fields_ = [("major", C.c_uint16), ("minor", C.c_uint16), ("patch", C.c_uint16)]


class TensorRef(C.Structure):
    _fields_ = [
        ("logical_id", C.c_uint64),
        ("dtype", C.c_uint32),
        ("rank", C.c_uint32),
        ("dims", C.c_uint64 * ABI_MAX_RANK),
        ("strides", C.c_uint64 * ABI_MAX_RANK),
        ("data", C.c_void_p),
        ("byte_len", C.c_uint64),
    ]


class TensorMut(C.Structure):
    _fields_ = [
        ("dtype", C.c_uint32),
        ("rank", C.c_uint32),
        ("dims", C.c_uint64 * ABI_MAX_RANK),
        ("strides", C.c_uint64 * ABI_MAX_RANK),
        ("data", C.c_void_p),
        ("byte_len", C.c_uint64),
    ]


class OpAttrs(C.Structure):
    _fields_ = [
        ("eps", C.c_float),
        ("rope_base", C.c_float),
        ("rope_dim", C.c_uint32),
        ("rope_pairing", C.c_uint32),
        ("n_heads", C.c_uint32),
        ("n_kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32),
        ("position", C.c_uint32),
        ("past_len", C.c_uint32),
        ("scale", C.c_float),
        ("cast_to", C.c_uint32),
        ("temperature", C.c_float),
        ("top_k", C.c_uint32),
        ("top_p", C.c_float),
        ("seed", C.c_uint64),
        ("n_experts", C.c_uint32),
        ("n_expert_used", C.c_uint32),
        ("expert_gating_func", C.c_uint32),
        ("routed_scaling_factor", C.c_float),
        ("norm_topk_prob", C.c_uint32),
        ("shortconv_l_cache", C.c_uint32),
        ("n_embd", C.c_uint32),
        ("block_size", C.c_uint32),
        ("kv_slot", C.c_uint32),
        ("layer_ord", C.c_uint32),
        ("attention_mode", C.c_uint32),
        ("attention_window", C.c_uint32),
        ("query_len", C.c_uint32),
        ("kv_len", C.c_uint32),
        ("prefix_len", C.c_uint32),
        ("softcap", C.c_float),
        ("custom_op_id", C.c_uint32),
        ("gdn_inner_size", C.c_uint32),
        ("gdn_state_size", C.c_uint32),
        ("gdn_conv_kernel", C.c_uint32),
    ]


class PagedKvSnapshot(C.Structure):
    _fields_ = [
        ("arena", C.c_void_p),
        ("arena_len", C.c_size_t),
        ("block_table", C.c_void_p),
        ("n_block_table", C.c_size_t),
        ("n_logical_blocks", C.c_size_t),
        ("n_layers", C.c_size_t),
        ("tokens_stride", C.c_size_t),
        ("block_bytes", C.c_size_t),
        ("block_size", C.c_size_t),
        ("elem_bytes", C.c_size_t),
        ("device_arena", C.c_void_p),
        ("device_arena_len", C.c_size_t),
        ("device_block_table", C.c_void_p),
        ("n_device_block_table", C.c_size_t),
        ("device_logical_stride", C.c_size_t),
        ("batch_size", C.c_size_t),
        ("row_positions", C.c_void_p),
        ("row_lengths", C.c_void_p),
        ("row_rope_positions", C.c_void_p),
    ]


SnapshotPagedFn = C.CFUNCTYPE(C.c_int, C.POINTER(PagedKvSnapshot))


class HostContext(C.Structure):
    _fields_ = [
        ("abi_version", AbiVersion),
        ("device_handle", C.c_uint64),
        ("default_stream", C.c_uint64),
        ("allocator_opaque", C.c_void_p),
        ("backend_id", C.c_char * PLUGIN_NAME_MAX),
        ("snapshot_paged", SnapshotPagedFn),
    ]


class PluginManifestJson(C.Structure):
    _fields_ = [("ptr", C.c_void_p), ("len", C.c_size_t)]


PluginLaunchFn = C.CFUNCTYPE(
    C.c_int, C.POINTER(OpAttrs), C.POINTER(TensorRef), C.c_uint32, C.POINTER(TensorMut), C.c_uint32, C.c_uint64
)


class PluginOpRegistration(C.Structure):
    _fields_ = [
        ("op_kind", C.c_uint32),
        ("n_input_dtypes", C.c_uint32),
        ("input_dtypes", C.c_uint32 * PLUGIN_MAX_INPUT_DTYPES),
        ("output_dtype", C.c_uint32),
        ("launch", C.c_void_p),
    ]


RegisterOpFn = C.CFUNCTYPE(C.c_int, C.c_void_p, C.POINTER(PluginOpRegistration))


class KernelRegistryVtable(C.Structure):
    _fields_ = [("registry", C.c_void_p), ("register_op", RegisterOpFn)]


class DeviceStepParams(C.Structure):
    _pack_ = 8
    _fields_ = [
        ("token_id", C.c_uint32),
        ("position", C.c_uint32),
        ("sequence_length", C.c_uint32),
        ("active_batch", C.c_uint32),
        ("kv_write_block", C.c_uint32),
        ("kv_write_slot", C.c_uint32),
        ("temperature", C.c_float),
        ("top_p", C.c_float),
        ("top_k", C.c_uint32),
        ("recent_count", C.c_uint32),
        ("seed", C.c_uint64),
    ]


# Expected sizes, the same numbers the C header pins with static asserts.
LAYOUT = {
    "TensorRef": (TensorRef, 112),
    "TensorMut": (TensorMut, 104),
    "OpAttrs": (OpAttrs, 144),
    "PagedKvSnapshot": (PagedKvSnapshot, 152),
    "HostContext": (HostContext, 104),
    "PluginOpRegistration": (PluginOpRegistration, 88),
    "DeviceStepParams": (DeviceStepParams, 48),
    "AbiVersion": (AbiVersion, 6),
}

# Launch return codes (plugins/cuda_kernels/src/launchers.rs, lib.rs).
ERR_ARITY = -1
ERR_SHAPE = -2
ERR_ALLOC = -3
ERR_LAUNCH = -4
ERR_DTYPE = -10
ERR_PAGED_MISSING = -20
ERR_PAGED_NO_DEVICE = -21
ERR_PAGED_RANGE = -22
ERR_PANIC = -99


def tensor_ref(data_ptr: int, byte_len: int, dtype: int, dims, logical_id: int = 0) -> TensorRef:
    """Row-major TensorRef over ``byte_len`` bytes at ``data_ptr``."""
    t = TensorRef()
    t.logical_id = logical_id
    t.dtype = int(dtype)
    t.rank = len(dims)
    stride = 1
    strides = []
    for d in reversed(dims):
        strides.append(stride)
        stride *= int(d)
    for i, (d, s) in enumerate(zip(dims, reversed(strides))):
        t.dims[i] = int(d)
        t.strides[i] = s
    t.data = data_ptr
    t.byte_len = byte_len
    return t


def tensor_mut(data_ptr: int, byte_len: int, dtype: int, dims) -> TensorMut:
    r = tensor_ref(data_ptr, byte_len, dtype, dims)
    t = TensorMut()
    t.dtype, t.rank = r.dtype, r.rank
    for i in range(ABI_MAX_RANK):
        t.dims[i] = r.dims[i]
        t.strides[i] = r.strides[i]
    t.data, t.byte_len = r.data, r.byte_len
    return t
