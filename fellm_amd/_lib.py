"""Loads libfellm_rocm_kernels.so and declares its C entry points.

There is no fallback: if the library is missing, every op raises.  The
library is loaded after ``torch`` when torch is importable, so both share
one HIP runtime (they carry the same SONAME, libamdhip64.so.7).
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

from . import abi

# FELLM_ROCM_LIB overrides the library path (e.g. to compare builds).
LIB_PATH = Path(os.environ.get("FELLM_ROCM_LIB") or Path(__file__).resolve().parent / "libfellm_rocm_kernels.so")

_lib: C.CDLL | None = None

P = C.c_void_p
U32 = C.c_uint32
U64 = C.c_uint64
F32 = C.c_float
I32 = C.c_int


class FellmRocmPagedKv(C.Structure):
    """Mirror of FellmRocmPagedKv (include/fellm_rocm.h)."""

    _fields_ = [
        ("arena", P),
        ("arena_len", U64),
        ("block_table", P),
        ("n_block_table", U64),
        ("n_logical_blocks", U32),
        ("n_layers", U32),
        ("layer", U32),
        ("block_size", U32),
        ("block_bytes", U64),
        ("stride", U32),
        ("kv_dtype", U32),
    ]


class FellmRocmDecodeStep(C.Structure):
    """Mirror of FellmRocmDecodeStep (include/fellm_rocm.h)."""

    _fields_ = [
        ("act_dtype", U32),
        ("q", P), ("q_out", P), ("n_q_heads", U32), ("k", P), ("k_out", P), ("v", P), ("n_kv_heads", U32),
        ("batch", U32), ("head_dim", U32), ("rope_dim", U32), ("pairing", U32), ("inv_freqs", P),
        ("rope_positions", P), ("kv_positions", P), ("kv", C.POINTER(FellmRocmPagedKv)), ("err_flag", P),
        ("x", P), ("residual", P), ("h_out", P), ("norm_weight", P), ("group", U32), ("y", P), ("norm_elems", U64),
        ("eps", F32),
        ("gate", P), ("up", P), ("act_out", P), ("swiglu_elems", U64),
    ]


_SIGNATURES = {
    "fellm_rocm_version": (C.c_char_p, []),
    "fellm_rocm_add_rmsnorm": (I32, [P, P, P, U32, P, U32, P, U32, U64, F32, P]),
    "fellm_rocm_silu_gate": (I32, [P, P, U32, P, U32, U64, P]),
    "fellm_rocm_add": (I32, [P, P, U32, P, U32, U64, P]),
    "fellm_rocm_embedding": (I32, [P, U32, U64, U32, P, U32, P, U32, P, P]),
    "fellm_rocm_embedding_rmsnorm": (I32, [P, U32, U64, U32, P, U32, P, F32, P, P, U32, P, P]),
    "fellm_rocm_rope": (I32, [P, P, U32, P, P, U32, U32, U32, U32, U32, U32, P, P, U32, P]),
    "fellm_rocm_kv_write": (I32, [P, U32, U32, P, C.POINTER(FellmRocmPagedKv), U32, P, P]),
    "fellm_rocm_rope_kv_write": (
        I32,
        [P, P, U32, P, P, P, U32, U32, U32, U32, U32, U32, P, P, P, C.POINTER(FellmRocmPagedKv), P, P],
    ),
    "fellm_rocm_router_topk": (I32, [P, U32, U32, U32, U32, U32, F32, P, P, P]),
    "fellm_rocm_expf": (I32, [P, P, U64, P]),
    "fellm_rocm_sincosf": (I32, [P, P, P, U64, P]),
    "fellm_rocm_mathf": (I32, [U32, P, P, U64, P]),
    "fellm_rocm_timing_arm": (I32, [P, P]),
    "fellm_rocm_attention_f32kv": (I32, [P, P, U32, U32, U32, U32, P, P, U32, U32, P, P, U32, F32, P]),
    "fellm_rocm_attention_f32kv_rows": (I32, [P, P, U32, U32, U32, U32, P, P, U32, F32, U32, U32, P]),
    "fellm_rocm_decode_step": (I32, [C.POINTER(FellmRocmDecodeStep), P]),
    "fellm_rocm_stream_probe": (I32, [P, P, U64, P, U64, U32, P]),
    "fellm_rocm_timing_disarm": (None, []),
    "fellm_rocm_silu_fast_bound": (I32, [P, P]),
    "fellm_rocm_silu_fast_dist": (U32, []),
    "fellm_rocm_gate_up_swiglu": (I32, [P, U32, P, U32, U32, U32, P, P, P]),
    "fellm_rocm_matvec_kquant": (I32, [P, U32, U32, U32, P, P, P]),
    "fellm_rocm_paged_attention_workspace": (U64, [U32, U32, U32, U32, U32]),
    "fellm_rocm_paged_attention": (I32, [P, U32, P, U32, U32, U32, U32, U32, P, U32, F32, U32, U32,
                                         C.POINTER(FellmRocmPagedKv), P, U64, P]),
    "fellm_rocm_cast": (I32, [P, U32, P, U32, U64, P]),
    "fellm_rocm_q8k_bytes": (U64, [U32]),
    "fellm_rocm_quantize_q8k": (I32, [P, U32, P, P]),
    "fellm_rocm_gate_up_swiglu_q8k": (I32, [P, U32, P, U32, U32, U32, P, P, P]),
    "fellm_rocm_matvec_kquant_q8k": (I32, [P, U32, U32, U32, P, P, P]),
    "fellm_rocm_moe_dispatch_workspace": (U64, [U64, U32, U32]),
    "fellm_rocm_moe_dispatch": (I32, [P, U64, U32, U32, P, P, P, P, P, P, U64, P]),
    "fellm_rocm_moe_dispatch_noalloc_max_bytes": (U64, []),
    "fellm_rocm_moe_dispatch_noalloc": (I32, [P, U64, U32, U32, P, P, P, P, P, P]),
    "fellm_rocm_moe_gather": (I32, [P, U32, U64, U32, U64, P, P, P, P]),
    "fellm_rocm_moe_combine": (I32, [P, P, P, P, P, U64, U32, U64, P, P]),
    "fellm_rocm_step_kv_position": (I32, [P, U32, P, P]),
    "fellm_rocm_graph_begin": (I32, [P]),
    "fellm_rocm_graph_end": (I32, [P, P]),
    "fellm_rocm_graph_abort": (I32, [P]),
    "fellm_rocm_graph_launch": (I32, [P, P]),
    "fellm_rocm_graph_destroy": (None, [P]),
    "fellm_rocm_stream_is_capturing": (I32, [P]),
    # plugin ABI
    "_fellm_plugin_abi_version": (abi.AbiVersion, []),
    "_fellm_plugin_manifest_json": (abi.PluginManifestJson, []),
    "_fellm_plugin_init": (I32, [C.POINTER(abi.HostContext)]),
    "_fellm_plugin_register_kernels": (I32, [C.POINTER(abi.KernelRegistryVtable)]),
    "_fellm_plugin_shutdown": (None, []),
    "_fellm_plugin_invalidate_f32": (None, [P, C.c_size_t]),
    "_fellm_plugin_device_stream": (U64, []),
    "_fellm_plugin_update_step_params": (I32, [C.POINTER(abi.DeviceStepParams)]),
    "_fellm_plugin_register_device_tensor": (I32, [P, C.c_size_t, U64]),
}

EXPORTED = tuple(_SIGNATURES)


class FellmRocmError(RuntimeError):
    def __init__(self, fn: str, code: int):
        super().__init__(f"{fn} failed with code {code}")
        self.fn = fn
        self.code = code


def lib() -> C.CDLL:
    """The loaded kernel library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m fellm_amd.build`")
        try:  # share torch's HIP runtime when torch is present
            import torch  # noqa: F401
        except ImportError:
            pass
        handle = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def call(name: str, *args) -> None:
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        raise FellmRocmError(name, rc)
