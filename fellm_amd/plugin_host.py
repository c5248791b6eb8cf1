"""Python restatement of fellm-plugin-host for the kernel plugin.

Follows crates/fellm-plugin-host/src/loader.rs:357-437 (activate_path:
dlopen, verify_abi, read_manifest, init, register_kernels, optional symbols)
and src/registry.rs:160-240 (KernelRegistry::register / lookup / launch,
exact-match keys (op, input dtypes, output dtype), nonzero launch return
codes become errors).  The host owns the paged-KV context and hands the
plugin a snapshot callback, as crates/fellm-plugin-abi/src/paged_ctx.rs:55-95
does with its process-wide PAGED_CTX.
"""
from __future__ import annotations

import ctypes as C
import json
from dataclasses import dataclass, field
from pathlib import Path

from . import abi
from ._lib import LIB_PATH


class PluginError(RuntimeError):
    def __init__(self, msg: str, code: int | None = None):
        super().__init__(msg)
        self.code = code


@dataclass
class PagedKvContext:
    """Host-side paged context (paged_ctx.rs:178-215).  Arrays are kept alive here."""

    arena_ptr: int
    arena_len: int
    block_table: "object"          # numpy uint32 array, host
    n_logical_blocks: int
    n_layers: int
    tokens_stride: int
    block_bytes: int
    block_size: int
    row_positions: "object"        # numpy uint32 [batch]
    row_rope_positions: "object"   # numpy uint32 [batch]
    row_lengths: "object" = None
    device_arena_ptr: int = 0
    device_arena_len: int = 0
    elem_bytes: int = 2
    device_block_table_ptr: int = 0     # device u32 table (engine.rs:3060-3087), 0 = none
    n_device_block_table: int = 0
    device_logical_stride: int = 0


@dataclass
class Registration:
    op: int
    input_dtypes: tuple
    output_dtype: int
    launch_ptr: int


@dataclass
class KernelRegistry:
    entries: dict = field(default_factory=dict)   # key -> Registration
    by_handle: dict = field(default_factory=dict)  # handle -> key
    next_handle: int = 1

    def register(self, reg: abi.PluginOpRegistration) -> int:
        op = reg.op_kind
        if not (op <= 22 or op & 0x80000000):  # OpKind::from_u32
            return -1
        if not reg.launch:
            return -2
        n = reg.n_input_dtypes
        if n > abi.PLUGIN_MAX_INPUT_DTYPES:
            return -3
        key = (op, tuple(reg.input_dtypes[:n]), reg.output_dtype)
        handle = self.next_handle
        self.next_handle += 1
        self.by_handle[handle] = key
        self.entries[key] = Registration(op, key[1], key[2], reg.launch)
        return 0

    def lookup(self, op: int, input_dtypes, output_dtype: int) -> int | None:
        key = (int(op), tuple(int(d) for d in input_dtypes), int(output_dtype))
        if key not in self.entries:
            return None
        for h, k in self.by_handle.items():
            if k == key:
                return h
        return None


def validate_manifest(m: dict) -> None:
    """V1 manifest rules of crates/fellm-plugin-host/src/manifest.rs:110-165."""
    schema = m.get("schema", m.get("schema_version"))
    if schema is None:
        raise PluginError("plugin manifest is missing schema/schema_version")
    if "schema" in m and "schema_version" in m and m["schema"] != m["schema_version"]:
        raise PluginError("plugin manifest schema fields disagree")
    if schema != 1:
        raise PluginError(f"unsupported plugin manifest schema {schema}")
    if not str(m.get("id", "")).strip():
        raise PluginError("plugin manifest id is empty")
    if not str(m.get("version", "")).strip():
        raise PluginError("plugin has an empty version")
    provides = m.get("provides") or []
    if not provides:
        raise PluginError("plugin declares no provided components")
    for c in provides:
        kind = c.get("type")
        if kind in ("backend", "architecture", "capability", "capabilities") and not c.get("id"):
            raise PluginError(f"component {kind} is missing id")
        if kind in ("kernels", "kernel-provider") and not (c.get("id") or c.get("backend")):
            raise PluginError("kernels component needs id or backend")


class PluginHost:
    """Loads one kernel plugin and launches its ops."""

    def __init__(self, path: str | Path = LIB_PATH, backend_id: str = "rocm"):
        self.path = Path(path)
        self.registry = KernelRegistry()
        self.paged: PagedKvContext | None = None
        self._snap_keep = None
        # ctypes callbacks must outlive the plugin.
        self._snapshot_cb = abi.SnapshotPagedFn(self._snapshot)
        self._register_cb = abi.RegisterOpFn(self._register)
        self.lib = C.CDLL(str(self.path))
        self._verify_abi()
        self.manifest = self._read_manifest()
        init = self.lib._fellm_plugin_init
        init.restype = C.c_int
        init.argtypes = [C.POINTER(abi.HostContext)]
        self.ctx = abi.HostContext()
        self.ctx.abi_version = abi.AbiVersion(*abi.ABI_VERSION)
        self.ctx.device_handle = 0
        self.ctx.default_stream = 0
        self.ctx.allocator_opaque = None
        self.ctx.backend_id = backend_id.encode()[: abi.PLUGIN_NAME_MAX - 1]
        self.ctx.snapshot_paged = self._snapshot_cb
        rc = init(C.byref(self.ctx))
        if rc != 0:
            raise PluginError(f"plugin init failed ({rc})", rc)
        reg = self.lib._fellm_plugin_register_kernels
        reg.restype = C.c_int
        reg.argtypes = [C.POINTER(abi.KernelRegistryVtable)]
        vt = abi.KernelRegistryVtable()
        vt.registry = None
        vt.register_op = self._register_cb
        rc = reg(C.byref(vt))
        if rc != 0:
            self.shutdown()
            raise PluginError(f"plugin kernel registration failed ({rc})", rc)
        # Optional symbols (loader.rs:387-406).
        self.invalidate = getattr(self.lib, "_fellm_plugin_invalidate_f32", None)
        if self.invalidate is not None:
            self.invalidate.restype = None
            self.invalidate.argtypes = [C.c_void_p, C.c_size_t]
        self.device_stream = getattr(self.lib, "_fellm_plugin_device_stream", None)
        if self.device_stream is not None:
            self.device_stream.restype = C.c_uint64
            self.device_stream.argtypes = []
        self._update_step_params = getattr(self.lib, "_fellm_plugin_update_step_params", None)
        if self._update_step_params is not None:
            self._update_step_params.restype = C.c_int
            self._update_step_params.argtypes = [C.POINTER(abi.DeviceStepParams)]
        self.register_device_tensor = getattr(self.lib, "_fellm_plugin_register_device_tensor", None)
        if self.register_device_tensor is not None:
            self.register_device_tensor.restype = C.c_int
            self.register_device_tensor.argtypes = [C.c_void_p, C.c_size_t, C.c_uint64]

    # -- activation -----------------------------------------------------------
    def _verify_abi(self) -> None:
        fn = self.lib._fellm_plugin_abi_version
        fn.restype = abi.AbiVersion
        fn.argtypes = []
        v = fn()
        if (v.major, v.minor, v.patch) != abi.ABI_VERSION:
            raise PluginError(f"plugin ABI {v.major}.{v.minor}.{v.patch} incompatible with host 0.9.0")

    def _read_manifest(self) -> dict:
        fn = self.lib._fellm_plugin_manifest_json
        fn.restype = abi.PluginManifestJson
        fn.argtypes = []
        raw = fn()
        if not raw.ptr or raw.len == 0:
            raise PluginError("empty plugin manifest")
        manifest = json.loads(C.string_at(raw.ptr, raw.len).decode())
        validate_manifest(manifest)
        return manifest

    def _register(self, _registry, reg_ptr) -> int:
        return self.registry.register(reg_ptr.contents)

    def shutdown(self) -> None:
        fn = self.lib._fellm_plugin_shutdown
        fn.restype = None
        fn()

    # -- paged context (paged_ctx.rs:55-95) -----------------------------------
    def set_paged_context(self, ctx: PagedKvContext | None) -> None:
        self.paged = ctx

    def _snapshot(self, out) -> int:
        if not out:
            return -1
        ctx = self.paged
        if ctx is None:
            return 1
        s = out.contents
        s.arena = ctx.arena_ptr
        s.arena_len = ctx.arena_len
        s.block_table = ctx.block_table.ctypes.data
        s.n_block_table = ctx.block_table.size
        s.n_logical_blocks = ctx.n_logical_blocks
        s.n_layers = ctx.n_layers
        s.tokens_stride = ctx.tokens_stride
        s.block_bytes = ctx.block_bytes
        s.block_size = ctx.block_size
        s.elem_bytes = ctx.elem_bytes
        s.device_arena = ctx.device_arena_ptr or None
        s.device_arena_len = ctx.device_arena_len
        s.device_block_table = ctx.device_block_table_ptr or None
        s.n_device_block_table = ctx.n_device_block_table
        s.device_logical_stride = ctx.device_logical_stride
        s.batch_size = max(ctx.row_positions.size, 1)
        s.row_positions = ctx.row_positions.ctypes.data
        s.row_lengths = ctx.row_lengths.ctypes.data if ctx.row_lengths is not None else None
        s.row_rope_positions = ctx.row_rope_positions.ctypes.data
        return 0

    # -- device plan (loader.rs:212-224, backend-cuda backend.rs:140-152) ------
    def update_step_params(self, params: abi.DeviceStepParams) -> None:
        """Upload the one device-resident step block read by single-row decode
        launches (and by every replay of a captured step)."""
        if self._update_step_params is None:
            raise PluginError("plugin has no _fellm_plugin_update_step_params")
        rc = self._update_step_params(C.byref(params))
        if rc != 0:
            raise PluginError(f"plugin step-parameter update failed ({rc})", rc)

    def stream(self):
        """The plugin's compute stream as a torch stream (for capture and sync)."""
        import torch

        if self.device_stream is None:
            raise PluginError("plugin has no capture-capable device stream")
        return torch.cuda.ExternalStream(self.device_stream())

    def begin_graph_capture(self):
        """Start capturing the plugin stream (CudaBackend::begin_graph_capture);
        `finish()` on the result returns a replayable graph."""
        from .graph import GraphCapture

        return GraphCapture(self.stream()).begin()

    # -- registry -------------------------------------------------------------
    def lookup(self, op: int, input_dtypes, output_dtype: int) -> int | None:
        return self.registry.lookup(op, input_dtypes, output_dtype)

    def launch_raw(self, handle: int, attrs: abi.OpAttrs, inputs, outputs, stream: int = 0) -> int:
        key = self.registry.by_handle.get(handle)
        if key is None:
            raise PluginError(f"unknown plugin kernel handle {handle}")
        fn = abi.PluginLaunchFn(self.registry.entries[key].launch_ptr)
        ins = (abi.TensorRef * max(len(inputs), 1))(*inputs)
        outs = (abi.TensorMut * max(len(outputs), 1))(*outputs)
        rc = fn(C.byref(attrs), ins, len(inputs), outs, len(outputs), stream)
        for i, o in enumerate(outputs):  # reflect any pointer updates
            outputs[i] = outs[i]
        return rc

    def launch(self, handle: int, attrs: abi.OpAttrs, inputs, outputs, stream: int = 0) -> None:
        rc = self.launch_raw(handle, attrs, inputs, outputs, stream)
        if rc != 0:
            raise PluginError(f"plugin kernel launch failed ({rc})", rc)
