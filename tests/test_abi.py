"""CPU tests of the drop-in boundary: ABI layouts, exported symbols, plugin
activation and registration, and launch error paths that return before any
GPU work (no compute calls: these run where no GPU exists)."""
from __future__ import annotations

import ctypes as C
import json
import re
import subprocess
from pathlib import Path

import pytest

from fellm_amd import abi
from fellm_amd._lib import EXPORTED, LIB_PATH
from fellm_amd.plugin_host import PluginHost

ROOT = Path(__file__).resolve().parent.parent
GOLD = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())


def test_ctypes_layouts_match_reference_sizes():
    for name, (cls, size) in abi.LAYOUT.items():
        assert C.sizeof(cls) == size, name
    assert abi.TensorRef.data.offset == 96 and abi.TensorRef.byte_len.offset == 104
    assert abi.TensorMut.data.offset == 88
    assert abi.OpAttrs.seed.offset == 56 and abi.OpAttrs.block_size.offset == 92
    assert abi.OpAttrs.custom_op_id.offset == 128
    assert abi.PagedKvSnapshot.device_arena.offset == 80 and abi.PagedKvSnapshot.batch_size.offset == 120
    assert abi.HostContext.snapshot_paged.offset == 96
    assert abi.PluginOpRegistration.launch.offset == 80


def test_c_header_static_asserts_compile(tmp_path):
    src = tmp_path / "t.c"
    src.write_text('#include "fellm_abi.h"\n#include "fellm_rocm.h"\nint main(void){return 0;}\n')
    for cc, std in (("gcc", "-std=c11"), ("g++", "-std=c++17")):
        r = subprocess.run([cc, std, "-x", "c" if cc == "gcc" else "c++", f"-I{ROOT / 'include'}", str(src),
                            "-o", str(tmp_path / "t")], capture_output=True, text=True)
        assert r.returncode == 0, r.stderr


def _declared_functions():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b((?:_fellm_plugin|fellm_rocm)_\w+)\s*\(", text, re.M):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol():
    assert LIB_PATH.exists(), "build the library first: python -m fellm_amd.build"
    out = subprocess.run(["nm", "-D", "--defined-only", str(LIB_PATH)], capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    declared = _declared_functions()
    assert declared, "no declarations parsed"
    assert declared <= exported, declared - exported
    assert set(EXPORTED) <= exported
    # nothing else leaks out of the version script
    assert all(n.startswith(("_fellm_plugin_", "fellm_rocm_")) for n in exported), exported


def test_custom_op_ids_follow_fnv1a():
    # independent FNV-1a over "ns:name" (op.rs:69-80)
    def fnv(s):
        h = 2166136261
        for b in s.encode():
            h = ((h ^ b) * 16777619) % 2**32
        return h | 0x80000000
    a = abi.custom_op(*GOLD["custom_op_ids"]["pairs"][0])
    b = abi.custom_op(*GOLD["custom_op_ids"]["pairs"][1])
    assert a == fnv("example:fused_bias") and b == fnv("other:fused_bias") and a != b
    assert a & 0x80000000
    assert abi.OP_ADD_RMSNORM == fnv("rocm:add_rmsnorm")


@pytest.fixture(scope="module")
def host():
    h = PluginHost()
    yield h
    h.shutdown()


def test_manifest_validation_rules():
    from fellm_amd.plugin_host import PluginError, validate_manifest

    good = {"schema": 1, "id": "x", "version": "1", "provides": [{"type": "kernels", "backend": "rocm"}]}
    validate_manifest(good)
    for bad in ({**good, "schema": 2}, {**good, "id": " "}, {**good, "version": ""}, {**good, "provides": []},
                {**good, "provides": [{"type": "backend"}]}, {**good, "schema_version": 3}):
        with pytest.raises(PluginError):
            validate_manifest(bad)


def test_plugin_activation(host):
    assert host.manifest["schema"] == 1
    assert host.manifest["id"] == "fellm.rocm"
    assert {"type": "kernels", "backend": "rocm"} in host.manifest["provides"]
    assert host.invalidate is not None and host.device_stream is not None


REFERENCE_KEYS = [
    # plugins/cuda_kernels/src/lib.rs:337-720 keys this library serves
    (abi.OpKind.RMSNORM, [abi.DType.F32, abi.DType.F32], abi.DType.F32),
    (abi.OpKind.SILU_GATE, [abi.DType.F32, abi.DType.F32], abi.DType.F32),
    (abi.OpKind.ROPE, [abi.DType.F32, abi.DType.F32], abi.DType.F32),
    (abi.OpKind.KV_WRITE, [abi.DType.F32, abi.DType.F32], abi.DType.F32),
    (abi.OpKind.ADD, [abi.DType.F32, abi.DType.F32], abi.DType.F32),
    (abi.OpKind.CAST, [abi.DType.F32], abi.DType.F32),
    (abi.OpKind.EMBEDDING, [abi.DType.F32, abi.DType.U32], abi.DType.F32),
    (abi.OpKind.EMBEDDING, [abi.DType.BF16, abi.DType.U32], abi.DType.F32),
    (abi.OpKind.EMBEDDING, [abi.DType.Q4K, abi.DType.U32], abi.DType.F32),
    (abi.OpKind.EMBEDDING, [abi.DType.Q6K, abi.DType.U32], abi.DType.F32),
    (abi.OpKind.EMBEDDING, [abi.DType.Q5K, abi.DType.U32], abi.DType.F32),
    # load_cuda_kernels.rs:107-111 asserts this key on the CUDA plugin.
    (abi.OpKind.EMBEDDING, [abi.DType.Q8_0, abi.DType.U32], abi.DType.F32),
]
NEW_KEYS = [
    (abi.OpKind.RMSNORM, [abi.DType.F16, abi.DType.F32], abi.DType.F16),
    (abi.OpKind.SILU_GATE, [abi.DType.BF16, abi.DType.BF16], abi.DType.BF16),
    (abi.OpKind.EMBEDDING, [abi.DType.Q4K, abi.DType.U32], abi.DType.F16),
    (abi.OpKind.EMBEDDING, [abi.DType.Q5K, abi.DType.U32], abi.DType.F16),
    (abi.OpKind.EMBEDDING, [abi.DType.Q8_0, abi.DType.U32], abi.DType.F16),
    (abi.OpKind.CAST, [abi.DType.Q5K], abi.DType.F32),
    (abi.OpKind.CAST, [abi.DType.Q8_0], abi.DType.F32),
    (abi.OP_ADD_RMSNORM, [abi.DType.F16, abi.DType.F16, abi.DType.F32], abi.DType.F16),
    (abi.OP_ROPE_KV_WRITE, [abi.DType.BF16, abi.DType.BF16, abi.DType.BF16, abi.DType.F32], abi.DType.BF16),
    (abi.OP_ROUTER_TOPK, [abi.DType.F32], abi.DType.U32),
    (abi.OP_EMBEDDING_RMSNORM, [abi.DType.Q4K, abi.DType.U32, abi.DType.F32], abi.DType.F16),
]


@pytest.mark.parametrize("op,ins,out", REFERENCE_KEYS + NEW_KEYS)
def test_registry_keys(host, op, ins, out):
    assert host.lookup(op, ins, out) is not None


def test_registry_exact_match_only(host):
    assert host.lookup(abi.OpKind.RMSNORM, [abi.DType.F32], abi.DType.F32) is None
    assert host.lookup(abi.OpKind.MATMUL, [abi.DType.Q4K, abi.DType.F32], abi.DType.F32) is None


def _launch(host, op, ins_dt, out_dt, attrs, ins, outs):
    h = host.lookup(op, ins_dt, out_dt)
    return host.launch_raw(h, attrs, ins, outs)


def _f32(n):
    import numpy as np

    return np.zeros(n, np.float32)


def test_launch_error_paths_before_gpu(host):
    import numpy as np

    attrs = abi.OpAttrs()
    x, w, y = _f32(10), _f32(3), _f32(10)
    tr = lambda a, dt=abi.DType.F32: abi.tensor_ref(a.ctypes.data, a.nbytes, dt, [a.size])
    tm = lambda a, dt=abi.DType.F32: abi.tensor_mut(a.ctypes.data, a.nbytes, dt, [a.size])
    rms = (abi.OpKind.RMSNORM, [abi.DType.F32, abi.DType.F32], abi.DType.F32)
    # x.len() % w.len() != 0 -> -2 (launchers.rs:357-359)
    assert _launch(host, *rms, attrs, [tr(x), tr(w)], [tm(y)]) == abi.ERR_SHAPE
    # arity
    assert _launch(host, *rms, attrs, [tr(x)], [tm(y)]) == abi.ERR_ARITY
    # dtype mismatch between registration and tensors
    assert _launch(host, *rms, attrs, [tr(x, abi.DType.F16), tr(w)], [tm(y)]) == abi.ERR_DTYPE
    # embedding: token id >= vocab -> -2 (launchers.rs:618-621)
    table = _f32(4 * 8)
    ids = np.array([1, 4], np.uint32)
    emb = (abi.OpKind.EMBEDDING, [abi.DType.F32, abi.DType.U32], abi.DType.F32)
    out = _f32(2 * 8)
    tref = abi.tensor_ref(table.ctypes.data, table.nbytes, abi.DType.F32, [4, 8])
    iref = abi.tensor_ref(ids.ctypes.data, ids.nbytes, abi.DType.U32, [2])
    assert _launch(host, *emb, attrs, [tref, iref], [tm(out)]) == abi.ERR_SHAPE
    # RoPE: x.len() not a multiple of n_heads * head_dim -> -2
    attrs_r = abi.OpAttrs(n_heads=1, head_dim=4, rope_dim=4)
    rope = (abi.OpKind.ROPE, [abi.DType.F32, abi.DType.F32], abi.DType.F32)
    assert _launch(host, *rope, attrs_r, [tr(x), tr(_f32(5))], [tm(y)]) == abi.ERR_SHAPE
    # fused RoPE + KV write without a paged context -> -20
    q, k = _f32(8), _f32(8)
    rkv = (abi.OP_ROPE_KV_WRITE, [abi.DType.F32] * 4, abi.DType.F32)
    assert _launch(host, *rkv, abi.OpAttrs(n_heads=1, n_kv_heads=1, head_dim=8, rope_dim=8),
                   [tr(q), tr(k), tr(k), tr(_f32(4))], [tm(_f32(8))]) == abi.ERR_PAGED_MISSING
    # router: logits not a multiple of n_experts
    rt = (abi.OP_ROUTER_TOPK, [abi.DType.F32], abi.DType.U32)
    assert _launch(host, *rt, abi.OpAttrs(n_experts=3, n_expert_used=2), [tr(x)],
                   [tm(_f32(4), abi.DType.U32), tm(_f32(4))]) == abi.ERR_SHAPE


def test_entry_points_reject_null(host):
    lib = host.lib
    lib._fellm_plugin_init.restype = C.c_int
    assert lib._fellm_plugin_init(None) == abi.ERR_ARITY
    lib._fellm_plugin_register_kernels.restype = C.c_int
    assert lib._fellm_plugin_register_kernels(None) == abi.ERR_ARITY
    lib._fellm_plugin_register_device_tensor.restype = C.c_int
    lib._fellm_plugin_register_device_tensor.argtypes = [C.c_void_p, C.c_size_t, C.c_uint64]
    assert lib._fellm_plugin_register_device_tensor(None, 0, 0) == abi.ERR_ARITY
    host.invalidate(None, 0)  # no-op, must not crash
    attrs = abi.OpAttrs()
    h = host.lookup(abi.OpKind.ADD, [abi.DType.F32, abi.DType.F32], abi.DType.F32)
    fn = abi.PluginLaunchFn(host.registry.entries[host.registry.by_handle[h]].launch_ptr)
    assert fn(C.byref(attrs), None, 0, None, 0, 0) == abi.ERR_ARITY


def test_device_api_validates_before_launch():
    from fellm_amd import _lib

    lib = _lib.lib()
    assert lib.fellm_rocm_version().startswith(b"fellm-rocm")
    assert lib.fellm_rocm_add_rmsnorm(None, None, None, 1, None, 16, None, 1, 32, 1e-5, None) == abi.ERR_ARITY
    assert lib.fellm_rocm_router_topk(C.c_void_p(16), 1, 600, 8, 1, 1, 0.0, C.c_void_p(16), C.c_void_p(16),
                                      None) == abi.ERR_SHAPE
    assert lib.fellm_rocm_router_topk(C.c_void_p(16), 1, 0, 2, 4, 1, 0.0, C.c_void_p(16), C.c_void_p(16),
                                      None) == abi.ERR_SHAPE
    assert lib.fellm_rocm_embedding(C.c_void_p(16), 99, 10, 16, C.c_void_p(16), 1, C.c_void_p(16), 0, None,
                                    None) == abi.ERR_DTYPE
    assert lib.fellm_rocm_rope(C.c_void_p(16), C.c_void_p(16), 1, None, None, 0, 0, 1, 8, 10, 0, C.c_void_p(16),
                               None, 0, None) == abi.ERR_SHAPE
