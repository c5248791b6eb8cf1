"""The allocation-free MoE dispatch (fellm_rocm_moe_dispatch_noalloc) against
the workspace entry point (fellm_rocm_moe_dispatch), both through the C ABI:
counts, offsets, order and inv must be bit-identical.  Two calls in a row
share the library's per-GPU count buffer, the second with a smaller input
(fewer blocks and experts, so stale counts of the first call lie in the
buffer past what the second writes); then a single-block call that needs no
buffer at all, the largest expert count, and an input with invalid ids."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def _call(fn, ids, n_experts, workspace=None):
    from fellm_amd import _lib

    tokens, k = ids.shape
    dev = ids.device
    out = [torch.full((n,), -7, dtype=torch.int32, device=dev) for n in (n_experts, n_experts + 1, tokens * k,
                                                                         tokens * k)]
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    lib = _lib.lib()
    if fn == "noalloc":
        rc = lib.fellm_rocm_moe_dispatch_noalloc(ids.data_ptr(), tokens, k, n_experts, *(t.data_ptr() for t in out),
                                                 flag.data_ptr(), stream)
    else:
        ws_bytes = 0 if workspace is None else workspace.numel()
        rc = lib.fellm_rocm_moe_dispatch(ids.data_ptr(), tokens, k, n_experts, *(t.data_ptr() for t in out),
                                         flag.data_ptr(), None if workspace is None else workspace.data_ptr(),
                                         ws_bytes, stream)
    assert rc == 0, f"{fn}: rc {rc}"
    torch.cuda.synchronize()
    return [t.cpu().numpy() for t in out] + [int(flag.item())]


def _ids(gen, tokens, k, n_experts, dev):
    ids = torch.argsort(torch.rand(tokens, n_experts, generator=gen), dim=1)[:, :k].to(torch.int32)
    return ids.contiguous().to(dev)


def _compare(ids, n_experts):
    from fellm_amd import _lib

    need = _lib.lib().fellm_rocm_moe_dispatch_workspace(ids.shape[0], ids.shape[1], n_experts)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=ids.device) if need else None
    ref = _call("workspace", ids, n_experts, ws)
    got = _call("noalloc", ids, n_experts)
    for name, g, r in zip(("counts", "offsets", "order", "inv", "err_flag"), got, ref):
        assert np.array_equal(g, r), f"{name} differs ({ids.shape}, E {n_experts})"
    return got


def test_noalloc_dispatch_matches_workspace_dispatch(dev):
    from fellm_amd import _lib

    assert _lib.lib().fellm_rocm_moe_dispatch_noalloc_max_bytes() == 256 * 4096 * 4
    gen = torch.Generator().manual_seed(11)
    # 1: configs[4]'s shape, 16384 tokens x top-8 of 128 experts (64 blocks)
    _compare(_ids(gen, 16384, 8, 128, dev), 128)
    # 2: smaller, right after: 3000 x 4 of 60 experts (6 blocks)
    counts = _compare(_ids(gen, 3000, 4, 60, dev), 60)[0]
    assert counts.sum() == 3000 * 4
    # 3: one block (no count buffer), 64-token decode batch
    _compare(_ids(gen, 64, 8, 128, dev), 128)
    # 4: the most experts and a full 256-block grid
    ids = torch.randint(0, 4096, (65536, 16), generator=gen, dtype=torch.int32).to(dev)
    _compare(ids, 4096)
    # 5: invalid ids are left out of every group and flagged, as in the workspace form
    ids = torch.randint(0, 40, (5000, 2), generator=gen, dtype=torch.int32)
    ids[7, 1] = 40
    ids[4000, 0] = 1 << 20
    out = _compare(ids.to(dev), 40)
    assert out[-1] == 1


def test_noalloc_dispatch_rejects_bad_shapes(dev):
    from fellm_amd import _lib

    ids = torch.zeros((4, 2), dtype=torch.int32, device=dev)
    z = torch.zeros(4096 * 2, dtype=torch.int32, device=dev)
    lib = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    for e, k in ((4097, 2), (0, 2), (16, 0), (16, 65)):
        rc = lib.fellm_rocm_moe_dispatch_noalloc(ids.data_ptr(), 4, k, e, z.data_ptr(), z.data_ptr(), z.data_ptr(),
                                                 z.data_ptr(), None, stream)
        assert rc == -2, (e, k, rc)
