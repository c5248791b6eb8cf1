"""Torch-facing entry points for the gfx950 kernels.

Every function takes device tensors already resident in HBM, launches one
HIP kernel through the C ABI on torch's current stream and returns the
outputs.  There is no CPU path: tensors must live on a ROCm device and the
kernel library must be built (``python -m fellm_amd.build``).

Reference semantics are documented on the C entry points (include/fellm_rocm.h).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import NamedTuple

import torch

from . import _lib
from .abi import DType

_ACT = {torch.float32: DType.F32, torch.float16: DType.F16, torch.bfloat16: DType.BF16}
_TORCH = {v: k for k, v in _ACT.items()}
QTYPES = {"q4k": (DType.Q4K, 144), "q5k": (DType.Q5K, 176), "q6k": (DType.Q6K, 210)}


def _code(t: torch.Tensor) -> int:
    try:
        return int(_ACT[t.dtype])
    except KeyError as e:
        raise TypeError(f"unsupported activation dtype {t.dtype}") from e


def _dev(*ts: torch.Tensor | None) -> None:
    for t in ts:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError("fellm_amd ops need device tensors (no CPU fallback)")
        if not t.is_contiguous():
            raise ValueError("fellm_amd ops need contiguous tensors")


def _p(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def add_rmsnorm(x, residual, weight, eps: float, *, h_out=None, y_out=None, y_dtype=None, store_h=True):
    """h = x + residual (stored in x's dtype); y = rmsnorm(h) * weight.

    ``residual=None`` gives plain RMSNorm of ``x`` (returns ``(None, y)``).
    Rows are the last-dimension groups of ``weight.numel()`` elements.
    """
    _dev(x, residual, weight)
    group = weight.numel()
    if weight.dtype != torch.float32:
        raise TypeError("RMSNorm weight must be float32")
    y_dtype = y_dtype or x.dtype
    y = y_out if y_out is not None else torch.empty(x.shape, dtype=y_dtype, device=x.device)
    h = None
    if residual is not None and store_h:
        h = h_out if h_out is not None else torch.empty_like(x)
    if residual is not None and residual.dtype != x.dtype:
        raise TypeError("x and residual dtypes differ")
    _dev(y, h)
    _lib.call("fellm_rocm_add_rmsnorm", _p(x), _p(residual), _p(h), _code(x), _p(weight), group, _p(y),
              _code(y), x.numel(), eps, _stream())
    return h, y


def rmsnorm(x, weight, eps: float, out=None):
    return add_rmsnorm(x, None, weight, eps, y_out=out)[1]


def silu_gate(gate, up, out=None, out_dtype=None):
    """out = silu(gate) * up, elementwise."""
    _dev(gate, up)
    if gate.shape != up.shape or gate.dtype != up.dtype:
        raise ValueError("gate/up mismatch")
    out = out if out is not None else torch.empty(gate.shape, dtype=out_dtype or gate.dtype, device=gate.device)
    _dev(out)
    _lib.call("fellm_rocm_silu_gate", _p(gate), _p(up), _code(gate), _p(out), _code(out), gate.numel(), _stream())
    return out


def add(a, b, out=None):
    _dev(a, b)
    out = out if out is not None else torch.empty_like(a)
    _lib.call("fellm_rocm_add", _p(a), _p(b), _code(a), _p(out), _code(out), a.numel(), _stream())
    return out


# Quantized embedding tables: the K-quants and Q8_0 (34-byte blocks of 32).
TABLE_QTYPES = {**{k: v[0] for k, v in QTYPES.items()}, "q8_0": DType.Q8_0}


def _table_code(table: torch.Tensor, qtype: str | None) -> int:
    if qtype is None:
        return _code(table)
    return int(TABLE_QTYPES[qtype])


def embedding(table, ids, *, dim: int | None = None, qtype: str | None = None, out=None,
              out_dtype=torch.float32, err_flag=None):
    """Gather rows ``table[ids]``.

    Dense tables are ``[vocab, dim]`` f32/f16/bf16 tensors.  Quantized tables
    (``qtype`` "q4k", "q5k", "q6k" or "q8_0") are uint8 ``[vocab, row_bytes]`` with ``dim``
    elements per row.  ``ids`` is int32 (read as u32).
    """
    _dev(table, ids)
    vocab = table.shape[0]
    dim = dim if dim is not None else table.shape[1]
    out = out if out is not None else torch.empty((ids.numel(), dim), dtype=out_dtype, device=table.device)
    _dev(out)
    _lib.call("fellm_rocm_embedding", _p(table), _table_code(table, qtype), vocab, dim, _p(ids), ids.numel(),
              _p(out), _code(out), _p(err_flag), _stream())
    return out


def embedding_rmsnorm(table, ids, weight, eps: float, *, dim: int | None = None, qtype: str | None = None,
                      out_dtype=torch.float16, h_out=None, y_out=None, store_h=True, err_flag=None):
    """Gather fused with RMSNorm of each gathered row: returns (h, y)."""
    _dev(table, ids, weight)
    vocab = table.shape[0]
    dim = dim if dim is not None else table.shape[1]
    y = y_out if y_out is not None else torch.empty((ids.numel(), dim), dtype=out_dtype, device=table.device)
    h = None
    if store_h:
        h = h_out if h_out is not None else torch.empty_like(y)
    _lib.call("fellm_rocm_embedding_rmsnorm", _p(table), _table_code(table, qtype), vocab, dim, _p(ids),
              ids.numel(), _p(weight), eps, _p(h), _p(y), _code(y), _p(err_flag), _stream())
    return h, y


def rope(x1, inv_freqs, *, head_dim: int, rope_dim: int | None = None, pairing: int = 0, positions=None,
         position0: int = 0, x2=None, out1=None, out2=None, inplace: bool = False):
    """RoPE over ``x1`` (and ``x2``, sharing positions).  Shapes ``[rows, heads*head_dim]``."""
    _dev(x1, x2, inv_freqs, positions)
    rope_dim = head_dim if rope_dim is None else rope_dim
    rows = x1.shape[0]
    nh1 = x1.shape[-1] // head_dim
    out1 = x1 if inplace else (out1 if out1 is not None else torch.empty_like(x1))
    nh2 = 0
    if x2 is not None:
        nh2 = x2.shape[-1] // head_dim
        out2 = x2 if inplace else (out2 if out2 is not None else torch.empty_like(x2))
    _lib.call("fellm_rocm_rope", _p(x1), _p(out1), nh1, _p(x2), _p(out2), nh2, _code(x1), rows, head_dim, rope_dim,
              pairing, _p(inv_freqs), _p(positions), position0, _stream())
    return (out1, out2) if x2 is not None else out1


@dataclass
class PagedKvCache:
    """Device paged KV arena in FeLLM's layout (paged_ctx.rs:341-360).

    ``arena`` is a uint8 device tensor of ``n_blocks * block_bytes``; each
    block holds ``block_size`` K rows then ``block_size`` V rows of
    ``stride`` elements (f16 as in the reference, or bf16).
    ``block_table`` is an int32 device tensor (read as u32) of
    ``batch * n_layers * n_logical_blocks`` physical block ids.
    """

    arena: torch.Tensor
    block_table: torch.Tensor
    n_layers: int
    n_logical_blocks: int
    block_size: int
    block_bytes: int
    stride: int
    kv_dtype: torch.dtype = torch.float16

    @staticmethod
    def block_bytes_for(stride: int, block_size: int = 16) -> int:
        """round_up(2 * block_size * stride * 2, 64) (backend-cuda/src/vram_pool.rs:31-35)."""
        return (2 * block_size * stride * 2 + 63) // 64 * 64

    def c_struct(self, layer: int) -> _lib.FellmRocmPagedKv:
        s = _lib.FellmRocmPagedKv()
        s.arena = self.arena.data_ptr()
        s.arena_len = self.arena.numel()
        s.block_table = self.block_table.data_ptr()
        s.n_block_table = self.block_table.numel()
        s.n_logical_blocks = self.n_logical_blocks
        s.n_layers = self.n_layers
        s.layer = layer
        s.block_size = self.block_size
        s.block_bytes = self.block_bytes
        s.stride = self.stride
        s.kv_dtype = int(_ACT[self.kv_dtype])
        return s


def kv_write(rows, kv_positions, cache: PagedKvCache, *, layer: int = 0, is_v: bool = False, err_flag=None):
    """Write rows ``[batch, stride]`` into K (or V) slots at ``kv_positions``."""
    _dev(rows, kv_positions)
    kv = cache.c_struct(layer)
    _lib.call("fellm_rocm_kv_write", _p(rows), _code(rows), rows.shape[0], _p(kv_positions), C.byref(kv),
              int(is_v), _p(err_flag), _stream())


def rope_kv_write(q, k, v, inv_freqs, kv_positions, cache: PagedKvCache, *, head_dim: int,
                  rope_dim: int | None = None, pairing: int = 0, rope_positions=None, layer: int = 0,
                  q_out=None, k_out=None, inplace_q: bool = False, err_flag=None):
    """Fused RoPE(q), RoPE(k) and paged append of rotated K and V."""
    _dev(q, k, v, inv_freqs, kv_positions, rope_positions)
    rope_dim = head_dim if rope_dim is None else rope_dim
    batch = q.shape[0]
    nq = q.numel() // (batch * head_dim)
    nkv = k.numel() // (batch * head_dim)
    q_out = q if inplace_q else (q_out if q_out is not None else torch.empty_like(q))
    kv = cache.c_struct(layer)
    _lib.call("fellm_rocm_rope_kv_write", _p(q), _p(q_out), nq, _p(k), _p(k_out), _p(v), nkv, _code(q), batch,
              head_dim, rope_dim, pairing, _p(inv_freqs), _p(rope_positions), _p(kv_positions), C.byref(kv),
              _p(err_flag), _stream())
    return q_out


def decode_step(q, k, v, inv_freqs, kv_positions, cache: PagedKvCache, x, residual, norm_weight, eps: float,
                gate, up, *, head_dim: int, rope_dim: int | None = None, pairing: int = 0, rope_positions=None,
                layer: int = 0, q_out=None, k_out=None, h_out=None, y_out=None, act_out=None, err_flag=None):
    """One launch for a decode step's RoPE(q, k) + paged K/V append, residual
    add + RMSNorm and SwiGLU (fellm_rocm_decode_step).  Returns (q_out, h, y, act)."""
    _dev(q, k, v, inv_freqs, kv_positions, rope_positions, x, residual, norm_weight, gate, up)
    rope_dim = head_dim if rope_dim is None else rope_dim
    batch = q.shape[0]
    q_out = q_out if q_out is not None else torch.empty_like(q)
    h_out = h_out if h_out is not None else torch.empty_like(x)
    y_out = y_out if y_out is not None else torch.empty_like(x)
    act_out = act_out if act_out is not None else torch.empty_like(gate)
    kv = cache.c_struct(layer)
    st = _lib.FellmRocmDecodeStep(
        act_dtype=_code(q), q=_p(q), q_out=_p(q_out), n_q_heads=q.numel() // (batch * head_dim), k=_p(k),
        k_out=_p(k_out), v=_p(v), n_kv_heads=k.numel() // (batch * head_dim), batch=batch, head_dim=head_dim,
        rope_dim=rope_dim, pairing=pairing, inv_freqs=_p(inv_freqs), rope_positions=_p(rope_positions),
        kv_positions=_p(kv_positions), kv=C.pointer(kv), err_flag=_p(err_flag),
        x=_p(x), residual=_p(residual), h_out=_p(h_out), norm_weight=_p(norm_weight), group=norm_weight.numel(),
        y=_p(y_out), norm_elems=x.numel(), eps=eps, gate=_p(gate), up=_p(up), act_out=_p(act_out),
        swiglu_elems=gate.numel())
    _lib.call("fellm_rocm_decode_step", C.byref(st), _stream())
    return q_out, h_out, y_out, act_out


def paged_attention(q, row_lengths, cache: PagedKvCache, *, n_heads: int, n_kv_heads: int, head_dim: int,
                    max_seq: int, layer: int = 0, scale: float = 0.0, causal: bool = True, window: int = 0,
                    out=None, out_dtype=None, workspace=None):
    """Paged decode attention: q [batch, n_heads*head_dim] against each row's cache
    (row_lengths int32 device [batch], max_seq >= every length).  Returns out
    [batch, n_heads*head_dim] in out_dtype (default: q's dtype)."""
    _dev(q, row_lengths)
    batch = q.shape[0]
    out_dtype = out_dtype or q.dtype
    out = out if out is not None else torch.empty((batch, n_heads * head_dim), dtype=out_dtype, device=q.device)
    need = _lib.lib().fellm_rocm_paged_attention_workspace(batch, n_heads, n_kv_heads, head_dim, max_seq)
    if workspace is None and need:
        workspace = torch.empty(need // 4, dtype=torch.float32, device=q.device)
    ws_bytes = workspace.numel() * 4 if workspace is not None else 0
    kv = cache.c_struct(layer)
    _lib.call("fellm_rocm_paged_attention", _p(q), _code(q), _p(out), _code(out), batch, n_heads, n_kv_heads,
              head_dim, _p(row_lengths), max_seq, scale, int(causal), window, C.byref(kv), _p(workspace), ws_bytes,
              _stream())
    return out


def router_topk(logits, k: int, *, gating_func: int = 1, norm_topk_prob: bool = True,
                routed_scaling_factor: float = 0.0, ids=None, weights=None):
    """Softmax/sigmoid gate + top-k + renorm: returns (ids int32 [T, k], weights f32 [T, k])."""
    _dev(logits)
    if logits.dtype != torch.float32:
        raise TypeError("router logits must be float32")
    tokens, n_exp = logits.shape
    kk = min(k, n_exp)
    ids = ids if ids is not None else torch.empty((tokens, kk), dtype=torch.int32, device=logits.device)
    weights = weights if weights is not None else torch.empty((tokens, kk), dtype=torch.float32, device=logits.device)
    _lib.call("fellm_rocm_router_topk", _p(logits), tokens, n_exp, k, gating_func, int(norm_topk_prob),
              routed_scaling_factor, _p(ids), _p(weights), _stream())
    return ids, weights


class MoeDispatch(NamedTuple):
    """Per-expert grouping of the routed assignments (all int32 tensors on the device)."""

    counts: torch.Tensor   # [E]
    offsets: torch.Tensor  # [E + 1]
    order: torch.Tensor    # [A], A = tokens * top_k
    inv: torch.Tensor      # [A]


def moe_dispatch(ids, n_experts: int, *, err_flag=None, workspace=None, out: MoeDispatch | None = None) -> MoeDispatch:
    """Stable per-expert grouping of the router's ids [tokens, top_k]
    (moe.rs:839-848 order; replaces oxide_kernels.rs:2283-2327).  `out`
    reuses the tensors of an earlier result of the same shape."""
    _dev(ids)
    if ids.dtype != torch.int32 or ids.dim() != 2 or not ids.is_contiguous():
        raise TypeError("ids must be a contiguous int32 [tokens, top_k] tensor")
    tokens, k = ids.shape
    dev = ids.device
    if out is not None:
        counts, offsets, order, inv = out
        if counts.numel() != n_experts or offsets.numel() != n_experts + 1 or order.numel() != tokens * k \
                or inv.numel() != tokens * k:
            raise ValueError("out does not match ids / n_experts")
    else:
        counts = torch.empty(n_experts, dtype=torch.int32, device=dev)
        offsets = torch.empty(n_experts + 1, dtype=torch.int32, device=dev)
        order = torch.empty(tokens * k, dtype=torch.int32, device=dev)
        inv = torch.empty(tokens * k, dtype=torch.int32, device=dev)
    need = _lib.lib().fellm_rocm_moe_dispatch_workspace(tokens, k, n_experts)
    if workspace is None and need:
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    _lib.call("fellm_rocm_moe_dispatch", _p(ids), tokens, k, n_experts, _p(counts), _p(offsets), _p(order), _p(inv),
              _p(err_flag), _p(workspace), ws_bytes, _stream())
    return MoeDispatch(counts, offsets, order, inv)


def moe_gather(x, order, top_k: int, *, inv=None, out=None):
    """grouped[p] = x[order[p] // top_k] (moe.rs:954-957), any 1/2/4-byte dtype.
    With the dispatch's inv, each x row is read once and scattered."""
    _dev(x, order, inv)
    tokens, hidden = x.shape
    if not x.is_contiguous() or order.numel() != tokens * top_k:
        raise ValueError("x must be contiguous [tokens, hidden] and order [tokens * top_k]")
    out = out if out is not None else torch.empty((tokens * top_k, hidden), dtype=x.dtype, device=x.device)
    _lib.call("fellm_rocm_moe_gather", _p(x), x.element_size(), tokens, top_k, hidden, _p(order), _p(inv), _p(out),
              _stream())
    return out


def moe_combine(expert_out, weights, *, ids=None, inv=None, y0=None, out=None):
    """y = y0 + sum_s weights[:, s] * row(t, s) in f32 without FMA.  With inv
    (grouped rows) the slots are added in ascending expert id (moe.rs:1024-1033);
    without, rows are per assignment and added in slot order
    (moe_weighted_reduce, oxide_kernels.rs:2507-2532)."""
    _dev(expert_out, weights, ids, inv, y0)
    tokens, k = weights.shape
    hidden = expert_out.shape[1]
    if expert_out.dtype != torch.float32 or weights.dtype != torch.float32:
        raise TypeError("expert_out and weights must be float32")
    if expert_out.shape[0] != tokens * k:
        raise ValueError("expert_out must hold tokens * top_k rows")
    if inv is not None and ids is None:
        raise ValueError("the expert-order combine needs ids")
    out = out if out is not None else torch.empty((tokens, hidden), dtype=torch.float32, device=expert_out.device)
    _lib.call("fellm_rocm_moe_combine", _p(y0), _p(expert_out), _p(ids), _p(weights), _p(inv), tokens, k, hidden,
              _p(out), _stream())
    return out


def quantize_q8k(x, out=None):
    """x (f32 vector, cols % 256 == 0) -> Q8_K blob (uint8 tensor) for the
    *_q8k GEMVs: qs int8 [cols], bsums int16 [cols/16], d f32 [cols/256]."""
    _dev(x)
    if x.dtype != torch.float32 or x.dim() != 1:
        raise TypeError("x must be a float32 vector")
    n = _lib.lib().fellm_rocm_q8k_bytes(x.numel())
    out = out if out is not None else torch.empty(n, dtype=torch.uint8, device=x.device)
    _lib.call("fellm_rocm_quantize_q8k", _p(x), x.numel(), _p(out), _stream())
    return out


def _q8k_cols(xq) -> int:
    if xq.dtype != torch.uint8 or xq.numel() % 292:
        raise ValueError("xq must be a Q8_K blob from quantize_q8k")
    return xq.numel() // 292 * 256


def gate_up_swiglu_q8k(gate_w, up_w, xq, *, qtype: str = "q4k", up_qtype: str | None = None, out=None):
    """gate_up_swiglu over an activation already quantized by quantize_q8k."""
    _dev(gate_w, up_w, xq)
    cols = _q8k_cols(xq)
    rows = gate_w.shape[0]
    g = _kquant_code(qtype, gate_w, cols)
    u = _kquant_code(up_qtype or qtype, up_w, cols)
    out = out if out is not None else torch.empty(rows, dtype=torch.float32, device=xq.device)
    _lib.call("fellm_rocm_gate_up_swiglu_q8k", _p(gate_w), g, _p(up_w), u, rows, cols, _p(xq), _p(out), _stream())
    return out


def matvec_kquant_q8k(w, xq, *, qtype: str = "q4k", out=None):
    """matvec_kquant over an activation already quantized by quantize_q8k."""
    _dev(w, xq)
    cols = _q8k_cols(xq)
    rows = w.shape[0]
    code = _kquant_code(qtype, w, cols)
    out = out if out is not None else torch.empty(rows, dtype=torch.float32, device=xq.device)
    _lib.call("fellm_rocm_matvec_kquant_q8k", _p(w), code, rows, cols, _p(xq), _p(out), _stream())
    return out


def step_kv_position(params, block_size: int, out=None):
    """KV position of the single decode row from a device DeviceStepParams
    block (uint8 [48] tensor): ((sequence_length - 1) // block_size) *
    block_size + kv_write_slot (oxide_kernels.rs:4203-4214)."""
    _dev(params)
    out = out if out is not None else torch.empty(1, dtype=torch.int32, device=params.device)
    _lib.call("fellm_rocm_step_kv_position", _p(params), block_size, _p(out), _stream())
    return out


def step_field(params, name: str):
    """A u32 field of a device DeviceStepParams block as a 1-element int32 view
    (token_id, position, sequence_length, ...), usable as the ids /
    positions / row_lengths array of a decode launch."""
    from .abi import DeviceStepParams

    off = getattr(DeviceStepParams, name).offset
    return params[off:off + 4].view(torch.int32)


def _kquant_code(qtype: str, w, cols: int) -> int:
    code, bb = QTYPES[qtype]
    if w.dtype != torch.uint8 or w.dim() != 2 or w.shape[1] != cols // 256 * bb:
        raise ValueError(f"{qtype} weights must be uint8 [rows, cols/256*{bb}]")
    return int(code)


def gate_up_swiglu(gate_w, up_w, x, *, qtype: str = "q4k", up_qtype: str | None = None, out=None):
    """out[r] = silu(gate_w[r] . x) * (up_w[r] . x) with x quantized to Q8_K
    (GateUpSwiGlu, backend.rs:944-1002).  Weights: uint8 GGUF K-quant rows."""
    _dev(gate_w, up_w, x)
    if x.dtype != torch.float32 or x.dim() != 1:
        raise TypeError("x must be a float32 vector")
    cols = x.numel()
    rows = gate_w.shape[0]
    g = _kquant_code(qtype, gate_w, cols)
    u = _kquant_code(up_qtype or qtype, up_w, cols)
    if up_w.shape[0] != rows:
        raise ValueError("gate and up must have the same number of rows")
    out = out if out is not None else torch.empty(rows, dtype=torch.float32, device=x.device)
    _lib.call("fellm_rocm_gate_up_swiglu", _p(gate_w), g, _p(up_w), u, rows, cols, _p(x), _p(out), _stream())
    return out


def matvec_kquant(w, x, *, qtype: str = "q4k", out=None):
    """y = W x for one activation vector, x quantized to Q8_K (matvec_quant, matmul.rs:534-600)."""
    _dev(w, x)
    if x.dtype != torch.float32 or x.dim() != 1:
        raise TypeError("x must be a float32 vector")
    cols = x.numel()
    code = _kquant_code(qtype, w, cols)
    rows = w.shape[0]
    out = out if out is not None else torch.empty(rows, dtype=torch.float32, device=x.device)
    _lib.call("fellm_rocm_matvec_kquant", _p(w), code, rows, cols, _p(x), _p(out), _stream())
    return out


def expf(x):
    """Device glibc-exact expf (self-check of the restatement)."""
    _dev(x)
    out = torch.empty_like(x)
    _lib.call("fellm_rocm_expf", _p(x), _p(out), x.numel(), _stream())
    return out


def logf(x):
    """Device glibc-exact logf (self-check of the restatement the router uses)."""
    _dev(x)
    out = torch.empty_like(x)
    _lib.call("fellm_rocm_mathf", 0, _p(x), _p(out), x.numel(), _stream())
    return out


def sqrtf(x):
    """Device correctly rounded sqrtf (self-check; the router's sqrt-softplus uses it)."""
    _dev(x)
    out = torch.empty_like(x)
    _lib.call("fellm_rocm_mathf", 1, _p(x), _p(out), x.numel(), _stream())
    return out


def bf16_store_bits(x):
    """bf16 bits (int32 tensor) of the device's bf16 activation store of f32 ``x`` (self-check)."""
    _dev(x)
    out = torch.empty_like(x)
    _lib.call("fellm_rocm_mathf", 2, _p(x), _p(out), x.numel(), _stream())
    return out.view(torch.int32)


def sincosf(x):
    """Device glibc-exact (sinf(x), cosf(x)) (self-check of the restatement RoPE uses)."""
    _dev(x)
    s, c = torch.empty_like(x), torch.empty_like(x)
    _lib.call("fellm_rocm_sincosf", _p(x), _p(s), _p(c), x.numel(), _stream())
    return s, c


def silu_fast_bound():
    """(largest measured bit distance between the fast and the exact silu over
    every f32 gate of the fast domain, the distance the SwiGLU 16-bit path
    assumes).  The path is bit-exact iff the first does not exceed the second."""
    m = torch.zeros(1, dtype=torch.int32, device="cuda")
    _lib.call("fellm_rocm_silu_fast_bound", _p(m), _stream())
    return int(m.cpu().item()) & 0xFFFFFFFF, int(_lib.lib().fellm_rocm_silu_fast_dist())


def rope_inv_freqs(theta: float, rope_dim: int) -> torch.Tensor:
    """inv_freq[i] = theta ** (-(2i) / rope_dim) in f32 with libm powf
    (crates/fellm-model/src/rope.rs:13-40, no scaling), as a CPU tensor."""
    import ctypes.util

    libm = C.CDLL(ctypes.util.find_library("m") or "libm.so.6")
    libm.powf.restype = C.c_float
    libm.powf.argtypes = [C.c_float, C.c_float]
    out = []
    for i in range(rope_dim // 2):
        e = C.c_float(-float(2 * i)).value / C.c_float(float(rope_dim)).value
        e = C.c_float(e).value
        out.append(libm.powf(theta, e))
    return torch.tensor(out, dtype=torch.float32)
