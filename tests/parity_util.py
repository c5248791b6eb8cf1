"""Helpers shared by the parity tests: host<->device transfer of stored
activations and the comparison rules with their stated tolerances.

Tolerances (from the contract of the path):
  * integer, byte and index results, embedding gathers, KV slot bytes:
    bit-exact;
  * f32 results of RMSNorm: |gpu - ref| <= 1e-5 * |ref| elementwise;
  * f16 / bf16 results after f32 accumulation: within 1 ulp of the output
    dtype (ordered-integer distance of the bit patterns <= 1);
  * RoPE and the rotated K slots: bit-exact (the device sin/cos restate
    glibc's sinf/cosf, and the rotation is evaluated without contraction).
"""
from __future__ import annotations

import numpy as np
import torch

KINDS = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def to_dev(stored: np.ndarray, kind: str, dev) -> torch.Tensor:
    """Stored form (f32 values or 16-bit bit patterns) -> device tensor of `kind`."""
    if kind == "f32":
        return torch.from_numpy(np.ascontiguousarray(stored, np.float32)).to(dev)
    bits = torch.from_numpy(np.ascontiguousarray(stored, np.uint16).view(np.int16)).to(dev)
    return bits.view(KINDS[kind])


def from_dev(t: torch.Tensor) -> np.ndarray:
    """Device tensor -> stored form (f32 values or uint16 bit patterns)."""
    t = t.detach().contiguous().cpu()
    if t.dtype == torch.float32:
        return t.numpy()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.int32:
        return t.numpy().view(np.uint32)
    return t.numpy()


def random_stored(rng: np.random.Generator, shape, kind: str, sigma: float = 1.0) -> np.ndarray:
    x = rng.normal(0.0, sigma, size=shape).astype(np.float32)
    import oracle

    return oracle.narrow(x, kind)


def ordered16(bits: np.ndarray) -> np.ndarray:
    b = bits.astype(np.int64)
    return np.where(b & 0x8000, -(b & 0x7FFF), b & 0x7FFF)


def assert_exact(got: np.ndarray, ref: np.ndarray, what: str = "") -> None:
    got = np.asarray(got)
    ref = np.asarray(ref)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    gv = got.view(np.uint32) if got.dtype == np.float32 else got
    rv = ref.view(np.uint32) if ref.dtype == np.float32 else ref
    bad = np.nonzero(gv != rv)
    n = len(bad[0])
    assert n == 0, f"{what}: {n} mismatches, first at {tuple(b[0] for b in bad)}: got {got[bad][:4]} ref {ref[bad][:4]}"


def assert_close(got: np.ndarray, ref: np.ndarray, kind: str, rel: float = 1e-5, what: str = "") -> None:
    if kind == "f32":
        err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
        lim = rel * np.abs(ref.astype(np.float64))
        bad = err > lim
        assert not bad.any(), f"{what}: {bad.sum()} beyond {rel} rel; worst {err.max():.3e} at ref {ref[bad][:3]}"
    else:
        d = np.abs(ordered16(got) - ordered16(ref))
        assert d.max(initial=0) <= 1, f"{what}: max ulp distance {d.max()} ({(d > 1).sum()} elems)"
