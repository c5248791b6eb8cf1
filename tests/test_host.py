"""CPU tests of the host-side helpers: synthetic generators and bench.py's contract."""
from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import numpy as np

import oracle
from fellm_amd import synth

ROOT = Path(__file__).resolve().parent.parent


def test_q4k_table_scales_roundtrip():
    rng = np.random.default_rng(0)
    t = synth.q4k_table(rng, 3, 512)
    assert t.shape == (3, 2 * 144)
    ls = rng.integers(0, 64, size=8)
    lm = rng.integers(0, 64, size=8)
    packed = synth.pack_scale_min_k4(ls, lm)
    for j in range(8):
        assert oracle.get_scale_min_k4(j, packed.tobytes()) == (ls[j], lm[j])
    d = t.reshape(3, 2, 144)[..., 0:2].copy().view(np.float16)
    assert np.all(d >= 0) and np.all(np.isfinite(d.astype(np.float32)))


def test_q6k_table_shape_and_scale():
    t = synth.q6k_table(np.random.default_rng(1), 4, 768)
    assert t.shape == (4, 3 * 210)
    d = t.reshape(4, 3, 210)[..., 208:210].copy().view(np.float16).astype(np.float32)
    assert np.all(d >= 0) and np.all(d < 0.1)


def test_zipf_ids_range_and_skew():
    ids = synth.zipf_ids(np.random.default_rng(2), 20000, 1000, 1.1)
    assert ids.dtype == np.uint32 and ids.max() < 1000
    counts = np.bincount(ids, minlength=1000)
    assert counts[0] > counts[10] > counts[500]


def test_paged_layout_distinct_blocks():
    pos, table, n_logical = synth.paged_layout(np.random.default_rng(3), 256, 65536, 16, 32768)
    assert n_logical == 2048 and table.size == 256 * 2048
    t = table.reshape(256, 2048)
    phys = t[np.arange(256), pos // 16]
    assert len(set(phys.tolist())) == 256  # a permutation: no two rows share a block


def test_bench_refuses_multi_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_bench_cpu_baseline_contract():
    sys.path.insert(0, str(ROOT))
    import bench

    cb = bench.cpu_baseline(0.2)
    assert cb["kind"] == "port" and cb["cores"] == 1 and cb["unit"] == "tokens/s" and cb["value"] > 0
    json.dumps(cb)


def test_bench_traffic_summary_parses():
    sys.path.insert(0, str(ROOT))
    import bench

    t = bench.read_traffic()
    assert t is None or 300e6 < t < 400e6


def test_bench_cpu_suite_reports_every_op():
    """bench.py --suite's CPU leg: every op of a config is timed through the
    oracle and reported with rows/s and the full-config extrapolation; the
    GPU speedup appears only where a GPU time for the op is given."""
    import bench

    out = bench.cpu_suite("c1", {"swiglu": {"us_median": 10.0}}, budget_s=0.01)
    assert set(out) == {"embedding_f32", "add_rmsnorm", "rope_qk", "swiglu"}
    for name, rec in out.items():
        assert rec["rows_per_s"] > 0 and rec["us_full_config_est"] > 0
        assert ("gpu_speedup" in rec) == (name == "swiglu")
