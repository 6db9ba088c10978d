"""Host-side pieces of the measurement: the synthetic workloads and bench.py's CLI contract."""
from __future__ import annotations

import json
import os
import subprocess
import sys

import numpy as np

from vllm_webgpu_amd import workloads as W

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_headline_workload_shape_and_bytes():
    w = W.config(3, scale=0.02)              # same construction as the full C3, smaller
    B, V = w.shape
    assert w.logits.dtype == np.float32 and w.output_ids.dtype == np.int32
    assert np.all(w.temperature == np.float32(0.7)) and np.all(w.top_k == 50)
    assert np.all(w.top_p == np.float32(0.9)) and np.all(w.repetition == np.float32(1.1))
    assert w.uniforms.min() > 0 and w.uniforms.max() < 1
    # algorithmic bytes of the full C3 with 50 survivors per row: 131,918,848
    z = np.zeros(256, np.float32)
    full = W.Workload("c3", np.zeros((256, 128256), np.float32), "f32", z + 0.7, z, z, z, z, z,
                      z, np.zeros((256, 512), np.int32), np.zeros((1, 1), np.float32))
    assert W.algorithmic_bytes(full, np.full(256, 50)) == 131_918_848


def test_workloads_are_deterministic():
    a, b = W.config(2, 0.1), W.config(2, 0.1)
    assert np.array_equal(a.logits, b.logits) and np.array_equal(a.uniforms, b.uniforms)
    c4 = W.config(4, 0.02)
    assert c4.dtype == "bf16" and c4.logits.dtype == np.uint16
    assert (c4.temperature == 0).sum() == c4.shape[0] // 8


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    msg = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in msg["error"]


def test_bench_reads_the_committed_traffic():
    """roofline.traffic comes from the committed rocprofv3 summary of the headline workload: the
    summary must name the sampling kernel and give a per-launch figure near the algorithmic
    bytes (no re-reads)."""
    import bench
    from vllm_webgpu_amd import workloads as W

    t = bench.pmc_traffic_bytes(3)
    assert t is not None
    w = W.config(3)
    alg = W.algorithmic_bytes(w, np.full(w.shape[0], 24))
    assert 0.95 * alg < t < 1.15 * alg
    for c in (2, 4, 5):  # every parity configuration has its own summary, traffic >= algorithmic
        wc = W.config(c, 0.01)
        t = bench.pmc_traffic_bytes(c)
        assert t is not None and t > 0
    assert bench.pmc_traffic_bytes(9) is None
