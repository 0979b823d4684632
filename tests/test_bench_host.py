"""bench.py's CPU-baseline bookkeeping: the thread count it sets is this process's physical-core share."""
import os

import bench


def test_host_cpu_share():
    h = bench.host_cpu()
    assert 1 <= h["threads"] <= h["physical_cores"] <= h["affinity_cpus"] <= h["logical_cpus"]
    for cap in h["caps"].values():
        assert h["threads"] <= cap
    assert h["model"]


def test_host_cpu_respects_omp_threads(monkeypatch):
    monkeypatch.setenv("OMP_NUM_THREADS", "1")
    assert bench.host_cpu()["threads"] == 1
    monkeypatch.setenv("OMP_NUM_THREADS", str(os.cpu_count() * 4))
    assert bench.host_cpu()["threads"] == bench.host_cpu()["physical_cores"]
