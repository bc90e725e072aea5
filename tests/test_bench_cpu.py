"""CPU tests of bench.py's host logic: the C5 table draw and its buckets, and the CPU-baseline helpers
(timed on tiny inputs here; on the GPU box they time bounded samples of the benchmark's inputs)."""
import numpy as np
import pytest
import torch

import bench
from oracle import attention as O


def test_c5_tables_follow_the_config():
    # 64 tables, n_train log-uniform in [500, 10000], n_test = 10% of it, fixed seed
    n_train, n_test = bench.c5_tables()
    assert len(n_train) == len(n_test) == 64
    assert n_train.min() >= 500 and n_train.max() <= 10000
    np.testing.assert_array_equal(n_test, np.round(0.1 * n_train).astype(int))
    a, _ = bench.c5_tables()
    np.testing.assert_array_equal(a, n_train)  # deterministic


def test_c5_buckets_are_powers_of_two_above_the_rows():
    n_train, n_test = bench.c5_tables()
    for n, m in zip(n_train, n_test):
        b = bench.c5_bucket(int(n + m))
        assert b in bench.C5_BUCKETS and b >= n + m and (b == 1024 or b // 2 < n + m)
    with pytest.raises(ValueError):
        bench.c5_bucket(40000)  # above the config's largest bucket


def test_median_time_runs_and_returns_the_result():
    calls = []

    def fn():
        calls.append(1)
        return len(calls)

    sec, out, reps = bench._median_time(fn, budget_s=10.0)
    assert reps == 3 and len(calls) == 4 and out == 4 and sec >= 0.0


def test_cpu_baseline_small_sample(monkeypatch):
    # the C4 CPU baseline on a tiny stand-in of one estimator's blocks: scaled by the estimator count,
    # error against a GPU-side output computed here by the same oracle is zero
    monkeypatch.setattr(bench, "TEST", 1200)
    g = torch.Generator().manual_seed(5)
    qs = [torch.randn(1, 8, 1200, 64, generator=g) for _ in range(2)]
    kvs = [(torch.randn(1, 8, 300, 64, generator=g), torch.randn(1, 8, 300, 64, generator=g)) for _ in range(2)]
    outs = [O.splash_sdpa_torch(q, k, v) for q, (k, v) in zip(qs, kvs)]
    rec = bench.cpu_baseline(qs, kvs, outs)
    assert rec["unit"] == "ms" and rec["kind"] == "port" and rec["value"] > 0
    assert rec["max_abs_err_gpu_vs_cpu"] == 0.0
    assert f"scaled x{bench.EST}" in rec["sample"] and "all 2 blocks" in rec["sample"]
