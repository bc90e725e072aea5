"""Bucket pickers against the reference's own examples and rules (scripts/tabicl_tpu_bucketed.py:
36-61 constants and pick_bucket, :74-80 pick_row_bucket docstring, :86-92 pick_feature_bucket
docstring) and its best preset's steps (scripts/benchmark_inference.py:239: rows 4096, features 4)."""
import sys
from pathlib import Path

import pytest

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "tabiclv2-torchtpu-v5p-benchmark_amd"))
import tabicl_mi355_buckets as bk  # noqa: E402


def test_pick_bucket_rules():
    assert bk.pick_bucket(0, bk.ROW_BUCKETS) == 1024
    assert bk.pick_bucket(-5, bk.TEST_ROW_BUCKETS) == 256
    assert bk.pick_bucket(1024, bk.ROW_BUCKETS) == 1024
    assert bk.pick_bucket(1025, bk.ROW_BUCKETS) == 2048
    assert bk.pick_bucket(45000, bk.ROW_BUCKETS) == 65536
    # above the largest bucket: next multiple of 1024
    assert bk.pick_bucket(600000, bk.ROW_BUCKETS) == 600064
    assert bk.pick_bucket(17, bk.FEATURE_BUCKETS) == 32
    assert bk.pick_bucket(513, bk.FEATURE_BUCKETS) == 1024


def test_row_bucket_step(monkeypatch):
    monkeypatch.delenv("TABICL_TPU_ROW_BUCKET_STEP", raising=False)
    assert bk.pick_row_bucket(45000) == 65536
    assert bk.pick_row_bucket(50000) == 65536
    # the docstring's examples for N = 8192
    assert bk.pick_row_bucket(45000, step=8192) == 49152
    assert bk.pick_row_bucket(50000, step=8192) == 57344
    # the best preset (row step 4096): 45,000 train rows -> 45,056 cache rows
    assert bk.pick_row_bucket(45000, step=4096) == 45056
    # at or below 16384 the power-of-two buckets hold
    assert bk.pick_row_bucket(10000, step=8192) == 16384
    monkeypatch.setenv("TABICL_TPU_ROW_BUCKET_STEP", "8192")
    assert bk.pick_row_bucket(45000) == 49152


def test_feature_bucket_step(monkeypatch):
    monkeypatch.delenv("TABICL_TPU_FEATURE_STEP", raising=False)
    assert bk.pick_feature_bucket(100) == 128
    assert bk.pick_feature_bucket(100, step=8) == 104
    assert bk.pick_feature_bucket(3, step=8) == 16
    assert bk.pick_feature_bucket(100, step=4) == 100  # the best preset (feature step 4)
    monkeypatch.setenv("TABICL_TPU_FEATURE_STEP", "8")
    assert bk.pick_feature_bucket(100) == 104


@pytest.mark.parametrize("fn,val,want", [
    (bk.pick_test_row_bucket, 5000, 8192),
    (bk.pick_test_row_bucket, 100, 256),
    (bk.pick_estimator_bucket, 8, 8),
    (bk.pick_estimator_bucket, 2, 4),
    (bk.pick_batch_bucket, 3, 4),
])
def test_other_buckets(fn, val, want):
    assert fn(val) == want
