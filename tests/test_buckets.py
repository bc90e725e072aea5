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


# ---- dispatch plan (reference scripts/tabicl_tpu_bucketed.py:83, 1160-1162, 1184, 1222, 1298-1336) ----

def test_plan_prefill_fused_and_tiled(monkeypatch):
    monkeypatch.delenv("TABICL_TPU_ROW_BUCKET_STEP", raising=False)
    # small: 4 x 1024 x (16 + 4) = 81,920 elements, fused: the ICL stage takes the whole batch
    p = bk.plan_prefill(3, 700, 10)
    assert (p.batch_bkt, p.rows_bkt, p.features_bkt, p.tiled, p.icl_step) == (4, 1024, 16, False, 4)
    assert p.chunks() == [(0, 4)]
    # C4's fit: 8 x 65536 x 132 elements, tiled, 65536 padded rows: one estimator per ICL call
    p = bk.plan_prefill(8, 45000, 100)
    assert (p.batch_bkt, p.rows_bkt, p.features_bkt, p.tiled, p.icl_step) == (8, 65536, 128, True, 1)
    assert p.chunks() == [(i, i + 1) for i in range(8)]
    # tiled with 32768 <= rows < 65536: two per call
    p = bk.plan_prefill(8, 20000, 100)
    assert (p.rows_bkt, p.tiled, p.icl_step) == (32768, True, 2)
    assert p.chunks() == [(0, 2), (2, 4), (4, 6), (6, 8)]
    # tiled below 32768 rows: the whole batch
    p = bk.plan_prefill(32, 10000, 100)
    assert (p.rows_bkt, p.tiled, p.icl_step) == (16384, True, 32)
    # with a row step the one-per-call threshold is 40960 padded rows: 45,000 -> 45,056 (step 4096)
    p = bk.plan_prefill(8, 45000, 100, row_step=4096, feature_step=4)
    assert (p.rows_bkt, p.features_bkt, p.icl_step) == (45056, 100, 1)
    p = bk.plan_prefill(8, 40000, 100, row_step=4096)
    assert (p.rows_bkt, p.icl_step) == (40960, 1)
    p = bk.plan_prefill(8, 36000, 100, row_step=4096)
    assert (p.rows_bkt, p.icl_step) == (36864, 2)
    assert bk.icl_step_min_rows(0) == 65536 and bk.icl_step_min_rows(4096) == 40960


def test_plan_query_steps():
    pre = bk.plan_prefill(3, 700, 10)
    q = bk.plan_query(pre, 300)
    # test rows to 512; the batch (4) and feature (16) buckets come from the prefill
    assert (q.batch, q.batch_bkt, q.rows, q.rows_bkt, q.features_bkt, q.train_bkt) == (3, 4, 300, 512, 16, 1024)
    assert q.icl_step == 4  # 4 x 512 x 20 = 40,960 elements
    # the element count rule: B T_test (H + 4) above max_fused_elements -> one per call
    assert bk.plan_query(pre, 300, max_fused_elements=40959).icl_step == 1
    assert bk.plan_query(pre, 300, max_fused_elements=40960).icl_step == 4
    # a cache spanning 65536 padded train rows: one per call whatever the test rows
    big = bk.plan_prefill(8, 45000, 100)
    assert bk.plan_query(big, 256, max_fused_elements=10 ** 12, row_step=0).icl_step == 1


def test_pad_batch_and_unpad_output():
    import torch
    pre = bk.plan_prefill(3, 5, 6)
    x = torch.arange(3 * 5 * 6, dtype=torch.float64).view(3, 5, 6) + 1
    xp = bk.pad_batch(x, pre)
    assert xp.shape == (4, 1024, 16) and xp.dtype == torch.float32
    assert torch.equal(xp[:3, :5, :6], x.float())
    assert float(xp[:3, 5:].abs().sum()) == 0 and float(xp[:3, :, 6:].abs().sum()) == 0
    assert torch.equal(xp[3], xp[0])  # the padded element repeats element 0
    y = torch.ones(3, 5)
    assert bk.pad_batch(y, pre).shape == (4, 1024)
    reps = torch.randn(3, 5, 7)
    assert bk.pad_batch(reps, pre, pad_features=False).shape == (4, 1024, 7)
    with pytest.raises(ValueError):
        bk.pad_batch(torch.zeros(2, 5, 6), pre)
    q = bk.plan_query(pre, 5)
    raw = torch.randn(4, 256, 10)
    out = bk.unpad_output(raw, q)
    assert torch.equal(out, raw[:3, :5])
    out = bk.unpad_output(raw, q, num_classes=4)
    assert torch.equal(out, raw[:3, :5, :4])
    prob = bk.unpad_output(raw, q, num_classes=4, return_logits=False, softmax_temperature=0.5)
    e = torch.exp(raw[:3, :5, :4] * 2.0)
    assert torch.allclose(prob, e / e.sum(-1, keepdim=True), atol=1e-6)
