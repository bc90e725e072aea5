"""Host logic of the composed cached-KV query (tabicl_mi355_query) on the CPU: the column and row stages
run with the HIP attention calls replaced by the oracle (pk_cross_ref / pk_self_ref in float64) and
float64 weights, and must equal the float64 restatement of tests/query_ref.py to rounding. This pins the
composition itself (feature grouping and its wrap-around past the real features, the reserved skip
columns, the skip-column refill, pre-norm residual layers, CLS tokens, the feature key mask, the CLS-only
last row block with RoPE on both sides, out-LayerNorm and flattening); the kernels are pinned by the GPU
tests. Bar: 1e-9 absolute (both sides compute in float64 with the same oracle)."""
import types

import numpy as np
import pytest
import torch

from oracle import attention as O
from query_ref import C, NI, E, H, Rope, as_f64, column_ref, grouping_loops, model, row_ref

B, T, NF = 2, 12, 10


def _fake_pk():
    def pk_cross_attention(q, kv, h, key_bias, rope, scale, q_len=None):
        lead, Lq, Lk = q.shape[:-2], q.shape[-2], kv.shape[-2]
        q3, kv3 = q.reshape(-1, Lq, E), kv.reshape(-1, Lk, 2 * E)
        kb = None if key_bias is None else np.broadcast_to(
            key_bias.double().numpy().reshape(*key_bias.shape[:-1], Lk), (*lead, Lk)).reshape(-1, Lk)
        tq = tk = None
        if rope is not None:
            tq = O.rope_tables_ref(rope.freqs.double().numpy(), Lq, E, h, rope.interleaved)
            tk = O.rope_tables_ref(rope.freqs.double().numpy(), Lk, E, h, rope.interleaved)
        out = O.pk_cross_ref(q3, kv3, h, kb, tq, tk, scale)
        return torch.from_numpy(out).to(q.dtype).reshape(*lead, Lq, E)

    def pk_self_attention(qkv, h, key_bias, rope, scale):
        lead, L = qkv.shape[:-2], qkv.shape[-2]
        kb = None if key_bias is None else np.broadcast_to(
            key_bias.double().numpy().reshape(*key_bias.shape[:-1], L), (*lead, L)).reshape(-1, L)
        tabs = None if rope is None else O.rope_tables_ref(rope.freqs.double().numpy(), L, E, h, rope.interleaved)
        out = O.pk_self_ref(qkv.reshape(-1, L, 3 * E), h, kb, tabs, scale)
        return torch.from_numpy(out).to(qkv.dtype).reshape(*lead, L, E)

    return types.SimpleNamespace(pk_cross_attention=pk_cross_attention, pk_self_attention=pk_self_attention)


@pytest.fixture()
def Q(monkeypatch):
    import tabicl_mi355_query as q
    monkeypatch.setattr(q, "_pk", _fake_pk())
    monkeypatch.setattr(q._nat, "require_device", lambda *ts: None)
    return q


def test_feature_grouping_matches_index_loops(Q):
    g = torch.Generator().manual_seed(1)
    X = torch.randn(3, 5, 11, generator=g, dtype=torch.float64)
    d = torch.tensor([11, 7, 1])
    got = Q.feature_grouping(X, d)
    assert torch.equal(got, torch.from_numpy(grouping_loops(X.numpy(), d.numpy())))
    assert torch.equal(Q.feature_grouping(X), Q.feature_grouping(X, torch.tensor([11, 11, 11])))


@pytest.mark.parametrize("d", [[NF, NF], [NF, NF - 3]], ids=["all_real", "padded_features"])
def test_column_and_row_stages_match_restatement(Q, d):
    w, g = model(torch.float64, seed=91)
    w = as_f64(w)  # LayerNorm weights too: the norms compute in their weights' dtype
    X = torch.randn(B, T, NF, generator=g, dtype=torch.float64)
    d = torch.tensor(d)
    cache = Q.ColumnKVCache(3, B, NF + C, NI, E, torch.float64, "cpu")
    for b in range(3):
        cache.append_projected(b, torch.randn(B, NF + C, NI, E, generator=g, dtype=torch.float64), w.column.blocks[b])
    src = Q.column_stage(X, d, cache, w.column)
    ref = column_ref(X, d, cache.kv, w.column)
    assert src.shape == (B, NF + C, T, E)
    assert torch.equal(src[:, :C], torch.full_like(src[:, :C], -100.0))
    assert float((src - ref).abs().max()) <= 1e-9
    reprs = Q.row_stage(src, d, w.row, Rope())
    ref_r = row_ref(src, d, w.row, Rope())
    assert reprs.shape == (B, T, C * E)
    assert float((reprs - ref_r).abs().max()) <= 1e-9


def test_padded_feature_slots_do_not_reach_the_cls_rows(Q):
    # the row stage's key mask hides token slots >= d + num_cls: changing their column output changes
    # nothing in the row representation
    w, g = model(torch.float64, seed=92)
    w = as_f64(w)
    src = torch.randn(B, NF + C, T, E, generator=g, dtype=torch.float64)
    d = torch.tensor([NF - 4, NF - 4])
    a = Q.row_stage(src, d, w.row, Rope())
    src2 = src.clone()
    src2[:, C + NF - 4:] = torch.randn(B, 4, T, E, generator=g, dtype=torch.float64) * 5
    b = Q.row_stage(src2, d, w.row, Rope())
    assert float((a - b).abs().max()) <= 1e-12
