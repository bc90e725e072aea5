"""GPU parity of the small-head kernels (hx, hxq, pk_self, pk_cross) against the CPU oracle.

Shapes follow the reference's own test matrix (scripts/tests/test_pallas_attn.py:371-403) plus edge
cases. Bars (tests/parity.py): max abs error <= 2e-2 for bf16 inputs with
fp32 accumulation, <= 1e-4 for fp32 inputs, and <= 2e-2 (bf16) / 1e-3 (fp32) times max |ref|, against
the fp32/fp64 oracle on the same inputs.
"""
import numpy as np
import pytest
import torch

from oracle import attention as O
from parity import check

H = 8
E = 128

pytestmark = pytest.mark.gpu


def _attn():
    import tabicl_mi355_attn as pk
    return pk


def _gen(seed):
    return torch.Generator().manual_seed(seed)


class _Rope:
    """Minimal stand-in for upstream RotaryEmbedding (get_seq_pos / interleaved / freqs / forward)."""

    def __init__(self, dim=16, theta=100000.0, interleaved=False):
        self.interleaved = interleaved
        self.freqs = torch.tensor(O.textbook_freqs(dim, theta), dtype=torch.float32)

    def get_seq_pos(self, L, device=None, dtype=torch.float32):
        return torch.arange(L, device=device, dtype=dtype)

    def forward(self, seq, seq_len=None):
        f = seq.float().unsqueeze(-1) * self.freqs.to(seq.device)
        return f.repeat_interleave(2, dim=-1)


def _rope_np(rope, L):
    freqs = rope.freqs.double().numpy()
    return O.rope_tables_ref(freqs, L, E, H, rope.interleaved)


@pytest.mark.parametrize("name,B,Lq,Lk,dtype,bias", [
    ("col2_bf16", 4, 1024, 128, torch.bfloat16, False),
    ("col2_fp32", 4, 1024, 128, torch.float32, False),
    ("col1_bf16", 4, 128, 576, torch.bfloat16, False),
    ("row_bf16", 16, 104, 104, torch.bfloat16, False),
    ("row_bf16_bias", 16, 104, 104, torch.bfloat16, True),
    ("row_fp32_bias", 16, 108, 108, torch.float32, True),
    ("cls_bf16", 16, 4, 104, torch.bfloat16, False),
    ("ragged_bf16_bias", 3, 77, 1500, torch.bfloat16, True),
    ("one_key_fp32", 2, 5, 1, torch.float32, False),
])
def test_hx(dev, name, B, Lq, Lk, dtype, bias):
    pk = _attn()
    g = _gen(0)
    q = (torch.randn(B, Lq, E, generator=g) * 0.25).to(dtype)
    k = torch.randn(B, Lk, E, generator=g).to(dtype)
    v = torch.randn(B, Lk, E, generator=g).to(dtype)
    kb = None
    if bias:
        kb = torch.zeros(B, Lk)
        kb[:, Lk - 9:] = -1e30
    print(f"[hx] {name} B={B} Lq={Lq} Lk={Lk} {dtype}", flush=True)
    out = pk.hx_attention(q.to(dev), k.to(dev), v.to(dev), H, None if kb is None else kb.to(dev))
    torch.cuda.synchronize()
    ref = O.hx_ref(q, k, v, H, kb)
    assert out.shape == q.shape and out.dtype == dtype
    check(out, ref, dtype, "hx")


def test_hx_fp32_long_queries(dev):
    pk = _attn()
    g = _gen(1)
    q = torch.randn(2, 53248, E, generator=g) * 0.25
    k = torch.randn(2, 128, E, generator=g)
    v = torch.randn(2, 128, E, generator=g)
    out = pk.hx_attention(q.to(dev), k.to(dev), v.to(dev), H)
    ref = O.ref_attn(q, k, v, H).double().numpy()
    check(out, ref, torch.float32, "hx_fp32_long_queries")


def test_hx_shared_bias_matches_broadcast(dev):
    pk = _attn()
    g = _gen(2)
    q = (torch.randn(3, 40, E, generator=g) * 0.25).to(torch.bfloat16).to(dev)
    k = torch.randn(3, 200, E, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(3, 200, E, generator=g).to(torch.bfloat16).to(dev)
    kb = torch.randn(200, generator=g).to(dev)
    a = pk.hx_attention(q, k, v, H, kb)
    b = pk.hx_attention(q, k, v, H, kb.expand(3, 200).contiguous())
    assert torch.equal(a, b)


@pytest.mark.parametrize("name,B,Lq,Lk,valid,dtype", [
    ("col1_small_fp32", 4, 128, 4096, 3000, torch.float32),
    ("col1_small_bf16", 4, 128, 4096, 3000, torch.bfloat16),
    ("valid_full", 2, 128, 1000, 1000, torch.bfloat16),
    ("valid_not_tile_aligned", 2, 64, 777, 129, torch.bfloat16),
    ("valid_beyond_lk_clamped", 2, 16, 300, 100000, torch.float32),
    ("short_keys_resident", 3, 200, 100, 37, torch.bfloat16),
    ("short_keys_resident_none_valid", 2, 64, 128, 0, torch.bfloat16),
])
def test_hxq(dev, name, B, Lq, Lk, valid, dtype):
    pk = _attn()
    g = _gen(3)
    q = (torch.randn(B, Lq, E, generator=g) * 0.25).to(dtype)
    kv = torch.randn(B, Lk, 2 * E, generator=g).to(dtype)
    print(f"[hxq] {name}", flush=True)
    out = pk.hxq_attention(q.to(dev), kv.to(dev), torch.tensor(valid, dtype=torch.int32).to(dev), H)
    ref = O.hxq_ref(q, kv, np.array([min(valid, Lk)]), H)
    check(out, ref, dtype, "hxq")


def test_hxq_ragged_valid_and_empty(dev):
    pk = _attn()
    g = _gen(4)
    B, Lq, Lk = 4, 128, 2048
    q = (torch.randn(B, Lq, E, generator=g) * 0.25).to(torch.bfloat16)
    kv = torch.randn(B, Lk, 2 * E, generator=g).to(torch.bfloat16)
    valid = torch.tensor([2048, 1, 0, 1000], dtype=torch.int32)
    out = pk.hxq_attention(q.to(dev), kv.to(dev), valid.to(dev), H)
    ref = O.hxq_ref(q, kv, valid.numpy(), H)
    check(out, ref, torch.bfloat16, "hxq_ragged_valid_and_empty")
    assert torch.all(out[2] == 0)


def test_hxq_ragged_valid_and_empty_fp32(dev):
    # fp32 kernel: per-batch valid lengths (all keys, one key, none, a partial 128-key tile)
    pk = _attn()
    g = _gen(22)
    B, Lq, Lk = 4, 128, 2048
    q = torch.randn(B, Lq, E, generator=g) * 0.25
    kv = torch.randn(B, Lk, 2 * E, generator=g)
    valid = torch.tensor([2048, 1, 0, 1000], dtype=torch.int32)
    out = pk.hxq_attention(q.to(dev), kv.to(dev), valid.to(dev), H)
    ref = O.hxq_ref(q, kv, valid.numpy(), H)
    check(out, ref, torch.float32, "hxq_ragged_valid_and_empty_fp32")
    assert torch.all(out[2] == 0)


def test_fp32_stream_long_runs_with_bias(dev):
    # fp32 kernel over 128-key tiles with runs of 8 query blocks (4 per wave carried across the
    # tiles), a key bias with masked keys, and keys not a multiple of the tile
    pk = _attn()
    g = _gen(21)
    B, Lq, Lk = 512, 128, 300
    q = torch.randn(B, Lq, E, generator=g) * 0.25
    k = torch.randn(B, Lk, E, generator=g)
    v = torch.randn(B, Lk, E, generator=g)
    kb = torch.randn(B, Lk, generator=g)
    kb[:, 290:] = -1e30
    out = pk.hx_attention(q.to(dev), k.to(dev), v.to(dev), H, kb.to(dev)).cpu()
    for b in (0, 255, 511):
        ref = O.hx_ref(q[b:b + 1], k[b:b + 1], v[b:b + 1], H, kb[b:b + 1])
        check(out[b:b + 1], ref, torch.float32, "fp32_stream_long_runs_with_bias")


def test_hxq_inference_tile_subset(dev):
    # reference shape col1_infer_tile54 (54 x 128 queries over 53248 keys, 45000 valid); 6 of the
    # 54 batch elements keep the CPU oracle within seconds
    pk = _attn()
    g = _gen(5)
    B, Lq, Lk, valid = 6, 128, 53248, 45000
    q = (torch.randn(B, Lq, E, generator=g) * 0.25).to(torch.bfloat16)
    kv = torch.randn(B, Lk, 2 * E, generator=g).to(torch.bfloat16)
    out = pk.hxq_attention(q.to(dev), kv.to(dev), torch.tensor(valid).to(dev), H)
    ref = O.ref_attn(q.float(), kv[:, :valid, :E].float(), kv[:, :valid, E:].float(), H).double().numpy()
    check(out, ref, torch.bfloat16, "hxq_inference_tile_subset")


@pytest.mark.parametrize("name,B,L,dtype,interleaved,bias", [
    ("self_bf16_rope_halves", 16, 104, torch.bfloat16, False, False),
    ("self_bf16_rope_halves_bias", 16, 104, torch.bfloat16, False, True),
    ("self_fp32_rope_halves_bias", 16, 108, torch.float32, False, True),
    ("self_fp32_rope_pairs", 8, 104, torch.float32, True, False),
    ("self_bf16_norope", 4, 300, torch.bfloat16, None, False),
])
def test_pk_self(dev, name, B, L, dtype, interleaved, bias):
    pk = _attn()
    g = _gen(6)
    x = torch.randn(B, L, 3 * E, generator=g).to(dtype)
    rope = None if interleaved is None else _Rope(interleaved=interleaved)
    kb = None
    if bias:
        kb = torch.zeros(B, L)
        kb[:, L - 7:] = -1e30
    print(f"[pk_self] {name}", flush=True)
    out = pk.pk_self_attention(x.to(dev), H, None if kb is None else kb.to(dev), rope, 16 ** -0.5)
    ref = O.pk_self_ref(x, H, kb, None if rope is None else _rope_np(rope, L), 16 ** -0.5)
    assert out.shape == (B, L, E)
    check(out, ref, dtype, "pk_self")


@pytest.mark.parametrize("name,B,L,dtype,interleaved", [
    ("self_bf16_rot8_halves", 8, 104, torch.bfloat16, False),
    ("self_bf16_rot8_pairs", 8, 104, torch.bfloat16, True),
    ("self_fp32_rot8_halves", 4, 108, torch.float32, False),
])
def test_pk_self_partial_rotary(dev, name, B, L, dtype, interleaved):
    # rotary embedding over the first 8 of each head's 16 dims (cos = 1, sin = 0 beyond): the forms
    # other than full-width pairs / halves take the tiled kernel's generic RoPE
    pk = _attn()
    g = _gen(16)
    x = torch.randn(B, L, 3 * E, generator=g).to(dtype)
    rope = _Rope(dim=8, interleaved=interleaved)
    print(f"[pk_self partial rotary] {name}", flush=True)
    out = pk.pk_self_attention(x.to(dev), H, None, rope, 16 ** -0.5)
    ref = O.pk_self_ref(x, H, None, _rope_np(rope, L), 16 ** -0.5)
    check(out, ref, dtype, "pk_self_partial_rotary")


@pytest.mark.parametrize("name,B,Lq,Lk,dtype,interleaved", [
    ("cross_cls_bf16_rope", 16, 4, 104, torch.bfloat16, False),
    ("cross_col2_bf16", 4, 1024, 128, torch.bfloat16, None),
    ("cross_col1_bf16", 4, 128, 576, torch.bfloat16, None),
    ("cross_col2_fp32", 2, 4096, 128, torch.float32, None),
    ("cross_cls_bf16_rope_pairs", 16, 4, 104, torch.bfloat16, True),
])
def test_pk_cross(dev, name, B, Lq, Lk, dtype, interleaved):
    pk = _attn()
    g = _gen(7)
    x = torch.randn(B, Lq, E, generator=g).to(dtype)
    y = torch.randn(B, Lk, 2 * E, generator=g).to(dtype)
    rope = None if interleaved is None else _Rope(interleaved=interleaved)
    print(f"[pk_cross] {name}", flush=True)
    out = pk.pk_cross_attention(x.to(dev), y.to(dev), H, None, rope, 16 ** -0.5)
    rq = None if rope is None else _rope_np(rope, Lq)
    rk = None if rope is None else _rope_np(rope, Lk)
    ref = O.pk_cross_ref(x, y, H, None, rq, rk, 16 ** -0.5)
    check(out, ref, dtype, "pk_cross")


def test_pk_cross_broadcast_query_no_copy(dev):
    # inducing points expanded over the batch (batch stride 0) are read once by the kernel
    pk = _attn()
    g = _gen(8)
    ind = torch.randn(1, 128, E, generator=g).to(torch.bfloat16)
    kv = torch.randn(5, 300, 2 * E, generator=g).to(torch.bfloat16)
    q_exp = ind.to(dev).expand(5, 128, E)
    out = pk.pk_cross_attention(q_exp, kv.to(dev), H, None, None, 0.25)
    ref = O.pk_cross_ref(ind, kv, H, None, None, None, 0.25)
    assert out.shape == (5, 128, E)
    check(out, ref, torch.bfloat16, "pk_cross_broadcast_query_no_copy")


def test_all_keys_masked_by_bias_is_uniform(dev):
    # every key at -1e30: the reference's fp32 softmax sees equal scores -> uniform weights
    pk = _attn()
    g = _gen(9)
    q = torch.randn(2, 8, E, generator=g) * 0.25
    k = torch.randn(2, 20, E, generator=g)
    v = torch.randn(2, 20, E, generator=g)
    kb = torch.full((2, 20), -1e30)
    out = pk.hx_attention(q.to(dev), k.to(dev), v.to(dev), H, kb.to(dev))
    want = v.mean(dim=1, keepdim=True).expand_as(out.cpu())
    assert float((out.cpu() - want).abs().max()) <= 1e-4
    assert torch.isfinite(out).all()


@pytest.mark.parametrize("Lk", [100, 700])
def test_fp32_sharp_key_far_above_first_keys(dev, Lk):
    # fp32 kernel, resident (Lk <= 128) and streaming: one key per head whose score lies up to ~150 nats above
    # the first 16 keys' maximum (the fast pass's fixed reference) overflows its row-sum bound; those
    # blocks must come out of the exact pass equal to the oracle
    pk = _attn()
    g = _gen(12)
    q = torch.randn(3, 40, E, generator=g) * 0.25
    k = torch.randn(3, Lk, E, generator=g)
    v = torch.randn(3, Lk, E, generator=g)
    k[:, Lk - 5] = q[:, 7] * 80.0  # key Lk-5 aligns with query 7: score ~ 80 |q_7|^2 (30-150 nats) per head
    out = pk.hx_attention(q.to(dev), k.to(dev), v.to(dev), H)
    ref = O.hx_ref(q, k, v, H)
    assert torch.isfinite(out).all()
    check(out, ref, torch.float32, "fp32_sharp_key_far_above_first_keys")


def test_no_nan_with_garbage_past_valid(dev):
    # NaN/inf in key/value rows past valid must not leak into the output
    pk = _attn()
    g = _gen(10)
    q = (torch.randn(2, 32, E, generator=g) * 0.25).to(torch.bfloat16)
    kv = torch.randn(2, 500, 2 * E, generator=g).to(torch.bfloat16)
    kv[:, 300:] = float("nan")
    out = pk.hxq_attention(q.to(dev), kv.to(dev), torch.tensor(300).to(dev), H)
    assert torch.isfinite(out.float()).all()
    ref = O.hxq_ref(q, kv[:, :300], np.array([300]), H)
    check(out, ref, torch.bfloat16, "no_nan_with_garbage_past_valid")


# --- streaming kernel (bf16, Lk > 128, no RoPE / key bias): reference-point moves, key splits ---

@pytest.mark.parametrize("name,B,Lq,Lk", [
    ("multi_query_groups", 2, 300, 700),
    ("ragged_queries", 3, 77, 1500),
    ("one_tile_past_resident", 2, 64, 129),
])
def test_stream_shapes(dev, name, B, Lq, Lk):
    pk = _attn()
    g = _gen(11)
    q = (torch.randn(B, Lq, E, generator=g) * 0.25).to(torch.bfloat16)
    k = torch.randn(B, Lk, E, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Lk, E, generator=g).to(torch.bfloat16)
    print(f"[stream] {name}", flush=True)
    out = pk.hx_attention(q.to(dev), k.to(dev), v.to(dev), H)
    check(out, O.hx_ref(q, k, v, H), torch.bfloat16, "stream_shapes")


@pytest.mark.parametrize("name,qscale,kshift", [
    ("large_scores", 3.0, 0.0),          # scores reach ~2^70 over the first tile's scale
    ("very_negative_scores", -3.0, 5.0),  # every score ~ -240 nats: exp underflows without a move
])
def test_stream_reference_moves(dev, name, qscale, kshift):
    pk = _attn()
    g = _gen(12)
    B, Lq, Lk = 2, 128, 3000
    if kshift:
        q = torch.full((B, Lq, E), qscale) + 0.1 * torch.randn(B, Lq, E, generator=g)
    else:
        q = qscale * torch.randn(B, Lq, E, generator=g)
    q = q.to(torch.bfloat16)
    kv = (torch.randn(B, Lk, 2 * E, generator=g) + torch.cat(
        [torch.full((E,), kshift), torch.zeros(E)])).to(torch.bfloat16)
    print(f"[stream] {name}", flush=True)
    out = pk.hxq_attention(q.to(dev), kv.to(dev), torch.tensor(2900, dtype=torch.int32).to(dev), H)
    assert torch.isfinite(out.float()).all()
    check(out, O.hxq_ref(q, kv, np.array([2900]), H), torch.bfloat16, "stream_reference_moves")


def test_stream_split_matches_unsplit(dev):
    # the key-split path (workspace given) against the one-pass path (no workspace) of the same
    # library call, and both against the oracle on a subset of rows
    import tabicl_mi355_native as nat
    pk = _attn()
    g = _gen(13)
    B, Lq, Lk = 2, 128, 40000
    q = (torch.randn(B, Lq, E, generator=g) * 0.25).to(torch.bfloat16).to(dev)
    kv = torch.randn(B, Lk, 2 * E, generator=g).to(torch.bfloat16).to(dev)
    valid = torch.tensor([39000, 20001], dtype=torch.int32).to(dev)
    nbytes = int(nat.load().tabicl_hxq_workspace_bytes(B, Lq, Lk, E, H, 0))
    assert nbytes > 0, "this shape should split its keys"
    split = pk.hxq_attention(q, kv, valid, H)
    one = torch.empty_like(q)
    nat.call("tabicl_hxq_fwd", valid.data_ptr(), B, q.data_ptr(), kv.data_ptr(), one.data_ptr(), B, Lq, Lk, E,
             H, 0, None, 0, nat.stream_of(q))
    torch.cuda.synchronize()
    assert float((split.float() - one.float()).abs().max()) <= 1e-2
    ref = O.hxq_ref(q[:, :16].cpu(), kv.cpu(), valid.cpu().numpy(), H)
    check(split[:, :16], ref, torch.bfloat16, "stream_split_matches_unsplit")
    check(one[:, :16], ref, torch.bfloat16, "stream_split_matches_unsplit")


def test_c5_style_bucket_group(dev):
    # BASELINE config 5 in miniature: tables of different train sizes padded to one row bucket,
    # several sequences per table, hxq with valid = n_train per sequence, then pk_cross of all rows
    pk = _attn()
    g = _gen(14)
    L, per = 2048, 3
    n_train = [1100, 1900, 1337]
    B = per * len(n_train)
    valid = torch.tensor(n_train, dtype=torch.int32).repeat_interleave(per)
    q = (torch.randn(B, 128, E, generator=g) * 0.25).to(torch.bfloat16)
    kv = torch.randn(B, L, 2 * E, generator=g).to(torch.bfloat16)
    out = pk.hxq_attention(q.to(dev), kv.to(dev), valid.to(dev), H)
    check(out, O.hxq_ref(q, kv, valid.numpy(), H), torch.bfloat16, "c5_style_bucket_group")
    rows = torch.randn(B, L, E, generator=g).to(torch.bfloat16)
    ind = torch.randn(B, 128, 2 * E, generator=g).to(torch.bfloat16)
    out2 = pk.pk_cross_attention(rows.to(dev), ind.to(dev), H, None, None, 0.25)
    sub = slice(0, 300)
    check(out2[:, sub], O.pk_cross_ref(rows[:, sub], ind, H, None, None, None, 0.25), torch.bfloat16, "c5_style_bucket_group")


# --- resident kernel (bf16, Lk <= 128): key-group counts, masking modes, recompute, long runs ---

@pytest.mark.parametrize("name,B,Lq,Lk,bias", [
    ("one_key", 3, 40, 1, False),                 # one 32-key group, keys past Lk masked
    ("one_group_full", 3, 40, 32, False),         # no masking at all
    ("two_groups_ragged", 3, 40, 50, False),
    ("three_groups_full", 3, 40, 96, False),
    ("four_groups_key_bias", 4, 104, 104, True),  # key bias: the additive term on every group
])
def test_resident_key_groups(dev, name, B, Lq, Lk, bias):
    pk = _attn()
    g = _gen(15)
    q = (torch.randn(B, Lq, E, generator=g) * 0.25).to(torch.bfloat16)
    k = torch.randn(B, Lk, E, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Lk, E, generator=g).to(torch.bfloat16)
    kb = None
    if bias:
        kb = torch.randn(B, Lk, generator=g) * 2.0
        kb[:, Lk - 5:] = -1e30
    print(f"[resident] {name}", flush=True)
    out = pk.hx_attention(q.to(dev), k.to(dev), v.to(dev), H, None if kb is None else kb.to(dev))
    check(out, O.hx_ref(q, k, v, H, kb), torch.bfloat16, "resident_key_groups")


def test_resident_sums_out_of_range(dev):
    # rows whose exp2 sums leave [2^-64, 2^64] are recomputed with the row maximum subtracted:
    # batch 0 has every key at bias -60 (sums underflow), batch 1 has every other query scaled
    # x120 (sums overflow, waves mix recomputed and kept rows), batch 2 stays in range
    pk = _attn()
    g = _gen(16)
    B, Lq, Lk = 3, 80, 128
    q = torch.randn(B, Lq, E, generator=g) * 0.25
    q[1, 0::2] *= 120.0
    q = q.to(torch.bfloat16)
    k = torch.randn(B, Lk, E, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Lk, E, generator=g).to(torch.bfloat16)
    kb = torch.zeros(B, Lk)
    kb[0] = -60.0
    out = pk.hx_attention(q.to(dev), k.to(dev), v.to(dev), H, kb.to(dev))
    assert torch.isfinite(out.float()).all()
    check(out, O.hx_ref(q, k, v, H, kb), torch.bfloat16, "resident_sums_out_of_range")


def test_resident_all_keys_masked_bf16_is_uniform(dev):
    pk = _attn()
    g = _gen(17)
    q = (torch.randn(2, 24, E, generator=g) * 0.25).to(torch.bfloat16)
    k = torch.randn(2, 20, E, generator=g).to(torch.bfloat16)
    v = torch.randn(2, 20, E, generator=g).to(torch.bfloat16)
    kb = torch.full((2, 20), -1e30)
    out = pk.hx_attention(q.to(dev), k.to(dev), v.to(dev), H, kb.to(dev))
    want = v.double().mean(dim=1, keepdim=True).expand(2, 24, E).numpy()
    check(out, want, torch.bfloat16, "resident_all_keys_masked_bf16_is_uniform")


def test_resident_long_query_runs(dev):
    # enough 16-query blocks that each workgroup walks several (two-buffer loop, odd tail block,
    # a partial last block of 6 rows)
    pk = _attn()
    g = _gen(18)
    B, Lq, Lk = 80, 3990, 128
    x = torch.randn(B, Lq, E, generator=g).to(torch.bfloat16)
    y = torch.randn(B, Lk, 2 * E, generator=g).to(torch.bfloat16)
    out = pk.pk_cross_attention(x.to(dev), y.to(dev), H, None, None, 0.25).cpu()
    for b in (0, 41, 79):
        ref = O.pk_cross_ref(x[b:b + 1], y[b:b + 1], H, None, None, None, 0.25)
        check(out[b:b + 1], ref, torch.bfloat16, "resident_long_query_runs")


def test_resident_long_runs_rope(dev):
    # C2-like row attention with RoPE, several 16-query blocks per workgroup
    pk = _attn()
    g = _gen(19)
    B, L = 2048, 104
    x = torch.randn(B, L, 3 * E, generator=g).to(torch.bfloat16)
    rope = _Rope(interleaved=False)
    out = pk.pk_self_attention(x.to(dev), H, None, rope, 16 ** -0.5).cpu()
    tabs = _rope_np(rope, L)
    for b in (0, 1023, 2047):
        ref = O.pk_self_ref(x[b:b + 1], H, None, tabs, 16 ** -0.5)
        check(out[b:b + 1], ref, torch.bfloat16, "resident_long_runs_rope")


@pytest.mark.parametrize("name,Lk,bias,hot", [
    ("four_groups", 128, False, False),              # no b2 term
    ("four_groups_key_bias", 128, True, False),      # b2 on every group (key bias, masked tail)
    ("four_groups_last_partial", 120, False, False),  # b2 on the last group only
    ("two_groups_last_partial", 60, False, False),
    ("one_group", 32, False, False),
    ("sums_out_of_range", 128, True, True),          # exact-maximum recompute, mixed waves
])
def test_resident_exact_scale_long_runs(dev, name, Lk, bias, hot):
    # runs of more than 8 16-query blocks per workgroup with a power-of-two scale: the K operand
    # carries scale log2e as bf16 high parts and remainders (the exact-scale form the column ISAB-2
    # takes at C3 / C5 sizes), under every b2 mode and the exact-maximum recompute.
    # 70 x 16000 queries: odd runs of 9 blocks, and the last run of each element holds 10 rows
    pk = _attn()
    g = torch.Generator(device=dev)
    g.manual_seed(21)
    B, Lq = 70, 16000
    q = torch.randn(B, Lq, E, generator=g, device=dev) * 0.25
    if hot:
        q[1, 0::2] *= 120.0  # sums past 2^64 on every other query
    q = q.to(torch.bfloat16)
    k = torch.randn(B, Lk, E, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(B, Lk, E, generator=g, device=dev).to(torch.bfloat16)
    kb = None
    if bias:
        kb = torch.randn(B, Lk, generator=g, device=dev) * 2.0
        kb[:, Lk - 5:] = -1e30
        if hot:
            kb[0] = -60.0  # sums below 2^-64
    print(f"[resident exact] {name}", flush=True)
    out = pk.hx_attention(q, k, v, H, kb).cpu()
    assert torch.isfinite(out.float()).all()
    qc, kc, vc = q.cpu(), k.cpu(), v.cpu()
    kbc = None if kb is None else kb.cpu()
    for b in (0, 1, 69):
        rows = np.r_[0:200, Lq - 300:Lq]
        ref = O.hx_ref(qc[b:b + 1, rows], kc[b:b + 1], vc[b:b + 1], H, None if kbc is None else kbc[b:b + 1])
        check(out[b:b + 1, rows], ref, torch.bfloat16, "resident_exact_scale_long_runs")


@pytest.mark.parametrize("interleaved", [False, True])
def test_resident_long_runs_cross_rope(dev, interleaved):
    # pk_cross with RoPE (positions 0..L-1 on both sides) and runs of several 16-query blocks per
    # workgroup (the cos / sin buffer refilled block by block), keys not a multiple of 32
    pk = _attn()
    g = _gen(20)
    B, Lq, Lk = 80, 3990, 100
    x = torch.randn(B, Lq, E, generator=g).to(torch.bfloat16)
    y = torch.randn(B, Lk, 2 * E, generator=g).to(torch.bfloat16)
    rope = _Rope(interleaved=interleaved)
    out = pk.pk_cross_attention(x.to(dev), y.to(dev), H, None, rope, 16 ** -0.5).cpu()
    rq, rk = _rope_np(rope, Lq), _rope_np(rope, Lk)
    for b in (0, 41, 79):
        ref = O.pk_cross_ref(x[b:b + 1], y[b:b + 1], H, None, rq, rk, 16 ** -0.5)
        check(out[b:b + 1], ref, torch.bfloat16, "resident_long_runs_cross_rope")
