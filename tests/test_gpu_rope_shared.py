"""GPU check of the shared-table RoPE form (TABICL_ROPE_SHARED_TABLES): the forward kernels given one
head's [L, 16] columns of rope_tables' output must return exactly (bit for bit) what they return for
the tiled [L, 128] tables, for every forward kernel that reads tables: the resident bf16 kernel (row
stage, 104 tokens; CLS cross attention), the general bf16 kernel (keys past the resident limit, and a
partial-rotary form) and the fp32 kernel; and the backward kernels likewise (the fused short kernel,
the tiled dq / dk-dv pair, partial rotary, fp32). The tiled-table results are checked against the
oracle by test_gpu_smallhead.py and test_gpu_smallhead_bwd.py; the wrappers always pass the shared
form (the gradient tests run through it).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


class _Rope:
    def __init__(self, interleaved, rot=16):
        import numpy as np

        from oracle import attention as O
        self.interleaved = interleaved
        self.freqs = torch.tensor(np.asarray(O.textbook_freqs(rot, 10000.0)), dtype=torch.float32)

    def get_seq_pos(self, L, device=None, dtype=torch.float32):
        return torch.arange(L, device=device, dtype=dtype)

    def forward(self, seq, seq_len=None):
        f = (seq.float().unsqueeze(-1) * self.freqs.to(seq.device))
        return f.repeat_interleave(2, dim=-1) if self.interleaved else torch.cat([f, f], dim=-1)


@pytest.mark.parametrize("name,B,L,dtype,interleaved,rot", [
    ("row_resident_halves", 64, 104, torch.bfloat16, False, 16),
    ("row_resident_pairs", 16, 104, torch.bfloat16, True, 16),
    ("long_general_bf16", 4, 300, torch.bfloat16, False, 16),
    ("partial_rotary_bf16", 8, 104, torch.bfloat16, False, 8),
    ("fp32", 8, 104, torch.float32, False, 16),
])
def test_pk_self_shared_tables(dev, name, B, L, dtype, interleaved, rot):
    import tabicl_mi355_attn as pk
    g = torch.Generator().manual_seed(21)
    qkv = torch.randn(B, L, 384, generator=g).to(dtype).to(dev)
    bias = torch.zeros(B, 1, L, device=dev)
    bias[:, :, L - 3:] = -1e30
    rope = _Rope(interleaved, rot)
    cos, sin, rc, half, r = pk.rope_tables(rope, L, 128, 8, dev)
    lkp = -(-L // 128) * 128
    full = pk.PK_SELF(qkv, bias, cos, sin, 8, lkp, rc, half, r, 0, 0.25)
    cs, sn, rcs = pk._shared_tables(cos, sin, rc, 16)
    shared = pk.PK_SELF(qkv, bias, cs, sn, 8, lkp, rcs, half, r, 0, 0.25)
    torch.cuda.synchronize()
    assert torch.equal(full, shared), name


def test_pk_cross_shared_tables_cls(dev):
    import tabicl_mi355_attn as pk
    g = torch.Generator().manual_seed(22)
    q = torch.randn(256, 4, 128, generator=g).to(torch.bfloat16).to(dev)
    kv = torch.randn(256, 104, 256, generator=g).to(torch.bfloat16).to(dev)
    rope = _Rope(False)
    cq, sq, rc, half, r = pk.rope_tables(rope, 4, 128, 8, dev)
    ck, sk, _, _, _ = pk.rope_tables(rope, 104, 128, 8, dev)
    none = torch.empty(0, device=dev)
    full = pk.PK_CROSS(q, kv, none, cq, sq, ck, sk, 8, 128, 4, rc, half, r, 0, 0.25)
    cqs, sqs, _ = pk._shared_tables(cq, sq, rc, 16)
    cks, sks, rcs = pk._shared_tables(ck, sk, rc, 16)
    shared = pk.PK_CROSS(q, kv, none, cqs, sqs, cks, sks, 8, 128, 4, rcs, half, r, 0, 0.25)
    torch.cuda.synchronize()
    assert torch.equal(full, shared)


@pytest.mark.parametrize("name,B,Lq,Lk,dtype", [
    ("general_bf16", 4, 200, 300, torch.bfloat16),  # keys past the resident limit
    ("fp32", 4, 100, 200, torch.float32),
])
def test_pk_cross_shared_tables_general(dev, name, B, Lq, Lk, dtype):
    import tabicl_mi355_attn as pk
    g = torch.Generator().manual_seed(23)
    q = (torch.randn(B, Lq, 128, generator=g) * 0.5).to(dtype).to(dev)
    kv = torch.randn(B, Lk, 256, generator=g).to(dtype).to(dev)
    rope = _Rope(False)
    cq, sq, rc, half, r = pk.rope_tables(rope, Lq, 128, 8, dev)
    ck, sk, _, _, _ = pk.rope_tables(rope, Lk, 128, 8, dev)
    none = torch.empty(0, device=dev)
    lkp = -(-Lk // 128) * 128
    bq = pk._pick_bq(Lq, lkp)
    prec = pk._fp32_prec_code() if dtype == torch.float32 else 0
    full = pk.PK_CROSS(q, kv, none, cq, sq, ck, sk, 8, lkp, bq, rc, half, r, prec, 0.25)
    cqs, sqs, _ = pk._shared_tables(cq, sq, rc, 16)
    cks, sks, rcs = pk._shared_tables(ck, sk, rc, 16)
    shared = pk.PK_CROSS(q, kv, none, cqs, sqs, cks, sks, 8, lkp, bq, rcs, half, r, prec, 0.25)
    torch.cuda.synchronize()
    assert torch.equal(full, shared), name


@pytest.mark.parametrize("name,B,Lq,Lk,dtype,q_len", [
    ("resident_cls", 6, 40, 104, torch.bfloat16, [0, 1, 17, 40, 100, 16]),
    ("general_bf16", 3, 200, 300, torch.bfloat16, [200, 77, 0]),
    ("fp32", 3, 100, 128, torch.float32, [3, 100, 64]),
])
def test_pk_cross_ragged_with_rope(dev, name, B, Lq, Lk, dtype, q_len):
    # a ragged call with a RoPE module: the live rows are bit-identical to the plain call (both read the
    # shared tables), and the plain call matches the oracle on batch 0 (2e-2 bf16, 1e-4 fp32)
    import numpy as np

    import tabicl_mi355_attn as pk
    from oracle import attention as O
    g = torch.Generator().manual_seed(24)
    q = (torch.randn(B, Lq, 128, generator=g) * 0.5).to(dtype).to(dev)
    kv = torch.randn(B, Lk, 256, generator=g).to(dtype).to(dev)
    rope = _Rope(False)
    with torch.no_grad():
        ref = pk.pk_cross_attention(q, kv, 8, None, rope, 0.25)
        out = pk.pk_cross_attention(q, kv, 8, None, rope, 0.25, q_len=torch.tensor(q_len, dtype=torch.int32,
                                                                                    device=dev))
    torch.cuda.synchronize()
    for b in range(B):
        n = min(q_len[b], Lq)
        assert torch.equal(out[b, :n], ref[b, :n]), (name, b)
    freqs = rope.freqs.double().numpy()
    rq = O.rope_tables_ref(freqs, Lq, 128, 8, False)
    rk = O.rope_tables_ref(freqs, Lk, 128, 8, False)
    exp = O.pk_cross_ref(q[:1].cpu(), kv[:1].cpu(), 8, None, rq, rk, 0.25)
    err = float(np.abs(ref[:1].double().cpu().numpy() - exp).max())
    assert err <= (2e-2 if dtype == torch.bfloat16 else 1e-4), (name, err)


@pytest.mark.parametrize("name,B,L,dtype,interleaved,rot", [
    ("fused_short_halves", 16, 104, torch.bfloat16, False, 16),
    ("fused_short_pairs", 8, 104, torch.bfloat16, True, 16),
    ("tiled_long_bf16", 2, 300, torch.bfloat16, False, 16),
    ("partial_rotary_bf16", 4, 104, torch.bfloat16, False, 8),
    ("fp32", 4, 104, torch.float32, False, 16),
])
def test_pk_self_bwd_shared_tables(dev, name, B, L, dtype, interleaved, rot):
    import tabicl_mi355_attn as pk
    g = torch.Generator().manual_seed(25)
    qkv = torch.randn(B, L, 384, generator=g).to(dtype).to(dev)
    do = torch.randn(B, L, 128, generator=g).to(dtype).to(dev)
    bias = torch.zeros(B, 1, L, device=dev)
    bias[:, :, L - 3:] = -1e30
    rope = _Rope(interleaved, rot)
    cos, sin, rc, half, r = pk.rope_tables(rope, L, 128, 8, dev)
    lkp = -(-L // 128) * 128
    o = pk.PK_SELF(qkv, bias, cos, sin, 8, lkp, rc, half, r, 0, 0.25)
    full = pk.PK_SELF_BWD(qkv, bias, cos, sin, o, do, 8, lkp, rc, half, r, 0, 0.25)
    cs, sn, rcs = pk._shared_tables(cos, sin, rc, 16)
    shared = pk.PK_SELF_BWD(qkv, bias, cs, sn, o, do, 8, lkp, rcs, half, r, 0, 0.25)
    torch.cuda.synchronize()
    assert torch.isfinite(full.float()).all() and torch.equal(full, shared), name


@pytest.mark.parametrize("name,B,Lq,Lk", [("cls_fused_short", 64, 4, 104), ("tiled", 4, 200, 300)])
def test_pk_cross_bwd_shared_tables(dev, name, B, Lq, Lk):
    import tabicl_mi355_attn as pk
    g = torch.Generator().manual_seed(26)
    q = (torch.randn(B, Lq, 128, generator=g) * 0.5).to(torch.bfloat16).to(dev)
    kv = torch.randn(B, Lk, 256, generator=g).to(torch.bfloat16).to(dev)
    do = torch.randn(B, Lq, 128, generator=g).to(torch.bfloat16).to(dev)
    rope = _Rope(False)
    cq, sq, rc, half, r = pk.rope_tables(rope, Lq, 128, 8, dev)
    ck, sk, _, _, _ = pk.rope_tables(rope, Lk, 128, 8, dev)
    none = torch.empty(0, device=dev)
    lkp = -(-Lk // 128) * 128
    bq = pk._pick_bq(Lq, lkp)
    o = pk.PK_CROSS(q, kv, none, cq, sq, ck, sk, 8, lkp, bq, rc, half, r, 0, 0.25)
    full = pk.PK_CROSS_BWD(q, kv, none, cq, sq, ck, sk, o, do, 8, lkp, bq, rc, half, r, 0, 0.25)
    cqs, sqs, _ = pk._shared_tables(cq, sq, rc, 16)
    cks, sks, rcs = pk._shared_tables(ck, sk, rc, 16)
    shared = pk.PK_CROSS_BWD(q, kv, none, cqs, sqs, cks, sks, o, do, 8, lkp, bq, rcs, half, r, 0, 0.25)
    torch.cuda.synchronize()
    for a, b in zip(full, shared):
        assert torch.isfinite(a.float()).all() and torch.equal(a, b), name
