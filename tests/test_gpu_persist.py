"""GPU parity of the persistent resident-keys kernel (sh_persist_kernel), which takes bf16 calls over
many batch elements of 97..112 keys with 1 or 7 query blocks per element: the row stage's 104-token
self attention (pk_self, hx), the CLS queries (pk_cross) and few-query hxq over short key sets.

Each case is checked two ways:
  - against the fp64 oracle on a few batch elements (first, middle, last): max abs error <= 2e-2;
  - bit for bit against the one-element-per-workgroup resident kernel on the same elements. That
    kernel runs when the batch is smaller than two elements per persistent workgroup (a prefix of the
    same inputs) or when the RoPE tables are the tiled [L, 128] form.
Batches of 1100 and 4100 elements leave some workgroups an extra element. Rows of K / V past an
element's valid length hold NaN: they must never be read.
"""
import numpy as np
import pytest
import torch

from oracle import attention as O

pytestmark = pytest.mark.gpu
H, E = 8, 128
TOL = 2e-2


class _Rope:
    def __init__(self, interleaved):
        self.interleaved = interleaved
        self.freqs = torch.tensor(np.asarray(O.textbook_freqs(16, 10000.0)), dtype=torch.float32)

    def get_seq_pos(self, L, device=None, dtype=torch.float32):
        return torch.arange(L, device=device, dtype=dtype)

    def forward(self, seq, seq_len=None):
        f = seq.float().unsqueeze(-1) * self.freqs.to(seq.device)
        return f.repeat_interleave(2, dim=-1) if self.interleaved else torch.cat([f, f], dim=-1)


def _rope_np(rope, L):
    return O.rope_tables_ref(rope.freqs.double().numpy(), L, E, H, rope.interleaved)


def _err(out, ref):
    return float(np.abs(out.detach().double().cpu().numpy() - ref).max())


def _sample(B):
    return sorted({0, 1, B // 2, B - 1})


@pytest.mark.parametrize("name,B,interleaved,bias", [
    ("rope_halves", 1100, False, False),
    ("rope_pairs_bias", 1100, True, True),
    ("rope_halves_bias", 4100, False, True),  # the row stage with padded feature slots
    ("rope_pairs", 1100, True, False),
])
def test_pk_self_row_stage(dev, name, B, interleaved, bias):
    import tabicl_mi355_attn as pk
    g = torch.Generator().manual_seed(90)
    L = 104
    x = torch.randn(B, L, 3 * E, generator=g).to(torch.bfloat16)
    kb = None
    if bias:
        kb = torch.randn(B, L, generator=g)
        kb[:, L - 3:] = float(torch.finfo(torch.float32).min)  # padded feature slots
        kb[torch.rand(B, L, generator=g) < 0.05] = -1e30
    rope = _Rope(interleaved)
    xd, kbd = x.to(dev), None if kb is None else kb.to(dev)
    print(f"[persist] pk_self {name}", flush=True)
    with torch.no_grad():
        out = pk.pk_self_attention(xd, H, kbd, rope, 0.25)  # shared tables: persistent kernel
        cos, sin, rc, half, r = pk.rope_tables(rope, L, E, H, dev)  # tiled tables: the other kernel
        tiled = pk.PK_SELF(xd, pk._bias_arg(kbd, (B,), L, dev), cos, sin, H, 128, rc, half, r, 0, 0.25)
    torch.cuda.synchronize()
    assert torch.equal(out, tiled), name
    for b in _sample(B):
        ref = O.pk_self_ref(x[b:b + 1], H, None if kb is None else kb[b:b + 1], _rope_np(rope, L), 0.25)
        assert _err(out[b:b + 1], ref) <= TOL, (name, b)


def test_hx_no_rope_matches_prefix_call(dev):
    import tabicl_mi355_attn as pk
    g = torch.Generator().manual_seed(91)
    B, L = 1100, 104
    q = (torch.randn(B, L, E, generator=g) * 0.25).to(torch.bfloat16)
    k = torch.randn(B, L, E, generator=g).to(torch.bfloat16)
    v = torch.randn(B, L, E, generator=g).to(torch.bfloat16)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    print("[persist] hx 104 keys", flush=True)
    out = pk.hx_attention(qd, kd, vd, H)
    part = pk.hx_attention(qd[:300], kd[:300], vd[:300], H)  # 300 elements: the other kernel
    torch.cuda.synchronize()
    assert torch.equal(out[:300], part)
    for b in _sample(B):
        assert _err(out[b:b + 1], O.hx_ref(q[b:b + 1], k[b:b + 1], v[b:b + 1], H)) <= TOL, b


@pytest.mark.parametrize("shared_len", [False, True])
def test_hxq_short_keys_per_element_valid(dev, shared_len):
    # one query block per element over 104 packed keys, valid length per element (0 included: zeros)
    # or one for all; rows past it hold NaN
    import tabicl_mi355_attn as pk
    g = torch.Generator().manual_seed(92)
    B, Lq, Lk = 4100, 16, 104
    q = (torch.randn(B, Lq, E, generator=g) * 0.25).to(torch.bfloat16)
    kv = torch.randn(B, Lk, 2 * E, generator=g).to(torch.bfloat16)
    if shared_len:
        valid = np.array([77])
    else:
        valid = np.random.default_rng(3).integers(0, Lk + 1, B)
        valid[:4] = [0, 1, Lk, 50]
    for b in range(B):
        kv[b, int(valid[0] if shared_len else valid[b]):] = float("nan")
    vt = torch.tensor(valid, dtype=torch.int32, device=dev)
    qd, kvd = q.to(dev), kv.to(dev)
    print(f"[persist] hxq shared_len={shared_len}", flush=True)
    out = pk.hxq_attention(qd, kvd, vt, H)
    part = pk.hxq_attention(qd[:300], kvd[:300], vt if shared_len else vt[:300], H)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    assert torch.equal(out[:300], part)
    for b in _sample(B) + [2, 3]:
        vb = int(valid[0] if shared_len else valid[b])
        if vb == 0:
            assert float(out[b].abs().max()) == 0.0
            continue
        ref = O.hxq_ref(q[b:b + 1], kv[b:b + 1, :vb], np.array([vb]), H)
        assert _err(out[b:b + 1], ref) <= TOL, b


def test_pk_cross_cls_rope(dev):
    # the CLS queries: 4 rows over the 104 tokens, RoPE on both (q tables staged apart from the key
    # tables), one query block per element
    import tabicl_mi355_attn as pk
    g = torch.Generator().manual_seed(93)
    B, Lq, Lk = 4100, 4, 104
    q = (torch.randn(B, Lq, E, generator=g) * 0.5).to(torch.bfloat16)
    kv = torch.randn(B, Lk, 2 * E, generator=g).to(torch.bfloat16)
    rope = _Rope(False)
    qd, kvd = q.to(dev), kv.to(dev)
    print("[persist] pk_cross cls", flush=True)
    with torch.no_grad():
        out = pk.pk_cross_attention(qd, kvd, H, None, rope, 0.25)
        cq, sq, rc, half, r = pk.rope_tables(rope, Lq, E, H, dev)
        ck, sk, _, _, _ = pk.rope_tables(rope, Lk, E, H, dev)
        none = torch.empty(0, device=dev)
        tiled = pk.PK_CROSS(qd, kvd, none, cq, sq, ck, sk, H, 128, 4, rc, half, r, 0, 0.25)
    torch.cuda.synchronize()
    assert torch.equal(out, tiled)
    for b in _sample(B):
        ref = O.pk_cross_ref(q[b:b + 1], kv[b:b + 1], H, None, _rope_np(rope, Lq), _rope_np(rope, Lk), 0.25)
        assert _err(out[b:b + 1], ref) <= TOL, b


def test_repeat_calls_identical(dev):
    # the workgroups' element order and the LDS copies in flight must not leak between calls
    import tabicl_mi355_attn as pk
    g = torch.Generator().manual_seed(94)
    x = torch.randn(2048, 104, 3 * E, generator=g).to(torch.bfloat16).to(dev)
    rope = _Rope(False)
    with torch.no_grad():
        a = pk.pk_self_attention(x, H, None, rope, 0.25)
        b = pk.pk_self_attention(x, H, None, rope, 0.25)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_pk_cross_cls_rope_with_feature_mask(dev):
    # the CLS queries as the row stage runs them: a per-sequence key mask over the padded feature slots
    # (finfo.min, results/tpu_patch.diff:1253-1271) on top of RoPE
    import tabicl_mi355_attn as pk
    g = torch.Generator().manual_seed(95)
    B, Lq, Lk = 4100, 4, 104
    q = (torch.randn(B, Lq, E, generator=g) * 0.5).to(torch.bfloat16)
    kv = torch.randn(B, Lk, 2 * E, generator=g).to(torch.bfloat16)
    kb = torch.zeros(B, Lk)
    real = torch.randint(1, Lk + 1, (B,), generator=g)
    for b in range(B):
        kb[b, int(real[b]):] = float(torch.finfo(torch.float32).min)
    rope = _Rope(False)
    qd, kvd, kbd = q.to(dev), kv.to(dev), kb.to(dev)
    print("[persist] pk_cross cls masked", flush=True)
    with torch.no_grad():
        out = pk.pk_cross_attention(qd, kvd, H, kbd, rope, 0.25)
        cq, sq, rc, half, r = pk.rope_tables(rope, Lq, E, H, dev)
        ck, sk, _, _, _ = pk.rope_tables(rope, Lk, E, H, dev)
        tiled = pk.PK_CROSS(qd, kvd, pk._bias_arg(kbd, (B,), Lk, dev), cq, sq, ck, sk, H, 128, 4, rc, half, r, 0,
                            0.25)
    torch.cuda.synchronize()
    assert torch.equal(out, tiled)
    for b in _sample(B):
        ref = O.pk_cross_ref(q[b:b + 1], kv[b:b + 1], H, kb[b:b + 1], _rope_np(rope, Lq), _rope_np(rope, Lk), 0.25)
        assert _err(out[b:b + 1], ref) <= TOL, b


def test_hxq_short_keys_valid_and_key_mask(dev):
    # both a per-element valid length and a per-element key mask (random terms and finfo.min entries)
    import tabicl_mi355_attn as pk
    g = torch.Generator().manual_seed(96)
    B, Lq, Lk = 4100, 16, 104
    q = (torch.randn(B, Lq, E, generator=g) * 0.25).to(torch.bfloat16)
    kv = torch.randn(B, Lk, 2 * E, generator=g).to(torch.bfloat16)
    valid = torch.randint(1, Lk + 1, (B,), generator=g).to(torch.int32)
    kb = torch.randn(B, Lk, generator=g)
    kb[torch.rand(B, Lk, generator=g) < 0.1] = float(torch.finfo(torch.float32).min)
    kb[:, 0] = 0.0  # one finite key per row (a fully masked row has no defined softmax in fp64)
    for b in range(B):
        kv[b, int(valid[b]):] = float("nan")
    qd, kvd, vd, kbd = q.to(dev), kv.to(dev), valid.to(dev), kb.to(dev)
    print("[persist] hxq valid + mask", flush=True)
    out = pk.hxq_attention(qd, kvd, vd, H, kbd)
    part = pk.hxq_attention(qd[:300], kvd[:300], vd[:300], H, kbd[:300])
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    assert torch.equal(out[:300], part)
    for b in _sample(B):
        vb = int(valid[b])
        ref = O.attention_f64(q[b:b + 1].double().numpy(), kv[b:b + 1, :vb, :E].double().numpy(),
                              kv[b:b + 1, :vb, E:].double().numpy(), H, kb[b:b + 1, :vb].double().numpy())
        assert _err(out[b:b + 1], ref) <= TOL, b
