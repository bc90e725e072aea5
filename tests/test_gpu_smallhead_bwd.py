"""GPU parity of the small-head backward kernels (hx_bwd, pk_self_bwd, pk_cross_bwd) through torch
autograd, against the float64 oracle of the reference's backward (oracle.attention.*_bwd_ref).

Shapes follow the reference's gradient checks (scripts/tests/test_pallas_attn.py:51-78, 202-249 and
the matrix at :371-403), plus keys past the reference's 1024-key limit, a query set broadcast over
the batch, and fully masked keys. The upstream gradient is random N(0, 1); the kernel receives it in
the output dtype, and the oracle gets the same rounded values. Tolerance (written here): max abs
error <= 2e-2 * max(1, max |grad|) for bf16 inputs, <= 1e-4 * max(1, max |grad|) for fp32 inputs
(the forward's absolute bar, scaled by the gradient's magnitude when that exceeds 1).
"""
import numpy as np
import pytest
import torch

from oracle import attention as O

H = 8
E = 128
TOL = {torch.bfloat16: 2e-2, torch.float32: 1e-4}

pytestmark = pytest.mark.gpu


def _attn():
    import tabicl_mi355_attn as pk
    return pk


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _check(name, got, ref, dtype):
    got = got.detach().double().cpu().numpy()
    scale = max(1.0, float(np.abs(ref).max()))
    err = float(np.abs(got - ref).max())
    print(f"  {name}: max abs err {err:.3e} (ref max {np.abs(ref).max():.3e})", flush=True)
    assert err <= TOL[dtype] * scale, (name, err, scale)


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
    return O.rope_tables_ref(rope.freqs.double().numpy(), L, E, H, rope.interleaved)


@pytest.mark.parametrize("name,B,Lq,Lk,dtype,bias", [
    ("col2_bf16", 4, 1024, 128, torch.bfloat16, False),
    ("col2_fp32", 4, 1024, 128, torch.float32, False),
    ("col1_bf16", 4, 128, 576, torch.bfloat16, False),
    ("row_bf16", 16, 104, 104, torch.bfloat16, False),
    ("row_fp32_bias", 16, 108, 108, torch.float32, True),
    ("cls_bf16", 16, 4, 104, torch.bfloat16, False),
    ("long_keys_bf16", 2, 200, 3000, torch.bfloat16, True),   # past the reference's 1024-key limit
    ("long_keys_fp32", 2, 70, 1500, torch.float32, False),
    # fused short-sequence kernel (both lengths <= 128, bf16): edges of its range
    ("short_max_bf16_bias", 5, 128, 128, torch.bfloat16, True),
    ("short_one_bf16", 3, 1, 1, torch.bfloat16, False),
    ("short_ragged_bf16_bias", 7, 33, 77, torch.bfloat16, True),
    ("short_keys_past_128_bf16", 3, 40, 129, torch.bfloat16, False),
])
def test_hx_bwd(dev, name, B, Lq, Lk, dtype, bias):
    pk = _attn()
    g = _gen(30)
    q = (torch.randn(B, Lq, E, generator=g) * 0.25).to(dtype)
    k = torch.randn(B, Lk, E, generator=g).to(dtype)
    v = torch.randn(B, Lk, E, generator=g).to(dtype)
    kb = None
    if bias:
        kb = torch.zeros(B, Lk)
        kb[:, Lk - 9:] = -1e30
    go = torch.randn(B, Lq, E, generator=g)
    print(f"[hx_bwd] {name}", flush=True)
    qr, kr, vr = (t.to(dev).requires_grad_(True) for t in (q, k, v))
    out = pk.hx_attention(qr, kr, vr, H, None if kb is None else kb.to(dev))
    out.float().backward(go.to(dev))
    do = go.to(dtype)
    dq, dk, dv = O.hx_bwd_ref(q, k, v, H, do, kb)
    _check("dq", qr.grad, dq, dtype)
    _check("dk", kr.grad, dk, dtype)
    _check("dv", vr.grad, dv, dtype)


@pytest.mark.parametrize("name,B,L,dtype,interleaved,bias", [
    ("self_bf16_rope_halves", 16, 104, torch.bfloat16, False, False),
    ("self_fp32_rope_halves_bias", 16, 108, torch.float32, False, True),
    ("self_fp32_rope_pairs", 8, 104, torch.float32, True, False),
    ("self_bf16_norope_long", 2, 700, torch.bfloat16, None, False),
    ("self_bf16_rope_pairs", 8, 104, torch.bfloat16, True, False),
    ("self_bf16_rope_halves_bias_128", 4, 128, torch.bfloat16, False, True),
    # past 128 tokens with RoPE: the tiled dq / dk-dv kernels' RoPE instances (two key sweeps)
    ("self_bf16_rope_halves_long", 2, 300, torch.bfloat16, False, False),
    ("self_fp32_rope_pairs_long_bias", 2, 260, torch.float32, True, True),
])
def test_pk_self_bwd(dev, name, B, L, dtype, interleaved, bias):
    pk = _attn()
    g = _gen(31)
    x = torch.randn(B, L, 3 * E, generator=g).to(dtype)
    rope = None if interleaved is None else _Rope(interleaved=interleaved)
    kb = None
    if bias:
        kb = torch.zeros(B, L)
        kb[:, L - 7:] = -1e30
    go = torch.randn(B, L, E, generator=g)
    print(f"[pk_self_bwd] {name}", flush=True)
    xr = x.to(dev).requires_grad_(True)
    out = pk.pk_self_attention(xr, H, None if kb is None else kb.to(dev), rope, 16 ** -0.5)
    out.float().backward(go.to(dev))
    ref = O.pk_self_bwd_ref(x, H, kb, None if rope is None else _rope_np(rope, L), 16 ** -0.5, go.to(dtype))
    _check("dqkv", xr.grad, ref, dtype)


@pytest.mark.parametrize("name,B,L,dtype,interleaved", [
    ("self_bf16_rot8_halves", 8, 104, torch.bfloat16, False),
    ("self_fp32_rot8_pairs", 4, 100, torch.float32, True),
])
def test_pk_self_bwd_partial_rotary(dev, name, B, L, dtype, interleaved):
    # rotary embedding over the first 8 of each head's 16 dims: the tiled backward's generic RoPE
    pk = _attn()
    g = _gen(35)
    x = torch.randn(B, L, 3 * E, generator=g).to(dtype)
    rope = _Rope(dim=8, interleaved=interleaved)
    go = torch.randn(B, L, E, generator=g)
    print(f"[pk_self_bwd partial rotary] {name}", flush=True)
    xr = x.to(dev).requires_grad_(True)
    out = pk.pk_self_attention(xr, H, None, rope, 16 ** -0.5)
    out.float().backward(go.to(dev))
    ref = O.pk_self_bwd_ref(x, H, None, _rope_np(rope, L), 16 ** -0.5, go.to(dtype))
    _check("dqkv", xr.grad, ref, dtype)


@pytest.mark.parametrize("name,B,Lq,Lk,dtype,interleaved,shared_q", [
    ("cross_cls_bf16_rope", 16, 4, 104, torch.bfloat16, False, False),
    ("cross_col2_bf16", 4, 1024, 128, torch.bfloat16, None, False),
    ("cross_col1_bf16", 4, 128, 576, torch.bfloat16, None, False),
    ("cross_col2_fp32", 2, 4096, 128, torch.float32, None, False),
    ("cross_shared_q_bf16", 6, 128, 300, torch.bfloat16, None, True),   # ISAB inducing points
    ("cross_shared_q_fp32_rope", 3, 16, 50, torch.float32, True, True),
    ("cross_shared_q_bf16_short", 6, 128, 100, torch.bfloat16, None, True),
    ("cross_shared_q_bf16_rope_pairs", 3, 16, 50, torch.bfloat16, True, True),
])
def test_pk_cross_bwd(dev, name, B, Lq, Lk, dtype, interleaved, shared_q):
    pk = _attn()
    g = _gen(32)
    x = torch.randn(1 if shared_q else B, Lq, E, generator=g).to(dtype)
    y = torch.randn(B, Lk, 2 * E, generator=g).to(dtype)
    rope = None if interleaved is None else _Rope(interleaved=interleaved)
    go = torch.randn(B, Lq, E, generator=g)
    print(f"[pk_cross_bwd] {name}", flush=True)
    xr = x.to(dev).requires_grad_(True)
    yr = y.to(dev).requires_grad_(True)
    q_in = xr.expand(B, Lq, E) if shared_q else xr
    out = pk.pk_cross_attention(q_in, yr, H, None, rope, 16 ** -0.5)
    out.float().backward(go.to(dev))
    rq = None if rope is None else _rope_np(rope, Lq)
    rk = None if rope is None else _rope_np(rope, Lk)
    dq, dkv = O.pk_cross_bwd_ref(x, y, H, None, rq, rk, 16 ** -0.5, go.to(dtype))
    assert xr.grad.shape == x.shape
    _check("dq", xr.grad, dq, dtype)
    _check("dkv", yr.grad, dkv, dtype)


@pytest.mark.parametrize("Lq,Lk", [(24, 20), (40, 200)], ids=["fused_short", "tiled"])
def test_bwd_all_keys_masked_is_uniform(dev, Lq, Lk):
    # every key at -1e30: P is uniform (the reference's finite sentinel); gradients stay finite
    pk = _attn()
    g = _gen(33)
    B = 2
    q = (torch.randn(B, Lq, E, generator=g) * 0.25).to(torch.bfloat16)
    k = torch.randn(B, Lk, E, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Lk, E, generator=g).to(torch.bfloat16)
    kb = torch.full((B, Lk), -1e30)
    go = torch.randn(B, Lq, E, generator=g)
    qr, kr, vr = (t.to(dev).requires_grad_(True) for t in (q, k, v))
    out = pk.hx_attention(qr, kr, vr, H, kb.to(dev))
    out.float().backward(go.to(dev))
    for t in (qr, kr, vr):
        assert torch.isfinite(t.grad.float()).all()
    # uniform P: dv_j = (1 / Lk) sum_i dO_i for every key j (closed form)
    want_dv = go.to(torch.bfloat16).double().sum(dim=1, keepdim=True).expand(B, Lk, E).numpy() / Lk
    _check("dv", vr.grad, want_dv, torch.bfloat16)
    # dq, dk: the reference's formula with that uniform P (dS = P (dP - D) is not zero)
    dq, dk, _ = O.hx_bwd_ref(q, k, v, H, go.to(torch.bfloat16), kb)
    _check("dq", qr.grad, dq, torch.bfloat16)
    _check("dk", kr.grad, dk, torch.bfloat16)


def test_bwd_through_compiled_loss(dev):
    # the reference's training benchmark pattern: loss = out.float().square().mean(), twice in a row
    pk = _attn()
    g = _gen(34)
    q = (torch.randn(3, 256, E, generator=g) * 0.25).to(torch.bfloat16).to(dev).requires_grad_(True)
    k = torch.randn(3, 128, E, generator=g).to(torch.bfloat16).to(dev).requires_grad_(True)
    v = torch.randn(3, 128, E, generator=g).to(torch.bfloat16).to(dev).requires_grad_(True)
    grads = []
    for _ in range(2):
        q.grad = k.grad = v.grad = None
        pk.hx_attention(q, k, v, H).float().square().mean().backward()
        grads.append([t.grad.clone() for t in (q, k, v)])
    for a, b in zip(*grads):
        assert torch.equal(a, b)  # deterministic: no atomics
