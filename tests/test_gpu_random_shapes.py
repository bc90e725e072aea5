"""Seeded random shapes through every forward op family (hx, hxq, pk_self, pk_cross, the d = 64 ICL
attention) and the small-head backward (hx, pk_self, pk_cross through autograd), against the float64
oracle. Each case draws, from its own seed: batch size, query and key lengths (half the time one of the
kernels' route and tile boundaries: 1, 15-17, 31-33, 63-65, 96/97, 104, 112/113, 127-129, 255-257, 576,
1023-1025), valid lengths (incl. 0), a key mask (none, prefix, scattered finfo.min-like entries, finite
terms), a RoPE form (none, pairs, halves), bf16 or fp32 and the query sharpness. The draw is printed
before each launch. Bars: tests/parity.py's for the forwards (2e-2 / 1e-4 times max |ref| for bf16 /
fp32), with the absolute bar (2e-2 / 1e-4) taken times max(1, max |ref|): inputs drawn up to 2x N(0, 1)
give outputs up to ~5, where half an ulp of the bf16 output alone is 1.6e-2; for the gradients 2e-2 /
1e-4 times max(1, max |grad|), as in test_gpu_smallhead_bwd.py. The packed ops' oracle rounds q' and k'
to the input dtype where the reference's kernel does (`cast=`).
"""
import numpy as np
import pytest
import torch

from oracle import attention as O
from parity import ABS, check, errors

pytestmark = pytest.mark.gpu
H, E = 8, 128
EDGES = [1, 15, 16, 17, 31, 32, 33, 63, 64, 65, 96, 97, 104, 112, 113, 127, 128, 129, 255, 256, 257, 576,
         1023, 1024, 1025]
GTOL = {torch.bfloat16: 2e-2, torch.float32: 1e-4}
SEEDS = range(8)


class _Rope:
    """RotaryEmbedding stand-in (get_seq_pos / interleaved / freqs / forward)."""

    def __init__(self, interleaved):
        self.interleaved = interleaved
        self.freqs = torch.tensor(O.textbook_freqs(16, 100000.0), dtype=torch.float32)

    def get_seq_pos(self, L, device=None, dtype=torch.float32):
        return torch.arange(L, device=device, dtype=dtype)

    def forward(self, seq, seq_len=None):
        f = seq.float().unsqueeze(-1) * self.freqs.to(seq.device)
        return f.repeat_interleave(2, dim=-1)


def _len(rng, hi):
    if rng.random() < 0.5:
        c = [x for x in EDGES if x <= hi]
        return int(rng.choice(c))
    return int(rng.integers(1, hi + 1))


def _dtype(rng):
    return torch.bfloat16 if rng.random() < 0.65 else torch.float32


def _mask(rng, rows, L, g, allow_finite=True):
    kind = rng.choice(["none", "prefix", "scattered", "finite"] if allow_finite else ["none", "prefix", "scattered"])
    if kind == "none":
        return kind, None
    b = torch.zeros(rows, L)
    if kind == "prefix":
        for r in range(rows):
            b[r, int(rng.integers(1, L + 1)):] = -1e30
    elif kind == "scattered":
        b[torch.rand(rows, L, generator=g) < 0.15] = -1e30
    else:
        b = torch.randn(rows, L, generator=g) * 2.0
    return kind, b


def _rope(rng):
    r = rng.choice(["none", "pairs", "halves"])
    return r, (None if r == "none" else _Rope(r == "pairs"))


def _rope_np(rope, L):
    return None if rope is None else O.rope_tables_ref(rope.freqs.double().numpy(), L, E, H, rope.interleaved)


def _check(out, ref, dtype, what):
    _, scale = errors(out, ref)
    check(out, ref, dtype, what, abs_tol=ABS[dtype] * max(1.0, scale))


def _gcheck(name, got, ref, dtype):
    got = got.detach().double().cpu().numpy()
    scale = max(1.0, float(np.abs(ref).max()))
    err = float(np.abs(got - ref).max())
    print(f"  {name}: max abs err {err:.3e} (ref max {np.abs(ref).max():.3e})", flush=True)
    assert err <= GTOL[dtype] * scale, (name, err, scale)


@pytest.mark.parametrize("seed", SEEDS)
def test_hx_random(dev, seed):
    import tabicl_mi355_attn as pk
    rng = np.random.default_rng(7000 + seed)
    g = torch.Generator().manual_seed(7000 + seed)
    B, Lq, Lk, dtype = int(rng.integers(1, 5)), _len(rng, 1100), _len(rng, 2100), _dtype(rng)
    qs = float(rng.uniform(0.1, 1.0))
    kind, kb = _mask(rng, B, Lk, g)
    print(f"[random] hx seed={seed}: B={B} Lq={Lq} Lk={Lk} {dtype} mask={kind} q x{qs:.2f}", flush=True)
    q = (torch.randn(B, Lq, E, generator=g) * qs).to(dtype)
    k = torch.randn(B, Lk, E, generator=g).to(dtype)
    v = torch.randn(B, Lk, E, generator=g).to(dtype)
    out = pk.hx_attention(q.to(dev), k.to(dev), v.to(dev), H, None if kb is None else kb.to(dev))
    torch.cuda.synchronize()
    _check(out, O.hx_ref(q, k, v, H, kb), dtype, f"hx_random_{seed}")


@pytest.mark.parametrize("seed", SEEDS)
def test_hxq_random(dev, seed):
    import tabicl_mi355_attn as pk
    rng = np.random.default_rng(7100 + seed)
    g = torch.Generator().manual_seed(7100 + seed)
    B, Lq, Lk, dtype = int(rng.integers(1, 6)), _len(rng, 300), _len(rng, 9000), _dtype(rng)
    qs = float(rng.uniform(0.1, 1.0))
    valid = rng.integers(0, Lk + 1, B)
    if rng.random() < 0.3:
        valid[int(rng.integers(0, B))] = 0
    print(f"[random] hxq seed={seed}: B={B} Lq={Lq} Lk={Lk} {dtype} valid={valid.tolist()} q x{qs:.2f}", flush=True)
    q = (torch.randn(B, Lq, E, generator=g) * qs).to(dtype)
    kv = torch.randn(B, Lk, 2 * E, generator=g).to(dtype)
    kvn = kv.clone()
    for b in range(B):
        kvn[b, int(valid[b]):] = float("nan")  # never read
    out = pk.hxq_attention(q.to(dev), kvn.to(dev), torch.tensor(valid, dtype=torch.int32).to(dev), H)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    _check(out, O.hxq_ref(q, kv, valid, H), dtype, f"hxq_random_{seed}")


@pytest.mark.parametrize("seed", SEEDS)
def test_pk_self_random(dev, seed):
    import tabicl_mi355_attn as pk
    rng = np.random.default_rng(7200 + seed)
    g = torch.Generator().manual_seed(7200 + seed)
    B, L, dtype = int(rng.integers(1, 25)), _len(rng, 300), _dtype(rng)
    xs = float(rng.uniform(0.5, 2.0))
    rname, rope = _rope(rng)
    kind, kb = _mask(rng, B, L, g)
    print(f"[random] pk_self seed={seed}: B={B} L={L} {dtype} rope={rname} mask={kind} x{xs:.2f}", flush=True)
    x = (torch.randn(B, L, 3 * E, generator=g) * xs).to(dtype)
    out = pk.pk_self_attention(x.to(dev), H, None if kb is None else kb.to(dev), rope, 16 ** -0.5)
    torch.cuda.synchronize()
    _check(out, O.pk_self_ref(x, H, kb, _rope_np(rope, L), 16 ** -0.5, cast=dtype), dtype, f"pk_self_random_{seed}")


@pytest.mark.parametrize("seed", SEEDS)
def test_pk_cross_random(dev, seed):
    import tabicl_mi355_attn as pk
    rng = np.random.default_rng(7300 + seed)
    g = torch.Generator().manual_seed(7300 + seed)
    B, Lq, Lk, dtype = int(rng.integers(1, 13)), _len(rng, 600), _len(rng, 600), _dtype(rng)
    xs = float(rng.uniform(0.5, 2.0))
    rname, rope = _rope(rng)
    kind, kb = _mask(rng, B, Lk, g)
    shared = rng.random() < 0.3
    print(f"[random] pk_cross seed={seed}: B={B} Lq={Lq} Lk={Lk} {dtype} rope={rname} mask={kind} "
          f"shared_q={shared} x{xs:.2f}", flush=True)
    x = (torch.randn(1 if shared else B, Lq, E, generator=g) * xs).to(dtype)
    y = torch.randn(B, Lk, 2 * E, generator=g).to(dtype)
    xd = x.to(dev)
    out = pk.pk_cross_attention(xd.expand(B, Lq, E) if shared else xd, y.to(dev), H,
                                None if kb is None else kb.to(dev), rope, 16 ** -0.5)
    torch.cuda.synchronize()
    ref = O.pk_cross_ref(x, y, H, kb, _rope_np(rope, Lq), _rope_np(rope, Lk), 16 ** -0.5, cast=dtype)
    _check(out, ref, dtype, f"pk_cross_random_{seed}")


@pytest.mark.parametrize("seed", SEEDS)
def test_icl_random(dev, seed):
    import tabicl_mi355_icl as icl
    rng = np.random.default_rng(7400 + seed)
    g = torch.Generator().manual_seed(7400 + seed)
    N, Hh, Tq, Tkv, dtype = int(rng.integers(1, 4)), int(rng.integers(1, 9)), _len(rng, 700), _len(rng, 3000), \
        _dtype(rng)
    qs = float(rng.uniform(0.5, 4.0))
    valid = None if rng.random() < 0.5 else rng.integers(0, Tkv + 1, N)
    kind, kb = _mask(rng, N, Tkv, g)
    print(f"[random] icl seed={seed}: N={N} H={Hh} Tq={Tq} Tkv={Tkv} {dtype} "
          f"valid={None if valid is None else valid.tolist()} mask={kind} q x{qs:.2f}", flush=True)
    q = (torch.randn(N, Hh, Tq, 64, generator=g) * qs).to(dtype)
    k = torch.randn(N, Hh, Tkv, 64, generator=g).to(dtype)
    v = torch.randn(N, Hh, Tkv, 64, generator=g).to(dtype)
    vt = None if valid is None else torch.tensor(valid, dtype=torch.int32)
    out = icl.icl_sdpa(q.to(dev), k.to(dev), v.to(dev), None if vt is None else vt.to(dev),
                       None if kb is None else kb.to(dev))
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    _check(out, O.splash_sdpa_ref(q, k, v, vt, kb), dtype, f"icl_random_{seed}")


@pytest.mark.parametrize("seed", SEEDS)
def test_hx_bwd_random(dev, seed):
    import tabicl_mi355_attn as pk
    rng = np.random.default_rng(7500 + seed)
    g = torch.Generator().manual_seed(7500 + seed)
    B, Lq, Lk, dtype = int(rng.integers(1, 5)), _len(rng, 400), _len(rng, 1500), _dtype(rng)
    qs = float(rng.uniform(0.1, 0.6))
    kind, kb = _mask(rng, B, Lk, g, allow_finite=False)
    print(f"[random] hx_bwd seed={seed}: B={B} Lq={Lq} Lk={Lk} {dtype} mask={kind} q x{qs:.2f}", flush=True)
    q = (torch.randn(B, Lq, E, generator=g) * qs).to(dtype)
    k = torch.randn(B, Lk, E, generator=g).to(dtype)
    v = torch.randn(B, Lk, E, generator=g).to(dtype)
    go = torch.randn(B, Lq, E, generator=g)
    qr, kr, vr = (t.to(dev).requires_grad_(True) for t in (q, k, v))
    out = pk.hx_attention(qr, kr, vr, H, None if kb is None else kb.to(dev))
    out.float().backward(go.to(dev))
    dq, dk, dv = O.hx_bwd_ref(q, k, v, H, go.to(dtype), kb)
    _gcheck("dq", qr.grad, dq, dtype)
    _gcheck("dk", kr.grad, dk, dtype)
    _gcheck("dv", vr.grad, dv, dtype)


@pytest.mark.parametrize("seed", SEEDS)
def test_pk_self_bwd_random(dev, seed):
    import tabicl_mi355_attn as pk
    rng = np.random.default_rng(7600 + seed)
    g = torch.Generator().manual_seed(7600 + seed)
    B, L, dtype = int(rng.integers(1, 13)), _len(rng, 300), _dtype(rng)
    rname, rope = _rope(rng)
    kind, kb = _mask(rng, B, L, g, allow_finite=False)
    print(f"[random] pk_self_bwd seed={seed}: B={B} L={L} {dtype} rope={rname} mask={kind}", flush=True)
    x = torch.randn(B, L, 3 * E, generator=g).to(dtype)
    go = torch.randn(B, L, E, generator=g)
    xr = x.to(dev).requires_grad_(True)
    out = pk.pk_self_attention(xr, H, None if kb is None else kb.to(dev), rope, 16 ** -0.5)
    out.float().backward(go.to(dev))
    ref = O.pk_self_bwd_ref(x, H, kb, _rope_np(rope, L), 16 ** -0.5, go.to(dtype))
    _gcheck("dqkv", xr.grad, ref, dtype)


@pytest.mark.parametrize("seed", SEEDS)
def test_pk_cross_bwd_random(dev, seed):
    import tabicl_mi355_attn as pk
    rng = np.random.default_rng(7700 + seed)
    g = torch.Generator().manual_seed(7700 + seed)
    B, Lq, Lk, dtype = int(rng.integers(1, 9)), _len(rng, 500), _len(rng, 700), _dtype(rng)
    rname, rope = _rope(rng)
    shared = rng.random() < 0.4
    print(f"[random] pk_cross_bwd seed={seed}: B={B} Lq={Lq} Lk={Lk} {dtype} rope={rname} shared_q={shared}",
          flush=True)
    x = torch.randn(1 if shared else B, Lq, E, generator=g).to(dtype)
    y = torch.randn(B, Lk, 2 * E, generator=g).to(dtype)
    go = torch.randn(B, Lq, E, generator=g)
    xr = x.to(dev).requires_grad_(True)
    yr = y.to(dev).requires_grad_(True)
    out = pk.pk_cross_attention(xr.expand(B, Lq, E) if shared else xr, yr, H, None, rope, 16 ** -0.5)
    out.float().backward(go.to(dev))
    dq, dkv = O.pk_cross_bwd_ref(x, y, H, None, _rope_np(rope, Lq), _rope_np(rope, Lk), 16 ** -0.5, go.to(dtype))
    assert xr.grad.shape == x.shape
    _gcheck("dq", xr.grad, dq, dtype)
    _gcheck("dkv", yr.grad, dkv, dtype)
