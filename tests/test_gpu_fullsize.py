"""GPU checks at BASELINE's full sizes for the fp32 column attention (C1), the row attention (C2) and
both column ISAB legs (C3), configs that the other GPU tests run at reduced batch: the fp64 oracle on sampled sequences, and over
the whole output the size-independent properties of softmax attention: every output is finite and,
per head and dimension, lies between the smallest and largest value of V over the keys (a convex
combination), and a bit-identical rerun. Inputs come from a device generator (the CPU oracle gets
copies of the sampled sequences only).

Bar (written here): max abs error <= 2e-2 against the oracle (bf16 inputs), <= 1e-4 (fp32 inputs);
hull with 2e-2 slack for the bf16 rounding of the output (1e-4 for fp32).
"""
import pytest
import torch

from oracle import attention as O

pytestmark = pytest.mark.gpu
H, E = 8, 128


class _Rope:
    interleaved = False

    def __init__(self):
        self.freqs = 10000.0 ** (-torch.arange(0, 16, 2, dtype=torch.float32) / 16)

    def get_seq_pos(self, L, device=None, dtype=torch.float32):
        return torch.arange(L, device=device, dtype=dtype)


def _hull_ok(out, v, tol=2e-2):
    # out [B, Lq, E], v [B, Lk, E]: per (batch, dim) the output lies within V's range over the keys
    vmax = v.float().amax(dim=1, keepdim=True)
    vmin = v.float().amin(dim=1, keepdim=True)
    return bool((out.float() <= vmax + tol).all()) and bool((out.float() >= vmin - tol).all())


def test_c2_row_stage_full_size(dev):
    import numpy as np

    import tabicl_mi355_attn as pk
    g = torch.Generator(device=dev).manual_seed(1)
    B, L = 16384, 104
    qkv = torch.randn(B, L, 3 * E, generator=g, device=dev).to(torch.bfloat16)
    rope = _Rope()
    print("[fullsize] c2", flush=True)
    with torch.no_grad():
        out = pk.pk_self_attention(qkv, H, None, rope, 0.25)
        again = pk.pk_self_attention(qkv, H, None, rope, 0.25)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    assert torch.equal(out, again)
    assert _hull_ok(out, qkv[..., 2 * E:])
    tables = O.rope_tables_ref(rope.freqs.double().numpy(), L, E, H, False)
    for b in (0, 1, 4097, 9999, B - 1):
        ref = O.pk_self_ref(qkv[b:b + 1].cpu(), H, None, tables, 0.25)
        err = float(np.abs(out[b:b + 1].double().cpu().numpy() - ref).max())
        assert err <= 2e-2, (b, err)


def test_c3_isab2_full_size(dev):
    import numpy as np

    import tabicl_mi355_attn as pk
    g = torch.Generator(device=dev).manual_seed(2)
    B, T, NI = 800, 50000, 128
    q = torch.randn(B, T, E, generator=g, device=dev).to(torch.bfloat16)
    kv = torch.randn(B, NI, 2 * E, generator=g, device=dev).to(torch.bfloat16)
    print("[fullsize] c3 isab2", flush=True)
    with torch.no_grad():
        out = pk.pk_cross_attention(q, kv, H, None, None, 0.25)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    assert _hull_ok(out, kv[..., E:])
    rows = torch.arange(0, T, 997)
    for b in (0, 399, B - 1):
        ref = O.pk_cross_ref(q[b:b + 1, rows].cpu(), kv[b:b + 1].cpu(), H, None, None, None, 0.25)
        err = float(np.abs(out[b:b + 1, rows].double().cpu().numpy() - ref).max())
        assert err <= 2e-2, (b, err)
    del q, out


def test_c3_isab1_full_size(dev):
    # 800 sequences x 128 inducing queries over 50,000 rows of packed K|V, 45,000 valid; the rows past
    # the valid length hold NaN (never read). Hull over the valid keys, computed in bf16 (no fp32 copy).
    import numpy as np

    import tabicl_mi355_attn as pk
    g = torch.Generator(device=dev).manual_seed(3)
    B, T, VALID, NI = 800, 50000, 45000, 128
    q = (torch.randn(B, NI, E, generator=g, device=dev) * 0.25).to(torch.bfloat16)
    kv = torch.randn(B, T, 2 * E, generator=g, device=dev).to(torch.bfloat16)
    kv[:, VALID:] = float("nan")
    vt = torch.tensor([VALID], dtype=torch.int32, device=dev)
    print("[fullsize] c3 isab1", flush=True)
    with torch.no_grad():
        out = pk.hxq_attention(q, kv, vt, H)
        again = pk.hxq_attention(q, kv, vt, H)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    assert torch.equal(out, again)
    vmax = kv[:, :VALID, E:].amax(dim=1, keepdim=True).float()
    vmin = kv[:, :VALID, E:].amin(dim=1, keepdim=True).float()
    assert bool((out.float() <= vmax + 2e-2).all()) and bool((out.float() >= vmin - 2e-2).all())
    for b in (0, 399, B - 1):
        ref = O.hxq_ref(q[b:b + 1].cpu(), kv[b:b + 1, :VALID].cpu(), np.array([VALID]), H)
        err = float(np.abs(out[b:b + 1].double().cpu().numpy() - ref).max())
        assert err <= 2e-2, (b, err)
    del q, kv, out, again


@pytest.mark.parametrize("leg", ["isab1", "isab2"])
def test_c1_fp32_full_size(dev, leg):
    # BASELINE config 1 in fp32: 400 sequences, ISAB-1 = 128 queries over 1,024 keys (the streaming
    # kernel), ISAB-2 = 1,024 queries over 128 keys (the resident kernel), q pre-scaled by 1/4
    import numpy as np

    import tabicl_mi355_attn as pk
    g = torch.Generator(device=dev).manual_seed(4)
    B = 400
    Lq, Lk = (128, 1024) if leg == "isab1" else (1024, 128)
    q = torch.randn(B, Lq, E, generator=g, device=dev) * 0.25
    k = torch.randn(B, Lk, E, generator=g, device=dev)
    v = torch.randn(B, Lk, E, generator=g, device=dev)
    print(f"[fullsize] c1 {leg}", flush=True)
    with torch.no_grad():
        out = pk.hx_attention(q, k, v, H)
        again = pk.hx_attention(q, k, v, H)
    torch.cuda.synchronize()
    assert out.dtype == torch.float32 and torch.isfinite(out).all()
    assert torch.equal(out, again)
    assert bool((out <= v.amax(dim=1, keepdim=True) + 1e-4).all())
    assert bool((out >= v.amin(dim=1, keepdim=True) - 1e-4).all())
    for b in (0, 199, B - 1):
        ref = O.hx_ref(q[b:b + 1].cpu(), k[b:b + 1].cpu(), v[b:b + 1].cpu(), H)
        err = float(np.abs(out[b:b + 1].double().cpu().numpy() - ref).max())
        assert err <= 1e-4, (b, err)


def test_c5_ragged_buckets_full_size(dev):
    # BASELINE config 5 as bench.py draws it (64 tables, seed-fixed sizes): every ICL bucket at its full
    # shape (8 estimators x 8 heads per table, test rows padded to 1k over the train bucket, per-table
    # valid and test-row counts), and the column ISAB-2 buckets up to 4k rows (8 estimators x 100
    # features per table, per-sequence row counts). The ragged call's live rows equal the padded call's
    # bit for bit; sampled tables match the oracle; live outputs are finite.
    import numpy as np

    import bench
    import tabicl_mi355_attn as pk
    import tabicl_mi355_icl as icl
    n_train, n_test = bench.c5_tables()
    groups = {}
    for i in range(64):
        groups.setdefault(("isab", bench.c5_bucket(int(n_train[i] + n_test[i]))), []).append(i)
        groups.setdefault(("icl", bench.c5_bucket(int(n_train[i]))), []).append(i)
    g = torch.Generator(device=dev).manual_seed(5)
    for (kind, L), tabs in sorted(groups.items()):
        nt = [int(n_train[i]) for i in tabs]
        ns = [int(n_test[i]) for i in tabs]
        print(f"[fullsize] c5 {kind} bucket {L}: {len(tabs)} tables", flush=True)
        if kind == "icl":
            N, Tq = len(tabs) * 8, 1024
            valid = torch.tensor(nt, dtype=torch.int32).repeat_interleave(8).to(dev)
            qlen = torch.tensor(ns, dtype=torch.int32).repeat_interleave(8).to(dev)
            k = torch.randn(N, H, L, 64, generator=g, device=dev, dtype=torch.bfloat16)
            v = torch.randn(N, H, L, 64, generator=g, device=dev, dtype=torch.bfloat16)
            q = torch.randn(N, H, Tq, 64, generator=g, device=dev, dtype=torch.bfloat16)
            padded, ragged = torch.empty_like(q), torch.zeros_like(q)
            with torch.no_grad():
                icl.ICL_FWD_OUT(q, k, v, valid, 64 ** -0.5, padded)
                icl.ICL_FWD_RAGGED_OUT(q, k, v, valid, qlen, 64 ** -0.5, ragged)
            torch.cuda.synchronize()
            for n in range(N):
                m = ns[n // 8]
                assert torch.equal(ragged[n, :, :m], padded[n, :, :m]), (L, n)
                assert torch.isfinite(ragged[n, :, :m].float()).all()
            for n in (0, N - 1):
                m, vl = ns[n // 8], nt[n // 8]
                ref = O.splash_sdpa_ref(q[n:n + 1, :2, :m].cpu(), k[n:n + 1, :2].cpu(), v[n:n + 1, :2].cpu(),
                                        np.array([vl]))
                err = float(np.abs(ragged[n:n + 1, :2, :m].double().cpu().numpy() - ref).max())
                assert err <= 2e-2, (L, n, err)
            del k, v, q, padded, ragged
        elif L <= 4096:
            B = len(tabs) * 800
            rows = [a + b for a, b in zip(nt, ns)]
            qlen = torch.tensor(rows, dtype=torch.int32).repeat_interleave(800).to(dev)
            q2 = torch.randn(B, L, E, generator=g, device=dev, dtype=torch.bfloat16)
            kv2 = torch.randn(B, 128, 2 * E, generator=g, device=dev, dtype=torch.bfloat16)
            with torch.no_grad():
                padded = pk.pk_cross_attention(q2, kv2, H, None, None, 0.25)
                ragged = pk.pk_cross_attention(q2, kv2, H, None, None, 0.25, q_len=qlen)
            torch.cuda.synchronize()
            for t, r in enumerate(rows):
                sl = slice(800 * t, 800 * (t + 1))
                assert torch.equal(ragged[sl, :r], padded[sl, :r]), (L, t)
            for b in (0, B - 1):
                r = rows[b // 800]
                sel = torch.arange(0, r, 7)
                ref = O.pk_cross_ref(q2[b:b + 1, sel].cpu(), kv2[b:b + 1].cpu(), H, None, None, None, 0.25)
                err = float(np.abs(ragged[b:b + 1, sel].double().cpu().numpy() - ref).max())
                assert err <= 2e-2, (L, b, err)
            del q2, kv2, padded, ragged
        torch.cuda.empty_cache()
