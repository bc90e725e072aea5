"""GPU parity of the key-mask entry points against the CPU oracle: the ICL attention (head dim 64),
the few-query small-head attention (hxq) and the folded first-ISAB attention (hxf) with an additive
fp32 key mask, and the ICL cache's default valid length.

A prefix mask (0 on the first v keys, finfo.min or -inf after: what upstream builds from a tensor
train size, results/tpu_patch.diff:1526-1542) must give the same result as the valid length v, bit
for bit on the pipelined / streaming kernels (the device reads it as that length); any other mask
(random finite terms, scattered masked keys, a row masked everywhere) runs on the kernels that add it
term by term. Rows past the prefix hold NaN where the test says so: they must never be read.

Bars (tests/parity.py): max abs error <= 2e-2 for bf16 inputs, <= 1e-4 for fp32 inputs, and <= 2e-2
(bf16) / 1e-3 (fp32) times max |ref|.
"""
import numpy as np
import pytest
import torch

from oracle import attention as O
from parity import check

pytestmark = pytest.mark.gpu
FMIN = float(torch.finfo(torch.float32).min)
H, E = 8, 128


def _bias(kind, rows, L, g):
    b = torch.zeros(rows, L)
    if kind == "prefix":
        cut = [L - 1 - (r * 977) % (L // 2) for r in range(rows)]
        for r, c in enumerate(cut):
            b[r, c:] = FMIN
    elif kind == "prefix_inf":
        b[:, L // 3:] = float("-inf")
    elif kind == "random":
        b = torch.randn(rows, L, generator=g) * 2.0
        b[torch.rand(rows, L, generator=g) < 0.1] = FMIN
    elif kind == "mixed":  # row 0 prefix, row 1 random terms, row 2 masked everywhere, others all zero
        b[0, L // 2:] = FMIN
        b[1] = torch.randn(L, generator=g)
        if rows > 2:
            b[2] = FMIN
    return b


@pytest.mark.parametrize("name,N,Hh,Tq,Tkv,kind,rows,dtype", [
    ("prefix_shared_bf16", 2, 8, 300, 3000, "prefix", 1, torch.bfloat16),
    ("prefix_per_n_bf16", 3, 4, 200, 2500, "prefix", 3, torch.bfloat16),
    ("prefix_inf_bf16", 2, 8, 130, 1000, "prefix_inf", 1, torch.bfloat16),
    ("random_bf16", 2, 8, 300, 3000, "random", 2, torch.bfloat16),
    ("random_fp32", 2, 4, 100, 1000, "random", 1, torch.float32),
    ("mixed_rows_bf16", 3, 4, 256, 2000, "mixed", 3, torch.bfloat16),
    ("mixed_rows_fp32", 3, 2, 64, 700, "mixed", 3, torch.float32),
])
def test_icl_key_mask(dev, name, N, Hh, Tq, Tkv, kind, rows, dtype):
    import tabicl_mi355_icl as icl
    g = torch.Generator().manual_seed(60)
    q = torch.randn(N, Hh, Tq, 64, generator=g).to(dtype)
    k = torch.randn(N, Hh, Tkv, 64, generator=g).to(dtype)
    v = torch.randn(N, Hh, Tkv, 64, generator=g).to(dtype)
    b = _bias(kind, rows, Tkv, g)
    print(f"[keymask] icl {name}", flush=True)
    out = icl.icl_sdpa(q.to(dev), k.to(dev), v.to(dev), None, b.to(dev))
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    check(out, O.splash_sdpa_ref(q, k, v, None, b), dtype, "icl_key_mask")


def _scattered(case, N, Tkv, g):
    b = torch.zeros(N, Tkv)
    if case in ("scattered", "sharp", "key_split"):
        b[torch.rand(N, Tkv, generator=g) < 0.1] = FMIN
    elif case == "finite_terms":  # finite terms only, no key masked
        b = -4.0 * torch.rand(N, Tkv, generator=g)
    elif case == "head_masked":  # the first 40 keys masked (no reference from the first 32), then scattered
        b[:, :40] = FMIN
        b[torch.rand(N, Tkv, generator=g) < 0.05] = FMIN
    elif case == "inf_scattered":
        b[torch.rand(N, Tkv, generator=g) < 0.3] = float("-inf")
    elif case == "row_masked":  # row 0 masked everywhere (equal weights), row 1 scattered
        b[0] = FMIN
        b[1, torch.rand(Tkv, generator=g) < 0.5] = FMIN
    elif case == "nonpow2_scale":
        b[torch.rand(N, Tkv, generator=g) < 0.2] = -3.0
    return b


@pytest.mark.parametrize("case,N,Hh,Tq,Tkv,qscale", [
    ("scattered", 2, 8, 300, 3000, 1.0),
    ("sharp", 2, 8, 300, 3000, 6.0),
    ("finite_terms", 2, 8, 200, 2500, 3.0),
    ("head_masked", 2, 8, 256, 3000, 1.0),
    ("head_masked_sharp", 2, 8, 256, 3000, 8.0),
    ("inf_scattered", 3, 4, 130, 1000, 2.0),
    ("row_masked", 2, 8, 100, 1500, 2.0),
    ("key_split", 1, 2, 64, 20000, 4.0),
    ("nonpow2_scale", 2, 8, 200, 2000, 2.0),
])
def test_icl_scattered_mask_pipelined(dev, case, N, Hh, Tq, Tkv, qscale):
    # masks that are not prefix masks, bf16: with a power-of-two scale the pipelined kernel adds them as
    # the score product's accumulator input (rows that leave its trust range recomputed exactly); a
    # scale of 0.1 runs on the exact kernel. Sharp queries (x qscale) make the outputs O(0.3-1).
    import tabicl_mi355_icl as icl
    g = torch.Generator().manual_seed(64)
    q = (torch.randn(N, Hh, Tq, 64, generator=g) * qscale).to(torch.bfloat16)
    k = torch.randn(N, Hh, Tkv, 64, generator=g).to(torch.bfloat16)
    v = torch.randn(N, Hh, Tkv, 64, generator=g).to(torch.bfloat16)
    b = _scattered(case.replace("_sharp", ""), N, Tkv, g)
    print(f"[keymask] icl pipelined mask {case}: N={N} H={Hh} Tq={Tq} Tkv={Tkv}", flush=True)
    if case == "nonpow2_scale":
        out = icl.ICL_FWD(q.to(dev), k.to(dev), v.to(dev), None, 0.1, b.to(dev))
        ref = O.splash_sdpa_ref(q.double() * (0.1 / 0.125), k, v, None, b)
    else:
        out = icl.icl_sdpa(q.to(dev), k.to(dev), v.to(dev), None, b.to(dev))
        ref = O.splash_sdpa_ref(q, k, v, None, b)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    check(out, ref, torch.bfloat16, f"icl_pipelined_mask_{case}")


def test_icl_scattered_mask_with_valid_lengths(dev):
    # a scattered mask together with per-entry valid lengths (one of them 0): the masked instance runs to
    # the valid length, NaN keys past it are never read, the empty entry gives zeros
    import tabicl_mi355_icl as icl
    g = torch.Generator().manual_seed(65)
    N, Hh, Tq, Tkv = 4, 4, 150, 2600
    q = (torch.randn(N, Hh, Tq, 64, generator=g) * 3.0).to(torch.bfloat16)
    k = torch.randn(N, Hh, Tkv, 64, generator=g).to(torch.bfloat16)
    v = torch.randn(N, Hh, Tkv, 64, generator=g).to(torch.bfloat16)
    lens = [2600, 1777, 0, 65]
    kn, vn = k.clone(), v.clone()
    for n, L in enumerate(lens):
        kn[n, :, L:] = float("nan")
        vn[n, :, L:] = float("nan")
    b = torch.zeros(N, Tkv)
    b[torch.rand(N, Tkv, generator=g) < 0.15] = FMIN
    b[:, 1] = -2.5  # a finite term: no row is a prefix mask
    vt = torch.tensor(lens, dtype=torch.int32)
    print("[keymask] icl pipelined mask with valid lengths", flush=True)
    out = icl.icl_sdpa(q.to(dev), kn.to(dev), vn.to(dev), vt.to(dev), b.to(dev))
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    assert float(out[2].abs().max()) == 0.0
    check(out, O.splash_sdpa_ref(q, k, v, vt, b), torch.bfloat16, "icl_pipelined_mask_valid_lengths")


def test_icl_prefix_mask_is_the_valid_length(dev):
    # a prefix mask runs as the valid length on the pipelined kernel: identical bits to the length call,
    # and the NaN rows past the prefix are never read
    import tabicl_mi355_icl as icl
    g = torch.Generator().manual_seed(61)
    N, Hh, Tq, Tkv = 3, 8, 500, 6000
    q = torch.randn(N, Hh, Tq, 64, generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn(N, Hh, Tkv, 64, generator=g).to(torch.bfloat16)
    v = torch.randn(N, Hh, Tkv, 64, generator=g).to(torch.bfloat16)
    lens = [6000, 4321, 1]
    for n, L in enumerate(lens):
        k[n, :, L:] = float("nan")
        v[n, :, L:] = float("nan")
    k, v = k.to(dev), v.to(dev)
    b = torch.zeros(N, Tkv)
    for n, L in enumerate(lens):
        b[n, L:] = FMIN
    by_mask = icl.icl_sdpa(q, k, v, None, b.to(dev))
    by_len = icl.icl_sdpa(q, k, v, torch.tensor(lens, dtype=torch.int32, device=dev))
    assert torch.equal(by_mask, by_len)
    # with both: the shorter of the two
    b1 = torch.zeros(1, Tkv)
    b1[0, 3000:] = FMIN
    both = icl.icl_sdpa(q, k, v, torch.tensor(lens, dtype=torch.int32, device=dev), b1.to(dev))
    ref = icl.icl_sdpa(q, k, v, torch.tensor([min(L, 3000) for L in lens], dtype=torch.int32, device=dev))
    assert torch.equal(both, ref)


def test_icl_masked_view_of_block_output(dev):
    # the _out op with a key mask writes into a strided view of a [est, block, head, row, d] buffer
    import tabicl_mi355_icl as icl
    g = torch.Generator().manual_seed(62)
    q = torch.randn(2, 8, 90, 64, generator=g).to(torch.bfloat16)
    k = torch.randn(2, 8, 700, 64, generator=g).to(torch.bfloat16)
    v = torch.randn(2, 8, 700, 64, generator=g).to(torch.bfloat16)
    b = _bias("random", 2, 700, g)
    buf = torch.zeros(2, 3, 8, 90, 64, dtype=torch.bfloat16, device=dev)
    icl.ICL_FWD_OUT(q.to(dev), k.to(dev), v.to(dev), None, 0.125, buf[:, 1], b.to(dev))
    check(buf[:, 1], O.splash_sdpa_ref(q, k, v, None, b), torch.bfloat16, "icl_masked_view_of_block_output")
    assert float(buf[:, 0].abs().max()) == 0.0 and float(buf[:, 2].abs().max()) == 0.0


def test_icl_cache_default_length(dev):
    # 300 of 1000 rows appended into a NaN-filled cache: a query with no explicit length attends over them
    import tabicl_mi355_icl as icl
    g = torch.Generator().manual_seed(63)
    cache = icl.IclKVCache(2, 2, 8, 1000, 64, torch.bfloat16, dev)
    cache.keys.fill_(float("nan"))
    cache.values.fill_(float("nan"))
    k = torch.randn(2, 8, 300, 64, generator=g).to(torch.bfloat16)
    v = torch.randn(2, 8, 300, 64, generator=g).to(torch.bfloat16)
    cache.append(1, k[:, :, :200].to(dev), v[:, :, :200].to(dev))
    cache.append(1, k[:, :, 200:].to(dev), v[:, :, 200:].to(dev), row0=200)
    q = torch.randn(2, 8, 50, 64, generator=g).to(torch.bfloat16)
    out = cache.query(1, q.to(dev))
    assert cache.length(1) == 300
    assert torch.isfinite(out.float()).all()
    check(out, O.splash_sdpa_ref(q, k, v), torch.bfloat16, "icl_cache_default_length")
    with pytest.raises(ValueError):
        cache.query(0, q.to(dev))  # nothing appended to block 0


@pytest.mark.parametrize("name,B,Lq,Lk,kind,rows,valid,dtype", [
    ("stream_prefix_shared_bf16", 4, 128, 4096, "prefix", 1, None, torch.bfloat16),
    ("stream_prefix_per_b_bf16", 3, 128, 3000, "prefix", 3, None, torch.bfloat16),
    ("stream_mixed_bf16", 4, 128, 2048, "mixed", 4, None, torch.bfloat16),
    ("stream_prefix_and_valid_bf16", 3, 64, 1500, "prefix", 1, [1500, 700, 0], torch.bfloat16),
    ("resident_random_bf16", 3, 200, 100, "random", 3, None, torch.bfloat16),
    ("fp32_random", 3, 128, 1000, "random", 3, None, torch.float32),
    ("fp32_prefix", 2, 128, 700, "prefix", 1, None, torch.float32),
])
def test_hxq_key_mask(dev, name, B, Lq, Lk, kind, rows, valid, dtype):
    import tabicl_mi355_attn as pk
    g = torch.Generator().manual_seed(64)
    q = (torch.randn(B, Lq, E, generator=g) * 0.25).to(dtype)
    kv = torch.randn(B, Lk, 2 * E, generator=g).to(dtype)
    b = _bias(kind, rows, Lk, g)
    if kind == "mixed":
        b[2, : Lk // 4] = 0.0  # keep one unmasked key block in the masked-everywhere row: finite softmax in fp64
    vt = None if valid is None else torch.tensor(valid, dtype=torch.int32, device=dev)
    print(f"[keymask] hxq {name}", flush=True)
    out = pk.hxq_attention(q.to(dev), kv.to(dev), vt, H, b.to(dev))
    torch.cuda.synchronize()
    ref = O.attention_f64(q.double().numpy(), kv[..., :E].double().numpy(), kv[..., E:].double().numpy(), H,
                          np.broadcast_to(b.double().numpy(), (B, Lk)), valid=None if valid is None else np.array(valid))
    assert torch.isfinite(out.float()).all()
    check(out, ref, dtype, "hxq_key_mask")


def test_hxq_prefix_mask_is_the_valid_length(dev):
    import tabicl_mi355_attn as pk
    g = torch.Generator().manual_seed(65)
    B, Lq, Lk = 6, 128, 53248
    q = (torch.randn(B, Lq, E, generator=g) * 0.25).to(torch.bfloat16).to(dev)
    kv = torch.randn(B, Lk, 2 * E, generator=g).to(torch.bfloat16)
    kv[:, 45000:] = float("nan")  # the reference's inference shape: 53,248 padded rows, 45,000 train rows
    kv = kv.to(dev)
    b = torch.zeros(1, Lk)
    b[0, 45000:] = FMIN
    by_mask = pk.hxq_attention(q, kv, None, H, b.to(dev))
    by_len = pk.hxq_attention(q, kv, torch.tensor(45000, dtype=torch.int32, device=dev), H)
    assert torch.equal(by_mask, by_len)


@pytest.mark.parametrize("dtype,kind", [(torch.float32, "prefix"), (torch.float32, "random"),
                                        (torch.bfloat16, "prefix"), (torch.bfloat16, "random")])
def test_hxf_key_mask(dev, dtype, kind):
    import tabicl_mi355_attn as pk
    g = torch.Generator().manual_seed(66)
    B, hq, Lk = 3, 256, 900
    qf = (torch.randn(1, hq, E, generator=g) * 0.05).to(dtype)
    x = torch.randn(B, Lk, E, generator=g).to(dtype)
    b = _bias(kind, B, Lk, g)
    out = pk.hxf_attention(qf[0].to(dev), x.to(dev), None, b.to(dev))
    ref = O.attention_f64(np.broadcast_to(qf.double().numpy(), (B, hq, E)), x.double().numpy(), x.double().numpy(),
                          1, b.double().numpy())
    check(out, ref, dtype, "hxf_key_mask")
