"""GPU parity of the cached ICL query loop (IclKVCache.query_blocks: the loop of the reference's
scripts/tabicl_tpu_bucketed.py:803-817 around the attention kernel) against a CPU restatement.

The restatement follows the same dtype flow as the GPU path and the reference's bf16 autocast of the ICL
stage: LayerNorm in fp32 (SafeLayerNorm, results/tpu_patch.diff:1385-1397), every GEMM on bf16 inputs
with its output rounded to bf16, the residual stream in fp32, the attention from oracle.splash_sdpa_ref
(fp64) on the bf16 q and cache, rounded to bf16. So the two sides differ by GEMM accumulation order and
the kernel's own error (its bar: 2e-2 abs). Bar here (written here): max abs error <= 2e-2 x max(1, max
|reference|) after two blocks, since the residual stream grows and each GEMM output is a bf16 value of
that magnitude.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as O

pytestmark = pytest.mark.gpu
H, D = 8, 64
W = H * D


def _bf(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.bfloat16).float()


def _weights(nb: int, ff: int, g):
    import tabicl_mi355_icl as icl
    out = []
    for _ in range(nb):
        def lin(o, i):
            return (torch.randn(o, i, generator=g) * i ** -0.5).to(torch.bfloat16), \
                   (torch.randn(o, generator=g) * 0.1).to(torch.bfloat16)
        in_w, in_b = lin(3 * W, W)
        out_w, out_b = lin(W, W)
        f1w, f1b = lin(ff, W)
        f2w, f2b = lin(W, ff)
        out.append(icl.IclBlockWeights(1 + 0.1 * torch.randn(W, generator=g), 0.1 * torch.randn(W, generator=g), in_w,
                                       in_b, out_w, out_b, 1 + 0.1 * torch.randn(W, generator=g),
                                       0.1 * torch.randn(W, generator=g), f1w, f1b, f2w, f2b))
    return out


def _to(w, dev):
    import dataclasses
    return dataclasses.replace(w, **{f.name: getattr(w, f.name).to(dev) for f in dataclasses.fields(w)
                                     if isinstance(getattr(w, f.name), torch.Tensor)})


def _ssmax_standin(n: float, g):
    a = 0.05 * torch.randn(H, 1, D, generator=g)
    return a, (lambda q, _a=a: q * (1.0 + _a.to(q.device, q.dtype) * float(np.log(n))))


def _reference(x, blocks, kc, vc, valid, a):
    """CPU restatement of query_blocks with the GPU path's rounding points."""
    x = x.float()
    E_, Tq = x.shape[0], x.shape[1]
    for b, w in enumerate(blocks):
        h = _bf(F.layer_norm(x, (W,), w.ln1_w.float(), w.ln1_b.float(), w.eps))
        q = _bf(h @ w.in_w[:W].float().T + w.in_b[:W].float())
        q = q.view(E_, Tq, H, D).transpose(1, 2)
        q = _bf(q * (1.0 + _bf(a) * float(np.log(valid))))
        att = O.splash_sdpa_ref(q, kc[:, b].float(), vc[:, b].float(), valid)  # fp64 [E, H, Tq, D]
        att = _bf(torch.from_numpy(att).float()).transpose(1, 2).reshape(E_, Tq, W)
        x = x + _bf(att @ w.out_w.float().T + w.out_b.float())
        h = _bf(F.layer_norm(x, (W,), w.ln2_w.float(), w.ln2_b.float(), w.eps))
        f = _bf(F.gelu(_bf(h @ w.ff1_w.float().T + w.ff1_b.float())))
        x = x + _bf(f @ w.ff2_w.float().T + w.ff2_b.float())
    return x


def test_query_blocks_matches_restatement(dev):
    import tabicl_mi355_icl as icl
    g = torch.Generator().manual_seed(80)
    E_, NB, cap, train, Tq, ff = 2, 2, 1200, 1000, 300, 2 * W
    cache = icl.IclKVCache(E_, NB, H, cap, D, torch.bfloat16, dev)
    kc = torch.randn(E_, NB, H, train, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(E_, NB, H, train, D, generator=g).to(torch.bfloat16)
    for b in range(NB):
        cache.append(b, kc[:, b].to(dev), vc[:, b].to(dev))
    blocks = _weights(NB, ff, g)
    a, ssmax = _ssmax_standin(train, g)
    x = torch.randn(E_, Tq, W, generator=g)
    print("[icl_stage] 2 blocks", flush=True)
    with torch.no_grad():
        got = cache.query_blocks(x.to(dev), [_to(w, dev) for w in blocks], q_transform=ssmax)
    torch.cuda.synchronize()
    assert cache.length(0) == train and got.dtype == torch.float32
    ref = _reference(x, blocks, kc, vc, train, a)
    err = float((got.cpu() - ref).abs().max())
    assert torch.isfinite(got).all()
    assert err <= 2e-2 * max(1.0, float(ref.abs().max())), err


def test_attention_layer_strided_q_and_merged_output(dev):
    # attention_layer hands the kernel q as a strided head view and takes its output in merged-head order:
    # equal to the same attention computed on contiguous copies
    import tabicl_mi355_icl as icl
    g = torch.Generator().manual_seed(81)
    cache = icl.IclKVCache(2, 1, H, 700, D, torch.bfloat16, dev)
    cache.append(0, torch.randn(2, H, 700, D, generator=g).to(torch.bfloat16).to(dev),
                 torch.randn(2, H, 700, D, generator=g).to(torch.bfloat16).to(dev))
    w_in = (torch.randn(3 * W, W, generator=g) * W ** -0.5).to(torch.bfloat16).to(dev)
    w_out = (torch.randn(W, W, generator=g) * W ** -0.5).to(torch.bfloat16).to(dev)
    x = torch.randn(2, 130, W, generator=g).to(torch.bfloat16).to(dev)
    with torch.no_grad():
        got = cache.attention_layer(0, x, w_in, None, w_out, None, 650)
        q = F.linear(x, w_in[:W]).view(2, 130, H, D).transpose(1, 2).contiguous()
        o = icl.icl_sdpa(q, cache.keys[:, 0], cache.values[:, 0], 650).transpose(1, 2).reshape(2, 130, W)
        want = F.linear(o, w_out)
    assert torch.equal(got, want)


@pytest.mark.parametrize("max_fused", [40959, 10 ** 9])
def test_bucketed_dispatch_matches_unpadded_call(dev, max_fused):
    # The reference runner's call pattern around the ICL stage (scripts/tabicl_tpu_bucketed.py:1298-1382):
    # batch and test rows padded to their buckets (padded batch elements repeat element 0), the batch cut
    # into ICL calls by the plan (one estimator per call for max_fused 40959, all four in one for 1e9),
    # the real part sliced out. Here the same real rows come from one unpadded call over the real batch;
    # both match the CPU restatement (same bar as above), and the padded element matches element 0.
    import tabicl_mi355_buckets as bk
    import tabicl_mi355_icl as icl
    g = torch.Generator().manual_seed(82)
    pre = bk.plan_prefill(3, 700, 10)
    plan = bk.plan_query(pre, 300, max_fused_elements=max_fused)
    assert (pre.batch_bkt, pre.train_bkt, plan.rows_bkt) == (4, 1024, 512)
    assert plan.icl_step == (1 if max_fused < 40960 else 4)
    NB, ff = 2, 2 * W
    cache = icl.IclKVCache(pre.batch_bkt, NB, H, pre.train_bkt, D, torch.bfloat16, dev)
    kc = torch.randn(3, NB, H, 700, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(3, NB, H, 700, D, generator=g).to(torch.bfloat16)
    kp, vp = torch.cat([kc, kc[:1]]), torch.cat([vc, vc[:1]])  # the padded estimator's K/V repeat element 0's
    for b in range(NB):
        cache.append(b, kp[:, b].to(dev), vp[:, b].to(dev))
    blocks = [_to(w, dev) for w in _weights(NB, ff, g)]
    x = torch.randn(3, 300, W, generator=g)
    xp = bk.pad_batch(x, plan, pad_features=False)
    print(f"[icl_stage] bucketed dispatch, chunks {plan.chunks()}", flush=True)
    with torch.no_grad():
        raw = cache.query_chunked(xp.to(dev), blocks, plan.chunks())
        padded = bk.unpad_output(raw, plan)
        direct = cache.estimators(0, 3).query_blocks(x.to(dev), blocks)
    torch.cuda.synchronize()
    assert raw.shape == (4, 512, W) and padded.shape == direct.shape == (3, 300, W)
    ref = _reference(x, [_cpu(w) for w in blocks], kc, vc, 700, torch.zeros(H, 1, D))
    bar = 2e-2 * max(1.0, float(ref.abs().max()))
    for got in (padded, direct):
        assert torch.isfinite(got).all()
        assert float((got.cpu() - ref).abs().max()) <= bar
    assert float((padded - direct).abs().max()) <= bar
    assert float((raw[3] - raw[0]).abs().max()) <= bar


def _cpu(w):
    import dataclasses
    return dataclasses.replace(w, **{f.name: getattr(w, f.name).cpu() for f in dataclasses.fields(w)
                                     if isinstance(getattr(w, f.name), torch.Tensor)})
